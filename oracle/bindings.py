"""ctypes bindings for the CPU oracle (liboracle.so) and the compiled reference
(oracle/_ref/libref_*.so).  TEST INFRASTRUCTURE ONLY — see oracle/__init__.py.

All wrappers take and return numpy arrays; sizes are checked on the Python
side so a wrong call raises instead of reading past a buffer.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))


def oracle_lib_path() -> str:
    """liboracle.so, or the build MYTHOS_ORACLE_LIB names (the sanitizer
    build of `make -C oracle sanitize`)."""
    return os.environ.get("MYTHOS_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")


def ref_lib_path(variant: str = "avx2") -> str:
    return os.path.join(_HERE, "_ref", f"libref_{variant}.so")


def build(with_ref: bool | None = None) -> None:
    """Compile liboracle.so and, when the reference tree exists, oracle/_ref."""
    subprocess.run(["make", "-s", "-C", _HERE, "oracle"], check=True)
    ref_root = os.environ.get("MYTHOS_REFERENCE", "/root/reference")
    if with_ref is None:
        with_ref = os.path.isdir(os.path.join(ref_root, "src"))
    if with_ref:
        subprocess.run(["make", "-s", "-C", _HERE, "ref", f"REF={ref_root}", "-j4"], check=True)


def _p(a: np.ndarray, dtype) -> C.c_void_p:
    assert a.dtype == dtype, (a.dtype, dtype)
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


def i2s_bytes(M: int, K: int) -> int:
    """Bytes the i2s_gemm family reads: row m at m*(K/4), element k at byte
    k/4 of the row (src/kernel_i2s.cpp:54,207)."""
    return (M - 1) * (K // 4) + (K - 1) // 4 + 1


def _need(a: np.ndarray, n: int, name: str) -> None:
    if a.size < n:
        raise ValueError(f"{name}: {a.size} elements < {n} required")


I64, I32, F32, U64 = C.c_int64, C.c_int, C.c_float, C.c_uint64
VP = C.c_void_p


class DecoderConfig(C.Structure):
    _fields_ = [(n, C.c_int64) for n in ("vocab", "hidden", "layers", "heads", "kv_heads", "head_dim", "ffn",
                                         "max_seq", "cb_block")] + [("eps", C.c_float), ("theta", C.c_float),
                                                                    ("kv_bf16", C.c_int64)]


class DecoderLayer(C.Structure):
    _fields_ = [("attn_norm", VP), ("ffn_norm", VP), ("wq", VP), ("wk", VP), ("wv", VP), ("wo", VP),
                ("cbq", VP), ("cbk", VP), ("cbv", VP), ("cbo", VP), ("wgate", VP), ("wup", VP),
                ("cbgate", VP), ("cbup", VP), ("wdown", VP), ("down_scale", C.c_float)]


class DecoderModel(C.Structure):
    _fields_ = [("emb", VP), ("final_norm", VP), ("lm_idx", VP), ("lm_cb", VP), ("rope_cos", VP),
                ("rope_sin", VP), ("layers", C.POINTER(DecoderLayer))]


DECODER_CONFIG_KEYS = ("vocab", "hidden", "layers", "heads", "kv_heads", "head_dim", "ffn", "max_seq",
                       "cb_block", "eps", "theta")


class Oracle:
    """The C restatement (oracle.c, decoder.c)."""

    def __init__(self, path: str | None = None):
        path = path or oracle_lib_path()
        if not os.path.exists(path):
            build(with_ref=False)
        self.lib = L = C.CDLL(path)
        sig = {
            "orc_fp16_to_float_n": [VP, VP, I64],
            "orc_oil8_gemm_scalar": [VP, VP, VP, VP, I64, I64, I64],
            "orc_oil8_gemm_avx2": [VP, VP, VP, VP, I64, I64, I64],
            "orc_oil8_gemv": [VP, VP, VP, VP, I64, I64, I64, I32],
            "orc_oil4_gemm_scalar": [VP, VP, VP, VP, I64, I64, I64],
            "orc_oil4_gemm_avx2": [VP, VP, VP, VP, I64, I64, I64],
            "orc_oil4_gemv_blocked": [VP, VP, I64, VP, VP, I64, I64, I64, I32],
            "orc_quantize_per_token": [VP, VP, I64, I64, VP, VP],
            "orc_dequantize_per_tensor": [VP, VP, I64, F32],
            "orc_i2s_gemv": [VP, F32, VP, F32, VP, I64],
            "orc_i2s_gemm": [VP, VP, VP, I64, I64, I64],
            "orc_i2s_gemm_vnni": [VP, VP, VP, I64, I64, I64],
            "orc_i2s_gemv_f32": [VP, F32, VP, VP, I64, I64, I64, I32],
            "orc_tl1_gemm": [VP, VP, VP, I64, I64, I64],
            "orc_tl2_gemm": [VP, VP, VP, I64, I64, I64],
            "orc_tl1_precompute_lut": [VP, VP, I64],
            "orc_tl2_precompute_lut": [VP, VP, I64],
            "orc_gemv": [F32, VP, VP, F32, VP, I64, I64],
            "orc_gemm": [F32, VP, VP, F32, VP, I64, I64, I64],
            "orc_relu": [VP, VP, I64],
            "orc_gelu": [VP, VP, I64],
            "orc_scale": [F32, VP, VP, I64],
            "orc_layer_norm": [VP, VP, VP, F32, VP, I64, I64],
            "orc_softmax_axis": [VP, VP, I64, I64, I64],
            "orc_rms_norm": [VP, VP, F32, VP, I64, I64],
            "orc_silu": [VP, VP, I64],
            "orc_oil4_gemm_prefill": [VP, VP, VP, I64, VP, VP, I64, I64, I64, I32],
            "orc_softmax": [VP, VP, I64, I64],
            "orc_add": [VP, VP, VP, I64],
            "orc_mul": [VP, VP, VP, I64],
            "orc_silu_mul": [VP, VP, VP, I64],
            "orc_rope_tables": [I64, I64, F32, VP, VP],
            "orc_rope_apply": [VP, I64, I64, I64, VP, VP],
            "orc_attention_decode": [VP, VP, VP, VP, I64, I64, I64, I64, I64],
            "orc_decoder_step": [C.POINTER(DecoderConfig), C.POINTER(DecoderModel), VP, VP, I64, I32, VP, I32, I32],
            "orc_decoder_attn_half": [C.POINTER(DecoderConfig), C.POINTER(DecoderModel), I64, VP, VP, I64, VP, I32,
                                      I32],
            "orc_i2s_gemv_rows": [VP, F32, VP, F32, VP, I64, I64, I32],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = None
        L.orc_bf16_round.argtypes = [F32]
        L.orc_bf16_round.restype = F32
        L.orc_fp16_to_float.argtypes = [C.c_uint16]
        L.orc_fp16_to_float.restype = F32
        L.orc_half_to_float_codebook.argtypes = [C.c_uint16]
        L.orc_half_to_float_codebook.restype = F32
        L.orc_float_to_half_trunc.argtypes = [F32]
        L.orc_float_to_half_trunc.restype = C.c_uint16
        L.orc_rng_seed.argtypes = [VP, U64]
        L.orc_rng_next_u64.argtypes = [VP]
        L.orc_rng_next_u64.restype = U64
        L.orc_rng_uniform.argtypes = [VP]
        L.orc_rng_uniform.restype = F32
        L.orc_rng_normal.argtypes = [VP]
        L.orc_rng_normal.restype = F32
        L.orc_rng_uniform_int.argtypes = [VP, I32, I32]
        L.orc_rng_uniform_int.restype = I32
        L.orc_argmax.argtypes = [VP, I64]
        L.orc_argmax.restype = I32

    # -- rng ---------------------------------------------------------------
    def _rng(self, seed):
        st = (C.c_uint64 * 2)()
        self.lib.orc_rng_seed(C.cast(st, VP), seed)
        return st

    def rng_u64(self, seed: int, n: int) -> np.ndarray:
        st = self._rng(seed)
        return np.array([self.lib.orc_rng_next_u64(C.cast(st, VP)) for _ in range(n)], np.uint64)

    def rng_uniform(self, seed: int, n: int) -> np.ndarray:
        st = self._rng(seed)
        return np.array([self.lib.orc_rng_uniform(C.cast(st, VP)) for _ in range(n)], np.float32)

    def rng_normal(self, seed: int, n: int) -> np.ndarray:
        st = self._rng(seed)
        return np.array([self.lib.orc_rng_normal(C.cast(st, VP)) for _ in range(n)], np.float32)

    def rng_uniform_int(self, seed: int, lo: int, hi: int, n: int) -> np.ndarray:
        st = self._rng(seed)
        return np.array([self.lib.orc_rng_uniform_int(C.cast(st, VP), lo, hi) for _ in range(n)], np.int32)

    # -- fp16 ----------------------------------------------------------------
    def fp16_to_float(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, np.uint16)
        f = np.empty(h.shape, np.float32)
        self.lib.orc_fp16_to_float_n(_p(h, np.uint16), _p(f, np.float32), h.size)
        return f

    def half_to_float_codebook(self, h: int) -> float:
        return self.lib.orc_half_to_float_codebook(h)

    def float_to_half_trunc(self, f: float) -> int:
        return self.lib.orc_float_to_half_trunc(f)

    # -- oil8 ----------------------------------------------------------------
    def oil8_gemm(self, idx, cb, act, M, N, K, variant="avx2"):
        _need(idx, M * N * K, "idx"); _need(cb, 256, "cb"); _need(act, N * K, "act")
        out = np.empty(M * N, np.float32)
        f = self.lib.orc_oil8_gemm_avx2 if variant == "avx2" else self.lib.orc_oil8_gemm_scalar
        f(_p(idx, np.uint8), _p(cb, np.float32), _p(act, np.float32), _p(out, np.float32), M, N, K)
        return out

    def oil8_gemv(self, idx, cb, x, M, K, batch, threads=1):
        _need(idx, M * K, "idx"); _need(x, batch * K, "x")
        y = np.empty((batch, M), np.float32)
        self.lib.orc_oil8_gemv(_p(idx, np.uint8), _p(cb, np.float32), _p(x, np.float32),
                               _p(y, np.float32), M, K, batch, threads)
        return y

    # -- oil4 ----------------------------------------------------------------
    def oil4_gemm(self, nib, cb16, act, M, N, K, variant="scalar"):
        _need(nib, M * N * K // 2, "nib"); _need(cb16, 16, "cb16"); _need(act, N * K, "act")
        out = np.empty(M * N, np.float32)
        f = self.lib.orc_oil4_gemm_avx2 if variant == "avx2" else self.lib.orc_oil4_gemm_scalar
        f(_p(nib, np.uint8), _p(cb16, np.uint16), _p(act, np.float32), _p(out, np.float32), M, N, K)
        return out

    def oil4_gemv_blocked(self, nib, cb16, x, M, K, batch, block=128, threads=1):
        _need(nib, M * K // 2, "nib"); _need(cb16, M * (K // block) * 16, "cb16"); _need(x, batch * K, "x")
        y = np.empty((batch, M), np.float32)
        self.lib.orc_oil4_gemv_blocked(_p(nib, np.uint8), _p(cb16, np.uint16), block,
                                       _p(x, np.float32), _p(y, np.float32), M, K, batch, threads)
        return y

    def oil4_gemm_prefill(self, a_bf16, nib, cb16, M, N, K, block=128, threads=1):
        _need(a_bf16, M * K, "a"); _need(nib, N * K // 2, "nib")
        c16 = np.empty((M, N), np.uint16)
        c32 = np.empty((M, N), np.float32)
        self.lib.orc_oil4_gemm_prefill(_p(a_bf16, np.uint16), _p(nib, np.uint8), _p(cb16, np.uint16),
                                       block, _p(c16, np.uint16), _p(c32, np.float32), M, N, K, threads)
        return c16, c32

    # -- int8 / ternary --------------------------------------------------------
    def quantize_per_token(self, x, rows, cols):
        _need(x, rows * cols, "x")
        q = np.empty((rows, cols), np.int8)
        s = np.empty(rows, np.float32)
        inv = np.empty(rows, np.float32)
        self.lib.orc_quantize_per_token(_p(x, np.float32), _p(q, np.int8), rows, cols,
                                        _p(s, np.float32), _p(inv, np.float32))
        return q, s, inv

    def i2s_gemv(self, packed_row, w_scale, act, act_scale, K):
        _need(packed_row, K // 4, "packed"); _need(act, K, "act")
        out = np.empty(1, np.float32)
        self.lib.orc_i2s_gemv(_p(packed_row, np.uint8), w_scale, _p(act, np.int8), act_scale,
                              _p(out, np.float32), K)
        return float(out[0])

    def i2s_gemm(self, w, a, M, N, K):
        _need(w, i2s_bytes(M, K), "w"); _need(a, N * K, "a")
        o = np.empty(M * N, np.float32)
        self.lib.orc_i2s_gemm(_p(w, np.uint8), _p(a, np.float32), _p(o, np.float32), M, N, K)
        return o

    def i2s_gemm_vnni(self, w, a, M, N, K):
        _need(w, i2s_bytes(M, K), "w"); _need(a, N * K, "a")
        o = np.empty(M * N, np.float32)
        self.lib.orc_i2s_gemm_vnni(_p(w, np.uint8), _p(a, np.int8), _p(o, np.float32), M, N, K)
        return o

    def i2s_gemv_rows(self, packed, w_scale, q, inv, M, K, threads=1):
        """i2s_gemv over M rows for int8 activations q [K] and act_scale inv."""
        _need(packed, M * K // 4, "packed"); _need(q, K, "q")
        y = np.empty(M, np.float32)
        self.lib.orc_i2s_gemv_rows(_p(packed, np.uint8), w_scale, _p(q, np.int8), float(inv), _p(y, np.float32),
                                   M, K, threads)
        return y

    def bf16_round(self, f: float) -> float:
        return self.lib.orc_bf16_round(f)

    def i2s_gemv_f32(self, packed, w_scale, x, M, K, batch, threads=1):
        _need(packed, M * K // 4, "packed"); _need(x, batch * K, "x")
        y = np.empty((batch, M), np.float32)
        self.lib.orc_i2s_gemv_f32(_p(packed, np.uint8), w_scale, _p(x, np.float32),
                                  _p(y, np.float32), M, K, batch, threads)
        return y

    def tl1_gemm(self, w, a, M, N, K):
        _need(w, M * N * K // 4, "w"); _need(a, N * K, "a")
        o = np.empty(M * N, np.float32)
        self.lib.orc_tl1_gemm(_p(w, np.uint8), _p(a, np.float32), _p(o, np.float32), M, N, K)
        return o

    def tl2_gemm(self, w, a, M, N, K):
        if K % 3:
            raise ValueError("tl2_gemm is defined for K % 3 == 0")
        _need(w, M * N * ((2 * K + 7) // 8), "w"); _need(a, N * K, "a")
        o = np.empty(M * N, np.float32)
        self.lib.orc_tl2_gemm(_p(w, np.uint8), _p(a, np.float32), _p(o, np.float32), M, N, K)
        return o

    # -- dense -----------------------------------------------------------------
    def gemv(self, alpha, A, x, beta, y, M, N):
        y = np.array(y, np.float32, copy=True)
        self.lib.orc_gemv(alpha, _p(A, np.float32), _p(x, np.float32), beta, _p(y, np.float32), M, N)
        return y

    def rms_norm(self, x, g, eps, rows, dim):
        y = np.empty((rows, dim), np.float32)
        self.lib.orc_rms_norm(_p(x, np.float32), _p(g, np.float32), eps, _p(y, np.float32), rows, dim)
        return y

    def gemm(self, alpha, A, B, beta, C, M, N, K):
        C = np.array(C, np.float32, copy=True).reshape(M, N)
        self.lib.orc_gemm(alpha, _p(A, np.float32), _p(B, np.float32), beta, _p(C, np.float32), M, N, K)
        return C

    def relu(self, x):
        y = np.empty_like(x, dtype=np.float32)
        self.lib.orc_relu(_p(x, np.float32), _p(y, np.float32), x.size)
        return y

    def gelu(self, x):
        y = np.empty_like(x, dtype=np.float32)
        self.lib.orc_gelu(_p(x, np.float32), _p(y, np.float32), x.size)
        return y

    def scale(self, s, x):
        y = np.empty_like(x, dtype=np.float32)
        self.lib.orc_scale(s, _p(x, np.float32), _p(y, np.float32), x.size)
        return y

    def layer_norm(self, x, g, b, eps, rows, dim):
        y = np.empty((rows, dim), np.float32)
        self.lib.orc_layer_norm(_p(x, np.float32), _p(g, np.float32), _p(b, np.float32), eps, _p(y, np.float32),
                                rows, dim)
        return y

    def softmax_axis(self, x, outer, dim, inner):
        y = np.empty(outer * dim * inner, np.float32)
        self.lib.orc_softmax_axis(_p(x, np.float32), _p(y, np.float32), outer, dim, inner)
        return y

    # -- config-5 decoder (decoder.c) -------------------------------------
    def softmax(self, x, rows, dim):
        y = np.empty((rows, dim), np.float32)
        self.lib.orc_softmax(_p(x, np.float32), _p(y, np.float32), rows, dim)
        return y

    def silu_mul(self, g, u):
        y = np.empty_like(g)
        self.lib.orc_silu_mul(_p(g, np.float32), _p(u, np.float32), _p(y, np.float32), g.size)
        return y

    def rope_tables(self, head_dim, max_seq, theta=10000.0):
        c = np.empty((max_seq, head_dim // 2), np.float32)
        s = np.empty((max_seq, head_dim // 2), np.float32)
        self.lib.orc_rope_tables(head_dim, max_seq, theta, _p(c, np.float32), _p(s, np.float32))
        return c, s

    def rope_apply(self, x, heads, head_dim, pos, cos_t, sin_t):
        y = np.array(x, np.float32, copy=True)
        self.lib.orc_rope_apply(_p(y, np.float32), heads, head_dim, pos, _p(cos_t, np.float32), _p(sin_t, np.float32))
        return y

    def attention_decode(self, q, kc, vc, heads, kv_heads, head_dim, ctx, kv_stride):
        out = np.empty(heads * head_dim, np.float32)
        self.lib.orc_attention_decode(_p(q, np.float32), _p(kc, np.float32), _p(vc, np.float32),
                                      _p(out, np.float32), heads, kv_heads, head_dim, ctx, kv_stride)
        return out

    def argmax(self, logits) -> int:
        return int(self.lib.orc_argmax(_p(logits, np.float32), logits.size))

    def decoder(self, cfg: dict, model: dict):
        """A callable decoder over `model` (synth.decoder_model layout):
        step(kc, vc, pos, token, down_mode=0, threads=8) -> logits."""
        return _OracleDecoder(self, cfg, model)

    def silu(self, x):
        y = np.empty_like(x)
        self.lib.orc_silu(_p(x, np.float32), _p(y, np.float32), x.size)
        return y


class _OracleDecoder:
    def __init__(self, orc: "Oracle", cfg: dict, model: dict):
        self.orc, self.cfg = orc, cfg
        self.c = DecoderConfig(*[cfg[k] for k in DECODER_CONFIG_KEYS], int(cfg.get("kv_bf16", 0)))
        keep = []

        def ptr(a, dtype):
            a = np.ascontiguousarray(a)
            assert a.dtype == dtype, (a.dtype, dtype)
            keep.append(a)
            return a.ctypes.data

        cos_t, sin_t = orc.rope_tables(cfg["head_dim"], cfg["max_seq"], cfg["theta"])
        L = (DecoderLayer * cfg["layers"])()
        for i, ly in enumerate(model["layers"]):
            L[i] = DecoderLayer(ptr(ly["attn_norm"], np.float32), ptr(ly["ffn_norm"], np.float32),
                                ptr(ly["wq"], np.uint8), ptr(ly["wk"], np.uint8), ptr(ly["wv"], np.uint8),
                                ptr(ly["wo"], np.uint8), ptr(ly["cbq"], np.float32), ptr(ly["cbk"], np.float32),
                                ptr(ly["cbv"], np.float32), ptr(ly["cbo"], np.float32), ptr(ly["wgate"], np.uint8),
                                ptr(ly["wup"], np.uint8), ptr(ly["cbgate"], np.uint16), ptr(ly["cbup"], np.uint16),
                                ptr(ly["wdown"], np.uint8), float(ly["down_scale"]))
        self.m = DecoderModel(ptr(model["emb"], np.float32), ptr(model["final_norm"], np.float32),
                              ptr(model["lm_idx"], np.uint8), ptr(model["lm_cb"], np.float32),
                              ptr(cos_t, np.float32), ptr(sin_t, np.float32), L)
        self._keep, self._L = keep, L

    def new_cache(self):
        c = self.cfg
        shape = (c["layers"], c["kv_heads"], c["max_seq"], c["head_dim"])
        return np.zeros(shape, np.float32), np.zeros(shape, np.float32)

    def step(self, kc, vc, pos: int, token: int, down_mode: int = 0, threads: int = 8) -> np.ndarray:
        assert 0 <= pos < self.cfg["max_seq"]
        assert kc.shape == vc.shape == (self.cfg["layers"], self.cfg["kv_heads"], self.cfg["max_seq"],
                                        self.cfg["head_dim"])
        out = np.empty(self.cfg["vocab"], np.float32)
        self.orc.lib.orc_decoder_step(C.byref(self.c), C.byref(self.m), _p(kc, np.float32), _p(vc, np.float32),
                                      pos, token, _p(out, np.float32), down_mode, threads)
        return out

    def attn_half(self, kc, vc, layer: int, pos: int, x, append: bool = True, threads: int = 8) -> np.ndarray:
        """x + O(attention(rmsnorm(x))) of `layer` for one token at pos over
        kc/vc [layers][kv_heads][max_seq][head_dim]; with append, the
        position's K/V are computed and written into the cache first."""
        assert 0 <= pos < self.cfg["max_seq"] and 0 <= layer < self.cfg["layers"]
        assert kc.shape == vc.shape == (self.cfg["layers"], self.cfg["kv_heads"], self.cfg["max_seq"],
                                        self.cfg["head_dim"])
        y = np.array(x, np.float32, copy=True).ravel()
        assert y.size == self.cfg["hidden"]
        self.orc.lib.orc_decoder_attn_half(C.byref(self.c), C.byref(self.m), layer, _p(kc[layer], np.float32),
                                           _p(vc[layer], np.float32), pos, _p(y, np.float32), int(append), threads)
        return y


class Reference:
    """The reference's own kernels (oracle/_ref/libref_<variant>.so)."""

    def __init__(self, variant: str = "avx2"):
        path = ref_lib_path(variant)
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.variant = variant
        self.lib = L = C.CDLL(path)
        sig = {
            "ref_oil8_gemm": [VP, VP, VP, VP, I32, I32, I32],
            "ref_oil4_gemm": [VP, VP, VP, VP, I32, I32, I32],
            "ref_scalar_gemm": [VP, VP, VP, I32, I32, I32],
            "ref_i2s_init": [],
            "ref_i2s_gemv": [VP, F32, VP, F32, VP, I32],
            "ref_i2s_gemm": [VP, VP, VP, I32, I32, I32],
            "ref_i2s_gemm_vnni": [VP, VP, VP, I32, I32, I32],
            "ref_tl1_gemm": [VP, VP, VP, I32, I32, I32],
            "ref_tl2_gemm": [VP, VP, VP, I32, I32, I32],
            "ref_quantize_per_token": [VP, VP, I64, I64, VP, VP],
            "ref_rng_u64": [U64, VP, I64],
            "ref_rng_uniform": [U64, VP, I64],
            "ref_rng_normal": [U64, VP, I64],
            "ref_rng_uniform_int": [U64, I32, I32, VP, I64],
            "ref_gemv": [F32, VP, VP, F32, VP, I64, I64],
            "ref_rms_norm": [VP, VP, F32, VP, I64, I64],
            "ref_silu": [VP, VP, I64],
            "ref_softmax": [VP, VP, I64, I64],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = None
        L.ref_float_to_half.argtypes = [F32]
        L.ref_float_to_half.restype = C.c_uint16
        for name in ("ref_serialize_oil8", "ref_serialize_oil4"):
            getattr(L, name).argtypes = [VP, VP]
            getattr(L, name).restype = I64
        L.ref_oil_write.argtypes = [C.c_char_p, VP, C.c_uint32, C.c_int, VP, VP, VP, VP, VP, VP,
                                    C.c_int, C.POINTER(C.c_char_p), VP, VP]
        L.ref_oil_write.restype = None
        L.ref_oil_read_tensor.argtypes = [C.c_char_p, C.c_char_p, VP, I64]
        L.ref_oil_read_tensor.restype = I64
        L.ref_half_to_float.argtypes = [C.c_uint16]
        L.ref_half_to_float.restype = F32

    def oil8_gemm(self, idx, cb, act, M, N, K):
        _need(idx, M * N * K, "idx"); _need(act, N * K, "act")
        out = np.empty(M * N, np.float32)
        self.lib.ref_oil8_gemm(_p(idx, np.uint8), _p(cb, np.float32), _p(act, np.float32),
                               _p(out, np.float32), M, N, K)
        return out

    def oil4_gemm(self, nib, cb16, act, M, N, K):
        _need(nib, M * N * K // 2, "nib"); _need(act, N * K, "act")
        out = np.empty(M * N, np.float32)
        self.lib.ref_oil4_gemm(_p(nib, np.uint8), _p(cb16, np.uint16), _p(act, np.float32),
                               _p(out, np.float32), M, N, K)
        return out

    def scalar_gemm(self, A, B, M, N, K):
        """kernel::scalar_gemm: C[M][N] = A[M][K] @ B, B read as B[k*N + n]."""
        _need(A, M * K, "A"); _need(B, K * N, "B")
        out = np.empty(M * N, np.float32)
        self.lib.ref_scalar_gemm(_p(A, np.float32), _p(B, np.float32), _p(out, np.float32), M, N, K)
        return out

    def i2s_init(self):
        self.lib.ref_i2s_init()

    def i2s_gemv(self, packed_row, w_scale, act, act_scale, K):
        out = np.empty(1, np.float32)
        self.lib.ref_i2s_gemv(_p(packed_row, np.uint8), w_scale, _p(act, np.int8), act_scale,
                              _p(out, np.float32), K)
        return float(out[0])

    def i2s_gemm(self, w, a, M, N, K):
        o = np.empty(M * N, np.float32)
        self.lib.ref_i2s_gemm(_p(w, np.uint8), _p(a, np.float32), _p(o, np.float32), M, N, K)
        return o

    def i2s_gemm_vnni(self, w, a, M, N, K):
        o = np.full(M * N, np.nan, np.float32)
        self.lib.ref_i2s_gemm_vnni(_p(w, np.uint8), _p(a, np.int8), _p(o, np.float32), M, N, K)
        return o

    def tl1_gemm(self, w, a, M, N, K):
        o = np.empty(M * N, np.float32)
        self.lib.ref_tl1_gemm(_p(w, np.uint8), _p(a, np.float32), _p(o, np.float32), M, N, K)
        return o

    def tl2_gemm(self, w, a, M, N, K):
        o = np.empty(M * N, np.float32)
        self.lib.ref_tl2_gemm(_p(w, np.uint8), _p(a, np.float32), _p(o, np.float32), M, N, K)
        return o

    def quantize_per_token(self, x, rows, cols):
        q = np.empty((rows, cols), np.int8)
        s = np.empty(rows, np.float32)
        inv = np.empty(rows, np.float32)
        self.lib.ref_quantize_per_token(_p(x, np.float32), _p(q, np.int8), rows, cols,
                                        _p(s, np.float32), _p(inv, np.float32))
        return q, s, inv

    def float_to_half(self, f: float) -> int:
        return self.lib.ref_float_to_half(f)

    def half_to_float(self, h: int) -> float:
        return self.lib.ref_half_to_float(h)

    def rng_u64(self, seed, n):
        o = np.empty(n, np.uint64)
        self.lib.ref_rng_u64(seed, _p(o, np.uint64), n)
        return o

    def rng_uniform(self, seed, n):
        o = np.empty(n, np.float32)
        self.lib.ref_rng_uniform(seed, _p(o, np.float32), n)
        return o

    def rng_normal(self, seed, n):
        o = np.empty(n, np.float32)
        self.lib.ref_rng_normal(seed, _p(o, np.float32), n)
        return o

    def rng_uniform_int(self, seed, lo, hi, n):
        o = np.empty(n, np.int32)
        self.lib.ref_rng_uniform_int(seed, lo, hi, _p(o, np.int32), n)
        return o

    def gemv(self, alpha, A, x, beta, y, M, N):
        y = np.array(y, np.float32, copy=True)
        self.lib.ref_gemv(alpha, _p(A, np.float32), _p(x, np.float32), beta, _p(y, np.float32), M, N)
        return y

    def rms_norm(self, x, g, eps, rows, dim):
        y = np.empty((rows, dim), np.float32)
        self.lib.ref_rms_norm(_p(x, np.float32), _p(g, np.float32), eps, _p(y, np.float32), rows, dim)
        return y

    def silu(self, x):
        y = np.empty_like(x)
        self.lib.ref_silu(_p(x, np.float32), _p(y, np.float32), x.size)
        return y

    # ---- .oil container (src/oil_format.cpp, src/codebook.cpp) ----------
    def serialize_oil8(self, centroids) -> np.ndarray:
        out = np.zeros(4 + 1024, np.uint8)
        n = self.lib.ref_serialize_oil8(_p(np.asarray(centroids, np.float32), np.float32), _p(out, np.uint8))
        return out[:n]

    def serialize_oil4(self, centroids16) -> np.ndarray:
        out = np.zeros(4 + 32, np.uint8)
        n = self.lib.ref_serialize_oil4(_p(np.asarray(centroids16, np.uint16), np.uint16), _p(out, np.uint8))
        return out[:n]

    def oil_write(self, path, config: bytes, blocks, tensors) -> None:
        """blocks: [(format, num_weights, codebook bytes, index bytes)] in file
        order; tensors: [(name, block_start, num_blocks)]."""
        fm = np.array([b[0] for b in blocks], np.uint8)
        nw = np.array([b[1] for b in blocks], np.uint32)
        cbs = np.array([len(b[2]) for b in blocks], np.uint32)
        ids = np.array([len(b[3]) for b in blocks], np.uint32)
        cbd = np.concatenate([np.frombuffer(bytes(b[2]), np.uint8) for b in blocks] + [np.zeros(1, np.uint8)])
        idd = np.concatenate([np.frombuffer(bytes(b[3]), np.uint8) for b in blocks] + [np.zeros(1, np.uint8)])
        cfg = np.frombuffer(config + b"\0", np.uint8)
        names = (C.c_char_p * len(tensors))(*[t[0].encode() for t in tensors])
        bs = np.array([t[1] for t in tensors], np.uint32)
        nb = np.array([t[2] for t in tensors], np.uint32)
        self.lib.ref_oil_write(str(path).encode(), _p(cfg, np.uint8), len(config), len(blocks),
                               _p(fm, np.uint8), _p(nw, np.uint32), _p(cbs, np.uint32), _p(cbd, np.uint8),
                               _p(ids, np.uint32), _p(idd, np.uint8), len(tensors), names,
                               _p(bs, np.uint32), _p(nb, np.uint32))

    def oil_read_tensor(self, path, name: str, cap: int) -> np.ndarray:
        """OILReader::read_tensor(name) (the reference's FP32 dequantisation)."""
        out = np.zeros(max(cap, 1), np.float32)
        n = self.lib.ref_oil_read_tensor(str(path).encode(), name.encode(), _p(out, np.float32), cap)
        if n < 0:
            raise ValueError(f"reference OILReader rejected {path}")
        return out[:min(n, cap)]

    def softmax(self, x, rows, dim):
        """math::softmax over the last axis of a [rows][dim] tensor."""
        y = np.empty((rows, dim), np.float32)
        self.lib.ref_softmax(_p(np.ascontiguousarray(x, np.float32), np.float32), _p(y, np.float32), rows, dim)
        return y


class ReferenceModel:
    """The reference's DenseModel (oracle/_ref/libref_model.so)."""

    def __init__(self):
        path = ref_lib_path("model")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = C.CDLL(path)
        self.lib.ref_dense_model_run.argtypes = [VP, F32, F32, VP, C.POINTER(VP), VP, VP, VP, I64, VP]
        self.lib.ref_dense_model_run.restype = None

    def run(self, cfg: dict, emb, layers_inmajor, final_norm, lm_head_inmajor, ids) -> np.ndarray:
        """layers_inmajor: per layer [attn_norm, ffn_norm, q, k, v, o, gate,
        up, down] as float32 arrays, Linear weights input-major."""
        keep = [np.ascontiguousarray(a, np.float32) for ly in layers_inmajor for a in ly]
        ptrs = (VP * len(keep))(*[a.ctypes.data for a in keep])
        c = np.array([cfg[k] for k in ("vocab", "hidden", "layers", "heads", "head_dim", "ffn", "max_seq")], np.int64)
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((ids.size, cfg["vocab"]), np.float32)
        emb = np.ascontiguousarray(emb, np.float32)
        fn = np.ascontiguousarray(final_norm, np.float32)
        lm = np.ascontiguousarray(lm_head_inmajor, np.float32)
        self.lib.ref_dense_model_run(_p(c, np.int64), cfg["eps"], cfg["theta"], _p(emb, np.float32), ptrs,
                                     _p(fn, np.float32), _p(lm, np.float32), _p(ids, np.int32), ids.size,
                                     _p(out, np.float32))
        return out

