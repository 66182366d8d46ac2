"""Seeded synthetic inputs for the BASELINE configurations (host side).

One stream per configuration: MYTHOS.cpp's RNG (xoroshiro128+ seeded by
splitmix64, src/random.cpp:7-51) with seed 0x5EED0000 + config, drawn in
native code (libmythos_synth.so, host/synth.cpp).  Arrays are drawn one after
another from that stream:
  * OIL8 indices: next_u64() >> 56; codebook 256 x N(0, 0.02), sorted;
  * OIL4 nibbles: next_u64() >> 60; one 16-entry FP16 codebook per 128-weight
    row block, N(0, 0.02) converted with the reference's truncating
    float_to_half (src/codebook.cpp:16-34);
  * ternary codes t+1 = uniform_int(0, 2), packed four per byte, element 4i+j
    in bits 2j of byte i (src/kernel_i2s.cpp:13-30, tools/convert.cpp:329-342);
  * activations N(0, 1); normals from a double-precision Box-Muller over
    next_u64() >> 11;
  * the decoder stack (config 5): per layer Q, K, V, O as OIL8, gate and up
    as OIL4, down as ternary, drawn in that order after the FP32 embedding
    N(0, 1), then the OIL8 lm_head; prompt ids uniform_int(0, vocab - 1).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

SEED_BASE = 0x5EED0000
W_SCALE_TERNARY = 0.0159577  # E|N(0, 0.02)| = 0.02*sqrt(2/pi), the absmean scale

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmythos_synth.so")
if not os.path.exists(_LIB_PATH):
    raise ImportError(f"{_LIB_PATH} is not built; run make -C mythos.cpp_amd (or __graft_entry__.build())")
_lib = C.CDLL(_LIB_PATH)
_VP, _I64 = C.c_void_p, C.c_int64
_lib.mth_synth_seed.argtypes = [C.c_uint64, _VP]
_lib.mth_synth_u64.argtypes = [_VP, _VP, _I64]
_lib.mth_synth_bits.argtypes = [_VP, _VP, _I64, C.c_int]
_lib.mth_synth_uniform_int.argtypes = [_VP, _VP, _I64, C.c_int, C.c_int]
_lib.mth_synth_normal.argtypes = [_VP, _VP, _I64, C.c_double, C.c_double]
_lib.mth_synth_uniform_i32.argtypes = [_VP, _VP, _I64, C.c_int, C.c_int]
_lib.mth_synth_nibbles.argtypes = [_VP, _VP, _I64]
_lib.mth_synth_ternary.argtypes = [_VP, _VP, _I64]
_lib.mth_synth_normal_f16.argtypes = [_VP, _VP, _I64, C.c_double, C.c_double]
for _f in ("mth_synth_seed", "mth_synth_u64", "mth_synth_bits", "mth_synth_uniform_int", "mth_synth_normal",
           "mth_synth_uniform_i32", "mth_synth_nibbles", "mth_synth_ternary", "mth_synth_normal_f16"):
    getattr(_lib, _f).restype = None


class Stream:
    """One seeded stream; successive draws continue it."""

    def __init__(self, seed: int):
        self.st = np.zeros(2, np.uint64)
        _lib.mth_synth_seed(C.c_uint64(seed), self.st.ctypes.data)

    def u64(self, n: int) -> np.ndarray:
        out = np.empty(n, np.uint64)
        _lib.mth_synth_u64(self.st.ctypes.data, out.ctypes.data, n)
        return out

    def bits(self, shape, bits: int) -> np.ndarray:
        out = np.empty(shape, np.uint8)
        _lib.mth_synth_bits(self.st.ctypes.data, out.ctypes.data, out.size, bits)
        return out

    def uniform_int(self, shape, lo: int, hi: int) -> np.ndarray:
        out = np.empty(shape, np.int8)
        _lib.mth_synth_uniform_int(self.st.ctypes.data, out.ctypes.data, out.size, lo, hi)
        return out

    def uniform_i32(self, shape, lo: int, hi: int) -> np.ndarray:
        out = np.empty(shape, np.int32)
        _lib.mth_synth_uniform_i32(self.st.ctypes.data, out.ctypes.data, out.size, lo, hi)
        return out

    def nibbles(self, rows: int, cols: int) -> np.ndarray:
        """[rows][cols/2] packed 4-bit indices (= pack_nibbles(bits(.., 4)))."""
        out = np.empty((rows, cols // 2), np.uint8)
        _lib.mth_synth_nibbles(self.st.ctypes.data, out.ctypes.data, out.size)
        return out

    def ternary(self, rows: int, cols: int) -> np.ndarray:
        """[rows][cols/4] packed codes t+1 (= pack_ternary(uniform_int(.., 0, 2) - 1))."""
        out = np.empty((rows, cols // 4), np.uint8)
        _lib.mth_synth_ternary(self.st.ctypes.data, out.ctypes.data, out.size)
        return out

    def normal_f16(self, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        """FP16 bits of normal(shape) by the truncating float_to_half."""
        out = np.empty(shape, np.uint16)
        _lib.mth_synth_normal_f16(self.st.ctypes.data, out.ctypes.data, out.size, mean, std)
        return out

    def normal(self, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        out = np.empty(shape, np.float32)
        _lib.mth_synth_normal(self.st.ctypes.data, out.ctypes.data, out.size, mean, std)
        return out


def stream(config: int) -> Stream:
    return Stream(SEED_BASE + config)


def float_to_half_trunc(f: np.ndarray) -> np.ndarray:
    """Vectorised src/codebook.cpp:16-34 (round toward zero, no rounding)."""
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.int64)
    sign = ((u >> 16) & 0x8000).astype(np.int64)
    e = ((u >> 23) & 0xFF) - 127 + 15
    mant = u & 0x007FFFFF
    out = np.empty(u.shape, np.int64)
    den = e <= 0
    tiny = den & (e < -10)
    sub = den & ~tiny
    sh = np.clip(1 - e, 0, 31)
    out[tiny] = sign[tiny]
    out[sub] = sign[sub] | (((mant[sub] | 0x00800000) >> sh[sub]) >> 13)
    big = (~den) & (e >= 31)
    out[big] = sign[big] | 0x7C00 | np.where(mant[big] != 0, 0x0200, 0)
    nrm = (~den) & (e < 31)
    out[nrm] = sign[nrm] | (e[nrm] << 10) | (mant[nrm] >> 13)
    return out.astype(np.uint16)


def pack_nibbles(idx: np.ndarray) -> np.ndarray:
    """[..., K] indices 0..15 -> [..., K/2] bytes, even k in the low nibble."""
    idx = idx.astype(np.uint8)
    return (idx[..., 0::2] | (idx[..., 1::2] << 4)).astype(np.uint8)


def pack_ternary(t: np.ndarray) -> np.ndarray:
    """[..., K] values in {-1, 0, 1} -> [..., K/4] bytes with code t+1."""
    c = (t.astype(np.int16) + 1).astype(np.uint8)
    return (c[..., 0::4] | (c[..., 1::4] << 2) | (c[..., 2::4] << 4) | (c[..., 3::4] << 6)).astype(np.uint8)


def oil8(M: int, K: int, batch: int, config: int = 1):
    g = stream(config)
    idx = g.bits((M, K), 8)
    cb = np.sort(g.normal(256, 0.0, 0.02)).astype(np.float32)
    x = g.normal((batch, K))
    return idx, cb, x


def oil4(M: int, K: int, batch: int, block: int = 128, config: int = 2):
    g = stream(config)
    packed = pack_nibbles(g.bits((M, K), 4))
    ncb = M * (K // block) if block else 1
    cbs = g.normal_f16((ncb, 16), 0.0, 0.02)
    x = g.normal((batch, K))
    return packed, cbs.reshape(-1), x


def ternary(M: int, K: int, batch: int, config: int = 3):
    g = stream(config)
    t = g.uniform_int((M, K), 0, 2) - 1
    packed = pack_ternary(t)
    x = g.normal((batch, K))
    return packed, np.float32(W_SCALE_TERNARY), x


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """FP32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def prefill(M: int, N: int, K: int, block: int = 128, config: int = 4):
    g = stream(config)
    a = bf16_bits(g.normal((M, K)))
    packed = pack_nibbles(g.bits((N, K), 4))
    cbs = g.normal_f16((N * (K // block), 16), 0.0, 0.02)
    return a, packed, cbs.reshape(-1)


def fp16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    """IEEE binary16 -> FP32 (exact, subnormals included)."""
    return np.ascontiguousarray(h, np.uint16).view(np.float16).astype(np.float32)


def dequant_oil4(packed: np.ndarray, cbs: np.ndarray, rows: int, K: int, block: int) -> np.ndarray:
    """[rows][K] FP32 weights from nibbles + per-block codebooks (block 0 = shared)."""
    p = packed.reshape(rows, K // 2)
    nib = np.empty((rows, K), np.uint8)
    nib[:, 0::2] = p & 0xF
    nib[:, 1::2] = p >> 4
    table = fp16_bits_to_f32(cbs)
    if block == 0:
        return table[nib]
    nb = K // block
    blk = (np.arange(rows)[:, None] * nb + (np.arange(K)[None, :] // block)) * 16
    return table[blk + nib]


# ---- config 5: the mixed-format decoder stack ---------------------------------
DECODER_CONFIG5 = dict(vocab=32000, hidden=4096, layers=32, heads=32, kv_heads=32, head_dim=128, ffn=11008,
                       max_seq=192, cb_block=128, eps=1e-5, theta=10000.0)
PROMPT_LEN5, GEN_TOKENS5 = 64, 128


def decoder_config(**overrides) -> dict:
    c = dict(DECODER_CONFIG5)
    c.update(overrides)
    return c


def decoder_model(cfg: dict, config: int = 5, random_gamma: bool = False) -> dict:
    """Weights of the decoder stack in the kernels' layouts ([out][in] rows).
    Norm gains are 1 (the reference's RMSNorm init) unless random_gamma.
    gate and up are one array of 2*ffn rows (gate first) so that they can run
    as one GEMV; 'wgate'/'wup' are views of it."""
    g = stream(config)
    H, F, V = cfg["hidden"], cfg["ffn"], cfg["vocab"]
    QD, KD, B = cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"], cfg["cb_block"]

    def gamma():
        return g.normal(H, 1.0, 0.1) if random_gamma else np.ones(H, np.float32)

    def oil8(rows, cols):
        return g.bits((rows, cols), 8), np.sort(g.normal(256, 0.0, 0.02)).astype(np.float32)

    model = {"emb": g.normal((V, H)), "layers": []}
    for _ in range(cfg["layers"]):
        ly = {"attn_norm": gamma(), "ffn_norm": gamma()}
        for name, rows, cols in (("q", QD, H), ("k", KD, H), ("v", KD, H), ("o", H, QD)):
            ly["w" + name], ly["cb" + name] = oil8(rows, cols)
        gu = np.empty((2 * F, H // 2), np.uint8)
        half = F * (H // B) if B else 1      # codebooks per tensor
        cbs = np.empty((2 * half, 16), np.uint16)
        for i in range(2):
            gu[i * F:(i + 1) * F] = g.nibbles(F, H)
            cbs[i * half:(i + 1) * half] = g.normal_f16((half, 16), 0.0, 0.02)
        ly["wgate_up"], ly["cbgate_up"] = gu, cbs.reshape(-1)
        ly["wgate"], ly["wup"] = gu[:F], gu[F:]
        ly["cbgate"], ly["cbup"] = cbs[:half].reshape(-1), cbs[half:].reshape(-1)
        ly["wdown"] = g.ternary(H, F)
        ly["down_scale"] = np.float32(W_SCALE_TERNARY)
        model["layers"].append(ly)
    model["final_norm"] = gamma()
    model["lm_idx"], model["lm_cb"] = oil8(V, H)
    return model


def decoder_prompts(cfg: dict, batch: int, prompt_len: int, config: int = 5) -> np.ndarray:
    """[batch][prompt_len] ids uniform in [0, vocab), from the stream after the weights' seed + 100."""
    return stream(config + 100).uniform_i32((batch, prompt_len), 0, cfg["vocab"] - 1)


def dequant_oil8(idx: np.ndarray, cb: np.ndarray) -> np.ndarray:
    return cb[idx]


def dequant_ternary(packed: np.ndarray, rows: int, K: int, w_scale: float) -> np.ndarray:
    p = packed.reshape(rows, K // 4)
    codes = np.stack([(p >> (2 * j)) & 3 for j in range(4)], -1).reshape(rows, K).astype(np.int8)
    t = np.where(codes == 0, -1, np.where(codes == 1, 0, 1)).astype(np.float32)
    return t * np.float32(w_scale)


def decoder_digest(model: dict) -> str:
    """SHA-256 over every weight array of a decoder model, in a fixed order."""
    import hashlib
    h = hashlib.sha256()
    for k in ("emb", "final_norm", "lm_idx", "lm_cb"):
        h.update(np.ascontiguousarray(model[k]).tobytes())
    for ly in model["layers"]:
        for k in ("attn_norm", "ffn_norm", "wq", "cbq", "wk", "cbk", "wv", "cbv", "wo", "cbo", "wgate_up",
                  "cbgate_up", "wdown", "down_scale"):
            h.update(np.ascontiguousarray(ly[k]).tobytes())
    return h.hexdigest()


def decoder_dense(cfg: dict, model: dict) -> dict:
    """FP32 copies of every weight ([out][in]), for dense reference checks."""
    H, F, B = cfg["hidden"], cfg["ffn"], cfg["cb_block"]
    out = {"emb": model["emb"], "final_norm": model["final_norm"],
           "lm": dequant_oil8(model["lm_idx"], model["lm_cb"]), "layers": []}
    for ly in model["layers"]:
        d = {"attn_norm": ly["attn_norm"], "ffn_norm": ly["ffn_norm"]}
        for n in "qkvo":
            d[n] = dequant_oil8(ly["w" + n], ly["cb" + n])
        gu = dequant_oil4(ly["wgate_up"], ly["cbgate_up"], 2 * F, H, B)
        d["gate"], d["up"] = gu[:F], gu[F:]
        d["down"] = dequant_ternary(ly["wdown"], H, F, ly["down_scale"])
        out["layers"].append(d)
    return out

