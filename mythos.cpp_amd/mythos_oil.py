"""ctypes binding of libmythos_oil.so (include/mythos_oil.h) for Python callers.

Device memory and the stream come from torch (plumbing only): every function
takes torch CUDA tensors, checks dtype / size / contiguity on the host, and
calls the C ABI with raw device pointers on torch's current stream.  There is
no CPU fallback: importing this module raises if the library is missing, and
every non-zero status from the library raises MythosError with the library's
own message.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
# MYTHOS_OIL_LIB / MYTHOS_HOST_LIB select other builds of the two libraries
# (the sanitizer builds of `make -C mythos.cpp_amd sanitize`, for example).
LIB_PATH = os.environ.get("MYTHOS_OIL_LIB") or os.path.join(_HERE, "libmythos_oil.so")
HOST_LIB_PATH = os.environ.get("MYTHOS_HOST_LIB") or os.path.join(_HERE, "libmythos_host.so")

# Every extern "C" symbol declared in include/mythos_oil.h.
EXPORTS = (
    "mth_last_error", "mth_version", "mth_workspace_reserve",
    "mth_oil8_gemm", "mth_oil8_gemv",
    "mth_oil4_gemm", "mth_oil4_gemv", "mth_oil4_gemv_noalloc", "mth_oil4_gemm_prefill",
    "mth_quantize_per_token", "mth_dequantize_per_tensor",
    "mth_i2s_gemv", "mth_i2s_gemv_f32", "mth_i2s_gemm", "mth_i2s_gemm_vnni",
    "mth_tl1_gemm", "mth_tl2_gemm", "mth_tl_precompute_lut",
    "mth_rms_norm", "mth_add_rms_norm", "mth_silu", "mth_silu_mul", "mth_silu_mul_quant",
    "mth_oil4_gemv_swiglu", "mth_i2s_gemv_act", "mth_swiglu_batch_parts", "mth_oil4_gemv_swiglu_batch",
    "mth_i2s_gemv_act_batch", "mth_add", "mth_mul",
    "mth_softmax", "mth_softmax_axis", "mth_axpby", "mth_gemv_f32", "mth_relu", "mth_gelu", "mth_scale",
    "mth_layer_norm",
    "mth_rope_tables", "mth_rope_kv", "mth_attention_decode", "mth_argmax",
)

MTH_OK, MTH_EINVAL, MTH_EDEVICE, MTH_EUNSUPPORTED = 0, -1, -2, -3


class MythosError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def build() -> None:
    """Compile libmythos_oil.so / libmythos_host.so in-tree (gfx950)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-j8"], check=True)


def load_library(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built; run mythos_oil.build() (or __graft_entry__.build())")
    return C.CDLL(path)


# torch is loaded first so that libmythos_oil.so binds to the HIP runtime that
# already owns torch's device memory and streams: loading the library first
# would pull a second libamdhip64 into the process, whose context sees
# neither torch's allocations nor (on the GPU boxes) the device.
import torch as _torch_first  # noqa: E402,F401

_lib = load_library()
VP, I64, I32, F32 = C.c_void_p, C.c_int64, C.c_int, C.c_float
_SIG = {
    "mth_oil8_gemm": [VP, VP, VP, VP, I64, I64, I64, VP],
    "mth_oil8_gemv": [VP, VP, VP, VP, I64, I64, I64, VP],
    "mth_oil4_gemm": [VP, VP, VP, VP, I64, I64, I64, VP],
    "mth_oil4_gemv": [VP, VP, I64, VP, VP, I64, I64, I64, VP],
    "mth_oil4_gemv_noalloc": [VP, VP, I64, VP, VP, I64, I64, I64, VP],
    "mth_oil4_gemm_prefill": [VP, VP, VP, I64, VP, I64, I64, I64, VP],
    "mth_quantize_per_token": [VP, VP, VP, VP, I64, I64, VP],
    "mth_dequantize_per_tensor": [VP, VP, I64, F32, VP],
    "mth_i2s_gemv": [VP, F32, VP, VP, VP, I64, I64, I64, VP],
    "mth_i2s_gemv_f32": [VP, F32, VP, VP, I64, I64, I64, VP],
    "mth_i2s_gemm": [VP, VP, VP, I64, I64, I64, VP],
    "mth_i2s_gemm_vnni": [VP, VP, VP, I64, I64, I64, VP],
    "mth_tl1_gemm": [VP, VP, VP, I64, I64, I64, VP],
    "mth_tl2_gemm": [VP, VP, VP, I64, I64, I64, VP],
    "mth_tl_precompute_lut": [VP, VP, I64, I32, VP],
    "mth_rms_norm": [VP, VP, VP, I64, I64, F32, VP],
    "mth_add_rms_norm": [VP, VP, VP, VP, I64, I64, F32, VP],
    "mth_silu": [VP, VP, I64, VP],
    "mth_silu_mul": [VP, VP, VP, I64, I64, I64, I64, VP],
    "mth_silu_mul_quant": [VP, VP, VP, VP, I64, I64, I64, I64, VP],
    "mth_oil4_gemv_swiglu": [VP, VP, VP, VP, VP, I64, I64, VP],
    "mth_i2s_gemv_act": [VP, F32, VP, VP, VP, I64, I64, VP],
    "mth_oil4_gemv_swiglu_batch": [VP, VP, I64, VP, VP, VP, I64, I64, I64, VP],
    "mth_i2s_gemv_act_batch": [VP, F32, VP, I64, VP, VP, VP, I64, I64, I64, VP],
    "mth_add": [VP, VP, VP, I64, VP],
    "mth_mul": [VP, VP, VP, I64, VP],
    "mth_softmax": [VP, VP, I64, I64, VP],
    "mth_softmax_axis": [VP, VP, I64, I64, I64, VP],
    "mth_axpby": [F32, VP, F32, VP, I64, VP],
    "mth_gemv_f32": [F32, VP, VP, F32, VP, I64, I64, VP],
    "mth_relu": [VP, VP, I64, VP],
    "mth_gelu": [VP, VP, I64, VP],
    "mth_scale": [F32, VP, VP, I64, VP],
    "mth_layer_norm": [VP, VP, VP, VP, I64, I64, F32, VP],
    "mth_rope_tables": [I64, I64, F32, VP, VP],
    "mth_rope_kv": [VP, VP, VP, VP, VP, VP, VP, I64, I64, I64, I64, I64, I64, VP],
    "mth_attention_decode": [VP, VP, VP, VP, I64, I64, I64, I64, I64, I64, VP],
    "mth_argmax": [VP, VP, I64, I64, VP],
    "mth_workspace_reserve": [I64, VP],
}
for _n, _a in _SIG.items():
    _f = getattr(_lib, _n)
    _f.argtypes = _a
    _f.restype = I32
_lib.mth_last_error.argtypes = []
_lib.mth_last_error.restype = C.c_char_p
_lib.mth_version.argtypes = []
_lib.mth_version.restype = I32
_lib.mth_swiglu_batch_parts.argtypes = [I64]
_lib.mth_swiglu_batch_parts.restype = I64

lib = _lib


def version() -> int:
    return _lib.mth_version()


def last_error() -> str:
    return _lib.mth_last_error().decode()


def workspace_reserve(nbytes: int, stream=None) -> None:
    """Reserve the stream's device workspace before capturing batched calls."""
    _check(_lib.mth_workspace_reserve(int(nbytes), _stream(stream)))


def _check(rc: int) -> None:
    if rc != MTH_OK:
        raise MythosError(rc, last_error())


def _torch():
    import torch  # deferred: the library itself never needs torch
    return torch


def _stream(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _i2s_bytes(M: int, K: int) -> int:
    # row m at m*(K/4), element k at byte k/4 of the row (src/kernel_i2s.cpp:54,207)
    return (M - 1) * (K // 4) + (K - 1) // 4 + 1


def _ptr(t, dtype, numel: int, name: str) -> int:
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch tensor")
    if not t.is_cuda:
        raise ValueError(f"{name}: must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if t.numel() < numel:
        raise ValueError(f"{name}: {t.numel()} elements < {numel} required")
    return t.data_ptr()


# --------------------------------------------------------------------------
# Thin wrappers: outputs are passed in (preallocated) and overwritten.
# --------------------------------------------------------------------------
def oil8_gemm(indices, codebook, act, out, M, N, K, stream=None):
    t = _torch()
    _check(_lib.mth_oil8_gemm(_ptr(indices, t.uint8, M * N * K, "indices"), _ptr(codebook, t.float32, 256, "codebook"),
                              _ptr(act, t.float32, N * K, "act"), _ptr(out, t.float32, M * N, "out"),
                              M, N, K, _stream(stream)))


def oil8_gemv(indices, codebook, x, y, M, K, batch=1, stream=None):
    t = _torch()
    _check(_lib.mth_oil8_gemv(_ptr(indices, t.uint8, M * K, "indices"), _ptr(codebook, t.float32, 256, "codebook"),
                              _ptr(x, t.float32, batch * K, "x"), _ptr(y, t.float32, batch * M, "y"),
                              M, K, batch, _stream(stream)))


def oil4_gemm(packed, codebook, act, out, M, N, K, stream=None):
    t = _torch()
    _check(_lib.mth_oil4_gemm(_ptr(packed, t.uint8, (M * N * K + 1) // 2, "packed"),
                              _ptr(codebook, t.int16, 16, "codebook"),
                              _ptr(act, t.float32, N * K, "act"), _ptr(out, t.float32, M * N, "out"),
                              M, N, K, _stream(stream)))


def oil4_gemv(packed, codebooks, cb_block, x, y, M, K, batch=1, stream=None):
    t = _torch()
    ncb = M * (K // cb_block) * 16 if cb_block else 16
    _check(_lib.mth_oil4_gemv(_ptr(packed, t.uint8, M * K // 2, "packed"), _ptr(codebooks, t.int16, ncb, "codebooks"),
                              cb_block, _ptr(x, t.float32, batch * K, "x"), _ptr(y, t.float32, batch * M, "y"),
                              M, K, batch, _stream(stream)))


def oil4_gemv_noalloc(packed, codebooks, cb_block, x, y, M, K, batch=1, stream=None):
    """oil4_gemv whose scratch is a fixed per-GPU device array (no allocation)."""
    t = _torch()
    ncb = M * (K // cb_block) * 16 if cb_block else 16
    _check(_lib.mth_oil4_gemv_noalloc(_ptr(packed, t.uint8, M * K // 2, "packed"),
                                      _ptr(codebooks, t.int16, ncb, "codebooks"), cb_block,
                                      _ptr(x, t.float32, batch * K, "x"), _ptr(y, t.float32, batch * M, "y"),
                                      M, K, batch, _stream(stream)))


def oil4_gemm_prefill(a_bf16, packed, codebooks, cb_block, c_bf16, M, N, K, stream=None):
    t = _torch()
    _check(_lib.mth_oil4_gemm_prefill(_ptr(a_bf16, t.bfloat16, M * K, "a"), _ptr(packed, t.uint8, N * K // 2, "packed"),
                                      _ptr(codebooks, t.int16, N * (K // cb_block) * 16, "codebooks"), cb_block,
                                      _ptr(c_bf16, t.bfloat16, M * N, "c"), M, N, K, _stream(stream)))


def quantize_per_token(src, dst, scale, inv_scale, rows, cols, stream=None):
    t = _torch()
    _check(_lib.mth_quantize_per_token(_ptr(src, t.float32, rows * cols, "src"), _ptr(dst, t.int8, rows * cols, "dst"),
                                       _ptr(scale, t.float32, rows, "scale") if scale is not None else None,
                                       _ptr(inv_scale, t.float32, rows, "inv_scale") if inv_scale is not None else None,
                                       rows, cols, _stream(stream)))


def dequantize_per_tensor(src, dst, n, inv_scale, stream=None):
    t = _torch()
    _check(_lib.mth_dequantize_per_tensor(_ptr(src, t.int8, n, "src"), _ptr(dst, t.float32, n, "dst"), n,
                                          float(inv_scale), _stream(stream)))


def i2s_gemv(packed, w_scale, act, act_scale, y, M, K, batch=1, stream=None):
    t = _torch()
    _check(_lib.mth_i2s_gemv(_ptr(packed, t.uint8, M * K // 4, "packed"), float(w_scale),
                             _ptr(act, t.int8, batch * K, "act"), _ptr(act_scale, t.float32, batch, "act_scale"),
                             _ptr(y, t.float32, batch * M, "y"), M, K, batch, _stream(stream)))


def i2s_gemv_f32(packed, w_scale, x, y, M, K, batch=1, stream=None):
    t = _torch()
    _check(_lib.mth_i2s_gemv_f32(_ptr(packed, t.uint8, M * K // 4, "packed"), float(w_scale),
                                 _ptr(x, t.float32, batch * K, "x"), _ptr(y, t.float32, batch * M, "y"),
                                 M, K, batch, _stream(stream)))


def i2s_gemm(w, act, out, M, N, K, stream=None):
    t = _torch()
    _check(_lib.mth_i2s_gemm(_ptr(w, t.uint8, _i2s_bytes(M, K), "w"), _ptr(act, t.float32, N * K, "act"),
                             _ptr(out, t.float32, M * N, "out"), M, N, K, _stream(stream)))


def i2s_gemm_vnni(w, act, out, M, N, K, stream=None):
    t = _torch()
    _check(_lib.mth_i2s_gemm_vnni(_ptr(w, t.uint8, _i2s_bytes(M, K), "w"), _ptr(act, t.int8, N * K, "act"),
                                  _ptr(out, t.float32, M * N, "out"), M, N, K, _stream(stream)))


def tl1_gemm(w, act, out, M, N, K, stream=None):
    t = _torch()
    _check(_lib.mth_tl1_gemm(_ptr(w, t.uint8, (M * N * K) // 4, "w"), _ptr(act, t.float32, N * K, "act"),
                             _ptr(out, t.float32, M * N, "out"), M, N, K, _stream(stream)))


def tl2_gemm(w, act, out, M, N, K, stream=None):
    t = _torch()
    _check(_lib.mth_tl2_gemm(_ptr(w, t.uint8, M * N * ((2 * K + 7) // 8), "w"), _ptr(act, t.float32, N * K, "act"),
                             _ptr(out, t.float32, M * N, "out"), M, N, K, _stream(stream)))


def tl_precompute_lut(act, lut, K, group, stream=None):
    t = _torch()
    n = (K // group) * (9 if group == 2 else 27)
    _check(_lib.mth_tl_precompute_lut(_ptr(act, t.int8, K, "act"), _ptr(lut, t.int8, n, "lut"), K, group,
                                      _stream(stream)))


# ---- FP32 decode-step operators ---------------------------------------------
def rms_norm(x, gamma, y, rows, dim, eps=1e-5, stream=None):
    t = _torch()
    _check(_lib.mth_rms_norm(_ptr(x, t.float32, rows * dim, "x"), _ptr(gamma, t.float32, dim, "gamma"),
                             _ptr(y, t.float32, rows * dim, "y"), rows, dim, eps, _stream(stream)))


def add_rms_norm(x, res, gamma, y, rows, dim, eps=1e-5, stream=None):
    """x <- res + x, y = rms_norm(x) * gamma."""
    t = _torch()
    _check(_lib.mth_add_rms_norm(_ptr(x, t.float32, rows * dim, "x"), _ptr(res, t.float32, rows * dim, "res"),
                                 _ptr(gamma, t.float32, dim, "gamma"), _ptr(y, t.float32, rows * dim, "y"), rows, dim,
                                 eps, _stream(stream)))


def silu(x, y, n, stream=None):
    t = _torch()
    _check(_lib.mth_silu(_ptr(x, t.float32, n, "x"), _ptr(y, t.float32, n, "y"), n, _stream(stream)))


def silu_mul(g, u, y, rows, n, gstride=None, ustride=None, stream=None):
    t = _torch()
    gs, us = gstride or n, ustride or n
    _check(_lib.mth_silu_mul(_ptr(g, t.float32, (rows - 1) * gs + n, "g"), _ptr(u, t.float32, (rows - 1) * us + n, "u"),
                             _ptr(y, t.float32, rows * n, "y"), rows, n, gs, us, _stream(stream)))


def silu_mul_quant(g, u, q, inv_scale, rows, n, gstride=None, ustride=None, stream=None):
    t = _torch()
    gs, us = gstride or n, ustride or n
    _check(_lib.mth_silu_mul_quant(_ptr(g, t.float32, (rows - 1) * gs + n, "g"),
                                   _ptr(u, t.float32, (rows - 1) * us + n, "u"), _ptr(q, t.int8, rows * n, "q"),
                                   _ptr(inv_scale, t.float32, rows, "inv_scale"), rows, n, gs, us, _stream(stream)))


def oil4_gemv_swiglu(packed, codebooks, x, act, amax, F, K, stream=None):
    """Gate/up projections of one OIL4 weight of 2F rows (per-128 codebooks)
    and the SwiGLU: act[F] = silu(g) * u, amax[F // 8] = max |act| per 8."""
    t = _torch()
    _check(_lib.mth_oil4_gemv_swiglu(_ptr(packed, t.uint8, 2 * F * K // 2, "packed"),
                                     _ptr(codebooks, t.int16, 2 * F * (K // 128) * 16, "codebooks"),
                                     _ptr(x, t.float32, K, "x"), _ptr(act, t.float32, F, "act"),
                                     _ptr(amax, t.float32, F // 8, "amax"), F, K, _stream(stream)))


def i2s_gemv_act(packed, w_scale, act, amax, y, M, K, stream=None):
    """I2_S GEMV of quantize_per_token(act), amax as from oil4_gemv_swiglu."""
    t = _torch()
    _check(_lib.mth_i2s_gemv_act(_ptr(packed, t.uint8, M * K // 4, "packed"), float(w_scale),
                                 _ptr(act, t.float32, K, "act"), _ptr(amax, t.float32, K // 8, "amax"),
                                 _ptr(y, t.float32, M, "y"), M, K, _stream(stream)))


def swiglu_batch_parts(F):
    """Block maxima per token written by oil4_gemv_swiglu_batch (one per 256 columns)."""
    return int(_lib.mth_swiglu_batch_parts(F))


def oil4_gemv_swiglu_batch(packed, codebooks, cb_block, x, gu, amax, F, K, batch, stream=None):
    """Batches of 2..16: gate/up of one OIL4 weight of 2F rows and the SwiGLU;
    act of token t in gu[t, :F] (gu is [batch][2F]), amax [batch][parts]."""
    t = _torch()
    nb = K // cb_block if cb_block else 1
    _check(_lib.mth_oil4_gemv_swiglu_batch(
        _ptr(packed, t.uint8, 2 * F * K // 2, "packed"),
        _ptr(codebooks, t.int16, (2 * F * nb if cb_block else 1) * 16, "codebooks"), cb_block,
        _ptr(x, t.float32, batch * K, "x"), _ptr(gu, t.float32, batch * 2 * F, "gu"),
        _ptr(amax, t.float32, batch * swiglu_batch_parts(F), "amax"), F, K, batch, _stream(stream)))


def i2s_gemv_act_batch(packed, w_scale, act, lda, amax, inv_scale, y, M, K, batch, stream=None):
    """Batches of 2..16: I2_S GEMV of quantize_per_token(act rows, stride lda),
    amax as from oil4_gemv_swiglu_batch; inv_scale [batch] = max|act| / 127."""
    t = _torch()
    _check(_lib.mth_i2s_gemv_act_batch(
        _ptr(packed, t.uint8, M * K // 4, "packed"), float(w_scale), _ptr(act, t.float32, (batch - 1) * lda + K, "act"),
        lda, _ptr(amax, t.float32, batch * swiglu_batch_parts(K), "amax"),
        _ptr(inv_scale, t.float32, batch, "inv_scale"), _ptr(y, t.float32, batch * M, "y"), M, K, batch,
        _stream(stream)))


def add(a, b, c, n, stream=None):
    t = _torch()
    _check(_lib.mth_add(_ptr(a, t.float32, n, "a"), _ptr(b, t.float32, n, "b"), _ptr(c, t.float32, n, "c"), n,
                        _stream(stream)))


def mul(a, b, c, n, stream=None):
    t = _torch()
    _check(_lib.mth_mul(_ptr(a, t.float32, n, "a"), _ptr(b, t.float32, n, "b"), _ptr(c, t.float32, n, "c"), n,
                        _stream(stream)))


def softmax(x, y, rows, dim, stream=None):
    t = _torch()
    _check(_lib.mth_softmax(_ptr(x, t.float32, rows * dim, "x"), _ptr(y, t.float32, rows * dim, "y"), rows, dim,
                            _stream(stream)))


def softmax_axis(x, y, outer, dim, inner, stream=None):
    t = _torch()
    n = outer * dim * inner
    _check(_lib.mth_softmax_axis(_ptr(x, t.float32, n, "x"), _ptr(y, t.float32, n, "y"), outer, dim, inner,
                                 _stream(stream)))


def axpby(alpha, x, beta, y, n, stream=None):
    t = _torch()
    _check(_lib.mth_axpby(alpha, _ptr(x, t.float32, n, "x"), beta, _ptr(y, t.float32, n, "y"), n, _stream(stream)))


def gemv_f32(alpha, A, x, beta, y, M, N, stream=None):
    t = _torch()
    _check(_lib.mth_gemv_f32(alpha, _ptr(A, t.float32, M * N, "A"), _ptr(x, t.float32, N, "x"), beta,
                             _ptr(y, t.float32, M, "y"), M, N, _stream(stream)))


def relu(x, y, n, stream=None):
    t = _torch()
    _check(_lib.mth_relu(_ptr(x, t.float32, n, "x"), _ptr(y, t.float32, n, "y"), n, _stream(stream)))


def gelu(x, y, n, stream=None):
    t = _torch()
    _check(_lib.mth_gelu(_ptr(x, t.float32, n, "x"), _ptr(y, t.float32, n, "y"), n, _stream(stream)))


def scale(s, x, y, n, stream=None):
    t = _torch()
    _check(_lib.mth_scale(s, _ptr(x, t.float32, n, "x"), _ptr(y, t.float32, n, "y"), n, _stream(stream)))


def layer_norm(x, gamma, beta, y, rows, dim, eps=1e-5, stream=None):
    t = _torch()
    _check(_lib.mth_layer_norm(_ptr(x, t.float32, rows * dim, "x"), _ptr(gamma, t.float32, dim, "gamma"),
                               _ptr(beta, t.float32, dim, "beta"), _ptr(y, t.float32, rows * dim, "y"), rows, dim,
                               eps, _stream(stream)))


def rope_tables(head_dim, max_seq, theta=10000.0):
    """Host (numpy) cos/sin tables [max_seq][head_dim/2]."""
    import numpy as np
    c = np.empty((max_seq, head_dim // 2), np.float32)
    s = np.empty((max_seq, head_dim // 2), np.float32)
    _check(_lib.mth_rope_tables(head_dim, max_seq, theta, c.ctypes.data, s.ctypes.data))
    return c, s


def rope_kv(q, k, v, cos_t, sin_t, kcache, vcache, pos, batch, heads, kv_heads, head_dim, max_seq, stream=None):
    t = _torch()
    kv = batch * kv_heads * head_dim
    cache = batch * kv_heads * max_seq * head_dim
    _check(_lib.mth_rope_kv(_ptr(q, t.float32, batch * heads * head_dim, "q"), _ptr(k, t.float32, kv, "k"),
                            _ptr(v, t.float32, kv, "v"), _ptr(cos_t, t.float32, max_seq * head_dim // 2, "cos"),
                            _ptr(sin_t, t.float32, max_seq * head_dim // 2, "sin"),
                            _ptr(kcache, t.float32, cache, "kcache"), _ptr(vcache, t.float32, cache, "vcache"),
                            pos, batch, heads, kv_heads, head_dim, max_seq, _stream(stream)))


def attention_decode(q, kcache, vcache, out, batch, heads, kv_heads, head_dim, ctx, max_seq, stream=None):
    t = _torch()
    cache = batch * kv_heads * max_seq * head_dim
    _check(_lib.mth_attention_decode(_ptr(q, t.float32, batch * heads * head_dim, "q"),
                                     _ptr(kcache, t.float32, cache, "kcache"), _ptr(vcache, t.float32, cache, "vcache"),
                                     _ptr(out, t.float32, batch * heads * head_dim, "out"), batch, heads, kv_heads,
                                     head_dim, ctx, max_seq, _stream(stream)))


def argmax(logits, ids, rows, n, stream=None):
    t = _torch()
    _check(_lib.mth_argmax(_ptr(logits, t.float32, rows * n, "logits"), _ptr(ids, t.int32, rows, "ids"), rows, n,
                           _stream(stream)))

