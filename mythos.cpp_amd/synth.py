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
    next_u64() >> 11.
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
for _f in ("mth_synth_seed", "mth_synth_u64", "mth_synth_bits", "mth_synth_uniform_int", "mth_synth_normal"):
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
    cbs = float_to_half_trunc(g.normal((ncb, 16), 0.0, 0.02))
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
    cbs = float_to_half_trunc(g.normal((N * (K // block), 16), 0.0, 0.02))
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
