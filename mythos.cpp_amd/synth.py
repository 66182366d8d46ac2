"""Seeded synthetic inputs for the BASELINE configurations (numpy, host side).

Distributions follow the benchmark definitions: OIL8 indices uniform 0..255
into one sorted N(0, 0.02) FP32 codebook; OIL4 nibbles uniform 0..15 with one
16-entry FP16 codebook per 128-weight row block, N(0, 0.02) values converted
with the reference's truncating float_to_half (src/codebook.cpp:16-34);
ternary weights uniform over {-1, 0, +1} packed with code t+1, four per byte,
element 4i+j in bits 2j of byte i (src/kernel_i2s.cpp:13-30,
tools/convert.cpp:329-342); activations N(0, 1).  The generator is numpy's
PCG64 seeded with 0x5EED0000 + config number.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x5EED0000
W_SCALE_TERNARY = 0.0159577  # E|N(0, 0.02)| = 0.02*sqrt(2/pi), the absmean scale


def rng(config: int, salt: int = 0) -> np.random.Generator:
    return np.random.default_rng(SEED_BASE + config + (salt << 8))


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
    g = rng(config)
    idx = g.integers(0, 256, size=(M, K), dtype=np.uint8)
    cb = np.sort(g.normal(0.0, 0.02, 256)).astype(np.float32)
    x = g.normal(0.0, 1.0, (batch, K)).astype(np.float32)
    return idx, cb, x


def oil4(M: int, K: int, batch: int, block: int = 128, config: int = 2):
    g = rng(config)
    nib = g.integers(0, 16, size=(M, K), dtype=np.uint8)
    packed = pack_nibbles(nib)
    ncb = M * (K // block) if block else 1
    cbs = float_to_half_trunc(g.normal(0.0, 0.02, (ncb, 16)).astype(np.float32))
    x = g.normal(0.0, 1.0, (batch, K)).astype(np.float32)
    return packed, cbs.reshape(-1), x


def ternary(M: int, K: int, batch: int, config: int = 3):
    g = rng(config)
    t = g.integers(-1, 2, size=(M, K), dtype=np.int8)
    packed = pack_ternary(t)
    x = g.normal(0.0, 1.0, (batch, K)).astype(np.float32)
    return packed, np.float32(W_SCALE_TERNARY), x


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """FP32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def prefill(M: int, N: int, K: int, block: int = 128, config: int = 4):
    g = rng(config)
    a = bf16_bits(g.normal(0.0, 1.0, (M, K)).astype(np.float32))
    nib = g.integers(0, 16, size=(N, K), dtype=np.uint8)
    packed = pack_nibbles(nib)
    cbs = float_to_half_trunc(g.normal(0.0, 0.02, (N * (K // block), 16)).astype(np.float32))
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
