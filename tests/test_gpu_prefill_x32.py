"""GPU parity of the FP32-row MFMA GEMMs the prompt prefill runs (and the C
ABI's mth_oil8_gemv / mth_oil4_gemv for batches of 128 tokens and more)
against the CPU oracle.

Per token these are the decode GEMVs (src/kernel_oil8.cpp:14-27, 63-71;
src/kernel_oil4.cpp:31-54 with per-128 codebooks): FP32 products summed in
FP32.  The GEMMs split each row (and the OIL8 codebook) into FP16 hi + lo
parts after a power-of-two scale and sum the exact products in FP32, so the
bar is the FP32 one: 1e-5 of sum|w*x| per element.  Integer codebooks and
activations make every product and partial sum an exact integer, so those
cases must give the oracle's bits (a dropped or mis-scaled product term, a
wrong row shift or a swapped hi / lo group shows).
"""
import numpy as np
import pytest

import synth
from conftest import fp32_close
from test_gpu_gemv import empty, to_dev

pytestmark = pytest.mark.gpu


def run_oil8(mth, dev, idx, cb, x, M, K, B):
    import torch
    y = empty(B * M, torch.float32, dev)
    mth.oil8_gemv(to_dev(idx, dev), to_dev(cb, dev), to_dev(x, dev), y, M, K, B)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(B, M)


def absw8(idx, cb, x):
    with np.errstate(all="ignore"):
        return (np.abs(cb[idx]).astype(np.float64) @ np.abs(x.astype(np.float64)).T).T


# ------------------------------------------------------------------ OIL8 --
@pytest.mark.parametrize("M,K,B", [
    (4096, 4096, 256),   # config 1 weights, two M tiles of 128 tokens
    (4096, 4096, 1024),  # the b=16 x 64-token prompt chunk: 8 M tiles, one per XCD
    (320, 1024, 130),    # ragged last M tile (2 rows), 5 column tiles
    (64, 512, 128),      # one tile
    (192, 256, 1000),    # 8 M tiles, the last one partial
])
def test_oil8_gemm_x32(M, K, B, oracle, mth, dev):
    print(f"oil8 x32 GEMM M={M} K={K} B={B}", flush=True)
    idx, cb, x = synth.oil8(M, K, B)
    got = run_oil8(mth, dev, idx, cb, x, M, K, B)
    ref = oracle.oil8_gemv(idx, cb, x, M, K, B, threads=8)
    fp32_close(got, ref, absw8(idx, cb, x), 1e-5, "oil8 x32 GEMM")


# (4096, 512, 1024): tiles of 256 rows on 8 consumer waves (they fill a round of
# 256 workgroups); the others tiles of 128 rows on 4
@pytest.mark.parametrize("M,K,B", [(384, 2048, 200), (4096, 512, 1024)])
def test_oil8_gemm_x32_integer_bit_exact(M, K, B, oracle, mth, dev):
    g = np.random.default_rng(21)
    idx = g.integers(0, 256, (M, K), dtype=np.uint8)
    cb = (np.arange(256) - 128).astype(np.float32) * 3
    x = g.integers(-3, 4, (B, K)).astype(np.float32)
    print(f"oil8 x32 GEMM integer M={M} K={K} B={B}", flush=True)
    got = run_oil8(mth, dev, idx, cb, x, M, K, B)
    assert np.array_equal(got, oracle.oil8_gemv(idx, cb, x, M, K, B))


@pytest.mark.parametrize("M,K,B", [(256, 2048, 160), (4096, 256, 1024)])
def test_oil8_gemm_x32_range(M, K, B, oracle, mth, dev):
    """Codebook magnitudes 2^-60 .. 2^40 and row scales 2^-40 .. 2^40 (every
    product and sum a normal FP32 number), an all-zero row too: the
    power-of-two scales of rows and codebook put every hi / lo part in FP16's
    range, so the FP32 bar holds for every row."""
    g = np.random.default_rng(22)
    idx = g.integers(0, 256, (M, K), dtype=np.uint8)
    cb = (g.normal(0, 1, 256) * np.exp2(g.integers(-60, 40, 256))).astype(np.float32)
    x = (g.normal(0, 1, (B, K)) * np.exp2(np.linspace(-40, 40, B).round())[:, None]).astype(np.float32)
    x[B // 3] = 0.0
    print(f"oil8 x32 GEMM range M={M} K={K} B={B}", flush=True)
    got = run_oil8(mth, dev, idx, cb, x, M, K, B)
    ref = oracle.oil8_gemv(idx, cb, x, M, K, B, threads=8)
    aw = absw8(idx, cb, x)
    assert not got[B // 3].any()
    for t in range(B):
        fp32_close(got[t], ref[t], aw[t], 1e-5, f"oil8 x32 range row {t}")


@pytest.mark.parametrize("M,K,B", [(192, 1024, 300), (4096, 256, 1000)])
@pytest.mark.parametrize("where", ["codebook_inf", "codebook_nan", "x_inf", "x_nan"])
def test_oil8_gemm_x32_non_finite(where, M, K, B, oracle, mth, dev):
    """Workgroups whose codebook or rows hold Inf / NaN sum the reference's
    FP32 products directly: non-finite outputs match the oracle's class (NaN,
    +Inf, -Inf) element by element, finite ones the FP32 bar (the other M
    tiles keep the MFMA path).  (4096, 256, 1000): tiles of 256 rows."""
    g = np.random.default_rng(23)
    idx = g.integers(0, 256, (M, K), dtype=np.uint8)
    cb = g.normal(0, 0.02, 256).astype(np.float32)
    x = g.normal(0, 1, (B, K)).astype(np.float32)
    if where == "codebook_inf":
        cb[17], cb[200] = np.inf, -np.inf
        idx[idx == 17] = 18
        idx[idx == 200] = 201
        idx[:60, 5] = 17          # rows 0..59 only see +Inf, rows 60..119 only -Inf
        idx[60:120, 9] = 200
    elif where == "codebook_nan":
        cb[3] = np.nan
        idx[idx == 3] = 4
        idx[150:, 100] = 3
    elif where == "x_inf":
        x[1, 77] = np.inf
        x[290, 3] = -np.inf
    else:
        x[140, 200] = np.nan
    print(f"oil8 x32 GEMM non-finite {where}", flush=True)
    got = run_oil8(mth, dev, idx, cb, x, M, K, B)
    with np.errstate(all="ignore"):
        ref = oracle.oil8_gemv(idx, cb, x, M, K, B, threads=8)
    fin = np.isfinite(ref)
    assert (~fin).any() and fin.any()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fp32_close(got[fin], ref[fin], absw8(idx, cb, x)[fin], 1e-5, f"oil8 x32 finite outputs ({where})")


def test_oil8_gemm_x32_deterministic(mth, dev):
    import torch
    M, K, B = 512, 1024, 256
    idx, cb, x = synth.oil8(M, K, B)
    a = run_oil8(mth, dev, idx, cb, x, M, K, B)
    b = run_oil8(mth, dev, idx, cb, x, M, K, B)
    assert np.array_equal(a, b)
    assert torch.cuda.is_available()


# ------------------------------------------------------------------ OIL4 --
def run_oil4(mth, dev, packed, cbs, block, x, M, K, B):
    import torch
    y = empty(B * M, torch.float32, dev)
    mth.oil4_gemv(to_dev(packed, dev), to_dev(cbs, dev), block, to_dev(x, dev), y, M, K, B)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(B, M)


@pytest.mark.parametrize("M,K,B", [
    (11008, 4096, 256),  # config 2 weights
    (22016, 4096, 128),  # the decoder's fused gate / up at config 5, one M tile
    (448, 1024, 130),    # ragged last M tile
    (4096, 1024, 1024),  # 128-column tiles (a full round of 256 workgroups)
    (2048, 512, 2000),   # 128-column tiles, 16 M tiles, the last one ragged
])
def test_oil4_gemm_x32(M, K, B, oracle, mth, dev):
    print(f"oil4 x32 GEMM M={M} K={K} B={B}", flush=True)
    packed, cbs, x = synth.oil4(M, K, B, 128)
    got = run_oil4(mth, dev, packed, cbs, 128, x, M, K, B)
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, B, 128, threads=8)
    W = synth.dequant_oil4(packed, cbs, M, K, 128)
    absw = (np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64)).T).T
    fp32_close(got, ref, absw, 1e-5, "oil4 x32 GEMM")


@pytest.mark.parametrize("M,K,B", [(192, 1024, 140), (4096, 512, 1024)])
def test_oil4_gemm_x32_integer_bit_exact(M, K, B, oracle, mth, dev):
    g = np.random.default_rng(24)
    nib = g.integers(0, 16, (M, K), dtype=np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    vals = g.integers(-40, 41, M * (K // 128) * 16).astype(np.float32)
    cbs = synth.float_to_half_trunc(vals)
    x = g.integers(-3, 4, (B, K)).astype(np.float32)
    print(f"oil4 x32 GEMM integer M={M} K={K} B={B}", flush=True)
    got = run_oil4(mth, dev, packed, cbs, 128, x, M, K, B)
    assert np.array_equal(got, oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, B, 128))
