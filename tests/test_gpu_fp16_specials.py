"""GPU parity of the OIL4 kernels on FP16 codebook values at the edges of the
format: subnormals, signed zeros, the largest normal, +-Inf and NaN.

The reference decodes every codebook entry exactly, subnormals included
(fp16_to_float, src/kernel_oil4.cpp:15-29), and multiplies in FP32
(src/kernel_oil4.cpp:50).  Each case is run through every OIL4 kernel family,
chosen by shape (the launcher's dispatch rules):
  v2       batch 1, cb_block 128, K 4096      (oil4_gemv_v2, v_perm lookups)
  mfma     batch 1, cb_block 256              (oil4_gemv_mfma, LDS gathers)
  valu     batch 1, cb_block 64               (oil4_gemv_valu, FP32 FMA)
  generic  K = 1000, cb_block 100             (oil4_generic)
  bt       batch 4, cb_block 128              (oil4_gemv_bt, split-K MFMA)
  x32      batch 130, cb_block 128            (oil4_prefill_a16x + oil4_prefill_ws<X32>, the GEMM route)
  prefill  bf16 A: oil4_prefill_ws (N % 96 == 0), oil4_prefill_mfma, oil4_gemm_prefill_k

A flush of subnormals to zero would turn the all-subnormal case's outputs into
0 (relative error 1); the bar is 1e-5 of sum|w*x| per element.  NaN outputs
must be NaN exactly where the oracle's are, infinite outputs equal.  The
integer-codebook case has every partial sum an exact integer, so any
summation order gives the oracle's bits.
"""
import zlib

import numpy as np
import pytest

import synth
from conftest import fp32_close
from test_gpu_gemv import empty, to_dev

pytestmark = pytest.mark.gpu

GEMV_PATHS = [  # name, M, K, batch, cb_block
    ("v2", 256, 4096, 1, 128),
    ("mfma", 128, 2048, 1, 256),
    ("valu", 96, 1024, 1, 64),
    ("generic", 40, 1000, 1, 100),
    ("bt", 200, 2048, 4, 128),
    ("x32", 256, 1024, 130, 128),  # >= 128 tokens: the FP32-row MFMA GEMM (rows split into FP16 hi / lo)
]
# producer/consumer FP16-A kernel (N a multiple of 96), the LDS-staged kernel
# (N fits no tile of the former), the first kernel (codebook block 32)
PREFILL_PATHS = [("prefill_ws", 128, 96, 512, 128), ("prefill_mfma", 72, 100, 512, 128),
                 ("prefill_k", 64, 80, 256, 32)]


def codebooks(kind, rows, nblk, seed):
    """FP16 bit patterns [rows][nblk][16] of one kind of special values."""
    g = np.random.default_rng(seed)
    n = rows * nblk * 16
    normal = synth.float_to_half_trunc(g.normal(0, 0.02, n).astype(np.float32))
    if kind == "subnormal":   # only subnormals: exponent 0, mantissa 1..1023, either sign
        cb = (g.integers(1, 1024, n) | (g.integers(0, 2, n) << 15)).astype(np.uint16)
    elif kind == "edges":     # +-0, +-max normal, min normal, subnormals and normals mixed
        pool = np.array([0x0000, 0x8000, 0x7BFF, 0xFBFF, 0x0400, 0x8400, 0x0001, 0x83FF, 0x03FF], np.uint16)
        cb = np.where(g.random(n) < 0.5, pool[g.integers(0, len(pool), n)], normal).astype(np.uint16)
    elif kind in ("inf", "nan"):
        cb = normal.reshape(rows, nblk * 16).copy()
        special = [0x7C00, 0xFC00] if kind == "inf" else [0x7E00, 0xFE01]
        for r in range(0, rows, 5):  # every 5th row holds one special entry in one block
            cb[r, g.integers(0, nblk * 16)] = special[r // 5 % 2]
        cb = cb.ravel()
    else:
        raise ValueError(kind)
    return cb.astype(np.uint16)


def nonfinite_close(got, ref, absw, what):
    got, ref = np.asarray(got, np.float64).ravel(), np.asarray(ref, np.float64).ravel()
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r), f"{what}: NaN at {np.flatnonzero(nan_g != nan_r)[:8]}"
    inf_r = np.isinf(ref)
    assert np.array_equal(got[inf_r], ref[inf_r]), f"{what}: infinite outputs differ"
    fin = ~nan_r & ~inf_r
    assert fin.any() and (nan_r | inf_r).any(), f"{what}: case does not mix finite and non-finite rows"
    fp32_close(got[fin], ref[fin], np.asarray(absw).ravel()[fin], 1e-5, what)


@pytest.mark.parametrize("kind", ["subnormal", "edges", "inf", "nan"])
@pytest.mark.parametrize("path,M,K,batch,block", GEMV_PATHS)
def test_oil4_gemv_fp16_specials(path, M, K, batch, block, kind, oracle, mth, dev):
    import torch
    print(f"oil4 specials {kind} path={path} M={M} K={K} batch={batch} block={block}", flush=True)
    g = np.random.default_rng(zlib.crc32(f"{path}/{kind}".encode()))
    packed = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    cbs = codebooks(kind, M, K // block, 7)
    x = g.normal(0, 1, (batch, K)).astype(np.float32)
    y = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv(to_dev(packed, dev), to_dev(cbs, dev), block, to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
    with np.errstate(invalid="ignore", over="ignore"):
        W = synth.dequant_oil4(packed, cbs, M, K, block).astype(np.float64)
        absw = (np.abs(W) @ np.abs(x.astype(np.float64)).T).T
    got = y.cpu().numpy().reshape(batch, M)
    if kind in ("inf", "nan"):
        nonfinite_close(got, ref, absw, f"{path}/{kind}")
    else:
        fp32_close(got, ref, absw, 1e-5, f"{path}/{kind}")
        if kind == "subnormal":  # the values are far below the bar's floor: nothing flushed
            assert np.all(np.abs(ref) > 0) and np.all(np.abs(got) > 0)


@pytest.mark.parametrize("kind", ["subnormal", "edges", "inf"])
@pytest.mark.parametrize("path,M,N,K,block", PREFILL_PATHS)
def test_oil4_prefill_fp16_specials(path, M, N, K, block, kind, oracle, mth, dev):
    """Prefill: W exact in FP16 (specials included), A bf16 -> FP16 (exact
    for these N(0,1) values), FP32 sums, bf16 output; one bf16 rounding of the
    oracle's FP32 result per element."""
    import torch
    print(f"prefill specials {kind} path={path} M={M} N={N} K={K} block={block}", flush=True)
    g = np.random.default_rng(zlib.crc32(f"{path}/{kind}".encode()))
    a = synth.bf16_bits(g.normal(0, 1, (M, K)).astype(np.float32))
    packed = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    cbs = codebooks(kind, N, K // block, 9)
    c = torch.zeros(M * N, dtype=torch.bfloat16, device=dev)
    mth.oil4_gemm_prefill(to_dev(a, dev).view(torch.bfloat16), to_dev(packed, dev), to_dev(cbs, dev), block, c,
                          M, N, K)
    torch.cuda.synchronize()
    _, ref32 = oracle.oil4_gemm_prefill(a, packed, cbs, M, N, K, block, threads=8)
    got = synth.bf16_to_f32(c.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(M, N).astype(np.float64)
    ref = ref32.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        W = synth.dequant_oil4(packed, cbs, N, K, block).astype(np.float64)
        absw = np.abs(synth.bf16_to_f32(a).astype(np.float64)) @ np.abs(W).T
    if kind == "inf":
        nan_g, nan_r = np.isnan(got), np.isnan(ref)
        assert np.array_equal(nan_g, nan_r)
        inf_r = np.isinf(ref)
        assert inf_r.any() and np.array_equal(got[inf_r], ref[inf_r])
        fin = ~nan_r & ~inf_r
        got, ref, absw = got[fin], ref[fin], absw[fin]
    d = np.abs(got - ref)
    bound = 2.0 ** -8 * np.abs(ref) + 1e-5 * absw
    assert (d <= bound).all(), f"{path}/{kind}: {(d > bound).sum()} elements out of bound"
    if kind == "subnormal":
        assert np.all(got != 0)


@pytest.mark.parametrize("path,M,K,batch,block", GEMV_PATHS)
def test_oil4_integer_codebook_bit_exact(path, M, K, batch, block, oracle, mth, dev):
    """Integer codebook entries (-8..7, exact in FP16) and integer x in
    [-3, 3]: every product and partial sum is an integer below 2^24, so the
    result is exact in any summation order and must equal the oracle's bits."""
    import torch
    print(f"oil4 integer codebook path={path} M={M} K={K} batch={batch}", flush=True)
    g = np.random.default_rng(17)
    packed = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    vals = g.integers(-8, 8, M * (K // block) * 16).astype(np.float16)
    cbs = vals.view(np.uint16)
    x = g.integers(-3, 4, (batch, K)).astype(np.float32)
    y = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv(to_dev(packed, dev), to_dev(cbs, dev), block, to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
    assert np.array_equal(y.cpu().numpy().reshape(batch, M), ref)


@pytest.mark.parametrize("path,M,N,K,block", PREFILL_PATHS)
def test_oil4_prefill_integer_bit_exact(path, M, N, K, block, oracle, mth, dev):
    """Integer A and codebooks: the FP32 sums are exact integers, so the bf16
    output must be the round-to-nearest-even of the exact value, as the
    oracle's."""
    import torch
    g = np.random.default_rng(19)
    a = synth.bf16_bits(g.integers(-3, 4, (M, K)).astype(np.float32))
    packed = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    cbs = g.integers(-8, 8, N * (K // block) * 16).astype(np.float16).view(np.uint16)
    c = torch.zeros(M * N, dtype=torch.bfloat16, device=dev)
    mth.oil4_gemm_prefill(to_dev(a, dev).view(torch.bfloat16), to_dev(packed, dev), to_dev(cbs, dev), block, c,
                          M, N, K)
    torch.cuda.synchronize()
    ref16, _ = oracle.oil4_gemm_prefill(a, packed, cbs, M, N, K, block, threads=8)
    assert np.array_equal(c.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N), ref16)


@pytest.mark.parametrize("path,M,K,batch,block", GEMV_PATHS)
def test_oil4_gemv_x_wide_range(path, M, K, batch, block, oracle, mth, dev):
    """x with magnitudes spread over 2^-70 .. 2^6 (every binade, both signs,
    some exact zeros): the FP16 hi/lo split of the MFMA paths loses the
    bits of values far below max|x|, by at most max|c| max|x| 2^-40 per
    product, which the 1e-5 bar of sum|w*x| absorbs; the batch-1 kernel
    recomputes such waves with FP32 products."""
    import torch
    print(f"oil4 wide-range x path={path} M={M} K={K} batch={batch}", flush=True)
    g = np.random.default_rng(zlib.crc32(f"{path}/wide".encode()))
    packed = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    cbs = codebooks("edges", M, K // block, 11)
    x = (g.choice([-1.0, 1.0], (batch, K)) * np.exp2(g.uniform(-70, 6, (batch, K)))).astype(np.float32)
    x[:, ::37] = 0.0
    y = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv(to_dev(packed, dev), to_dev(cbs, dev), block, to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
    W = synth.dequant_oil4(packed, cbs, M, K, block).astype(np.float64)
    absw = (np.abs(W) @ np.abs(x.astype(np.float64)).T).T
    fp32_close(y.cpu().numpy().reshape(batch, M), ref, absw, 1e-5, f"{path}/wide")


# paths whose products come from an FP16 hi/lo split of x without an FP32
# fallback (batch >= 2, codebook blocks of 256): an infinite codebook entry
# times an x_k whose hi part underflows to 0 gives NaN, the reference +-Inf
HILO_NO_FALLBACK = {"mfma", "bt", "x32"}


@pytest.mark.parametrize("path,M,K,batch,block", GEMV_PATHS)
def test_oil4_gemv_inf_times_tiny_x(path, M, K, batch, block, oracle, mth, dev):
    """Every infinite codebook entry is selected only at columns where x is
    2^-60 times smaller than the rest, so the reference's products there are
    +-Inf (src/kernel_oil4.cpp:50).  The batch-1 kernel (its FP32 fallback),
    the FP32 and generic kernels give the oracle's +-Inf; the hi/lo kernels
    without a fallback give NaN in exactly those rows (pinned, documented)."""
    import torch
    print(f"oil4 inf x tiny path={path} M={M} K={K} batch={batch}", flush=True)
    g = np.random.default_rng(zlib.crc32(f"{path}/inftiny".encode()))
    nblk = K // block
    cbs = codebooks("inf", M, nblk, 13).reshape(M, nblk, 16)
    nib = g.integers(0, 16, (M, K), dtype=np.uint8)
    x = g.normal(0, 1, (batch, K)).astype(np.float32)
    x[:, 1::2] *= np.float32(2.0 ** -60)              # odd columns tiny
    isinf = np.isinf(synth.fp16_bits_to_f32(cbs.ravel()).reshape(M, nblk, 16))
    for r, b, e in zip(*np.nonzero(isinf)):            # infinite entry e of block b: only at odd columns
        cols = np.arange(b * block, (b + 1) * block)
        even = cols[(cols % 2 == 0) & (nib[r, cols] == e)]
        nib[r, even] = (e + 1) % 16
        nib[r, b * block + 1] = e                      # and used at least once
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    cbs = cbs.ravel()
    y = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv(to_dev(packed, dev), to_dev(cbs, dev), block, to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
    got = y.cpu().numpy().reshape(batch, M)
    with np.errstate(invalid="ignore", over="ignore"):
        W = synth.dequant_oil4(packed, cbs, M, K, block).astype(np.float64)
        absw = (np.abs(W) @ np.abs(x.astype(np.float64)).T).T
    inf_rows = np.isinf(ref)
    assert inf_rows.any()
    if path in HILO_NO_FALLBACK:
        assert np.isnan(got[inf_rows]).all(), f"{path}: pinned NaN-for-Inf divergence changed"
        fin = np.isfinite(ref)
        fp32_close(got[fin], ref[fin], absw[fin], 1e-5, f"{path}/inftiny finite rows")
    else:
        nonfinite_close(got, ref, absw, f"{path}/inftiny")


@pytest.mark.parametrize("path,M,N,K,block", PREFILL_PATHS)
def test_oil4_prefill_row_magnitudes(path, M, N, K, block, oracle, mth, dev):
    """Rows of A scaled by 2^-30 .. 2^30 (bf16 N(0,1) values times a power
    of two per row, an all-zero row too): FP16 holds neither end, so each row
    is scaled into FP16's range and the output row scaled back.  One bf16
    rounding of the oracle's FP32 result per element, as above; the largest
    rows' outputs are finite and the smallest rows' nonzero."""
    import torch
    print(f"prefill row magnitudes path={path} M={M} N={N} K={K}", flush=True)
    g = np.random.default_rng(zlib.crc32(f"{path}/rowmag".encode()))
    exps = np.linspace(-30, 30, M).round()
    a32 = (g.normal(0, 1, (M, K)) * np.exp2(exps)[:, None]).astype(np.float32)
    a32[M // 2] = 0.0
    a = synth.bf16_bits(a32)
    packed = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    cbs = synth.float_to_half_trunc(g.normal(0, 0.02, N * (K // block) * 16).astype(np.float32))
    c = torch.zeros(M * N, dtype=torch.bfloat16, device=dev)
    mth.oil4_gemm_prefill(to_dev(a, dev).view(torch.bfloat16), to_dev(packed, dev), to_dev(cbs, dev), block, c,
                          M, N, K)
    torch.cuda.synchronize()
    _, ref32 = oracle.oil4_gemm_prefill(a, packed, cbs, M, N, K, block, threads=8)
    got = synth.bf16_to_f32(c.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(M, N).astype(np.float64)
    ref = ref32.astype(np.float64)
    W = synth.dequant_oil4(packed, cbs, N, K, block).astype(np.float64)
    absw = np.abs(synth.bf16_to_f32(a).astype(np.float64)) @ np.abs(W).T
    assert np.isfinite(got).all()
    d = np.abs(got - ref)
    bound = 2.0 ** -8 * np.abs(ref) + 1e-5 * absw
    assert (d <= bound).all(), f"{path}: {(d > bound).sum()} elements out of bound, rows {np.unique(np.nonzero(d > bound)[0])[:8]}"
    assert (got[M // 2] == 0).all() and (got[0] != 0).all() and (got[-1] != 0).all()


@pytest.mark.parametrize("where", ["x_inf", "x_nan"])
@pytest.mark.parametrize("path,M,K,batch,block", GEMV_PATHS)
def test_oil4_gemv_nonfinite_x(path, M, K, batch, block, where, oracle, mth, dev):
    """Activations holding +-Inf or NaN (src/kernel_oil4.cpp:50 multiplies
    them in FP32): every output of such a token must be in the oracle's class
    (NaN, +Inf, -Inf), the other tokens' outputs within the FP32 bar."""
    import torch
    print(f"oil4 non-finite x {where} path={path} M={M} K={K} batch={batch}", flush=True)
    g = np.random.default_rng(zlib.crc32(f"{path}/{where}".encode()))
    packed = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    cbs = codebooks("edges", M, K // block, 17)
    x = g.normal(0, 1, (batch, K)).astype(np.float32)
    if where == "x_inf":
        x[0, 7] = np.inf
        x[-1, K // 2 + 3] = -np.inf
    else:
        x[0, 33] = np.nan
    y = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv(to_dev(packed, dev), to_dev(cbs, dev), block, to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    with np.errstate(invalid="ignore", over="ignore"):
        ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
        W = synth.dequant_oil4(packed, cbs, M, K, block).astype(np.float64)
        absw = (np.abs(W) @ np.abs(x.astype(np.float64)).T).T
    got = y.cpu().numpy().reshape(batch, M)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{path}/{where}: NaN classes differ"
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)), f"{path}/{where}: +Inf classes differ"
    assert np.array_equal(np.isneginf(got), np.isneginf(ref)), f"{path}/{where}: -Inf classes differ"
    fin = np.isfinite(ref)
    if fin.any():
        fp32_close(got[fin], ref[fin], absw[fin], 1e-5, f"{path}/{where} finite outputs")
