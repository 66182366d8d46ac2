"""GPU parity: decode GEMV kernels (OIL8, OIL4, I2_S) through the C ABI
against the CPU oracle on the same seeded inputs.

Bars: OIL8 FP32 within 1e-5 relative (norm-wise and
per element against sum|w*x|); OIL4 within 2e-3 (asserted here at 1e-5,
since the kernel accumulates in FP32 with exact FP16 codebook values);
ternary / int8 paths bit-exact.
"""
import numpy as np
import pytest

import synth
from conftest import fp32_close

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).to(dev)


def empty(n, dtype, dev):
    import torch
    return torch.full((n,), float("nan") if dtype.is_floating_point else 0, dtype=dtype, device=dev)


# ------------------------------------------------------------------ OIL8 --
@pytest.mark.parametrize("M,K,batch", [
    (4096, 4096, 1),     # config 1
    (300, 4096, 1),      # ragged row count
    (64, 1024, 1),       # one segment per lane
    (129, 2048, 3),      # batch > 1
    (4096, 4096, 16),    # decode batch 16
    (33, 1000, 2),       # K % 16 != 0 -> generic kernel
    (5, 4112, 1),        # K > 4096 -> generic kernel
    (32000, 4096, 16),   # lm_head of the decoder, one K slice
    (100, 512, 5),       # batched MFMA kernel, rows not a multiple of 64
    (4096, 4096, 2),
    (70, 4160, 17),      # two groups of tokens
])
def test_oil8_gemv(M, K, batch, oracle, mth, dev):
    import torch
    print(f"oil8_gemv M={M} K={K} batch={batch}", flush=True)
    idx, cb, x = synth.oil8(M, K, batch)
    y = empty(batch * M, torch.float32, dev)
    mth.oil8_gemv(to_dev(idx, dev), to_dev(cb, dev), to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.oil8_gemv(idx, cb, x, M, K, batch, threads=8)
    absw = np.abs(cb[idx]).astype(np.float64) @ np.abs(x.astype(np.float64)).T
    fp32_close(y.cpu().numpy().reshape(batch, M), ref, absw.T, 1e-5, "oil8_gemv")


@pytest.mark.parametrize("M,N,K", [(7, 3, 37), (16, 4, 256), (3, 1, 4096), (2, 5, 1)])
def test_oil8_gemm_reference_indexing(M, N, K, oracle, mth, dev):
    import torch
    print(f"oil8_gemm M={M} N={N} K={K}", flush=True)
    g = np.random.default_rng(11)
    idx = g.integers(0, 256, M * N * K, dtype=np.uint8)
    cb = g.normal(0, 0.02, 256).astype(np.float32)
    act = g.normal(0, 1, N * K).astype(np.float32)
    out = empty(M * N, torch.float32, dev)
    mth.oil8_gemm(to_dev(idx, dev), to_dev(cb, dev), to_dev(act, dev), out, M, N, K)
    torch.cuda.synchronize()
    ref = oracle.oil8_gemm(idx, cb, act, M, N, K, "avx2")
    W = np.abs(cb[idx.reshape(M * N, K)]).astype(np.float64)
    A = np.abs(act.reshape(N, K)).astype(np.float64)
    absw = np.einsum("rk,rk->r", W, A[np.arange(M * N) % N])
    fp32_close(out.cpu().numpy(), ref, absw, 1e-5, "oil8_gemm")


def test_oil8_integer_codebook_bit_exact(oracle, mth, dev):
    """cb[i] = i - 128 and integer x: every partial sum is an exact integer,
    so any summation order gives the reference's bits."""
    import torch
    M, K = 512, 4096
    g = np.random.default_rng(5)
    idx = g.integers(0, 256, (M, K), dtype=np.uint8)
    cb = (np.arange(256) - 128).astype(np.float32)
    x = g.integers(-3, 4, (1, K)).astype(np.float32)
    y = empty(M, torch.float32, dev)
    mth.oil8_gemv(to_dev(idx, dev), to_dev(cb, dev), to_dev(x, dev), y, M, K, 1)
    ref = oracle.oil8_gemv(idx, cb, x, M, K, 1)
    assert np.array_equal(y.cpu().numpy(), ref.ravel())


def run_oil8(mth, dev, idx, cb, x, M, K, batch):
    import torch
    y = empty(batch * M, torch.float32, dev)
    mth.oil8_gemv(to_dev(idx, dev), to_dev(cb, dev), to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(batch, M)


def test_oil8_batched_integer_codebook_bit_exact(oracle, mth, dev):
    """Batched kernel (FP16 hi/lo products): integer codebook and x keep every
    product and partial sum an exact integer, so the sum is the reference's
    bits whatever the order; a dropped or mis-scaled product term shows."""
    M, K, B = 640, 4096, 16
    g = np.random.default_rng(6)
    idx = g.integers(0, 256, (M, K), dtype=np.uint8)
    cb = (np.arange(256) - 128).astype(np.float32) * 3
    x = g.integers(-3, 4, (B, K)).astype(np.float32)
    print(f"oil8_gemv integer M={M} K={K} batch={B}", flush=True)
    got = run_oil8(mth, dev, idx, cb, x, M, K, B)
    assert np.array_equal(got, oracle.oil8_gemv(idx, cb, x, M, K, B))


def test_oil8_batched_codebook_range(oracle, mth, dev):
    """Codebook magnitudes over 2^-60 .. 2^40 and per-token activation
    scales from 2^-40 to 2^40 (every product and sum a normal FP32 number):
    the power-of-two scales put every hi / lo part in FP16 range, so the FP32
    bar holds for every token."""
    M, K, B = 256, 2048, 9
    g = np.random.default_rng(7)
    idx = g.integers(0, 256, (M, K), dtype=np.uint8)
    cb = (g.normal(0, 1, 256) * np.exp2(g.integers(-60, 40, 256))).astype(np.float32)
    x = (g.normal(0, 1, (B, K)) * np.exp2(np.linspace(-40, 40, B))[:, None]).astype(np.float32)
    print(f"oil8_gemv range M={M} K={K} batch={B}", flush=True)
    got = run_oil8(mth, dev, idx, cb, x, M, K, B)
    ref = oracle.oil8_gemv(idx, cb, x, M, K, B, threads=8)
    absw = (np.abs(cb[idx]).astype(np.float64) @ np.abs(x.astype(np.float64)).T).T
    for t in range(B):
        fp32_close(got[t], ref[t], absw[t], 1e-5, f"oil8 range token {t}")


@pytest.mark.parametrize("where", ["codebook_inf", "codebook_nan", "x_inf", "x_nan"])
def test_oil8_batched_non_finite(where, oracle, mth, dev):
    """A non-finite codebook entry or activation cannot take the hi / lo
    split (Inf - Inf is NaN): those workgroups sum the reference's FP32
    products directly.  Non-finite outputs must match the oracle's class
    (NaN, +Inf, -Inf); finite ones the FP32 bar."""
    M, K, B = 300, 1024, 4
    g = np.random.default_rng(8)
    idx = g.integers(0, 256, (M, K), dtype=np.uint8)
    cb = g.normal(0, 0.02, 256).astype(np.float32)
    x = g.normal(0, 1, (B, K)).astype(np.float32)
    if where == "codebook_inf":
        cb[17] = np.inf
        cb[200] = -np.inf
        idx[idx == 17] = 18                          # rows 0..99 only see +Inf, rows 100..199 only -Inf
        idx[idx == 200] = 201
        idx[:100, 5] = 17
        idx[100:200, 9] = 200
    elif where == "codebook_nan":
        cb[3] = np.nan
        idx[idx == 3] = 4
        idx[150:, 100] = 3
    elif where == "x_inf":
        x[1, 77] = np.inf
    else:
        x[2, 500] = np.nan
    print(f"oil8_gemv non-finite {where}", flush=True)
    got = run_oil8(mth, dev, idx, cb, x, M, K, B)
    with np.errstate(all="ignore"):
        ref = oracle.oil8_gemv(idx, cb, x, M, K, B, threads=8)
    fin = np.isfinite(ref)
    assert (~fin).any()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    with np.errstate(all="ignore"):
        absw = (np.abs(cb[idx]).astype(np.float64) @ np.abs(x.astype(np.float64)).T).T
    fp32_close(got[fin], ref[fin], absw[fin], 1e-5, f"oil8 finite outputs ({where})")


# ------------------------------------------------------------------ OIL4 --
@pytest.mark.parametrize("M,K,batch,block", [
    (11008, 4096, 1, 128),   # config 2, b=1
    (11008, 4096, 16, 128),  # config 2, b=16
    (100, 256, 3, 32),
    (257, 4096, 1, 0),       # one shared codebook
    (31, 2048, 2, 2048),
    (30, 100, 2, 50),        # K % 32 != 0 -> generic kernel
    (9, 4352, 1, 128),       # K > 4096 -> generic kernel
])
def test_oil4_gemv(M, K, batch, block, oracle, mth, dev):
    import torch
    print(f"oil4_gemv M={M} K={K} batch={batch} block={block}", flush=True)
    packed, cbs, x = synth.oil4(M, K, batch, block)
    y = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv(to_dev(packed, dev), to_dev(cbs, dev), block, to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    if block:
        ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
    else:
        ref = oracle.oil4_gemm(packed.ravel(), cbs, np.ascontiguousarray(x[0]), M, 1, K, "scalar").reshape(1, M)
    W = synth.dequant_oil4(packed, cbs, M, K, block)
    absw = np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64)).T
    fp32_close(y.cpu().numpy().reshape(batch, M), ref, absw.T, 1e-5, "oil4_gemv")


@pytest.mark.parametrize("M,K,batch,block", [
    (11008, 4096, 2, 128),   # 4 K slices, cross-workgroup sums
    (1000, 4096, 17, 128),   # two groups of tokens
    (130, 1024, 16, 128),    # 2 slices, rows not a multiple of 64
    (64, 512, 3, 128),       # one slice: no workspace
    (200, 1536, 8, 128),     # 3 slices of 512 columns
    (77, 3072, 4, 128),      # 3 slices of 1024 columns
    (300, 2048, 16, 0),      # one shared codebook
])
def test_oil4_gemv_batched(M, K, batch, block, oracle, mth, dev):
    """Batches >= 2 run the split-K MFMA kernel; FP32 accuracy as batch 1."""
    import torch
    print(f"oil4_gemv batched M={M} K={K} batch={batch} block={block}", flush=True)
    packed, cbs, x = synth.oil4(M, K, batch, block)
    y = empty(batch * M, torch.float32, dev)
    p_d, c_d, x_d = to_dev(packed, dev), to_dev(cbs, dev), to_dev(x, dev)
    mth.oil4_gemv(p_d, c_d, block, x_d, y, M, K, batch)
    torch.cuda.synchronize()
    if block:
        ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
    else:  # the shared codebook as one block per row
        ref = oracle.oil4_gemv_blocked(packed.ravel(), np.tile(cbs, M), x, M, K, batch, K, threads=8)
    W = synth.dequant_oil4(packed, cbs, M, K, block)
    absw = np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64)).T
    got = y.cpu().numpy().reshape(batch, M)
    fp32_close(got, ref, absw.T, 1e-5, "oil4_gemv batched")
    # deterministic: a second call gives the same bits
    y2 = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv(p_d, c_d, block, x_d, y2, M, K, batch)
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().reshape(batch, M), got)


def test_oil4_gemv_batched_two_streams(mth, dev):
    """Each stream has its own workspace; interleaved calls stay exact."""
    import torch
    M, K, batch = 2048, 4096, 8
    packed, cbs, x = synth.oil4(M, K, batch, 128)
    p_d, c_d, x_d = to_dev(packed, dev), to_dev(cbs, dev), to_dev(x, dev)
    y0 = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv(p_d, c_d, 128, x_d, y0, M, K, batch)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    ys = [empty(batch * M, torch.float32, dev) for _ in range(4)]
    for i, yy in enumerate(ys):
        mth.oil4_gemv(p_d, c_d, 128, x_d, yy, M, K, batch, stream=s1 if i % 2 == 0 else s2)
    torch.cuda.synchronize()
    for yy in ys:
        assert torch.equal(yy, y0)


@pytest.mark.parametrize("M,N,K", [(7, 3, 48), (5, 2, 33), (4, 1, 4096), (3, 4, 1)])
def test_oil4_gemm_reference_indexing(M, N, K, oracle, mth, dev):
    import torch
    print(f"oil4_gemm M={M} N={N} K={K}", flush=True)
    g = np.random.default_rng(12)
    nbytes = (M * N * K + 1) // 2
    packed = g.integers(0, 256, nbytes, dtype=np.uint8)
    cb = synth.float_to_half_trunc(g.normal(0, 0.02, 16).astype(np.float32))
    act = g.normal(0, 1, N * K).astype(np.float32)
    out = empty(M * N, torch.float32, dev)
    mth.oil4_gemm(to_dev(packed, dev), to_dev(cb, dev), to_dev(act, dev), out, M, N, K)
    torch.cuda.synchronize()
    ref = oracle.oil4_gemm(np.concatenate([packed, np.zeros(8, np.uint8)]), cb, act, M, N, K, "scalar")
    got = out.cpu().numpy()
    scale = np.abs(synth.fp16_bits_to_f32(cb)).max() * np.abs(act).sum()
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6 * scale), np.abs(got - ref).max()


# ------------------------------------------ FFN in two launches (batch 1) --
@pytest.mark.parametrize("F,K", [
    (11008, 4096),   # config 5's gate/up (four-wave workgroups)
    (2048, 1024),    # two waves per workgroup
    (64, 3072),      # six waves: norm-sum waves not a multiple of them
    (40, 512),       # one wave
    (8, 4096),       # one workgroup
])
def test_oil4_gemv_swiglu_bit_exact(F, K, oracle, mth, dev):
    """Gate/up GEMV with the SwiGLU in its epilogue: act bit-identical to
    mth_oil4_gemv over the 2F rows followed by mth_silu_mul; amax the exact
    maxima of |act| over groups of 8; the GEMV itself against the oracle."""
    import torch
    print(f"oil4_gemv_swiglu F={F} K={K}", flush=True)
    packed, cbs, x = synth.oil4(2 * F, K, 1, 128)
    p, c, xd = to_dev(packed, dev), to_dev(cbs, dev), to_dev(x, dev)
    act, amax = empty(F, torch.float32, dev), empty(F // 8, torch.float32, dev)
    mth.oil4_gemv_swiglu(p, c, xd, act, amax, F, K)
    y, ref_act = empty(2 * F, torch.float32, dev), empty(F, torch.float32, dev)
    mth.oil4_gemv(p, c, 128, xd, y, 2 * F, K)
    mth.silu_mul(y[:F], y[F:], ref_act, 1, F)
    torch.cuda.synchronize()
    got, want = act.cpu().numpy(), ref_act.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(amax.cpu().numpy(), np.abs(want).reshape(-1, 8).max(1))
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, 2 * F, K, 1, 128, threads=8)
    W = synth.dequant_oil4(packed, cbs, 2 * F, K, 128)
    absw = np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64)).T
    fp32_close(y.cpu().numpy().reshape(1, 2 * F), ref, absw.T, 1e-5, "oil4_gemv (2F rows)")


@pytest.mark.parametrize("M,K", [
    (4096, 11008),   # config 5's down projection
    (4096, 512),
    (100, 64),       # one segment
    (33, 12288),     # the largest K, rows not a multiple of 16
    (17, 8256),      # three segments per lane, the last partial; one row past a workgroup
])
def test_i2s_gemv_act_bit_exact(M, K, oracle, mth, dev):
    """The I2_S GEMV of quantize_per_token(act) with the quantisation inside
    the launch (max|act| from the per-8 maxima): bit-exact against the
    oracle's quantize_per_token + i2s_gemv; an all-zero act gives 0."""
    import torch
    print(f"i2s_gemv_act M={M} K={K}", flush=True)
    g = np.random.default_rng(M + K)
    packed = g.integers(0, 256, (M, K // 4), dtype=np.uint8)  # all four codes
    for act in (g.normal(0, 1, K).astype(np.float32), np.zeros(K, np.float32)):
        amax = np.abs(act).reshape(-1, 8).max(1)
        y = empty(M, torch.float32, dev)
        mth.i2s_gemv_act(to_dev(packed, dev), 0.0159577, to_dev(act, dev), to_dev(amax, dev), y, M, K)
        torch.cuda.synchronize()
        ref = oracle.i2s_gemv_f32(packed.ravel(), 0.0159577, act.reshape(1, K), M, K, 1, threads=8)
        assert np.array_equal(y.cpu().numpy().reshape(1, M), ref)


@pytest.mark.parametrize("M,K", [(int(m), 64 * int(k)) for m, k in
                                 zip(np.random.default_rng(5).integers(1, 300, 6),
                                     np.random.default_rng(6).integers(1, 193, 6))])
def test_i2s_gemv_act_random_shapes(M, K, oracle, mth, dev):
    """Seeded random (M, K): K % 64 == 0 up to 12288 (one to three segments per lane), ragged M."""
    test_i2s_gemv_act_bit_exact(M, K, oracle, mth, dev)


# ---------------------------------------- FFN in two launches (batches) --
@pytest.mark.parametrize("F,K,H,batch", [
    (11008, 4096, 4096, 16),   # config 5 at batch 16: 4 K slices of gate/up, 8 slices over 2 rounds of down
    (11008, 4096, 4096, 2),    # config 5 at batch 2
    (1024, 512, 512, 5),       # one K slice each (the in-place reduction, one round)
    (300, 2048, 200, 3),       # F not a multiple of 256, ragged down rows
])
def test_ffn_batch_bit_exact(F, K, H, batch, oracle, mth, dev):
    """The decoder's batched FFN pair through the C ABI, with real (all four
    codes) ternary down weights: act bit-identical to the batched OIL4 GEMV
    over 2F rows followed by mth_silu_mul, the block maxima exact, the GEMV
    against the oracle; the down projection of the GPU's act (quantised
    inside the launch from the block maxima) bit-exact against the oracle's
    quantize_per_token + i2s_gemv, and its act scales equal to the oracle's."""
    import torch
    print(f"ffn batch F={F} K={K} H={H} batch={batch}", flush=True)
    packed, cbs, x = synth.oil4(2 * F, K, batch, 128, config=5)
    p, c, xd = to_dev(packed, dev), to_dev(cbs, dev), to_dev(x, dev)
    parts = mth.swiglu_batch_parts(F)
    assert parts == -(-F // 256)
    gu, amax = empty(batch * 2 * F, torch.float32, dev), empty(batch * parts, torch.float32, dev)
    mth.oil4_gemv_swiglu_batch(p, c, 128, xd, gu, amax, F, K, batch)
    y, ref_act = empty(batch * 2 * F, torch.float32, dev), empty(batch * F, torch.float32, dev)
    mth.oil4_gemv(p, c, 128, xd, y, 2 * F, K, batch)
    mth.silu_mul(y, y[F:], ref_act, batch, F, 2 * F, 2 * F)
    g = np.random.default_rng(F + K + batch)
    wdown = g.integers(0, 256, (H, F // 4), dtype=np.uint8)
    # F % 256 != 0: pad the down projection's K to a multiple of 256 with zero activations
    Kd = -(-F // 256) * 256
    if Kd != F:
        wdown = np.concatenate([wdown, np.full((H, (Kd - F) // 4), 0x55, np.uint8)], axis=1)
        gu2 = torch.zeros(batch * 2 * Kd, dtype=torch.float32, device=dev)
        gu2.view(batch, 2 * Kd)[:, :F] = gu.view(batch, 2 * F)[:, :F]
        act_in, lda = gu2, 2 * Kd
    else:
        act_in, lda = gu, 2 * F
    down, inv = empty(batch * H, torch.float32, dev), empty(batch, torch.float32, dev)
    mth.i2s_gemv_act_batch(to_dev(wdown, dev), 0.0159577, act_in, lda, amax, inv, down, H, Kd, batch)
    torch.cuda.synchronize()
    got = gu.cpu().numpy().reshape(batch, 2 * F)[:, :F]
    want = ref_act.cpu().numpy().reshape(batch, F)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    pad = np.zeros((batch, parts * 256), np.float32)
    pad[:, :F] = np.abs(want)
    assert np.array_equal(amax.cpu().numpy().reshape(batch, parts), pad.reshape(batch, parts, 256).max(2))
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, 2 * F, K, batch, 128, threads=8)
    W = synth.dequant_oil4(packed, cbs, 2 * F, K, 128)
    absw = np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64)).T
    fp32_close(y.cpu().numpy().reshape(batch, 2 * F), ref, absw.T, 1e-5, "oil4_gemv (2F rows, batch)")
    a = np.zeros((batch, Kd), np.float32)
    a[:, :F] = got
    _, _, inv_ref = oracle.quantize_per_token(a, batch, Kd)
    assert np.array_equal(inv.cpu().numpy(), inv_ref)
    ref_down = oracle.i2s_gemv_f32(wdown.ravel(), 0.0159577, a, H, Kd, batch, threads=8)
    assert np.array_equal(down.cpu().numpy().reshape(batch, H), ref_down)


@pytest.mark.parametrize("M,K,batch", [(4096, 11008 // 256 * 256, 16), (130, 16384, 2), (64, 256, 9)])
def test_i2s_gemv_act_batch_inputs(M, K, batch, oracle, mth, dev):
    """mth_i2s_gemv_act_batch on activations of very different magnitudes
    per token (1e-30 .. 1e6, and an all-zero token: the 1e-10 floor), the
    largest K (64 block maxima), a row stride larger than K."""
    import torch
    print(f"i2s_gemv_act_batch M={M} K={K} batch={batch}", flush=True)
    g = np.random.default_rng(M + K + batch)
    packed = g.integers(0, 256, (M, K // 4), dtype=np.uint8)
    lda = K + 36
    act = np.zeros((batch, lda), np.float32)
    mags = [1e-30, 1e6, 0.0, 1.0, 3e-4, 7.5, 1e-12, 40.0, 1e3] * 2
    for t in range(batch):
        act[t, :K] = (g.normal(0, 1, K) * mags[t]).astype(np.float32)
    parts = -(-K // 256)
    amax = np.abs(act[:, :K]).reshape(batch, parts, 256).max(2)
    y, inv = empty(batch * M, torch.float32, dev), empty(batch, torch.float32, dev)
    mth.i2s_gemv_act_batch(to_dev(packed, dev), 0.0159577, to_dev(act.ravel(), dev), lda, to_dev(amax, dev), inv, y,
                           M, K, batch)
    torch.cuda.synchronize()
    a = np.ascontiguousarray(act[:, :K])
    _, _, inv_ref = oracle.quantize_per_token(a, batch, K)
    assert np.array_equal(inv.cpu().numpy(), inv_ref)
    ref = oracle.i2s_gemv_f32(packed.ravel(), 0.0159577, a, M, K, batch, threads=8)
    assert np.array_equal(y.cpu().numpy().reshape(batch, M), ref)


def test_ffn_building_blocks_reject_shapes(mth, dev):
    import torch
    p = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    c = torch.zeros(1 << 14, dtype=torch.int16, device=dev)
    f = torch.zeros(1 << 14, dtype=torch.float32, device=dev)
    with pytest.raises(mth.MythosError):
        mth.oil4_gemv_swiglu(p, c, f, f, f, 12, 1024)      # F % 8 != 0
    with pytest.raises(mth.MythosError):
        mth.oil4_gemv_swiglu(p, c, f, f, f, 8, 1280)      # K % 512 != 0
    with pytest.raises(mth.MythosError):
        mth.oil4_gemv_swiglu(p, c, f, f, f, 8, 8192)      # K > 4096
    with pytest.raises(mth.MythosError):
        mth.i2s_gemv_act(p, 1.0, f, f, f, 8, 1000)         # K % 64 != 0
    with pytest.raises(mth.MythosError):
        mth.i2s_gemv_act(p, 1.0, f[1:], f, f, 8, 64)       # act not 16-byte aligned


# ------------------------------------------------------------- int8/I2_S --
@pytest.mark.parametrize("rows,cols", [(1, 4096), (16, 11008), (3, 5), (2, 1)])
def test_quantize_per_token_bit_exact(rows, cols, oracle, mth, dev):
    import torch
    g = np.random.default_rng(rows * 1000 + cols)
    x = g.normal(0, 1, (rows, cols)).astype(np.float32)
    x[0, 0] = 0.0
    if rows > 2:
        x[2] = 0.0  # all-zero row: max_abs floor 1e-10
    q = empty(rows * cols, torch.int8, dev)
    s = empty(rows, torch.float32, dev)
    inv = empty(rows, torch.float32, dev)
    mth.quantize_per_token(to_dev(x, dev), q, s, inv, rows, cols)
    torch.cuda.synchronize()
    rq, rs, rinv = oracle.quantize_per_token(x, rows, cols)
    assert np.array_equal(q.cpu().numpy().reshape(rows, cols), rq)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(inv.cpu().numpy(), rinv)


@pytest.mark.parametrize("M,K,batch", [
    (4096, 4096, 1),    # config 3
    (4096, 11008, 1),   # decoder down projection shape
    (100, 256, 3),
    (77, 1024, 2),
    (50, 100, 2),       # K % 64 != 0 -> generic kernel
    (8, 20480, 1),      # K > 16384 -> generic kernel
])
def test_i2s_gemv_f32_bit_exact(M, K, batch, oracle, mth, dev):
    import torch
    print(f"i2s_gemv_f32 M={M} K={K} batch={batch}", flush=True)
    packed, w_scale, x = synth.ternary(M, K, batch)
    y = empty(batch * M, torch.float32, dev)
    mth.i2s_gemv_f32(to_dev(packed, dev), w_scale, to_dev(x, dev), y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.i2s_gemv_f32(packed.ravel(), float(w_scale), x, M, K, batch, threads=8)
    assert np.array_equal(y.cpu().numpy().reshape(batch, M), ref)


def test_i2s_code3_and_unfused_bit_exact(oracle, mth, dev):
    """Code 11 decodes to +1 (src/kernel_i2s.cpp:16-21); the unfused entry
    point takes int8 acts + act_scale like the reference i2s_gemv."""
    import torch
    M, K, batch = 640, 4096, 2
    g = np.random.default_rng(3)
    packed = g.integers(0, 256, (M, K // 4), dtype=np.uint8)  # all four codes
    x = g.normal(0, 1, (batch, K)).astype(np.float32)
    q, _, inv = oracle.quantize_per_token(x, batch, K)
    y = empty(batch * M, torch.float32, dev)
    mth.i2s_gemv(to_dev(packed, dev), 0.75, to_dev(q, dev), to_dev(inv, dev), y, M, K, batch)
    torch.cuda.synchronize()
    ref = np.array([[oracle.i2s_gemv(np.ascontiguousarray(packed[m]), 0.75, np.ascontiguousarray(q[t]),
                                     float(inv[t]), K) for m in range(M)] for t in range(batch)], np.float32)
    assert np.array_equal(y.cpu().numpy().reshape(batch, M), ref)
    y2 = empty(batch * M, torch.float32, dev)
    mth.i2s_gemv_f32(to_dev(packed, dev), 0.75, to_dev(x, dev), y2, M, K, batch)
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy().reshape(batch, M), ref)


@pytest.mark.parametrize("M,K,batch", [
    (4096, 11008, 16),   # decoder down projection, batch 16 (int8 MFMA kernel, 4 K slices)
    (4096, 11008, 2),
    (100, 512, 5),       # rows not a multiple of 64, 2 slices
    (64, 256, 17),       # one super-chunk, two groups of tokens
    (33, 1000, 3),       # K % 256 != 0 -> per-token kernel
])
def test_i2s_gemv_batched_bit_exact(M, K, batch, oracle, mth, dev):
    """int8 activations + act_scale (the unfused entry point, as the decoder
    calls it) for batches: bit-exact against quantize_per_token + i2s_gemv."""
    import torch
    print(f"i2s_gemv batched M={M} K={K} batch={batch}", flush=True)
    g = np.random.default_rng(M + K + batch)
    packed = g.integers(0, 256, (M, K // 4), dtype=np.uint8)  # all four codes
    x = g.normal(0, 1, (batch, K)).astype(np.float32)
    x[batch // 2] *= 1e-3
    q, _, inv = oracle.quantize_per_token(x, batch, K)
    y = empty(batch * M, torch.float32, dev)
    mth.i2s_gemv(to_dev(packed, dev), 0.0159577, to_dev(q, dev), to_dev(inv, dev), y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.i2s_gemv_f32(packed.ravel(), 0.0159577, x, M, K, batch, threads=8)
    assert np.array_equal(y.cpu().numpy().reshape(batch, M), ref)
