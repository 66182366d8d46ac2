"""GPU parity: OIL4 prefill GEMM (dequantise-in-LDS + MFMA) against the CPU
oracle (small shapes, every element) and against a float64 contraction of the
dequantised weights (config 4 shape, sampled rows and all columns).

Tolerance: 2e-3 relative for the OIL4/bf16 path.  The
production kernel (K a multiple of 256, the codebook block a multiple of 128,
N a multiple of 128, 112, 96 or 64) uses the FP16 codebook entries exactly and
converts A bf16 -> FP16 (exact in range), sums in FP32; the output is rounded
to bf16 (<= 2^-8 relative).  Asserted norm-wise
<= 2e-3 and per element |d| <= 2^-8*|ref| + 1e-3*sum|a*w|.  Other shapes run
the first FP16 kernel (same arithmetic, smaller tiles).
"""
import numpy as np
import pytest

import synth
from test_gpu_gemv import empty, to_dev

pytestmark = pytest.mark.gpu


def check(got_bits, ref_f64, absw, what):
    got = synth.bf16_to_f32(got_bits).astype(np.float64)
    d = np.abs(got - ref_f64)
    nrm = np.linalg.norm(got - ref_f64) / np.linalg.norm(ref_f64)
    assert nrm <= 2e-3, f"{what}: norm-wise rel err {nrm:.3e}"
    bound = 2.0 ** -8 * np.abs(ref_f64) + 1e-3 * absw
    assert (d <= bound).all(), f"{what}: {(d > bound).sum()} elements out of bound, worst {d.max():.3e}"
    return nrm


# producer/consumer kernel (the tile width with the best fill of 256 CUs): 128 (N = 32768), 112 (224; ragged M,
# block 256), 96 (288: two M tiles, M % 16 != 0; 96: three M tiles, the last of one row), 64 (N = 256, 128, 64;
# one row); block 64 and N = 130 / 250 take the one-wave kernel, K = 96 the first kernel
@pytest.mark.parametrize("M,N,K,block", [(128, 256, 256, 128), (64, 128, 1024, 128), (40, 224, 512, 256),
                                         (1, 128, 256, 128), (513, 96, 512, 128), (16, 32768, 256, 128),
                                         (270, 288, 1024, 128), (96, 256, 512, 64), (200, 130, 512, 64),
                                         (16, 64, 4096, 128), (300, 250, 1024, 128), (32, 48, 96, 32)])
def test_prefill_small_vs_oracle(M, N, K, block, oracle, mth, dev):
    import torch
    print(f"prefill M={M} N={N} K={K} block={block}", flush=True)
    a, packed, cbs = synth.prefill(M, N, K, block)
    c = torch.zeros(M * N, dtype=torch.bfloat16, device=dev)
    mth.oil4_gemm_prefill(to_dev(a, dev).view(torch.bfloat16), to_dev(packed, dev), to_dev(cbs, dev), block, c,
                          M, N, K)
    torch.cuda.synchronize()
    ref16, ref32 = oracle.oil4_gemm_prefill(a, packed, cbs, M, N, K, block, threads=8)
    W = synth.dequant_oil4(packed, cbs, N, K, block).astype(np.float64)
    A = synth.bf16_to_f32(a).astype(np.float64)
    absw = np.abs(A) @ np.abs(W).T
    got = c.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N)
    check(got, ref32.astype(np.float64), absw, "prefill vs oracle")


def _random_prefill_shapes(n, seed=11):
    """Seeded shapes for the producer/consumer kernel: N a multiple of one of its tile widths, K % 256 == 0,
    codebook blocks of 128 or 256, ragged M."""
    g = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        bn = int(g.choice([64, 96, 112, 128]))
        out.append((int(g.integers(1, 600)), bn * int(g.integers(1, 5)), 256 * int(g.integers(1, 5)),
                    int(g.choice([128, 256]))))
    return out


@pytest.mark.parametrize("M,N,K,block", _random_prefill_shapes(8))
def test_prefill_random_shapes_vs_oracle(M, N, K, block, oracle, mth, dev):
    if K % block:
        block = 128
    test_prefill_small_vs_oracle(M, N, K, block, oracle, mth, dev)


def test_prefill_config4_sampled(mth, dev):
    import torch
    M, N, K, block = 512, 14336, 4096, 128
    print(f"prefill M={M} N={N} K={K}", flush=True)
    a, packed, cbs = synth.prefill(M, N, K, block)
    c = torch.zeros(M * N, dtype=torch.bfloat16, device=dev)
    mth.oil4_gemm_prefill(to_dev(a, dev).view(torch.bfloat16), to_dev(packed, dev), to_dev(cbs, dev), block, c,
                          M, N, K)
    torch.cuda.synchronize()
    got = c.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N)
    rows = np.random.default_rng(0).choice(M, 24, replace=False)
    W = synth.dequant_oil4(packed, cbs, N, K, block).astype(np.float64)
    A = synth.bf16_to_f32(a[rows]).astype(np.float64)
    ref = A @ W.T
    absw = np.abs(A) @ np.abs(W).T
    check(got[rows], ref, absw, "prefill config 4")


def test_prefill_rejects_unsupported(mth, dev):
    import torch
    M, N, K = 4, 4, 48  # K % 32 != 0
    a = torch.zeros(M * K, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(N * K // 2, dtype=torch.uint8, device=dev)
    cb = torch.zeros(N * 16, dtype=torch.int16, device=dev)
    c = torch.zeros(M * N, dtype=torch.bfloat16, device=dev)
    with pytest.raises(mth.MythosError) as e:
        mth.oil4_gemm_prefill(a, w, cb, 48, c, M, N, K)
    assert e.value.code == mth.MTH_EUNSUPPORTED
