"""GPU parity: the ternary GEMM on int8 MFMA (mth_i2s_gemm_vnni for M, N >= 64
and K % 256 == 0, the prefill of the ternary down projection).

The reference's i2s_gemm_vnni (src/kernel_i2s.cpp:201-235) is an exact
integer dot product converted to FP32, so every output must equal the
oracle's bits.  At the full size (4096 weight rows x 512 tokens x K = 11008)
the oracle is replaced by a float64 contraction of the decoded weights: every
product and partial sum is an integer below 2^53, so it is exact, and its
FP32 rounding is the reference's value.
"""
import numpy as np
import pytest

import synth
from test_gpu_gemv import empty, to_dev

pytestmark = pytest.mark.gpu


def run(mth, dev, w, a, M, N, K):
    import torch
    out = empty(M * N, torch.float32, dev)
    mth.i2s_gemm_vnni(to_dev(w, dev), to_dev(a, dev), out, M, N, K)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("M,N,K", [(256, 128, 1024), (100, 70, 512), (64, 64, 256), (192, 300, 768),
                                   (130, 129, 2048), (512, 200, 1280), (1000, 130, 2816)])
def test_i2s_gemm_mfma_vs_oracle(M, N, K, oracle, mth, dev):
    print(f"i2s_gemm_vnni mfma M={M} N={N} K={K}", flush=True)
    g = np.random.default_rng(M * 7 + N * 3 + K)
    w = g.integers(0, 256, M * (K // 4), dtype=np.uint8)
    a = g.integers(-127, 128, N * K, dtype=np.int8)
    got = run(mth, dev, w, a, M, N, K)
    assert np.array_equal(got, oracle.i2s_gemm_vnni(w, a, M, N, K))


def test_i2s_gemm_mfma_extreme_values(oracle, mth, dev):
    """All weights +1 (codes 10 and 11) or -1 and activations at +-127/-128:
    the largest magnitudes the int32 sums take (127 * K)."""
    M, N, K = 64, 64, 4096
    w = np.full(M * (K // 4), 0xAA, np.uint8)
    w[: M * (K // 4) // 2] = 0xFF        # code 11 reads as +1
    w[-(K // 4):] = 0x00                 # last row all -1
    a = np.where(np.arange(N * K) % 3 == 0, -128, 127).astype(np.int8)
    got = run(mth, dev, w, a, M, N, K)
    assert np.array_equal(got, oracle.i2s_gemm_vnni(w, a, M, N, K))


def test_i2s_gemm_mfma_config_size(mth, dev):
    """4096 x 512 x 11008 (the ternary down projection over a 512-token
    prompt), exact float64 reference."""
    M, N, K = 4096, 512, 11008
    print(f"i2s_gemm_vnni mfma M={M} N={N} K={K}", flush=True)
    g = synth.stream(90)
    w = g.ternary(M, K).ravel()
    a = np.random.default_rng(91).integers(-127, 128, (N, K), dtype=np.int8)
    got = run(mth, dev, w, a.ravel(), M, N, K).reshape(M, N)
    t = synth.dequant_ternary(w, M, K, 1.0).astype(np.float64)
    want = (t @ a.astype(np.float64).T).astype(np.float32)
    assert np.array_equal(got, want)
