"""GPU parity: the reference's ternary GEMM-family drop-ins (i2s_gemm,
i2s_gemm_vnni, tl1_gemm, tl2_gemm, the TL LUT builders, dequantize) through
the C ABI against the CPU oracle.  Integer paths bit-exact; i2s_gemm (FP32
activations, reordered sums) within 1e-5 relative."""
import numpy as np
import pytest

from conftest import fp32_close
from test_gpu_gemv import empty, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(16, 8, 512), (7, 3, 260), (64, 1, 4096), (3, 2, 7)])
def test_i2s_gemm(M, N, K, oracle, mth, dev):
    import torch
    g = np.random.default_rng(M * N + K)
    w = g.integers(0, 256, M * (K // 4) + 1, dtype=np.uint8)
    a = g.normal(0, 1, N * K).astype(np.float32)
    out = empty(M * N, torch.float32, dev)
    mth.i2s_gemm(to_dev(w, dev), to_dev(a, dev), out, M, N, K)
    torch.cuda.synchronize()
    ref = oracle.i2s_gemm(w, a, M, N, K)
    absw = np.array([[np.abs(a[n * K:(n + 1) * K]).sum() for n in range(N)] for _ in range(M)]).ravel()
    fp32_close(out.cpu().numpy(), ref, absw, 1e-5, "i2s_gemm")


@pytest.mark.parametrize("M,N,K", [(16, 8, 512), (7, 3, 260), (64, 1, 4096), (3, 2, 7)])
def test_i2s_gemm_vnni_bit_exact(M, N, K, oracle, mth, dev):
    import torch
    g = np.random.default_rng(M * N + K + 1)
    w = g.integers(0, 256, M * (K // 4) + 1, dtype=np.uint8)
    a = g.integers(-127, 128, N * K, dtype=np.int8)
    out = empty(M * N, torch.float32, dev)
    mth.i2s_gemm_vnni(to_dev(w, dev), to_dev(a, dev), out, M, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), oracle.i2s_gemm_vnni(w, a, M, N, K))


@pytest.mark.parametrize("M,N,K", [(4, 4, 16), (5, 3, 40), (2, 2, 7), (8, 2, 1024)])
def test_tl1_gemm_bit_exact(M, N, K, oracle, mth, dev):
    import torch
    g = np.random.default_rng(M + N + K)
    w = g.integers(0, 256, (M * N * K) // 4 + 2, dtype=np.uint8)
    a = (g.normal(0, 1, N * K) * 0.5).astype(np.float32)
    out = empty(M * N, torch.float32, dev)
    mth.tl1_gemm(to_dev(w, dev), to_dev(a, dev), out, M, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), oracle.tl1_gemm(w, a, M, N, K))


# ceil(K / 4) % 16 == 0 (1023, 3069, 4095, 12285) takes the streaming v_dot4
# kernel over activations quantised once per row, the others one wave per
# output; codes past K (the last byte's spare fields) are random in both
@pytest.mark.parametrize("M,N,K", [(4, 4, 12), (5, 3, 36), (2, 2, 9), (8, 2, 1023), (64, 16, 3069), (33, 5, 4095),
                                   (256, 16, 12285), (17, 1, 1023)])
def test_tl2_gemm_bit_exact(M, N, K, oracle, mth, dev):
    import torch
    g = np.random.default_rng(M + N + K + 7)
    w = g.integers(0, 256, M * N * ((2 * K + 7) // 8), dtype=np.uint8)
    a = g.normal(0, 1, N * K).astype(np.float32)
    out = empty(M * N, torch.float32, dev)
    mth.tl2_gemm(to_dev(w, dev), to_dev(a, dev), out, M, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), oracle.tl2_gemm(w, a, M, N, K))


@pytest.mark.parametrize("group,K", [(2, 64), (2, 9), (3, 63)])
def test_tl_precompute_lut_bit_exact(group, K, oracle, mth, dev):
    import ctypes as C
    import torch
    g = np.random.default_rng(K)
    act = g.integers(-127, 128, K, dtype=np.int8)
    n = (K // group) * (9 if group == 2 else 27)
    lut = empty(n, torch.int8, dev)
    mth.tl_precompute_lut(to_dev(act, dev), lut, K, group)
    torch.cuda.synchronize()
    ref = np.zeros(n, np.int8)
    f = oracle.lib.orc_tl1_precompute_lut if group == 2 else oracle.lib.orc_tl2_precompute_lut
    f(C.c_void_p(act.ctypes.data), C.c_void_p(ref.ctypes.data), K)
    assert np.array_equal(lut.cpu().numpy(), ref)


def test_dequantize_per_tensor(oracle, mth, dev):
    import torch
    g = np.random.default_rng(9)
    q = g.integers(-128, 128, 10000, dtype=np.int8)
    out = empty(q.size, torch.float32, dev)
    mth.dequantize_per_tensor(to_dev(q, dev), out, q.size, 0.0123)
    torch.cuda.synchronize()
    ref = np.empty(q.size, np.float32)
    import ctypes as C
    oracle.lib.orc_dequantize_per_tensor(C.c_void_p(q.ctypes.data), C.c_void_p(ref.ctypes.data), q.size,
                                         C.c_float(0.0123))
    assert np.array_equal(out.cpu().numpy(), ref)
