"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the reference's own kernels compiled from its sources) replayed through
the oracle on the CPU and through libmythos_oil.so on the GPU.

Oracle bar: bit-exact, including the AVX2 lane order of oil8_gemm_avx2 /
oil4_gemm_avx2 (src/kernel_oil8.cpp:30-60, src/kernel_oil4.cpp:57-114).
GPU bar: bit-exact for integer work (quantize, i2s_gemv, vnni, tl1, tl2);
FP32 within 1e-5 (norm-wise and per element against sum|w*x|) for codebook
GEMMs, whose summation order differs from the CPU's.
"""
import hashlib
import os

import numpy as np
import pytest

from conftest import fp32_close

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, f"{name}.npz"))


def cases(z):
    for ci in range(int(z["ncases"])):
        yield ci, {k[len(f"c{ci}_"):]: z[k] for k in z.files if k.startswith(f"c{ci}_")}


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.uint32)
    b = np.ascontiguousarray(b, np.float32).view(np.uint32)
    return np.array_equal(a, b)


# --------------------------------------------------------------------------
# Oracle against the reference (CPU)
# --------------------------------------------------------------------------
def test_rng(oracle):
    z = load("rng")
    for i, s in enumerate(z["seeds"]):
        s = int(s)
        n = z["u64"].shape[1]
        assert np.array_equal(oracle.rng_u64(s, n), z["u64"][i])
        assert same_bits(oracle.rng_uniform(s, n), z["uniform"][i])
        assert same_bits(oracle.rng_normal(s, n), z["normal"][i])
        assert np.array_equal(oracle.rng_uniform_int(s, 0, 2, n), z["uint_0_2"][i])
        assert np.array_equal(oracle.rng_uniform_int(s, -5, 9, n), z["uint_m5_9"][i])


def test_fp16_codebook_conversions(oracle):
    z = load("fp16")
    got = np.array([oracle.half_to_float_codebook(int(h)) for h in z["half_bits"]], np.float32)
    assert np.array_equal(got.view(np.uint32), z["half_to_float_bits"])
    table = np.array([oracle.half_to_float_codebook(h) for h in range(65536)], np.float32)
    digest = hashlib.sha256(table.view(np.uint32).astype("<u4").tobytes()).digest()
    assert digest == bytes(z["table_sha256"])
    got = np.array([oracle.float_to_half_trunc(float(f)) for f in z["floats"]], np.uint16)
    assert np.array_equal(got, z["float_to_half"])


@pytest.mark.parametrize("variant", ["avx2", "scalar"])
def test_oil8_gemm(oracle, variant):
    for ci, c in cases(load("oil8")):
        M, N, K = (int(v) for v in c["shape"])
        got = oracle.oil8_gemm(c["idx"], c["cb"], c["act"], M, N, K, variant=variant)
        assert same_bits(got, c[variant]), (variant, ci)


@pytest.mark.parametrize("variant", ["avx2", "scalar"])
def test_oil4_gemm(oracle, variant):
    for ci, c in cases(load("oil4")):
        M, N, K = (int(v) for v in c["shape"])
        got = oracle.oil4_gemm(c["nib"], c["cb16"], c["act"], M, N, K, variant=variant)
        assert same_bits(got, c[variant]), (variant, ci)


def test_quantize_per_token(oracle):
    z = load("quant")
    rows, cols = z["x"].shape
    q, s, inv = oracle.quantize_per_token(z["x"], rows, cols)
    assert np.array_equal(q, z["q"])
    assert same_bits(s, z["scale"]) and same_bits(inv, z["inv_scale"])


def test_i2s_gemv(oracle):
    for ci, c in cases(load("i2s_gemv")):
        K = int(c["K"])
        q, _, inv = oracle.quantize_per_token(c["x"], 1, K)
        assert np.array_equal(q[0], c["act"]) and same_bits(inv, c["act_scale"])
        got = np.array([oracle.i2s_gemv(np.ascontiguousarray(c["packed"][m]), float(c["w_scale"]), c["act"],
                                        float(c["act_scale"][0]), K) for m in range(c["packed"].shape[0])],
                       np.float32)
        assert same_bits(got, c["y"]), ci
        # the fused decode op (quantize + per-row gemv) gives the same bits
        fused = oracle.i2s_gemv_f32(np.ascontiguousarray(c["packed"]), float(c["w_scale"]), c["x"],
                                    c["packed"].shape[0], K, 1)
        assert same_bits(fused[0], c["y"]), ci


def test_i2s_gemm_and_vnni(oracle):
    for ci, c in cases(load("i2s_gemm")):
        M, N, K = (int(v) for v in c["shape"])
        assert same_bits(oracle.i2s_gemm(c["w"], c["a"], M, N, K), c["gemm"]), ci
        assert same_bits(oracle.i2s_gemm_vnni(c["w"], c["ai"], M, N, K), c["vnni"]), ci


def test_tl1_tl2(oracle):
    for ci, c in cases(load("tl")):
        M, N, K = (int(v) for v in c["shape"])
        assert same_bits(oracle.tl1_gemm(c["w1"], c["a"], M, N, K), c["tl1"]), ci
        assert same_bits(oracle.tl2_gemm(c["w2"], c["a"], M, N, K), c["tl2"]), ci


def test_dense_math(oracle):
    """Bit-exact against the reference built without FMA contraction; within
    FP32 reordering tolerance of the -mfma build, whose contraction GCC picks."""
    z = load("math")
    M, N = z["A"].shape
    y = oracle.gemv(0.75, z["A"], z["x"], 0.5, z["y0"], M, N)
    assert same_bits(y, z["gemv"])
    absw = 0.75 * np.abs(z["A"]) @ np.abs(z["x"]) + 0.5 * np.abs(z["y0"])
    fp32_close(y, z["gemv_fma"], absw, rel=1e-6, what="gemv vs -mfma build")
    rows, dim = z["rms_x"].shape
    r = oracle.rms_norm(z["rms_x"], z["rms_g"], 1e-5, rows, dim)
    assert same_bits(r, z["rms"])
    np.testing.assert_allclose(r, z["rms_fma"], rtol=1e-6, atol=0)
    s = oracle.silu(z["silu_x"])
    assert same_bits(s, z["silu"])
    np.testing.assert_allclose(s, z["silu_fma"], rtol=1e-6, atol=1e-30)


# --------------------------------------------------------------------------
# GPU (C ABI) against the reference
# --------------------------------------------------------------------------
def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.gpu
def test_gpu_oil8_gemm_golden(mth, dev):
    import torch
    for ci, c in cases(load("oil8")):
        M, N, K = (int(v) for v in c["shape"])
        out = torch.empty(M * N, dtype=torch.float32, device=dev)
        mth.oil8_gemm(_t(c["idx"], dev), _t(c["cb"], dev), _t(c["act"], dev), out, M, N, K)
        w = np.abs(c["cb"][c["idx"].reshape(M, N, K)]) * np.abs(c["act"].reshape(1, N, K))
        fp32_close(out.cpu().numpy(), c["avx2"], w.sum(-1), what=f"oil8 case {ci}")


@pytest.mark.gpu
def test_gpu_oil4_gemm_golden(mth, dev):
    import torch
    from synth import fp16_bits_to_f32
    for ci, c in cases(load("oil4")):
        M, N, K = (int(v) for v in c["shape"])
        out = torch.empty(M * N, dtype=torch.float32, device=dev)
        mth.oil4_gemm(_t(c["nib"], dev), _t(c["cb16"].view(np.int16), dev), _t(c["act"], dev), out, M, N, K)
        nib = c["nib"]
        codes = np.stack([nib & 15, nib >> 4], -1).reshape(-1)[: M * N * K].reshape(M, N, K)
        w = np.abs(fp16_bits_to_f32(c["cb16"])[codes]) * np.abs(c["act"].reshape(1, N, K))
        fp32_close(out.cpu().numpy(), c["scalar"], w.sum(-1), what=f"oil4 case {ci}")


@pytest.mark.gpu
def test_gpu_quantize_golden(mth, dev):
    import torch
    z = load("quant")
    rows, cols = z["x"].shape
    q = torch.empty((rows, cols), dtype=torch.int8, device=dev)
    s = torch.empty(rows, dtype=torch.float32, device=dev)
    inv = torch.empty(rows, dtype=torch.float32, device=dev)
    mth.quantize_per_token(_t(z["x"], dev), q, s, inv, rows, cols)
    assert np.array_equal(q.cpu().numpy(), z["q"])
    assert same_bits(s.cpu().numpy(), z["scale"]) and same_bits(inv.cpu().numpy(), z["inv_scale"])


@pytest.mark.gpu
def test_gpu_i2s_gemv_golden(mth, dev):
    import torch
    for ci, c in cases(load("i2s_gemv")):
        K = int(c["K"])
        M = c["packed"].shape[0]
        y = torch.empty(M, dtype=torch.float32, device=dev)
        mth.i2s_gemv(_t(c["packed"], dev), float(c["w_scale"]), _t(c["act"], dev), _t(c["act_scale"], dev),
                     y, M, K)
        assert same_bits(y.cpu().numpy(), c["y"]), ci
        y2 = torch.empty(M, dtype=torch.float32, device=dev)
        mth.i2s_gemv_f32(_t(c["packed"], dev), float(c["w_scale"]), _t(c["x"], dev), y2, M, K)
        assert same_bits(y2.cpu().numpy(), c["y"]), ci


@pytest.mark.gpu
def test_gpu_i2s_gemm_golden(mth, dev):
    import torch
    for ci, c in cases(load("i2s_gemm")):
        M, N, K = (int(v) for v in c["shape"])
        o = torch.empty(M * N, dtype=torch.float32, device=dev)
        mth.i2s_gemm_vnni(_t(c["w"], dev), _t(c["ai"], dev), o, M, N, K)
        assert same_bits(o.cpu().numpy(), c["vnni"]), ci
        mth.i2s_gemm(_t(c["w"], dev), _t(c["a"], dev), o, M, N, K)
        codes = np.stack([(c["w"] >> (2 * j)) & 3 for j in range(4)], -1).reshape(-1)[: M * K]
        t = codes.reshape(M, K).astype(np.float64) - 1
        absw = np.abs(t) @ np.abs(c["a"].reshape(N, K).astype(np.float64)).T
        fp32_close(o.cpu().numpy(), c["gemm"], absw, what=f"i2s_gemm case {ci}")


@pytest.mark.gpu
def test_gpu_tl_golden(mth, dev):
    import torch
    for ci, c in cases(load("tl")):
        M, N, K = (int(v) for v in c["shape"])
        o = torch.empty(M * N, dtype=torch.float32, device=dev)
        mth.tl1_gemm(_t(c["w1"], dev), _t(c["a"], dev), o, M, N, K)
        assert same_bits(o.cpu().numpy(), c["tl1"]), ci
        mth.tl2_gemm(_t(c["w2"], dev), _t(c["a"], dev), o, M, N, K)
        assert same_bits(o.cpu().numpy(), c["tl2"]), ci
