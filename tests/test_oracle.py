"""Pins of the CPU oracle that do not come from the reference's outputs:
closed forms, exhaustive sweeps, brute force and the reference's own
known-answer tests.  Each check is chosen so that a plausible slip in the
oracle (a swapped nibble order, a wrong row offset, round-half-even instead of
half-away, a missing term) fails it; where that is not obvious the test shows
the slip's output is different.  CPU only.
"""
import numpy as np
import pytest

from conftest import fp32_close
from synth import fp16_bits_to_f32, pack_nibbles, pack_ternary


def rng(i):
    return np.random.default_rng(1234 + i)


def nibbles_of(nib, n):
    return np.stack([nib & 15, nib >> 4], -1).reshape(-1)[:n].astype(np.int64)


# ---------------------------------------------------------------- OIL8 ---
@pytest.mark.parametrize("variant", ["avx2", "scalar"])
@pytest.mark.parametrize("M,N,K", [(3, 1, 64), (2, 3, 67), (4, 2, 5), (1, 1, 4093)])
def test_oil8_integer_codebook_exact(oracle, variant, M, N, K):
    """cb[i] = i-128 and integer x: every partial sum is an integer < 2^24, so
    any summation order gives the exact integer (src/kernel_oil8.cpp:14-60)."""
    g = rng(0)
    idx = g.integers(0, 256, M * N * K, dtype=np.uint8)
    cb = (np.arange(256) - 128).astype(np.float32)
    x = g.integers(-8, 9, N * K).astype(np.float32)
    want = ((idx.reshape(M, N, K).astype(np.int64) - 128) * x.reshape(1, N, K).astype(np.int64)).sum(-1)
    got = oracle.oil8_gemm(idx, cb, x, M, N, K, variant=variant).reshape(M, N)
    assert np.array_equal(got, want.astype(np.float32))
    # a row offset of m*K instead of (m*N+n)*K is a different answer
    if N > 1:
        wrong = ((idx[: M * K].reshape(M, 1, K).astype(np.int64) - 128) * x.reshape(1, N, K)).sum(-1)
        assert not np.array_equal(got, wrong)


@pytest.mark.parametrize("variant", ["avx2", "scalar"])
def test_oil8_brute_force(oracle, variant):
    g = rng(1)
    M, N, K = 5, 2, 300
    idx = g.integers(0, 256, M * N * K, dtype=np.uint8)
    cb = np.sort(g.normal(0, 0.02, 256)).astype(np.float32)
    x = g.normal(0, 1, N * K).astype(np.float32)
    w = cb[idx.reshape(M, N, K)].astype(np.float64) * x.reshape(1, N, K)
    got = oracle.oil8_gemm(idx, cb, x, M, N, K, variant=variant)
    fp32_close(got, w.sum(-1), np.abs(w).sum(-1), rel=2e-6, what="oil8 vs float64")


def test_oil8_gemv_is_per_token_gemm(oracle):
    """The batched decode op = `batch` reference calls with N=1 and per-token
    act/out offsets (the weight-shared GEMV the decode configs run)."""
    g = rng(2)
    M, K, B = 7, 520, 3
    idx = g.integers(0, 256, M * K, dtype=np.uint8)
    cb = g.normal(0, 0.02, 256).astype(np.float32)
    x = g.normal(0, 1, B * K).astype(np.float32)
    y = oracle.oil8_gemv(idx, cb, x, M, K, B)
    for t in range(B):
        for m in range(M):
            ref = oracle.oil8_gemm(idx[m * K:(m + 1) * K], cb, x[t * K:(t + 1) * K], 1, 1, K)
            assert y[t, m].view(np.uint32) == ref[0].view(np.uint32)


# ---------------------------------------------------------------- OIL4 ---
def test_oil4_scalar_closed_form(oracle):
    """Element k = low nibble of byte k/2 for even k, high for odd k
    (src/kernel_oil4.cpp:45-48); integer-valued fp16 codebook -> exact."""
    g = rng(3)
    M, N, K = 3, 2, 70
    codes = g.integers(0, 16, M * N * K)
    nib = pack_nibbles(codes)
    cbv = np.arange(-8, 8).astype(np.float16)
    cb16 = cbv.view(np.uint16)
    x = g.integers(-4, 5, N * K).astype(np.float32)
    want = (cbv.astype(np.int64)[codes].reshape(M, N, K) * x.reshape(1, N, K).astype(np.int64)).sum(-1)
    got = oracle.oil4_gemm(nib, cb16, x, M, N, K, variant="scalar").reshape(M, N)
    assert np.array_equal(got, want.astype(np.float32))
    swapped = pack_nibbles(codes.reshape(-1, 2)[:, ::-1].reshape(-1))
    assert not np.array_equal(oracle.oil4_gemm(swapped, cb16, x, M, N, K, variant="scalar").reshape(M, N),
                              want.astype(np.float32))


def test_oil4_avx2_deviation_closed_form(oracle):
    """oil4_gemm_avx2 adds cb[0]*sum_{k < 16*floor(K/16)} x_k to every output
    (src/kernel_oil4.cpp:57-114): a zeroed lane is gathered as index 0."""
    g = rng(4)
    M, N, K = 4, 2, 70
    codes = g.integers(0, 16, M * N * K)
    nib = pack_nibbles(codes)
    cb16 = (np.arange(16) * 0.5 - 3).astype(np.float16).view(np.uint16)
    x = g.integers(-4, 5, N * K).astype(np.float32)
    sc = oracle.oil4_gemm(nib, cb16, x, M, N, K, variant="scalar").reshape(M, N)
    av = oracle.oil4_gemm(nib, cb16, x, M, N, K, variant="avx2").reshape(M, N)
    k16 = 16 * (K // 16)
    extra = fp16_bits_to_f32(cb16)[0] * x.reshape(N, K)[:, :k16].sum(-1)
    assert np.array_equal(av, sc + extra.reshape(1, N).astype(np.float32))
    assert np.any(extra != 0)


def test_oil4_blocked_brute_force(oracle):
    g = rng(5)
    M, K, B, blk = 6, 512, 2, 128
    codes = g.integers(0, 16, (M, K))
    nib = pack_nibbles(codes)
    cbf = g.normal(0, 0.02, (M, K // blk, 16)).astype(np.float16)
    x = g.normal(0, 1, (B, K)).astype(np.float32)
    w = np.take_along_axis(cbf.astype(np.float64).repeat(blk, axis=1), codes[..., None], -1)[..., 0]
    want = x.astype(np.float64) @ w.T
    got = oracle.oil4_gemv_blocked(nib.reshape(-1), cbf.view(np.uint16).reshape(-1), x.reshape(-1), M, K, B, blk)
    fp32_close(got, want, np.abs(x) @ np.abs(w).T, rel=2e-6, what="oil4 blocked vs float64")
    # one block spanning the row = the reference scalar kernel, bit for bit
    one = cbf[:, :1].copy()
    for m in range(M):
        y1 = oracle.oil4_gemv_blocked(nib[m], one[m].view(np.uint16).reshape(-1), x[0], 1, K, 1, K)
        ref = oracle.oil4_gemm(nib[m], one[m].view(np.uint16).reshape(-1), x[0], 1, 1, K, variant="scalar")
        assert y1[0, 0].view(np.uint32) == ref[0].view(np.uint32)


# ---------------------------------------------------------------- FP16 ---
def test_fp16_to_float_exhaustive(oracle):
    """src/kernel_oil4.cpp:15-29 is the exact IEEE conversion: all 65536 bit
    patterns against numpy's float16 (NaNs compared as NaN)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.fp16_to_float(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_half_to_float_codebook_normals(oracle):
    """src/codebook.cpp:36-64 agrees with IEEE on zeros, normals and infinities;
    its subnormal branch differs and is pinned by the golden table."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    e = (h >> 10) & 31
    sel = h[(e > 0) & (e < 31)][::7]
    got = np.array([oracle.half_to_float_codebook(int(v)) for v in sel], np.float32)
    assert np.array_equal(got.view(np.uint32), sel.view(np.float16).astype(np.float32).view(np.uint32))
    for v in (0x0000, 0x8000, 0x7C00, 0xFC00):
        assert oracle.half_to_float_codebook(v) == np.uint16(v).view(np.float16).astype(np.float32)


def test_float_to_half_truncates(oracle):
    """src/codebook.cpp:16-34 rounds toward zero: |half(f)| <= |f| < next."""
    g = rng(6)
    f = np.concatenate([g.normal(0, 0.02, 2000), g.normal(0, 300, 2000)]).astype(np.float32)
    h = np.array([oracle.float_to_half_trunc(float(v)) for v in f], np.uint16)
    hv = h.view(np.float16).astype(np.float64)
    nxt = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)   # same sign, one ulp further
    a = np.abs(f.astype(np.float64))
    ok = np.abs(hv) <= a
    ok &= (a < np.abs(nxt)) | (np.abs(hv) == 65504.0)
    ok &= np.signbit(hv) == np.signbit(f)
    assert ok.all()
    # round-to-nearest would differ on about half of these
    assert np.mean(h != f.astype(np.float16).view(np.uint16)) > 0.3


# --------------------------------------------------------- int8 quant ---
def test_quantize_round_half_away_and_floor(oracle):
    """q = (int8)round(x*127/max|x|) with std::round (ties away from zero);
    max|x| floored at 1e-10 (src/int8_quant.cpp:8-31)."""
    x = np.zeros((2, 8), np.float32)
    x[0] = [127.0, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, -127.0]
    q, s, inv = oracle.quantize_per_token(x, 2, 8)
    assert q[0].tolist() == [127, 64, -64, 1, -1, 2, -3, -127]
    assert s[0] == np.float32(1.0) and inv[0] == np.float32(1.0)
    assert q[1].tolist() == [0] * 8
    assert inv[1] == np.float32(np.float32(1e-10) / np.float32(127.0))


# ------------------------------------------------------------- ternary ---
def test_i2s_gemv_integer_closed_form(oracle):
    """(sum_i t_i*a_i) * w_scale * act_scale in FP32 with an exact integer sum;
    code = t+1, element 4i+j in bits 2j (src/kernel_i2s.cpp:13-40)."""
    g = rng(7)
    K = 1024
    t = g.integers(-1, 2, K)
    packed = pack_ternary(t)
    a = g.integers(-127, 128, K).astype(np.int8)
    S = int((t.astype(np.int64) * a.astype(np.int64)).sum())
    ws, asc = np.float32(0.0159577), np.float32(0.0213)
    got = oracle.i2s_gemv(packed, float(ws), a, float(asc), K)
    assert np.float32(got) == np.float32(np.float32(np.float32(S) * ws) * asc)
    # the fused op: x -> per-token int8 -> same value
    x = g.normal(0, 1, K).astype(np.float32)
    q, _, inv = oracle.quantize_per_token(x, 1, K)
    S2 = int((t.astype(np.int64) * q[0].astype(np.int64)).sum())
    y = oracle.i2s_gemv_f32(packed, float(ws), x, 1, K, 1)
    assert y[0, 0] == np.float32(np.float32(np.float32(S2) * ws) * inv[0])


def test_i2s_gemm_brute_force(oracle):
    g = rng(8)
    M, N, K = 3, 4, 260
    t = g.integers(-1, 2, (M, K))
    w = pack_ternary(t).reshape(-1)
    a = g.normal(0, 1, N * K).astype(np.float32)
    want = t.astype(np.float64) @ a.reshape(N, K).T.astype(np.float64)
    got = oracle.i2s_gemm(w, a, M, N, K).reshape(M, N)
    fp32_close(got, want, np.abs(t) @ np.abs(a.reshape(N, K)).T, rel=2e-6, what="i2s_gemm")
    ai = g.integers(-128, 128, N * K).astype(np.int8)
    exact = t.astype(np.int64) @ ai.reshape(N, K).T.astype(np.int64)
    assert np.array_equal(oracle.i2s_gemm_vnni(w, ai, M, N, K).reshape(M, N), exact.astype(np.float32))


def test_tl2_exact_integer(oracle):
    """tl2 = (float)sum(a_i8 * t) / (127/max|a|) for K % 3 == 0."""
    g = rng(9)
    M, N, K = 2, 3, 36
    t = g.integers(-1, 2, (M, N, K))
    w = pack_ternary(t).reshape(-1)
    a = g.normal(0, 0.5, N * K).astype(np.float32)
    mx = np.abs(a.reshape(N, K)).max(-1).astype(np.float32)
    sc = (np.float32(127.0) / mx).astype(np.float32)
    ai = np.array([np.float32(v) * sc[i // K] for i, v in enumerate(a)], np.float32)
    ai = np.where(ai >= 0, np.floor(ai + 0.5), np.ceil(ai - 0.5)).astype(np.int64).reshape(N, K)
    tot = (t.astype(np.int64) * ai[None]).sum(-1)
    want = (tot.astype(np.float32) / sc[None]).astype(np.float32)
    assert np.array_equal(oracle.tl2_gemm(w, a, M, N, K).reshape(M, N), want)


def test_tl1_reference_p5_finite(oracle):
    """tests/test_protected.cpp:177-196 (P5): TL1 on RNG(77) inputs is finite."""
    M, N, K = 4, 4, 16
    u = oracle.rng_uniform(77, M * K + K * N)
    w = (u[: M * K] * np.float32(3.0)).astype(np.uint8)
    a = ((u[M * K:] * np.float32(2.0) - np.float32(1.0)) * np.float32(0.5)).astype(np.float32)
    assert np.isfinite(oracle.tl1_gemm(w, a, M, N, K)).all()


# --------------------------------------------------------------- dense ---
def test_gemv_known_answer(oracle):
    """tests/test_math.cpp:74-91: A=[[1,2,3],[4,5,6]], x=[2,3,4] -> [20, 47]."""
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    x = np.array([2, 3, 4], np.float32)
    y = oracle.gemv(1.0, A, x, 0.0, np.ones(2, np.float32), 2, 3)
    assert y.tolist() == [20.0, 47.0]


def test_rms_norm_and_silu(oracle):
    g = rng(10)
    x = g.normal(0, 2, (3, 128)).astype(np.float32)
    gam = g.uniform(0.5, 1.5, 128).astype(np.float32)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-5) * gam
    np.testing.assert_allclose(oracle.rms_norm(x, gam, 1e-5, 3, 128), want, rtol=2e-6, atol=0)
    s = g.normal(0, 5, 1000).astype(np.float32)
    np.testing.assert_allclose(oracle.silu(s), s / (1 + np.exp(-s.astype(np.float64))), rtol=2e-6, atol=1e-30)


def test_gemm_closed_forms(oracle):
    """math::gemm (src/math.cpp:74-97): small-integer operands make every sum
    exact, so C = alpha*(A B) + beta*C must equal the integer product; a
    one-column B is math::gemv bit for bit (same sum order); C is read even
    with beta = 0, so NaN/Inf there reach the result as in the reference."""
    g = rng(21)
    M, N, K = 7, 5, 33
    A = g.integers(-8, 9, (M, K)).astype(np.float32)
    B = g.integers(-8, 9, (K, N)).astype(np.float32)
    C = g.integers(-8, 9, (M, N)).astype(np.float32)
    want = 2.0 * (A.astype(np.int64) @ B.astype(np.int64)) - 0.5 * C
    assert np.array_equal(oracle.gemm(2.0, A, B, -0.5, C, M, N, K), want.astype(np.float32))
    x = g.normal(0, 1, K).astype(np.float32)
    y0 = g.normal(0, 1, M).astype(np.float32)
    col = oracle.gemm(1.5, A, x.reshape(K, 1).copy(), 0.25, y0.reshape(M, 1), M, 1, K)
    assert np.array_equal(col.ravel(), oracle.gemv(1.5, A, x, 0.25, y0, M, K))
    Cn = np.zeros((M, N), np.float32)
    Cn[1, 2], Cn[3, 4] = np.nan, np.inf
    out = oracle.gemm(1.0, A, B, 0.0, Cn, M, N, K)
    assert np.isnan(out[1, 2]) and np.isnan(out[3, 4])  # 0 * NaN, 0 * Inf
    assert np.isfinite(np.delete(out.ravel(), [1 * N + 2, 3 * N + 4])).all()


def test_relu_gelu_scale(oracle):
    """relu / gelu / scale (src/math.cpp:99-117, :278-284): relu exactly
    max(x, 0) with NaN -> 0; gelu against float64 0.5 x (1 + erf(x/sqrt 2)),
    the FP32 bound one ulp of 1 in (1 + erf) times |x|/2 (the sum cancels for
    x << 0) plus a few ulps of the result; scale by powers of two is exact."""
    import math
    x = np.array([-3.0, -0.0, 0.0, 1e-30, 2.5, np.nan, np.inf, -np.inf], np.float32)
    r = oracle.relu(x)
    assert r.tolist()[:5] == [0.0, 0.0, 0.0, np.float32(1e-30), 2.5] and r[5] == 0.0
    assert r[6] == np.inf and r[7] == 0.0
    g = rng(22)
    v = np.concatenate([g.normal(0, 3, 4000), np.linspace(-12, 12, 97), [0.0]]).astype(np.float32)
    want = np.array([0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))) for t in v.astype(np.float64)])
    got = oracle.gelu(v).astype(np.float64)
    bound = 4e-7 * np.abs(want) + 2.5e-7 * np.abs(0.5 * v.astype(np.float64)) + 1e-37
    assert np.all(np.abs(got - want) <= bound), float(np.max(np.abs(got - want) - bound))
    assert oracle.gelu(np.array([0.0], np.float32))[0] == 0.0
    for s in (0.5, 4.0, -2.0):
        assert np.array_equal(oracle.scale(s, v), v * np.float32(s))


def test_layer_norm_properties(oracle):
    """layer_norm (src/math.cpp:148-180): gamma = 1, beta = 0 leaves every
    row with mean 0 and (biased) variance var / (var + eps); gamma and beta
    are an exact affine map of that output; against float64."""
    g = rng(23)
    rows, dim, eps = 5, 300, 1e-5
    x = (g.normal(0, 2, (rows, dim)) + g.normal(0, 10, (rows, 1))).astype(np.float32)
    one, zero = np.ones(dim, np.float32), np.zeros(dim, np.float32)
    z = oracle.layer_norm(x, one, zero, eps, rows, dim).astype(np.float64)
    xd = x.astype(np.float64)
    var = xd.var(axis=1, keepdims=True)
    assert np.abs(z.mean(axis=1)).max() < 1e-6
    np.testing.assert_allclose(z.var(axis=1, keepdims=True), var / (var + eps), rtol=1e-6)
    np.testing.assert_allclose(z, (xd - xd.mean(axis=1, keepdims=True)) / np.sqrt(var + eps), rtol=2e-6, atol=1e-6)
    gam = g.uniform(0.5, 1.5, dim).astype(np.float32)
    bet = g.normal(0, 1, dim).astype(np.float32)
    y = oracle.layer_norm(x, gam, bet, eps, rows, dim)
    assert np.array_equal(y, z.astype(np.float32) * gam + bet)


def test_softmax_axis(oracle):
    """softmax along any axis (src/math.cpp:207-249): inner = 1 is the
    row softmax bit for bit; along axis 0 of [dim][inner] it is the row
    softmax of the transpose bit for bit (same per-column order); every
    column sums to 1."""
    g = rng(24)
    outer, dim, inner = 3, 41, 7
    x = g.normal(0, 4, outer * dim * inner).astype(np.float32)
    rows = oracle.softmax(x, outer * inner * dim // dim, dim)
    assert np.array_equal(oracle.softmax_axis(x, outer * inner, dim, 1), rows.ravel())
    y = oracle.softmax_axis(x, outer, dim, inner).reshape(outer, dim, inner)
    xt = np.ascontiguousarray(x.reshape(outer, dim, inner).transpose(0, 2, 1)).ravel()
    yt = oracle.softmax(xt, outer * inner, dim).reshape(outer, inner, dim).transpose(0, 2, 1)
    assert np.array_equal(y, yt)
    np.testing.assert_allclose(y.astype(np.float64).sum(axis=1), 1.0, rtol=1e-6)


# -------------------------------------------------------------- prefill ---
def test_prefill_reference(oracle):
    """C = bf16(sum_k A[m][k] W[n][k]): against a float64 contraction of the
    dequantised weights and against the blocked GEMV row by row."""
    from synth import bf16_bits, bf16_to_f32
    g = rng(11)
    M, N, K, blk = 5, 6, 256, 128
    a = bf16_bits(g.normal(0, 1, (M, K)).astype(np.float32))
    codes = g.integers(0, 16, (N, K))
    nib = pack_nibbles(codes)
    cbf = g.normal(0, 0.02, (N, K // blk, 16)).astype(np.float16)
    c16, c32 = oracle.oil4_gemm_prefill(a.reshape(-1), nib.reshape(-1), cbf.view(np.uint16).reshape(-1),
                                        M, N, K, blk)
    w = np.take_along_axis(cbf.astype(np.float64).repeat(blk, axis=1), codes[..., None], -1)[..., 0]
    af = bf16_to_f32(a).astype(np.float64)
    fp32_close(c32, af @ w.T, np.abs(af) @ np.abs(w).T, rel=2e-6, what="prefill fp32")
    assert np.array_equal(c16, bf16_bits(c32.astype(np.float32)))
    y = oracle.oil4_gemv_blocked(nib.reshape(-1), cbf.view(np.uint16).reshape(-1),
                                 bf16_to_f32(a).reshape(-1), N, K, M, blk)
    fp32_close(c32, y, np.abs(af) @ np.abs(w).T, rel=2e-6, what="prefill vs gemv")
