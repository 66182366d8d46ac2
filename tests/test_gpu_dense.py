"""GPU parity of the FP32 decode-step operators (dense.hip) through the C ABI
against the CPU oracle (oracle/decoder.c, oracle.c) on seeded inputs.

Bars: elementwise add/mul, RoPE and the KV append, argmax bit-exact; RMSNorm
bit-exact up to one ulp (double sums in another order); SiLU/softmax within a
few ulp (device exp); attention within 1e-5 relative (FP32, reordered sums).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def dev_t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).copy()).to(dev)


def host(t):
    return t.cpu().numpy()


def ulp_diff(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-2**31) - a, a)
    b = np.where(b < 0, np.int64(-2**31) - b, b)
    return np.abs(a - b)


@pytest.mark.parametrize("rows,dim", [(1, 4096), (16, 4096), (3, 1000), (2, 37)])
def test_rms_norm(rows, dim, oracle, mth, dev):
    import torch
    print(f"rms_norm rows={rows} dim={dim}", flush=True)
    g = np.random.default_rng(rows * 7 + dim)
    x = (g.normal(0, 3, (rows, dim))).astype(np.float32)
    gm = g.uniform(0.5, 1.5, dim).astype(np.float32)
    dx, dg = dev_t(x, dev), dev_t(gm, dev)
    y = torch.empty_like(dx)
    mth.rms_norm(dx, dg, y, rows, dim, 1e-5)
    want = np.empty_like(x)
    oracle.lib.orc_rms_norm(x.ctypes.data, gm.ctypes.data, 1e-5, want.ctypes.data, rows, dim)
    assert ulp_diff(host(y), want).max() <= 1
    # residual add fused in: x <- t + x exactly, then the norm of the sum
    t = g.normal(0, 1, (rows, dim)).astype(np.float32)
    mth.add_rms_norm(dx, dev_t(t, dev), dg, y, rows, dim, 1e-5)
    s = t + x
    assert np.array_equal(host(dx), s)
    oracle.lib.orc_rms_norm(s.ctypes.data, gm.ctypes.data, 1e-5, want.ctypes.data, rows, dim)
    assert ulp_diff(host(y), want).max() <= 1
    # in place
    mth.rms_norm(dx, dg, dx, rows, dim, 1e-5)
    assert ulp_diff(host(dx), want).max() <= 1


def test_elementwise(oracle, mth, dev):
    import torch
    g = np.random.default_rng(5)
    n = 11008 * 3 + 5
    a = g.normal(0, 4, n).astype(np.float32)
    b = g.normal(0, 1, n).astype(np.float32)
    da, db = dev_t(a, dev), dev_t(b, dev)
    c = torch.empty_like(da)
    mth.add(da, db, c, n)
    assert np.array_equal(host(c), a + b)
    mth.mul(da, db, c, n)
    assert np.array_equal(host(c), a * b)
    mth.silu(da, c, n)
    want = np.empty_like(a)
    oracle.lib.orc_silu(a.ctypes.data, want.ctypes.data, n)
    assert ulp_diff(host(c), want).max() <= 4
    # SwiGLU over rows of a fused [gate | up] output
    rows, F = 3, 11008
    gu = g.normal(0, 2, (rows, 2 * F)).astype(np.float32)
    y = torch.empty((rows, F), dtype=torch.float32, device=dev)
    dgu = dev_t(gu, dev)
    mth.silu_mul(dgu.view(-1), dgu.view(-1)[F:], y, rows, F, 2 * F, 2 * F)
    want = oracle.silu_mul(np.ascontiguousarray(gu[:, :F]), np.ascontiguousarray(gu[:, F:]))
    assert ulp_diff(host(y), want).max() <= 4


@pytest.mark.parametrize("rows,n", [(1, 11008), (16, 11008), (2, 100), (3, 12288)])
def test_silu_mul_quant_bit_exact(rows, n, oracle, mth, dev):
    """The int8 activations and scales equal quantize_per_token of the
    device's own SwiGLU output (bit for bit); that output is checked against
    the oracle in test_elementwise."""
    import torch
    print(f"silu_mul_quant rows={rows} n={n}", flush=True)
    g = np.random.default_rng(n + rows)
    gu = g.normal(0, 2, (rows, 2 * n)).astype(np.float32)
    if rows > 1:
        gu[1] = 0.0                                   # all-zero row: max_abs floor 1e-10
    dgu = dev_t(gu, dev).view(-1)
    a = torch.empty((rows, n), dtype=torch.float32, device=dev)
    mth.silu_mul(dgu, dgu[n:], a, rows, n, 2 * n, 2 * n)
    q = torch.empty((rows, n), dtype=torch.int8, device=dev)
    inv = torch.empty(rows, dtype=torch.float32, device=dev)
    mth.silu_mul_quant(dgu, dgu[n:], q, inv, rows, n, 2 * n, 2 * n)
    ha = host(a)
    wq = np.empty((rows, n), np.int8)
    winv = np.empty(rows, np.float32)
    oracle.lib.orc_quantize_per_token(ha.ctypes.data, wq.ctypes.data, rows, n, None, winv.ctypes.data)
    assert np.array_equal(host(q), wq)
    assert np.array_equal(host(inv), winv)


@pytest.mark.parametrize("rows,dim", [(4, 192), (2, 32000), (3, 5)])
def test_softmax(rows, dim, oracle, mth, dev):
    import torch
    print(f"softmax rows={rows} dim={dim}", flush=True)
    g = np.random.default_rng(dim)
    x = (g.normal(0, 5, (rows, dim))).astype(np.float32)
    x[0, ::4] = -np.inf
    y = torch.empty((rows, dim), dtype=torch.float32, device=dev)
    mth.softmax(dev_t(x, dev), y, rows, dim)
    want = oracle.softmax(x, rows, dim)
    got = host(y)
    assert np.all(got[0, ::4] == 0)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)


# ---- the ComputeBackend vtable's remaining dense operators --------------------
@pytest.mark.parametrize("outer,dim,inner", [(3, 41, 7), (1, 1000, 1), (2, 5, 300), (1, 1, 9)])
def test_softmax_axis(outer, dim, inner, oracle, mth, dev):
    import torch
    print(f"softmax_axis {outer}x{dim}x{inner}", flush=True)
    g = np.random.default_rng(outer * 100 + dim + inner)
    x = g.normal(0, 5, outer * dim * inner).astype(np.float32)
    y = torch.empty(outer * dim * inner, dtype=torch.float32, device=dev)
    mth.softmax_axis(dev_t(x, dev), y, outer, dim, inner)
    np.testing.assert_allclose(host(y), oracle.softmax_axis(x, outer, dim, inner), rtol=2e-6, atol=1e-30)


def test_axpby_rounding_and_nan(oracle, mth, dev):
    """alpha*x + beta*y with each product and the sum rounded (the gemm/gemv
    epilogue, src/math.cpp:70,94): bit-exact against numpy's float32
    operations; y is read even with beta = 0, so NaN/Inf there propagate."""
    import torch
    g = np.random.default_rng(31)
    n = 70001
    x = g.normal(0, 3, n).astype(np.float32)
    y0 = g.normal(0, 3, n).astype(np.float32)
    for alpha, beta in ((1.7, -0.3), (1.0, 0.0), (0.0, 2.5)):
        y = dev_t(y0, dev)
        mth.axpby(alpha, dev_t(x, dev), beta, y, n)
        want = np.float32(alpha) * x + np.float32(beta) * y0
        assert np.array_equal(host(y), want), (alpha, beta)
    y0[[5, 17]] = np.nan, np.inf
    y = dev_t(y0, dev)
    mth.axpby(1.0, dev_t(x, dev), 0.0, y, n)
    got = host(y)
    assert np.isnan(got[5]) and np.isnan(got[17]) and np.array_equal(np.delete(got, [5, 17]), np.delete(x, [5, 17]))


@pytest.mark.parametrize("M,N", [(4096, 4096), (37, 1001), (1, 64), (300, 3)])
def test_gemv_f32(M, N, oracle, mth, dev):
    import torch
    from conftest import fp32_close
    print(f"gemv_f32 M={M} N={N}", flush=True)
    g = np.random.default_rng(M + 7 * N)
    A = g.normal(0, 1, (M, N)).astype(np.float32)
    x = g.normal(0, 1, N).astype(np.float32)
    y0 = g.normal(0, 1, M).astype(np.float32)
    y = dev_t(y0, dev)
    mth.gemv_f32(0.75, dev_t(A, dev), dev_t(x, dev), -1.25, y, M, N)
    want = oracle.gemv(0.75, A, x, -1.25, y0, M, N)
    absw = 0.75 * (np.abs(A.astype(np.float64)) @ np.abs(x.astype(np.float64))) + 1.25 * np.abs(y0)
    fp32_close(host(y), want, absw, 1e-5, "gemv_f32")
    # integers: exact in any order
    Ai = g.integers(-8, 9, (M, N)).astype(np.float32)
    xi = g.integers(-8, 9, N).astype(np.float32)
    y = dev_t(y0, dev)
    mth.gemv_f32(1.0, dev_t(Ai, dev), dev_t(xi, dev), 0.0, y, M, N)
    assert np.array_equal(host(y), oracle.gemv(1.0, Ai, xi, 0.0, y0, M, N))


def test_relu_gelu_scale(oracle, mth, dev):
    import torch
    g = np.random.default_rng(32)
    x = np.concatenate([g.normal(0, 3, 50000), np.linspace(-12, 12, 301),
                        [0.0, -0.0, np.inf, -np.inf, np.nan]]).astype(np.float32)
    n = x.size
    dx, y = dev_t(x, dev), torch.empty(n, dtype=torch.float32, device=dev)
    mth.relu(dx, y, n)
    assert np.array_equal(host(y), oracle.relu(x))
    mth.scale(-0.375, dx, y, n)
    assert np.array_equal(host(y), oracle.scale(-0.375, x), equal_nan=True)
    mth.gelu(dx, y, n)
    got, want = host(y).astype(np.float64), oracle.gelu(x).astype(np.float64)
    fin = np.isfinite(want)
    # device erff vs the C library's: a few ulps of erf, amplified by the
    # cancellation in 1 + erf for x << 0 (the reference's own FP32 form)
    bound = 4e-7 * np.abs(want[fin]) + 2.5e-7 * np.abs(0.5 * x[fin].astype(np.float64)) + 1e-37
    assert np.all(np.abs(got[fin] - want[fin]) <= bound)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)])


@pytest.mark.parametrize("rows,dim", [(4, 4096), (3, 1000), (1, 7)])
def test_layer_norm(rows, dim, oracle, mth, dev):
    import torch
    print(f"layer_norm rows={rows} dim={dim}", flush=True)
    g = np.random.default_rng(rows * 13 + dim)
    x = (g.normal(0, 2, (rows, dim)) + g.normal(0, 20, (rows, 1))).astype(np.float32)
    gm = g.uniform(0.5, 1.5, dim).astype(np.float32)
    bt = g.normal(0, 1, dim).astype(np.float32)
    y = torch.empty((rows, dim), dtype=torch.float32, device=dev)
    mth.layer_norm(dev_t(x, dev), dev_t(gm, dev), dev_t(bt, dev), y, rows, dim, 1e-5)
    want = oracle.layer_norm(x, gm, bt, 1e-5, rows, dim)
    # double statistics summed in another order: (float)(d * inv) may differ by
    # one ulp, then * gamma + beta (two roundings)
    z = np.abs(want.astype(np.float64) - bt)
    bound = 3 * np.finfo(np.float32).eps * (z + np.abs(want)) + 1e-30
    assert np.all(np.abs(host(y).astype(np.float64) - want) <= bound)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_rope_kv_bit_exact(D, oracle, mth, dev):
    import torch
    print(f"rope_kv D={D}", flush=True)
    B, H, KVH, S, pos = 2, 4, 2, 40, 33
    g = np.random.default_rng(D)
    cos_t, sin_t = mth.rope_tables(D, S)
    oc, os_ = oracle.rope_tables(D, S)
    assert np.array_equal(cos_t, oc) and np.array_equal(sin_t, os_)   # same float recipe
    q = g.normal(0, 1, (B, H * D)).astype(np.float32)
    k = g.normal(0, 1, (B, KVH * D)).astype(np.float32)
    v = g.normal(0, 1, (B, KVH * D)).astype(np.float32)
    kc = torch.zeros((B, KVH, S, D), dtype=torch.float32, device=dev)
    vc = torch.zeros_like(kc)
    dq = dev_t(q, dev)
    mth.rope_kv(dq, dev_t(k, dev), dev_t(v, dev), dev_t(cos_t, dev), dev_t(sin_t, dev), kc, vc, pos, B, H, KVH, D, S)
    for b in range(B):
        assert np.array_equal(host(dq)[b], oracle.rope_apply(q[b], H, D, pos, oc, os_))
        assert np.array_equal(host(kc)[b, :, pos].ravel(), oracle.rope_apply(k[b], KVH, D, pos, oc, os_))
        assert np.array_equal(host(vc)[b, :, pos].ravel(), v[b])
    assert not host(kc)[:, :, :pos].any() and not host(kc)[:, :, pos + 1:].any()


# contexts past the rows a thread preloads (the K rows of 192 positions, the V rows of 64 at D = 128) run the
# batched tail loops: ragged ends at 700, 1500, 333, 1999 and 1200 positions; max_seq > 1024 takes 16 waves
@pytest.mark.parametrize("D,ctx,S", [(128, 1, 192), (128, 37, 192), (128, 192, 192), (64, 100, 128),
                                     (256, 17, 32), (128, 700, 1024), (64, 1500, 2048), (256, 333, 512),
                                     (128, 1999, 2048), (256, 1200, 1500)])
def test_attention(D, ctx, S, oracle, mth, dev):
    import torch
    print(f"attention D={D} ctx={ctx} S={S}", flush=True)
    B, H, KVH = 2, 4, 2
    g = np.random.default_rng(ctx + D)
    q = g.normal(0, 1, (B, H * D)).astype(np.float32)
    kc = g.normal(0, 1, (B, KVH, S, D)).astype(np.float32)
    vc = g.normal(0, 1, (B, KVH, S, D)).astype(np.float32)
    out = torch.empty((B, H * D), dtype=torch.float32, device=dev)
    mth.attention_decode(dev_t(q, dev), dev_t(kc, dev), dev_t(vc, dev), out, B, H, KVH, D, ctx, S)
    got = host(out)
    for b in range(B):
        want = oracle.attention_decode(q[b], np.ascontiguousarray(kc[b]), np.ascontiguousarray(vc[b]), H, KVH, D,
                                       ctx, S)
        err = np.linalg.norm(got[b] - want) / np.linalg.norm(want)
        assert err < 1e-5, (b, err)


@pytest.mark.parametrize("rows,n", [(16, 32000), (1, 5), (2, 2049), (3, 6143)])
def test_argmax_shapes(rows, n, oracle, mth, dev):
    import torch
    g = np.random.default_rng(n)
    x = g.normal(0, 1, (rows, n)).astype(np.float32)
    x[0, n // 2] = x[0, n - 1] = 9.0                 # tie across chunks: the first wins
    ids = torch.empty(rows, dtype=torch.int32, device=dev)
    mth.argmax(dev_t(x, dev), ids, rows, n)
    assert list(host(ids)) == [oracle.argmax(r) for r in x]


def test_argmax_rules(oracle, mth, dev):
    import torch
    n = 32000
    g = np.random.default_rng(9)
    rows = [g.normal(0, 1, n).astype(np.float32) for _ in range(6)]
    rows[1][[5, 700, 31999]] = 50.0                  # ties: the first wins
    rows[2][:] = np.nan
    rows[3][:] = -np.inf
    rows[4][::2] = np.nan                            # NaNs never win
    rows[5][31999] = np.inf
    x = np.stack(rows)
    ids = torch.empty(6, dtype=torch.int32, device=dev)
    mth.argmax(dev_t(x, dev), ids, 6, n)
    assert list(host(ids)) == [oracle.argmax(r) for r in rows]
    assert host(ids)[1] == 5 and host(ids)[2] == 0 and host(ids)[3] == 0 and host(ids)[5] == 31999
