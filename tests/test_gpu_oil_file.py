"""GPU: a `.oil` model file read by libmythos_host.so straight into device
memory (mth_oil_upload) feeds the GEMV kernels, and the results match the
oracle on the weights the file holds.  The file is written by the test-side
writer that test_oil_file.py pins byte-for-byte to the reference's OILWriter.
"""
import numpy as np
import pytest

import synth
from conftest import fp32_close
from test_oil_file import oil4_cb_bytes, oil8_cb_bytes, pack_codes, write_oil

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    """OIL4 with per-128 codebooks (one block each), OIL8 split into blocks
    that share a codebook, and a ternary tensor."""
    M4, K4, B = 512, 1024, 128
    packed, cbs, _ = synth.oil4(M4, K4, 1, B)
    M8, K8 = 256, 1024
    idx, cb, _ = synth.oil8(M8, K8, 1)
    Mt, Kt = 128, 1024
    tpk, _, _ = synth.ternary(Mt, Kt, 1)
    blocks, tensors = [], []
    flat = packed.reshape(-1)
    tensors.append(("blk.0.ffn_gate.weight", 0, M4 * K4 // B))
    for b in range(M4 * K4 // B):
        blocks.append((2, B, oil4_cb_bytes(cbs.reshape(-1, 16)[b]), flat[b * B // 2:(b + 1) * B // 2].tobytes()))
    tensors.append(("blk.0.attn_v.weight", len(blocks), 4))
    q = M8 * K8 // 4
    for b in range(4):
        blocks.append((3, q, oil8_cb_bytes(cb), idx.reshape(-1)[b * q:(b + 1) * q].tobytes()))
    tensors.append(("blk.0.attn_o.weight", len(blocks), 1))
    blocks.append((1, Mt * Kt, np.array([-1, 0, 1], "<f4").tobytes(), tpk.tobytes()))
    p = tmp_path_factory.mktemp("gpu_oil") / "model.oil"
    write_oil(p, b"{}", blocks, tensors)
    return str(p), dict(oil4=(packed, cbs, M4, K4, B), oil8=(idx, cb, M8, K8), tern=(tpk, Mt, Kt))


def dev_x(batch, K, seed, dev):
    import torch
    x = np.random.default_rng(seed).normal(0, 1, (batch, K)).astype(np.float32)
    return x, torch.from_numpy(x).to(dev)


@pytest.mark.parametrize("batch", [1, 4])
def test_oil4_upload_gemv(batch, model, oracle, mth, dev):
    import torch
    import oil_file
    path, t = model
    packed, cbs, M, K, B = t["oil4"]
    print(f"oil upload oil4 M={M} K={K} batch={batch}", flush=True)
    with oil_file.OILReader(path) as r:
        d_nib, d_cbs, cbk = r.upload("blk.0.ffn_gate.weight", M, K, dev)
    assert cbk == B
    assert np.array_equal(d_nib.cpu().numpy(), packed)
    assert np.array_equal(d_cbs.cpu().numpy().view(np.uint16), cbs.reshape(-1))
    x, dx = dev_x(batch, K, 1, dev)
    y = torch.full((batch * M,), float("nan"), device=dev)
    mth.oil4_gemv(d_nib, d_cbs, cbk, dx, y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, B, threads=8)
    W = synth.dequant_oil4(packed, cbs, M, K, B)
    absw = np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64)).T
    fp32_close(y.cpu().numpy().reshape(batch, M), ref, absw.T, 1e-5, "oil4 from .oil")


def test_oil8_upload_gemv(model, oracle, mth, dev):
    import torch
    import oil_file
    path, t = model
    idx, cb, M, K = t["oil8"]
    print(f"oil upload oil8 M={M} K={K}", flush=True)
    with oil_file.OILReader(path) as r:
        d_idx, d_cb, _ = r.upload("blk.0.attn_v.weight", M, K, dev)
    x, dx = dev_x(1, K, 2, dev)
    y = torch.full((M,), float("nan"), device=dev)
    mth.oil8_gemv(d_idx, d_cb, dx, y, M, K, 1)
    torch.cuda.synchronize()
    ref = oracle.oil8_gemv(idx, cb, x, M, K, 1, threads=8)
    absw = np.abs(cb[idx]).astype(np.float64) @ np.abs(x[0].astype(np.float64))
    fp32_close(y.cpu().numpy().reshape(1, M), ref, absw[None], 1e-5, "oil8 from .oil")


def test_ternary_upload_gemv_bit_exact(model, oracle, mth, dev):
    import torch
    import oil_file
    path, t = model
    tpk, M, K = t["tern"]
    print(f"oil upload ternary M={M} K={K}", flush=True)
    with oil_file.OILReader(path) as r:
        d_pk, d_cb, _ = r.upload("blk.0.attn_o.weight", M, K, dev)
    assert np.array_equal(d_cb.cpu().numpy(), np.array([-1, 0, 1], np.float32))
    assert np.array_equal(d_pk.cpu().numpy(), tpk.reshape(-1))
    # the file's codebook {-1, 0, +1} is the I2_S decode with scale 1
    x, dx = dev_x(2, K, 3, dev)
    y = torch.full((2 * M,), float("nan"), device=dev)
    mth.i2s_gemv_f32(d_pk, 1.0, dx, y, M, K, 2)
    torch.cuda.synchronize()
    ref = oracle.i2s_gemv_f32(tpk.ravel(), 1.0, x, M, K, 2, threads=8)
    assert np.array_equal(y.cpu().numpy().reshape(2, M), ref)


def test_linear_weights_reproduce_reference_forward(oracle, mth, dev, tmp_path):
    """Input-major Linear weights (the reference model's layout) uploaded with
    in_major give the reference's Linear::forward outputs (golden y)."""
    import os
    import torch
    import oil_file
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oil_linear.npz"))
    p = tmp_path / "linear.oil"
    g["oil"].tofile(p)
    M, K, nt = (int(v) for v in g["shape"])
    print(f"oil upload linear M={M} K={K} batch={nt}", flush=True)
    x = g["x"]
    dx = torch.from_numpy(x.copy()).to(dev)
    with oil_file.OILReader(str(p)) as r:
        d_idx, d_cb, _ = r.upload("layers.0.attention.q_proj.weight", M, K, dev, in_major=True)
        d_nib, d_cb4, cbk = r.upload("layers.0.ffn.up_proj.weight", M, K, dev, in_major=True)
    y8 = torch.full((nt * M,), float("nan"), device=dev)
    y4 = torch.full((nt * M,), float("nan"), device=dev)
    mth.oil8_gemv(d_idx, d_cb, dx, y8, M, K, nt)
    mth.oil4_gemv(d_nib, d_cb4, cbk, dx, y4, M, K, nt)
    torch.cuda.synchronize()
    for i, y in ((0, y8), (1, y4)):
        w = g[f"w_{i}"].reshape(K, M).astype(np.float64)        # reader's tensor, input-major
        absw = np.abs(x.astype(np.float64)) @ np.abs(w)
        fp32_close(y.cpu().numpy().reshape(nt, M), g[f"y_{i}"].reshape(nt, M), absw, 1e-5, f"linear {i}")
