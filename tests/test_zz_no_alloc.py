"""mth_oil4_gemv_noalloc (include/mythos_oil.h): the OIL4 GEMV whose batched
path keeps its K-slice partial sums in a fixed per-GPU device array instead
of the allocated workspace.

Its results must be those of mth_oil4_gemv (the same kernels, so bit for bit)
and the oracle's to the OIL4 bar (1e-5 of sum|w*x|), on consecutive calls of
decreasing size (the array keeps the previous call's contents), including
inside a captured graph replayed with other work in between; shapes whose
partial sums do not fit are rejected.
"""
import numpy as np
import pytest

import synth
from conftest import fp32_close
from test_gpu_gemv import empty, to_dev

pytestmark = pytest.mark.gpu


def run_both(mth, oracle, dev, M, K, batch, block, config):
    import torch
    print(f"oil4_gemv_noalloc M={M} K={K} batch={batch} block={block}", flush=True)
    packed, cbs, x = synth.oil4(M, K, batch, block, config=config)
    p, c, xd = to_dev(packed, dev), to_dev(cbs, dev), to_dev(x, dev)
    y_na = empty(batch * M, torch.float32, dev)
    y_ws = empty(batch * M, torch.float32, dev)
    mth.oil4_gemv_noalloc(p, c, block, xd, y_na, M, K, batch)
    mth.oil4_gemv(p, c, block, xd, y_ws, M, K, batch)
    torch.cuda.synchronize()
    got, want = y_na.cpu().numpy(), y_ws.cpu().numpy()
    assert np.array_equal(got, want), f"noalloc differs from mth_oil4_gemv at {np.flatnonzero(got != want)[:8]}"
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
    W = synth.dequant_oil4(packed, cbs, M, K, block).astype(np.float64)
    absw = (np.abs(W) @ np.abs(x.astype(np.float64)).T).T
    fp32_close(got.reshape(batch, M), ref, absw, 1e-5, "oil4_gemv_noalloc")


def test_noalloc_matches_oil4_gemv_on_consecutive_calls(mth, oracle, dev):
    run_both(mth, oracle, dev, 11008, 4096, 16, 128, 81)   # 4 K slices: 2.8 MB of partial sums
    run_both(mth, oracle, dev, 1000, 2048, 5, 128, 82)     # smaller, over the first call's contents
    run_both(mth, oracle, dev, 300, 4096, 1, 128, 83)      # batch 1: no scratch


def test_noalloc_rejects_oversized_partials(mth, dev):
    import torch
    M, K, batch = 40000, 4096, 2                            # 4 x 16 x 40000 x 4 B = 10.2 MB > 8 MiB
    p = torch.zeros(M * K // 2, dtype=torch.uint8, device=dev)
    c = torch.zeros(M * (K // 128) * 16, dtype=torch.int16, device=dev)
    x = torch.zeros(batch * K, dtype=torch.float32, device=dev)
    y = torch.zeros(batch * M, dtype=torch.float32, device=dev)
    with pytest.raises(mth.MythosError) as e:
        mth.oil4_gemv_noalloc(p, c, 128, x, y, M, K, batch)
    assert e.value.code == mth.MTH_EINVAL and "scratch" in str(e.value)


def test_noalloc_inside_graph_capture(mth, oracle, dev):
    """Captured on a fresh stream with no workspace reserved; every replay is
    checked, with an eager call of another shape on the same GPU in between."""
    import torch
    M, K, batch, block = 2048, 4096, 8, 128
    packed, cbs, x = synth.oil4(M, K, batch, block, config=84)
    p, c, xd = to_dev(packed, dev), to_dev(cbs, dev), to_dev(x, dev)
    y = empty(batch * M, torch.float32, dev)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        mth.oil4_gemv_noalloc(p, c, block, xd, y, M, K, batch)
    torch.cuda.synchronize()
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, block, threads=8)
    W = synth.dequant_oil4(packed, cbs, M, K, block).astype(np.float64)
    absw = (np.abs(W) @ np.abs(x.astype(np.float64)).T).T
    for rep in range(3):
        print(f"oil4_gemv_noalloc graph replay {rep}", flush=True)
        run_both(mth, oracle, dev, 700, 2048, 3, 128, 85 + rep)
        y.fill_(float("nan"))
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        fp32_close(y.cpu().numpy().reshape(batch, M), ref, absw, 1e-5, f"graph replay {rep}")
