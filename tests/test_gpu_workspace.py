"""The C ABI's per-(device, stream) workspace (include/mythos_oil.h,
"Workspace") under HIP graph capture.

A graph captured from a batched GEMV keeps the workspace address of its
capture; a later, larger call on the same stream grows the workspace.  The
old block is retired, not freed, so replays of the graph stay correct.  A call
that would have to grow the workspace while its stream is capturing fails with
MTH_EUNSUPPORTED instead of allocating; mth_workspace_reserve sizes it ahead.
Every replay is checked against the oracle, with eager work in between.
"""
import numpy as np
import pytest

import synth
from conftest import fp32_close
from test_gpu_gemv import empty, to_dev

pytestmark = pytest.mark.gpu


def oil4_case(M, K, batch, dev, config):
    packed, cbs, x = synth.oil4(M, K, batch, 128, config=config)
    return (packed, cbs, x), (to_dev(packed, dev), to_dev(cbs, dev), to_dev(x, dev))


def check(y, host, M, K, batch, oracle, what):
    packed, cbs, x = host
    ref = oracle.oil4_gemv_blocked(packed.ravel(), cbs, x, M, K, batch, 128, threads=8)
    W = synth.dequant_oil4(packed, cbs, M, K, 128)
    absw = (np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64)).T).T
    fp32_close(y.cpu().numpy().reshape(batch, M), ref, absw, 1e-5, what)


def test_graph_replay_after_workspace_growth(oracle, mth, dev):
    import torch
    s = torch.cuda.Stream()
    M1, K1, B1 = 1000, 2048, 4          # 2 K slices: 128 KB of partial sums
    M2, K2, B2 = 11008, 4096, 16        # 4 K slices: 2.8 MB, grows the workspace
    h1, (p1, c1, x1) = oil4_case(M1, K1, B1, dev, 71)
    h2, (p2, c2, x2) = oil4_case(M2, K2, B2, dev, 72)
    y1 = empty(B1 * M1, torch.float32, dev)
    y2 = empty(B2 * M2, torch.float32, dev)
    with torch.cuda.stream(s):
        mth.oil4_gemv(p1, c1, 128, x1, y1, M1, K1, B1)     # sizes the workspace for the small call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        mth.oil4_gemv(p1, c1, 128, x1, y1, M1, K1, B1)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"workspace graph replay {rep}", flush=True)
        with torch.cuda.stream(s):
            mth.oil4_gemv(p2, c2, 128, x2, y2, M2, K2, B2)  # grows the workspace on the first pass
        torch.cuda.synchronize()
        check(y2, h2, M2, K2, B2, oracle, f"eager large call {rep}")
        y1.fill_(float("nan"))
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        check(y1, h1, M1, K1, B1, oracle, f"graph replay {rep}")


def test_growth_under_capture_is_refused_then_reserve(oracle, mth, dev):
    import torch
    M, K, B = 2048, 4096, 8
    h, (p, c, x) = oil4_case(M, K, B, dev, 73)
    y = empty(B * M, torch.float32, dev)
    s = torch.cuda.Stream()                                # a fresh stream: no workspace yet
    g = torch.cuda.CUDAGraph()
    with pytest.raises(mth.MythosError) as e:
        with torch.cuda.graph(g, stream=s):
            mth.oil4_gemv(p, c, 128, x, y, M, K, B)
    assert e.value.code == mth.MTH_EUNSUPPORTED and "mth_workspace_reserve" in str(e.value)
    torch.cuda.synchronize()
    s2 = torch.cuda.Stream()
    mth.workspace_reserve(4 * 16 * M * 4, stream=s2)       # 4 K slices x 16 tokens x M rows
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s2):
        mth.oil4_gemv(p, c, 128, x, y, M, K, B)
    torch.cuda.synchronize()
    for rep in range(2):
        y.fill_(float("nan"))
        with torch.cuda.stream(s2):
            g2.replay()
        torch.cuda.synchronize()
        check(y, h, M, K, B, oracle, f"reserved graph replay {rep}")
