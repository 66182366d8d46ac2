#!/usr/bin/env python3
"""bench.py — MI355X throughput of the quantized GEMV/GEMM hot path.

One "step" is one launch of the hot-path kernel over one batch of synthetic
input.  The headline workload is BASELINE config 2 (OIL4 GEMV, W 11008x4096,
per-128-weight FP16 codebooks, batch 1); the other configs are reported in
"extra", config 5 (the 32-layer decoder, greedy, batch 1 and 16) as tokens
per second.  Method, per workload:
  * inputs are generated once on the host (seeded) and resident in HBM before
    timing; the weight operand is replicated into >= 1 GiB of distinct copies
    and consecutive steps rotate over them, so every step streams its weights
    from HBM rather than the 256 MB MALL;
  * the launches of one rotation are captured in a HIP graph (the K mod
    copies launches after it in a second one) and replayed back to back; at
    least W warm-up steps, then exactly K timed steps bracketed by device
    synchronisation, timed with HIP events on the launch stream;
  * value = algorithmic bytes per launch / average launch time.
cpu_baseline: the CPU restatement of the reference kernel (oracle, "port"),
on the host's cores (up to 16 OpenMP threads; the one-thread figure in
extra), timed on a bounded sample of the same workload on this host.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mythos.cpp_amd"))

METRIC = "HBM GB/s (% peak) for OIL8/OIL4/I2_S GEMV 4096^2 b=1; 32-layer decode tok/s"
HBM_PEAK_GBS = 8000.0
F16_PEAK_TFLOPS = 2500.0
I8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 1 << 30


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def dev_copy(a: np.ndarray, dev):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).to(dev)


def replicate(t, nbytes_each):
    """>= ROTATE_BYTES of distinct copies of device tensor t (list)."""
    n = max(2, -(-ROTATE_BYTES // nbytes_each))
    return [t.clone() for _ in range(n)]


def time_graph(launch, n_copies, steps, warmup):
    """launch(i) enqueues step i (rotating copy i % n_copies) on the current
    stream.  Captures one rotation in a graph (and the steps % n_copies
    launches that follow it in a second one), replays at least `warmup`
    untimed launches, then times exactly `steps` launches: steps // n_copies
    replays of the rotation and one of the remainder.  Returns (avg seconds
    per step, steps timed)."""
    import torch
    steps = max(1, int(steps))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for i in range(n_copies):  # eager pass: first-touch, JIT-free check
            launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(n_copies):
            launch(i)
    full, rem = divmod(steps, n_copies)
    gr = None
    if rem:
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            for i in range(rem):
                launch(i)
    torch.cuda.synchronize()
    # warm-up: every graph the timed region replays is replayed first, and
    # the timed replays are queued behind the last warm-up replay (no
    # synchronisation in between), so the timed launches start on a busy
    # queue as in steady state
    reps_w = max(1, -(-warmup // n_copies))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        for _ in range(reps_w):
            g.replay()
        if gr is not None:
            gr.replay()
        e0.record(s)
        for _ in range(full):
            g.replay()
        if gr is not None:
            gr.replay()
        e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    return ms / 1e3 / steps, steps


def bench_oil4_gemv(mth, dev, M, K, batch, steps, warmup, block=128):
    import synth
    import torch
    packed, cbs, x = synth.oil4(M, K, batch, block)
    p_d, c_d = dev_copy(packed, dev), dev_copy(cbs, dev)
    x_d = dev_copy(x, dev)
    y_d = torch.empty(batch * M, dtype=torch.float32, device=dev)
    wbytes = packed.nbytes + cbs.nbytes
    ps, cs = replicate(p_d, wbytes), None
    cs = [c_d.clone() for _ in ps]
    sec, n = time_graph(lambda i: mth.oil4_gemv(ps[i], cs[i], block, x_d, y_d, M, K, batch), len(ps), steps, warmup)
    alg = packed.nbytes + cbs.nbytes + x.nbytes + 4 * M * batch
    return dict(sec=sec, steps=n, bytes=alg, copies=len(ps)), (packed, cbs, x)


def bench_oil8_gemv(mth, dev, M, K, batch, steps, warmup):
    import synth
    import torch
    idx, cb, x = synth.oil8(M, K, batch)
    i_d, cb_d, x_d = dev_copy(idx, dev), dev_copy(cb, dev), dev_copy(x, dev)
    y_d = torch.empty(batch * M, dtype=torch.float32, device=dev)
    ids = replicate(i_d, idx.nbytes)
    sec, n = time_graph(lambda i: mth.oil8_gemv(ids[i], cb_d, x_d, y_d, M, K, batch), len(ids), steps, warmup)
    alg = idx.nbytes + cb.nbytes + x.nbytes + 4 * M * batch
    return dict(sec=sec, steps=n, bytes=alg, copies=len(ids)), (idx, cb, x)


def bench_i2s_gemv(mth, dev, M, K, batch, steps, warmup):
    import synth
    import torch
    packed, w_scale, x = synth.ternary(M, K, batch)
    p_d, x_d = dev_copy(packed, dev), dev_copy(x, dev)
    y_d = torch.empty(batch * M, dtype=torch.float32, device=dev)
    ps = replicate(p_d, packed.nbytes)
    sec, n = time_graph(lambda i: mth.i2s_gemv_f32(ps[i], float(w_scale), x_d, y_d, M, K, batch), len(ps),
                        steps, warmup)
    alg = packed.nbytes + 4 + x.nbytes + 4 * M * batch
    return dict(sec=sec, steps=n, bytes=alg, copies=len(ps)), (packed, w_scale, x)


def bench_i2s_gemv_i8(mth, dev, M, K, batch, steps, warmup):
    """I2_S GEMV on int8 activations (the decoder's down projection)."""
    import synth
    import torch
    packed, w_scale, x = synth.ternary(M, K, batch)
    q = np.random.default_rng(7).integers(-127, 128, (batch, K), dtype=np.int8)
    inv = np.full(batch, 0.01, np.float32)
    p_d, q_d, inv_d = dev_copy(packed, dev), dev_copy(q, dev), dev_copy(inv, dev)
    y_d = torch.empty(batch * M, dtype=torch.float32, device=dev)
    ps = replicate(p_d, packed.nbytes)
    sec, n = time_graph(lambda i: mth.i2s_gemv(ps[i], float(w_scale), q_d, inv_d, y_d, M, K, batch), len(ps), steps,
                        warmup)
    alg = packed.nbytes + 4 + q.nbytes + inv.nbytes + 4 * M * batch
    return dict(sec=sec, steps=n, bytes=alg, copies=len(ps))


def stream_floor(dev, nbytes, steps, warmup):
    """The measured streaming floor for one launch that reads `nbytes` once:
    the fastest of a plain 16-byte streaming-read kernel
    (csrc/stream_probe.hip) over a few grid shapes, rotated over >= 1 GiB
    of copies and timed like the GEMVs.  Returns (seconds per launch, grid,
    unroll)."""
    import ctypes as C
    import torch
    lib = C.CDLL(os.path.join(ROOT, "mythos.cpp_amd", "libmythos_probe.so"))
    lib.mth_probe_stream_read.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    lib.mth_probe_stream_read.restype = C.c_int
    nb = -(-nbytes // 4096) * 4096
    n = max(2, -(-ROTATE_BYTES // nb))
    buf = torch.ones(n * nb, dtype=torch.uint8, device=dev)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    base, optr = buf.data_ptr(), out.data_ptr()
    best = None
    for grid in (512, 1024, 2048, 4096):
        for unroll in (1, 4):
            def launch(i, grid=grid, unroll=unroll):
                rc = lib.mth_probe_stream_read(base + i * nb, nbytes, grid, unroll, optr,
                                               torch.cuda.current_stream().cuda_stream)
                if rc != 0:
                    raise RuntimeError(f"stream probe failed ({rc})")
            sec, _ = time_graph(launch, n, steps, warmup)
            if best is None or sec < best[0]:
                best = (sec, grid, unroll)
    del buf
    torch.cuda.empty_cache()
    return best


def cpu_time(fn, budget_s):
    """Median seconds of fn() over repetitions filling ~budget_s (3 warm-ups
    and at least 10 timed calls, as bench/bench_oil_quant.cpp:23-32 of the
    reference times its kernels)."""
    for _ in range(3):
        fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < 10 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts)


def bench_prefill(mth, dev, M, N, K, steps, warmup, block=128):
    import synth
    import torch
    a, packed, cbs = synth.prefill(M, N, K, block)
    a_d = dev_copy(a, dev).view(torch.bfloat16)
    p_d, c_d = dev_copy(packed, dev), dev_copy(cbs, dev)
    c_out = torch.empty(M * N, dtype=torch.bfloat16, device=dev)
    n_cp = 4
    ps = [p_d.clone() for _ in range(n_cp)]
    cs = [c_d.clone() for _ in range(n_cp)]
    sec, n = time_graph(lambda i: mth.oil4_gemm_prefill(a_d, ps[i], cs[i], block, c_out, M, N, K), n_cp,
                        max(8, steps // 100), max(2, warmup // 100))
    flop = 2.0 * M * N * K
    return dict(sec=sec, steps=n, flop=flop, copies=n_cp)


def bench_tl2_gemm(mth, dev, M, N, K, steps, warmup):
    """tl2_gemm with the reference's per-(m,n) weight rows (src/kernel_tl.cpp:109-168):
    M*N rows of ceil(K/4) code bytes, each used once (a streaming kernel)."""
    import torch
    bpr = (2 * K + 7) // 8
    w = np.random.default_rng(9).integers(0, 256, M * N * bpr, dtype=np.uint8)
    a = np.random.default_rng(10).normal(0, 1, N * K).astype(np.float32)
    w_d, a_d = dev_copy(w, dev), dev_copy(a, dev)
    o = torch.empty(M * N, dtype=torch.float32, device=dev)
    ws = replicate(w_d, w.nbytes)
    sec, n = time_graph(lambda i: mth.tl2_gemm(ws[i], a_d, o, M, N, K), len(ws), steps, warmup)
    return dict(sec=sec, steps=n, bytes=w.nbytes + a.nbytes + 4 * M * N, copies=len(ws))


def bench_ternary_gemm(mth, dev, M, N, K, steps, warmup):
    """Ternary prefill GEMM (i2s_gemm_vnni, int8 MFMA): M weight rows x N
    tokens x K; weights rotated over 4 copies (the 5.6 MB of activations and
    11 MB of weights fit the 256 MB MALL either way: this is compute-bound)."""
    import torch
    import synth
    w = synth.stream(6).ternary(M, K)
    a = np.random.default_rng(6).integers(-127, 128, (N, K), dtype=np.int8)
    a_d = dev_copy(a, dev)
    o = torch.empty(M * N, dtype=torch.float32, device=dev)
    n_cp = 4
    ws = [dev_copy(w, dev) for _ in range(n_cp)]
    sec, n = time_graph(lambda i: mth.i2s_gemm_vnni(ws[i], a_d, o, M, N, K), n_cp, max(8, steps // 100),
                        max(2, warmup // 100))
    return dict(sec=sec, steps=n, ops=2.0 * M * N * K, copies=n_cp)


def bench_decode(dev, batches=(1, 16), kv_dtype="bf16"):
    """Config 5: the 32-layer mixed-format decoder, greedy, 64-token random
    prompts, 128 generated tokens per sequence, bf16 KV cache.  The prompt
    runs as one forward pass (mth_decoder_prefill: all B x 64 prompt rows
    through the layer stack, yielding the first token); the remaining 127
    tokens take 127 steps, timed with HIP events on the launch stream.  Each
    step is one replay of the captured step graph.  Roofline bytes per step: every weight byte once plus the KV cache
    rows the attention reads (positions 0 .. pos-1 of every layer, sequence
    and kv head, K and V) and the row it appends, averaged over the timed
    steps."""
    import torch
    import decoder
    import synth
    cfg = synth.decoder_config()
    t0 = time.time()
    model = synth.decoder_model(cfg, config=5)
    log(f"decode: weights generated in {time.time() - t0:.1f} s")
    dec = decoder.Decoder(cfg, max_batch=max(batches), kv_dtype=kv_dtype)
    dec.load(model)
    H, F, V, L = cfg["hidden"], cfg["ffn"], cfg["vocab"], cfg["layers"]
    layer_bytes = sum(model["layers"][0][k].nbytes for k in ("attn_norm", "ffn_norm", "wq", "cbq", "wk", "cbk", "wv",
                                                             "cbv", "wo", "cbo", "wgate_up", "cbgate_up", "wdown"))
    weight_bytes = L * layer_bytes + model["lm_idx"].nbytes + model["lm_cb"].nbytes + model["final_norm"].nbytes
    del model
    P, G = synth.PROMPT_LEN5, synth.GEN_TOKENS5
    out = {}
    s = torch.cuda.current_stream()
    for B in batches:
        prompts = synth.decoder_prompts(cfg, B, P)
        dec.start(prompts)                 # warm-up: graph capture + one full run
        dec.prefill()
        dec.step(G - 1)
        torch.cuda.synchronize()
        dec.start(prompts)
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record(s)
        dec.prefill()
        e[1].record(s)
        dec.step(G - 1)
        e[2].record(s)
        torch.cuda.synchronize()
        t_prompt, t_dec = e[0].elapsed_time(e[1]) / 1e3, e[1].elapsed_time(e[2]) / 1e3
        toks = dec.tokens()
        step_ms = t_dec / (G - 1) * 1e3
        # timed steps run at positions P .. P+G-2: step at pos reads pos cache rows and appends one
        row = 2 * L * B * cfg["kv_heads"] * cfg["head_dim"] * (2 if kv_dtype == "bf16" else 4)
        kv_bytes = row * (sum(range(P, P + G - 1)) + (G - 1)) / (G - 1)
        gbs = weight_bytes / (t_dec / (G - 1)) / 1e9
        tot = (weight_bytes + kv_bytes) / (t_dec / (G - 1)) / 1e9
        out[f"decode_config5_b{B}"] = dict(
            tok_per_s=B * (G - 1) / t_dec, ms_per_step=step_ms, prompt_ms=t_prompt * 1e3,
            end_to_end_tok_per_s=B * G / (t_prompt + t_dec), weight_bytes_per_step=weight_bytes,
            kv_bytes_per_step=kv_bytes, kv_dtype=kv_dtype, weight_GBps=gbs, GBps=tot, frac=tot / HBM_PEAK_GBS,
            weight_frac=gbs / HBM_PEAK_GBS, launches_per_step=dec.launches_per_step,
            generated=int(toks.shape[1] - P), first_tokens=[int(t) for t in toks[0, P:P + 8]])
        log(f"decode b={B}: {B * (G - 1) / t_dec:.1f} tok/s, {step_ms:.3f} ms/step, weights+KV {tot:.0f} GB/s "
            f"({tot / HBM_PEAK_GBS:.1%}), {dec.launches_per_step} launches/step")
    dec.close()
    return out


def cpu_baseline_oil4(packed, cbs, x, M, K, block, budget_s, threads=1):
    """Oracle (CPU restatement of src/kernel_oil4.cpp:31-54 with per-block
    codebooks; OpenMP over rows), whole GEMVs repeated for ~budget_s
    seconds on `threads` host threads."""
    sys.path.insert(0, ROOT)
    from oracle import Oracle
    o = Oracle()
    xb = np.ascontiguousarray(x[:1])
    pr = np.ascontiguousarray(packed.ravel())
    o.oil4_gemv_blocked(pr, cbs, xb, M, K, 1, block, threads=threads)  # warm-up
    t0, n = time.perf_counter(), 0
    while True:
        o.oil4_gemv_blocked(pr, cbs, xb, M, K, 1, block, threads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return el / n, n


def cpu_threads():
    """Host threads for the all-cores baseline: the cores this process may
    use, at most 16 (one GPU's share of the host on the measurement box)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_model():
    """The host CPU's model name (lscpu's), for the CPU baselines."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_reference_oil8(idx, cb, x, M, K, budget_s):
    """The reference's own oil8_gemm (AVX2 build, oracle/_ref) when present."""
    sys.path.insert(0, ROOT)
    try:
        from oracle import Reference
        r = Reference("avx2")
    except (OSError, FileNotFoundError):
        return None
    xb = np.ascontiguousarray(x[0])
    ib = np.ascontiguousarray(idx.ravel())
    r.oil8_gemm(ib, cb, xb, M, 1, K)
    t0, n = time.perf_counter(), 0
    while True:
        r.oil8_gemm(ib, cb, xb, M, 1, K)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return el / n, n


def load_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 PMC summary
    (profiles/<name>.pmc.json, written from FETCH_SIZE/WRITE_SIZE runs scaled
    by a copy-kernel calibration), or None."""
    p = os.path.join(ROOT, "profiles", f"{name}.pmc.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        d = json.load(f)
    return d.get("traffic_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3200)
    ap.add_argument("--warmup", type=int, default=320)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--only", default="", help="comma list: oil4,oil4b16,oil8,oil8b16,i2s,i2sb16,tl2,floor,prefill,"
                                               "ternary_gemm,decode (default all); floor: each GEMV's streaming floor")
    ap.add_argument("--decode-batches", default="1,16", help="comma list of decode batch sizes (config 5)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the path shards by weight rows with no exchange, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch
    import mythos_oil as mth
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    only = set(filter(None, args.only.split(",")))
    want = (lambda k: not only or k in only)

    extra = {}
    head = None
    floors = {}

    def floor_of(name, nbytes):
        """Streaming floor for nbytes, measured once per size (want("floor"))."""
        if not want("floor"):
            return None
        if nbytes not in floors:
            sec, grid, unroll = stream_floor(dev, nbytes, args.steps, args.warmup)
            floors[nbytes] = dict(us=sec * 1e6, GBps=nbytes / sec / 1e9, frac=nbytes / sec / 1e9 / HBM_PEAK_GBS,
                                  grid=grid, unroll=unroll)
            log(f"stream floor {nbytes} B: {sec*1e6:.2f} us ({nbytes / sec / 1e9:.0f} GB/s, grid {grid} x{unroll})")
        extra.setdefault("stream_floor", {})[name] = dict(bytes=nbytes, **floors[nbytes])
        return floors[nbytes]["us"]

    def gemv_entry(name, r):
        gbs = r["bytes"] / r["sec"] / 1e9
        e = dict(us=r["sec"] * 1e6, GBps=gbs, frac=gbs / HBM_PEAK_GBS, bytes=r["bytes"], copies=r["copies"],
                 traffic=load_traffic(name))
        fl = floor_of(name, r["bytes"])
        if fl is not None:
            e.update(floor_us=fl, frac_of_floor=fl / e["us"])
        return e

    if want("oil4"):
        M, K = 11008, 4096
        r, data = bench_oil4_gemv(mth, dev, M, K, 1, args.steps, args.warmup)
        gbs = r["bytes"] / r["sec"] / 1e9
        head = dict(r=r, gbs=gbs, data=data, M=M, K=K)
        log(f"oil4 b=1: {r['sec']*1e6:.2f} us/launch, {gbs:.0f} GB/s ({gbs/HBM_PEAK_GBS:.1%})")
        head["floor_us"] = floor_of("oil4_gemv_11008x4096_b1", r["bytes"])
    if want("oil4b16"):
        r, _ = bench_oil4_gemv(mth, dev, 11008, 4096, 16, args.steps, args.warmup)
        extra["oil4_gemv_11008x4096_b16"] = e = gemv_entry("oil4_gemv_11008x4096_b16", r)
        log(f"oil4 b=16: {e['us']:.2f} us/launch, {e['GBps']:.0f} GB/s")
    oil8_data = i2s_data = None
    if want("oil8"):
        r, oil8_data = bench_oil8_gemv(mth, dev, 4096, 4096, 1, args.steps, args.warmup)
        extra["oil8_gemv_4096x4096_b1"] = e = gemv_entry("oil8_gemv_4096x4096_b1", r)
        log(f"oil8 b=1: {e['us']:.2f} us/launch, {e['GBps']:.0f} GB/s")
    if want("oil8b16"):
        r, _ = bench_oil8_gemv(mth, dev, 4096, 4096, 16, args.steps, args.warmup)
        extra["oil8_gemv_4096x4096_b16"] = e = gemv_entry("oil8_gemv_4096x4096_b16", r)
        log(f"oil8 b=16: {e['us']:.2f} us/launch, {e['GBps']:.0f} GB/s")
    if want("i2s"):
        r, i2s_data = bench_i2s_gemv(mth, dev, 4096, 4096, 1, args.steps, args.warmup)
        extra["i2s_gemv_4096x4096_b1"] = e = gemv_entry("i2s_gemv_4096x4096_b1", r)
        log(f"i2s b=1: {e['us']:.2f} us/launch, {e['GBps']:.0f} GB/s")
    if want("i2sb16"):
        r = bench_i2s_gemv_i8(mth, dev, 4096, 11008, 16, args.steps, args.warmup)
        extra["i2s_gemv_4096x11008_b16_int8"] = e = gemv_entry("i2s_gemv_4096x11008_b16_int8", r)
        log(f"i2s b=16 (int8 acts, 4096x11008): {e['us']:.2f} us/launch, {e['GBps']:.0f} GB/s")
    if want("tl2"):
        r = bench_tl2_gemm(mth, dev, 4096, 4, 4095, args.steps, args.warmup)
        extra["tl2_gemm_4096x4x4095"] = e = gemv_entry("tl2_gemm_4096x4x4095", r)
        log(f"tl2 gemm (per-(m,n) rows, 4096x4x4095): {e['us']:.2f} us/launch, {e['GBps']:.0f} GB/s")
    if want("prefill"):
        r = bench_prefill(mth, dev, 512, 14336, 4096, args.steps, args.warmup)
        tf = r["flop"] / r["sec"] / 1e12
        extra["oil4_prefill_gemm_512x14336x4096"] = dict(us=r["sec"] * 1e6, TFLOPs=tf, frac=tf / F16_PEAK_TFLOPS,
                                                         steps=r["steps"])
        log(f"prefill: {r['sec']*1e6:.1f} us/launch, {tf:.0f} TFLOP/s ({tf/F16_PEAK_TFLOPS:.1%})")

    if want("ternary_gemm"):
        r = bench_ternary_gemm(mth, dev, 4096, 512, 11008, args.steps, args.warmup)
        tops = r["ops"] / r["sec"] / 1e12
        extra["i2s_gemm_vnni_4096x512x11008"] = dict(us=r["sec"] * 1e6, TOPs=tops, frac=tops / I8_PEAK_TOPS,
                                                     steps=r["steps"])
        log(f"ternary gemm: {r['sec']*1e6:.1f} us/launch, {tops:.0f} TOP/s ({tops/I8_PEAK_TOPS:.1%} of int8 MFMA)")

    if want("decode"):
        extra.update(bench_decode(dev, tuple(int(b) for b in args.decode_batches.split(","))))

    cpu = None
    if head is not None:
        packed, cbs, x = head["data"]
        nt = cpu_threads()
        sec_cpu, n_cpu = cpu_baseline_oil4(packed, cbs, x, head["M"], head["K"], 128, args.cpu_seconds / 2, nt)
        cpu = dict(value=head["r"]["bytes"] / sec_cpu / 1e9, unit="GB/s", cores=nt, kind="port",
                   sample=f"{n_cpu} whole OIL4 GEMVs 11008x4096 b=1 (oracle, {nt} OpenMP threads), "
                          f"{sec_cpu*1e3:.2f} ms each")
        log(f"cpu port, {nt} threads: {sec_cpu*1e3:.2f} ms/GEMV")
        sec1, n1 = cpu_baseline_oil4(packed, cbs, x, head["M"], head["K"], 128, args.cpu_seconds / 2, 1)
        extra["cpu_baseline_1thread"] = dict(value=head["r"]["bytes"] / sec1 / 1e9, unit="GB/s", cores=1,
                                             kind="port", sample=f"{n1} whole OIL4 GEMVs 11008x4096 b=1 "
                                                                 f"(oracle, 1 thread), {sec1*1e3:.1f} ms each")
        log(f"cpu port, 1 thread: {sec1*1e3:.1f} ms/GEMV")
    if oil8_data is not None:
        idx, cb, x = oil8_data
        ref = cpu_reference_oil8(idx, cb, x, 4096, 4096, min(4.0, args.cpu_seconds / 3))
        if ref:
            extra["cpu_reference_oil8_gemm_avx2"] = dict(ms=ref[0] * 1e3, GBps=16811008 / ref[0] / 1e9, calls=ref[1],
                                                         cores=1)
    # configs 1 and 3 on the host: the oracle's OIL8 GEMV (AVX2 lane order
    # of src/kernel_oil8.cpp:30-60) and its I2_S GEMV with the per-token
    # quantisation (src/kernel_i2s.cpp:32-40, src/int8_quant.cpp:24-31), one
    # thread and all cores, median of >= 10 calls
    if oil8_data is not None or i2s_data is not None:
        sys.path.insert(0, ROOT)
        from oracle import Oracle
        o = Oracle()
        nt = cpu_threads()
        budget = min(3.0, args.cpu_seconds / 4)
        jobs = []
        if oil8_data is not None:
            idx, cb, x = oil8_data
            ib, xb = np.ascontiguousarray(idx.ravel()), np.ascontiguousarray(x[:1])
            jobs.append(("cpu_oil8_gemv_4096x4096_b1", 16811008,
                         lambda th: o.oil8_gemv(ib, cb, xb, 4096, 4096, 1, threads=th)))
        if i2s_data is not None:
            packed, w_scale, x = i2s_data
            pb, xb3 = np.ascontiguousarray(packed.ravel()), np.ascontiguousarray(x[:1])
            jobs.append(("cpu_i2s_gemv_4096x4096_b1", 4227076,
                         lambda th: o.i2s_gemv_f32(pb, float(w_scale), xb3, 4096, 4096, 1, threads=th)))
        for name, nbytes, fn in jobs:
            e = {}
            for th in (1, nt):
                sec, n = cpu_time(lambda: fn(th), budget)
                e[f"threads_{th}"] = dict(ms=sec * 1e3, GBps=nbytes / sec / 1e9, calls=n)
                log(f"{name}, {th} thread(s): {sec*1e3:.2f} ms")
            e.update(kind="port", cores_all=nt, cpu=cpu_model())
            extra[name] = e

    if head is None:
        print(json.dumps(dict(metric=METRIC, extra=extra)))
        return
    r = head["r"]
    gbs = head["gbs"]
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": args.warmup,
        "ms_per_step": r["sec"] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (MYTHOS.cpp RNG xoroshiro128+, seed 0x5EED0000+config; weights resident in HBM, "
                "rotated over >=1 GiB of copies)",
        "config": {"workload": "OIL4 GEMV W 11008x4096, per-128-weight FP16 codebooks, batch 1 (BASELINE config 2)",
                   "M": head["M"], "K": head["K"], "batch": 1, "cb_block": 128,
                   "weight_copies": r["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic("oil4_gemv_11008x4096_b1"),
                     "floor_us": head.get("floor_us"),
                     "frac_of_floor": (round(head["floor_us"] / (r["sec"] * 1e6), 4) if head.get("floor_us")
                                       else None)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
