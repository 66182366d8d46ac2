"""Write the golden fixtures in tests/golden/*.npz from the reference's own
kernels, compiled from the reference sources by oracle/Makefile into
oracle/_ref/ (`make -C oracle ref`).  Run in a container that holds the
reference tree:

    python tests/golden/make_golden.py

Each fixture holds the inputs of a case and the reference's outputs for them;
tests/test_golden.py replays the inputs through the oracle (and, on the GPU,
through libmythos_oil.so) and compares.  Inputs come from numpy's seeded
generator, so rerunning the script reproduces the files bit for bit.

Library variants used (oracle/Makefile):
  avx2    the reference's Release build flags (-mavx2 -mfma, OIL_AVX2 macro
          undefined): oil8_gemm_avx2, oil4_gemm_avx2, and math.cpp with GCC's
          FMA contraction
  scalar  no AVX2 flags: oil8_gemm_scalar, oil4_gemm_scalar, math.cpp as
          written (no contraction)
  vnni    -DOIL_AVX2: the i2s_gemm_vnni body
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import Reference, build  # noqa: E402


def save(name: str, **arrays) -> None:
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **arrays)
    print(f"{name}.npz  {os.path.getsize(path)} bytes")


def pack_nibbles(v: np.ndarray) -> np.ndarray:
    """element k -> low nibble of byte k/2 for even k, high for odd k."""
    v = v.reshape(-1).astype(np.uint8)
    if v.size % 2:
        v = np.concatenate([v, np.zeros(1, np.uint8)])
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


def pack_codes(c: np.ndarray) -> np.ndarray:
    """2-bit codes, element 4i+j in bits 2j..2j+1 of byte i."""
    c = c.reshape(-1).astype(np.uint8)
    pad = (-c.size) % 4
    c = np.concatenate([c, np.zeros(pad, np.uint8)]).reshape(-1, 4)
    return (c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)).astype(np.uint8)


def main() -> None:
    build(with_ref=True)
    avx2, scalar, vnni = Reference("avx2"), Reference("scalar"), Reference("vnni")
    rng = np.random.default_rng(20260601)

    # ---- RNG (src/random.cpp) -------------------------------------------
    seeds = np.array([0, 1, 42, 77, 0x5EED0001, 0x5EED0003, 2**63 + 5], np.uint64)
    n = 256
    save("rng", seeds=seeds,
         u64=np.stack([avx2.rng_u64(int(s), n) for s in seeds]),
         uniform=np.stack([avx2.rng_uniform(int(s), n) for s in seeds]),
         normal=np.stack([avx2.rng_normal(int(s), n) for s in seeds]),
         uint_0_2=np.stack([avx2.rng_uniform_int(int(s), 0, 2, n) for s in seeds]),
         uint_m5_9=np.stack([avx2.rng_uniform_int(int(s), -5, 9, n) for s in seeds]))

    # ---- FP16 conversions (src/codebook.cpp:16-64) -----------------------
    allh = np.arange(65536, dtype=np.uint32)
    h2f = np.array([avx2.half_to_float(int(h)) for h in allh], np.float32)
    # all subnormal / zero / inf / NaN patterns verbatim, a sample of normals,
    # and a SHA-256 of the whole 65536-entry table (float32 bits, little endian)
    ex = (allh >> 10) & 31
    keep = np.nonzero((ex == 0) | (ex == 31))[0]
    keep = np.union1d(keep, rng.choice(65536, 2048, replace=False))
    digest = np.frombuffer(hashlib.sha256(h2f.view(np.uint32).astype("<u4").tobytes()).digest(), np.uint8)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 65504.0, 65520.0, 65535.0,
                         1e5, -1e5, 6.103515625e-05, 6.0e-05, 5.96e-08, 2.98e-08, 1e-9, 3.0e-38,
                         1.0009765625, 1.00048828125, 0.33333334, -2.5e-3], np.float32)
    f = np.concatenate([specials, rng.standard_normal(2048).astype(np.float32) * 0.02,
                        rng.standard_normal(1024).astype(np.float32) * 1000,
                        (rng.standard_normal(1024) * 1e-5).astype(np.float32)])
    f2h = np.array([avx2.float_to_half(float(x)) for x in f], np.uint16)
    save("fp16", half_bits=keep.astype(np.uint16), half_to_float_bits=h2f[keep].view(np.uint32),
         table_sha256=digest, floats=f, float_to_half=f2h)

    # ---- OIL8 (src/kernel_oil8.cpp) -------------------------------------
    cases = {}
    for ci, (M, N, K) in enumerate([(8, 1, 256), (5, 3, 67), (3, 2, 1000), (4, 1, 7), (2, 4, 16)]):
        idx = rng.integers(0, 256, M * N * K, dtype=np.uint8)
        cb = np.sort(rng.standard_normal(256).astype(np.float32) * 0.02)
        act = rng.standard_normal(N * K).astype(np.float32)
        cases.update({f"c{ci}_shape": np.array([M, N, K]), f"c{ci}_idx": idx, f"c{ci}_cb": cb,
                      f"c{ci}_act": act,
                      f"c{ci}_avx2": avx2.oil8_gemm(idx, cb, act, M, N, K),
                      f"c{ci}_scalar": scalar.oil8_gemm(idx, cb, act, M, N, K)})
    save("oil8", ncases=np.array(5), **cases)

    # ---- OIL4 (src/kernel_oil4.cpp) -------------------------------------
    cases = {}
    for ci, (M, N, K) in enumerate([(6, 1, 128), (4, 2, 70), (3, 3, 256), (2, 1, 16), (5, 1, 34)]):
        nib = pack_nibbles(rng.integers(0, 16, M * N * K))
        cbf = rng.standard_normal(16).astype(np.float32) * 0.02
        cb16 = np.array([avx2.float_to_half(float(x)) for x in cbf], np.uint16)
        act = rng.standard_normal(N * K).astype(np.float32)
        cases.update({f"c{ci}_shape": np.array([M, N, K]), f"c{ci}_nib": nib, f"c{ci}_cb16": cb16,
                      f"c{ci}_act": act,
                      f"c{ci}_avx2": avx2.oil4_gemm(nib, cb16, act, M, N, K),
                      f"c{ci}_scalar": scalar.oil4_gemm(nib, cb16, act, M, N, K)})
    save("oil4", ncases=np.array(5), **cases)

    # ---- int8 quantization (src/int8_quant.cpp) -------------------------
    rows, cols = 6, 300
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[1] = 0.0                                            # max_abs floor 1e-10
    x[2, :6] = [127.0, 63.5, -63.5, 0.5, -0.5, 1.5]       # exact .5 ties (scale 1)
    x[2, 6:] = rng.uniform(-127, 127, cols - 6).astype(np.float32)
    x[3] *= 1e-3
    x[4, 7] = -50.0                                       # negative max
    q, s, inv = avx2.quantize_per_token(x, rows, cols)
    save("quant", x=x, q=q, scale=s, inv_scale=inv)

    # ---- I2_S (src/kernel_i2s.cpp) --------------------------------------
    avx2.i2s_init()
    vnni.i2s_init()
    cases = {}
    for ci, K in enumerate([256, 512, 64]):
        M = 5
        codes = rng.integers(0, 3, (M, K))
        packed = np.stack([pack_codes(codes[m]) for m in range(M)])
        xf = rng.standard_normal(K).astype(np.float32)
        qa, _, inva = avx2.quantize_per_token(xf, 1, K)
        ws = np.float32(0.0159577)
        y = np.array([avx2.i2s_gemv(np.ascontiguousarray(packed[m]), float(ws), qa[0], float(inva[0]), K)
                      for m in range(M)], np.float32)
        cases.update({f"c{ci}_K": np.array(K), f"c{ci}_packed": packed, f"c{ci}_x": xf,
                      f"c{ci}_act": qa[0], f"c{ci}_act_scale": inva, f"c{ci}_w_scale": np.array(ws),
                      f"c{ci}_y": y})
    save("i2s_gemv", ncases=np.array(3), **cases)

    cases = {}
    for ci, (M, N, K) in enumerate([(4, 3, 128), (3, 2, 260), (2, 5, 40)]):
        w = pack_codes(rng.integers(0, 3, M * K))
        a = rng.standard_normal(N * K).astype(np.float32)
        ai = rng.integers(-128, 128, N * K, dtype=np.int8)
        cases.update({f"c{ci}_shape": np.array([M, N, K]), f"c{ci}_w": w, f"c{ci}_a": a, f"c{ci}_ai": ai,
                      f"c{ci}_gemm": avx2.i2s_gemm(w, a, M, N, K),
                      f"c{ci}_vnni": vnni.i2s_gemm_vnni(w, ai, M, N, K)})
    save("i2s_gemm", ncases=np.array(3), **cases)

    # ---- TL1 / TL2 (src/kernel_tl.cpp) ----------------------------------
    cases = {}
    for ci, (M, N, K) in enumerate([(3, 2, 48), (2, 3, 24), (4, 4, 12)]):
        w1 = rng.integers(0, 256, M * N * K // 4, dtype=np.uint8)
        bpr = (2 * K + 7) // 8
        w2 = pack_codes(rng.integers(0, 3, M * N * bpr * 4))[: M * N * bpr]
        a = (rng.standard_normal(N * K) * 0.5).astype(np.float32)
        cases.update({f"c{ci}_shape": np.array([M, N, K]), f"c{ci}_w1": w1, f"c{ci}_w2": w2, f"c{ci}_a": a,
                      f"c{ci}_tl1": avx2.tl1_gemm(w1, a, M, N, K),
                      f"c{ci}_tl2": avx2.tl2_gemm(w2, a, M, N, K)})
    save("tl", ncases=np.array(3), **cases)

    # ---- dense math (src/math.cpp) --------------------------------------
    M, N = 7, 33
    A = rng.standard_normal((M, N)).astype(np.float32)
    xv = rng.standard_normal(N).astype(np.float32)
    y0 = rng.standard_normal(M).astype(np.float32)
    xr = rng.standard_normal((3, 64)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    xs = np.concatenate([np.linspace(-20, 20, 161), rng.standard_normal(95) * 4]).astype(np.float32)
    # scalar build: the plain C++ order; avx2 build: the same source with
    # GCC's FMA contraction under -mfma (the reference's Release flags)
    save("math", A=A, x=xv, y0=y0, gemv=scalar.gemv(0.75, A, xv, 0.5, y0, M, N),
         gemv_fma=avx2.gemv(0.75, A, xv, 0.5, y0, M, N),
         rms_x=xr, rms_g=g, rms=scalar.rms_norm(xr, g, 1e-5, 3, 64), rms_fma=avx2.rms_norm(xr, g, 1e-5, 3, 64),
         silu_x=xs, silu=scalar.silu(xs), silu_fma=avx2.silu(xs))

    # ---- .oil container (src/oil_format.cpp OILWriter / OILReader) --------
    # A small model file written by the reference's own OILWriter, holding
    # every block format the quantised path reads, and the reference's
    # OILReader::read_tensor dequantisation of each tensor.
    def normal_cb16(n):
        v = rng.standard_normal(n).astype(np.float32) * 0.02
        v = np.where(np.abs(v) < 1e-3, np.float32(1e-3), v)      # keep FP16 normals
        return np.array([avx2.float_to_half(float(x)) for x in v], np.uint16)

    blocks, tensors, inputs = [], [], {}
    # OIL8, one block (the converter's layout: tools/convert.cpp:521-533)
    r, c = 6, 40
    cb8 = np.sort(rng.standard_normal(256).astype(np.float32) * 0.05)
    i8 = rng.integers(0, 256, r * c, dtype=np.uint8)
    tensors.append(("blk.0.attn_q.weight", len(blocks), 1))
    blocks.append((3, r * c, avx2.serialize_oil8(cb8).tobytes(), i8.tobytes()))
    inputs.update(oil8_idx=i8, oil8_cb=cb8, oil8_shape=np.array([r, c]))
    # OIL8, three blocks sharing one codebook (rows 4 x 96, blocks of 128)
    i8m = rng.integers(0, 256, 4 * 96, dtype=np.uint8)
    tensors.append(("blk.0.ffn_up.weight", len(blocks), 3))
    for b in range(3):
        blocks.append((3, 128, avx2.serialize_oil8(cb8).tobytes(), i8m[b * 128:(b + 1) * 128].tobytes()))
    inputs.update(oil8m_idx=i8m, oil8m_shape=np.array([4, 96]))
    # OIL4, per-128-weight blocks, each with its own codebook (rows 3 x 256)
    r, c, B = 3, 256, 128
    v4 = rng.integers(0, 16, r * c)
    cbs4 = np.stack([normal_cb16(16) for _ in range(r * c // B)])
    tensors.append(("blk.0.ffn_down.weight", len(blocks), r * c // B))
    for b in range(r * c // B):
        blocks.append((2, B, avx2.serialize_oil4(cbs4[b]).tobytes(), pack_nibbles(v4[b * B:(b + 1) * B]).tobytes()))
    inputs.update(oil4_vals=v4.astype(np.uint8), oil4_cbs=cbs4, oil4_shape=np.array([r, c, B]))
    # OIL4, one block for the whole tensor (rows 2 x 48)
    v4s = rng.integers(0, 16, 2 * 48)
    cb4s = normal_cb16(16)
    tensors.append(("output.weight", len(blocks), 1))
    blocks.append((2, 96, avx2.serialize_oil4(cb4s).tobytes(), pack_nibbles(v4s).tobytes()))
    inputs.update(oil4s_vals=v4s.astype(np.uint8), oil4s_cb=cb4s, oil4s_shape=np.array([2, 48]))
    # TERNARY, one block: codes q+1, 4 per byte, codebook {-1, 0, +1} as FP32
    # (tools/convert.cpp:329-341)
    tq = rng.integers(0, 3, 5 * 64)
    tensors.append(("blk.1.attn_k.weight", len(blocks), 1))
    blocks.append((1, 5 * 64, np.array([-1, 0, 1], np.float32).tobytes(), pack_codes(tq).tobytes()))
    inputs.update(tern_codes=tq.astype(np.uint8), tern_shape=np.array([5, 64]))
    # FP32 block (format byte 5)
    fw = rng.standard_normal(64).astype(np.float32)
    tensors.append(("token_norm.weight", len(blocks), 1))
    blocks.append((5, 64, b"", fw.tobytes()))
    inputs.update(fp32_vals=fw)
    import tempfile
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "tiny.oil")
        avx2.oil_write(path, b'{"arch":"mythos","n_layers":2}', blocks, tensors)
        raw = np.fromfile(path, np.uint8)
        reads = {f"read_{i}": avx2.oil_read_tensor(path, t[0], 1 << 16) for i, t in enumerate(tensors)}
    save("oil_file", oil=raw, names=np.array([t[0] for t in tensors]),
         block_start=np.array([t[1] for t in tensors]), num_blocks=np.array([t[2] for t in tensors]),
         **inputs, **reads)

    # ---- Linear weights as the reference's model keeps them ----------------
    # Linear::forward (src/transformer.cpp:62-70) multiplies with scalar_gemm,
    # which reads the weight input-major: element (out n, in k) at k*out + n.
    # A file holding such weights, the reference's read_tensor of each, and
    # scalar_gemm(x, W) as Linear::forward computes it.
    out_f, in_f, nb_tok = 48, 64, 3
    xl = rng.standard_normal((nb_tok, in_f)).astype(np.float32)
    l8 = rng.integers(0, 256, in_f * out_f, dtype=np.uint8)
    l4 = rng.integers(0, 16, in_f * out_f)
    l4cb = normal_cb16(16)
    lf = (rng.standard_normal(in_f * out_f) * 0.05).astype(np.float32)
    half = in_f * out_f // 2
    lblocks = [(3, in_f * out_f, avx2.serialize_oil8(cb8).tobytes(), l8.tobytes()),
               (2, half, avx2.serialize_oil4(l4cb).tobytes(), pack_nibbles(l4[:half]).tobytes()),
               (2, half, avx2.serialize_oil4(l4cb).tobytes(), pack_nibbles(l4[half:]).tobytes()),
               (5, half, b"", lf[:half].tobytes()),                  # DenseModel::save splits FP32
               (5, half, b"", lf[half:].tobytes())]                  # tensors into blocks
    ltensors = [("layers.0.attention.q_proj.weight", 0, 1), ("layers.0.ffn.up_proj.weight", 1, 2),
                ("layers.0.attention.o_proj.weight", 3, 2)]
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "linear.oil")
        avx2.oil_write(path, b"", lblocks, ltensors)
        lraw = np.fromfile(path, np.uint8)
        lw = [avx2.oil_read_tensor(path, t[0], 1 << 16) for t in ltensors]
    save("oil_linear", oil=lraw, shape=np.array([out_f, in_f, nb_tok]), x=xl, idx8=l8, cb8=cb8,
         vals4=l4.astype(np.uint8), cb4=l4cb, fp32=lf,
         **{f"w_{i}": w for i, w in enumerate(lw)},
         **{f"y_{i}": avx2.scalar_gemm(xl, w, nb_tok, out_f, in_f) for i, w in enumerate(lw)})

    # ---- decoder composition (src/model.cpp DenseModel::forward) -----------
    # A 2-layer model with the decoder's weight formats, dequantized to FP32
    # and loaded into the reference's own DenseModel (Linear weights
    # input-major, as it holds them), fed one token per forward call through
    # its KVCache; the logits of every step.  The weights are regenerated in
    # the tests from the seeded stream (synth.decoder_model), checked against
    # the stored digest.
    # The reference's attention output is not usable: its P*V loop indexes
    # V[t][2d] (vptr = vd + v_base + d, then vptr[t*head_dim + d],
    # src/transformer.cpp:325-342), reading past the cache.  The O projection
    # is therefore zero here (OIL8 codebook of zeros), which makes the
    # attention branch contribute exactly 0: the golden pins the embedding,
    # both residuals, the norms, the FFN and the lm_head; the attention and
    # RoPE are pinned against float64 definitions in the tests.
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "mythos.cpp_amd"))
    import synth
    from oracle import ReferenceModel
    cfg = synth.decoder_config(vocab=96, hidden=64, layers=2, heads=4, kv_heads=4, head_dim=16, ffn=128,
                               max_seq=16, cb_block=32)
    model = synth.decoder_model(cfg, config=50, random_gamma=True)
    for ly in model["layers"]:
        ly["cbo"] = np.zeros(256, np.float32)
    dense = synth.decoder_dense(cfg, model)
    ids = synth.decoder_prompts(cfg, 1, 12, config=50)[0]
    ids[3] = cfg["vocab"] + 5          # out of range: Embedding::forward reads row 0
    layers = [[d["attn_norm"], d["ffn_norm"]] + [np.ascontiguousarray(d[n].T) for n in
                                                  ("q", "k", "v", "o", "gate", "up", "down")]
              for d in dense["layers"]]
    runs = [ReferenceModel().run(cfg, dense["emb"], layers, dense["final_norm"],
                                 np.ascontiguousarray(dense["lm"].T), ids) for _ in range(2)]
    assert np.array_equal(runs[0], runs[1]) and np.isfinite(runs[0]).all()
    logits = runs[0]
    # math::softmax rows (src/math.cpp:207-249): wide range, ties, -inf entries
    sx = (rng.standard_normal((6, 75)) * 4).astype(np.float32)
    sx[1] = 0.0
    sx[2, ::3] = -np.inf
    sx[3] *= 30
    save("decoder", config=np.array(50), digest=np.frombuffer(bytes.fromhex(synth.decoder_digest(model)), np.uint8),
         ids=ids, logits=logits, softmax_x=sx, softmax=avx2.softmax(sx, 6, 75),
         **{f"cfg_{k}": np.array(v) for k, v in cfg.items()})


if __name__ == "__main__":
    main()
