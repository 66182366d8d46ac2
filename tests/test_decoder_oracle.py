"""The CPU restatement of the config-5 decoder (oracle/decoder.c) against the
reference's own DenseModel (golden logits from tests/golden/decoder.npz, made
by make_golden.py with the compiled reference) and against what the
mathematics fixes for its parts.  CPU only.
"""
import os

import numpy as np
import pytest

import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLD, "decoder.npz"))


def golden_cfg(g):
    c = {k[4:]: g[k].item() for k in g.files if k.startswith("cfg_")}
    for k in ("eps", "theta"):
        c[k] = float(c[k])
    return c


@pytest.fixture(scope="module")
def tiny(gold):
    cfg = golden_cfg(gold)
    model = synth.decoder_model(cfg, config=int(gold["config"]), random_gamma=True)
    return cfg, model


def test_decoder_matches_reference_dense_model(oracle, gold, tiny):
    """down_mode 1 (FP32 activations into the ternary projection) is the
    reference Linear's arithmetic: the logits of every step agree with the
    reference DenseModel's to FP32 rounding.  The golden model's O projection
    is zero (the reference's attention output indexes V[t][2d],
    src/transformer.cpp:325-342), so this pins everything but attention."""
    cfg, model = tiny
    model = dict(model, layers=[dict(ly, cbo=np.zeros(256, np.float32)) for ly in model["layers"]])
    assert synth.decoder_digest(model) == bytes(gold["digest"]).hex(), "synthetic weights changed: regenerate goldens"
    dec = oracle.decoder(cfg, model)
    kc, vc = dec.new_cache()
    for pos, tok in enumerate(gold["ids"]):
        got = dec.step(kc, vc, pos, int(tok), down_mode=1, threads=1).astype(np.float64)
        ref = gold["logits"][pos].astype(np.float64)
        err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert err < 2e-6, (pos, err)


def test_int8_down_projection_stays_close(oracle, gold, tiny):
    """down_mode 0 quantises the FFN activations to int8 per token (the I2_S
    path); the logits move by the quantisation error only."""
    cfg, model = tiny
    dec = oracle.decoder(cfg, model)
    k0, v0 = dec.new_cache()
    k1, v1 = dec.new_cache()
    for pos, tok in enumerate(gold["ids"][:6]):
        a = dec.step(k0, v0, pos, int(tok), down_mode=0, threads=1).astype(np.float64)
        b = dec.step(k1, v1, pos, int(tok), down_mode=1, threads=1).astype(np.float64)
        err = np.linalg.norm(a - b) / np.linalg.norm(b)
        assert 0 < err < 0.05, (pos, err)


def test_softmax_matches_reference(oracle, gold):
    x = gold["softmax_x"]
    assert np.array_equal(oracle.softmax(x, *x.shape), gold["softmax"])


def test_rope_properties(oracle):
    D, S = 16, 64
    cos_t, sin_t = oracle.rope_tables(D, S)
    g = np.random.default_rng(1)
    q = g.normal(0, 1, 2 * D).astype(np.float32)
    k = g.normal(0, 1, 2 * D).astype(np.float32)
    assert np.array_equal(oracle.rope_apply(q, 2, D, 0, cos_t, sin_t), q)      # position 0: identity
    # rotation: each pair (d, d + D/2) keeps its length
    r = oracle.rope_apply(q, 2, D, 37, cos_t, sin_t).reshape(2, 2, D // 2)
    q2 = q.reshape(2, 2, D // 2)
    np.testing.assert_allclose(np.hypot(r[:, 0], r[:, 1]), np.hypot(q2[:, 0], q2[:, 1]), rtol=1e-5)
    # scores depend on the position difference only
    def score(m, n):
        a = oracle.rope_apply(q[:D], 1, D, m, cos_t, sin_t).astype(np.float64)
        b = oracle.rope_apply(k[:D], 1, D, n, cos_t, sin_t).astype(np.float64)
        return a @ b
    for m, n, j in ((5, 2, 7), (20, 20, 11), (3, 9, 40)):
        assert abs(score(m, n) - score(m + j, n + j)) < 1e-4 * (1 + abs(score(m, n)))
    # the table's frequencies: angle pos * theta^(-2j/D)
    j = np.arange(D // 2)
    np.testing.assert_allclose(cos_t[9], np.cos(9 * 10000.0 ** (-2 * j / D)), atol=2e-6)


def test_attention_against_float64(oracle):
    g = np.random.default_rng(2)
    H, KVH, D, S, ctx = 4, 2, 16, 10, 7
    q = g.normal(0, 1, H * D).astype(np.float32)
    kc = g.normal(0, 1, (KVH, S, D)).astype(np.float32)
    vc = g.normal(0, 1, (KVH, S, D)).astype(np.float32)
    got = oracle.attention_decode(q, kc, vc, H, KVH, D, ctx, S).reshape(H, D)
    for h in range(H):
        kh = h % KVH
        s = kc[kh, :ctx].astype(np.float64) @ q[h * D:(h + 1) * D].astype(np.float64) / np.sqrt(D)
        w = np.exp(s - s.max())
        w /= w.sum()
        np.testing.assert_allclose(got[h], w @ vc[kh, :ctx].astype(np.float64), rtol=1e-5, atol=1e-6)


def test_argmax_is_first_maximum(oracle):
    a = np.array([1.0, 3.0, 3.0, 2.0], np.float32)
    assert oracle.argmax(a) == 1
    assert oracle.argmax(np.array([np.nan, 0.5, np.nan, 0.5], np.float32)) == 1
    assert oracle.argmax(np.full(5, np.nan, np.float32)) == 0
    assert oracle.argmax(np.full(5, -np.inf, np.float32)) == 0


def test_decoder_greedy_uses_argmax(oracle, tiny):
    """A free-running greedy continuation feeds each step's argmax back."""
    cfg, model = tiny
    dec = oracle.decoder(cfg, model)
    kc, vc = dec.new_cache()
    tok, seq = 7, []
    for pos in range(6):
        logits = dec.step(kc, vc, pos, tok, threads=1)
        tok = oracle.argmax(logits)
        seq.append(tok)
    kc2, vc2 = dec.new_cache()
    ids = [7] + seq[:-1]
    for pos, t in enumerate(ids):
        assert oracle.argmax(dec.step(kc2, vc2, pos, t, threads=1)) == seq[pos]


def np_decoder(cfg, dense, ids, down_int8=False):
    """The decoder stack from its mathematical definition in float64:
    pre-norm blocks, rotate-half RoPE at each token's position, causal
    softmax attention with scale 1/sqrt(D), SwiGLU FFN, final norm, lm_head."""
    H, D, NH, KVH = cfg["hidden"], cfg["head_dim"], cfg["heads"], cfg["kv_heads"]
    eps = cfg["eps"]
    j = np.arange(D // 2)
    inv_freq = cfg["theta"] ** (-2.0 * j / D)

    def rms(x, g):
        return x / np.sqrt((x * x).mean() + eps) * g

    def rope(v, pos):
        v = v.reshape(-1, D)
        c, s = np.cos(pos * inv_freq), np.sin(pos * inv_freq)
        a, b = v[:, :D // 2], v[:, D // 2:]
        return np.concatenate([a * c - b * s, a * s + b * c], 1)

    K = [[] for _ in dense["layers"]]
    Vc = [[] for _ in dense["layers"]]
    out = []
    for pos, tok in enumerate(ids):
        x = dense["emb"][tok if 0 <= tok < cfg["vocab"] else 0].astype(np.float64)
        for li, d in enumerate(dense["layers"]):
            h = rms(x, d["attn_norm"])
            q = rope(d["q"] @ h, pos)
            K[li].append(rope(d["k"] @ h, pos))
            Vc[li].append((d["v"] @ h).reshape(-1, D))
            k_all, v_all = np.stack(K[li]), np.stack(Vc[li])          # [t][kvh][D]
            att = np.empty((NH, D))
            for hh in range(NH):
                sc = k_all[:, hh % KVH] @ q[hh] / np.sqrt(D)
                w = np.exp(sc - sc.max())
                att[hh] = (w / w.sum()) @ v_all[:, hh % KVH]
            x = x + d["o"] @ att.ravel()
            h = rms(x, d["ffn_norm"])
            gg, u = d["gate"] @ h, d["up"] @ h
            x = x + d["down"] @ (gg / (1 + np.exp(-gg)) * u)
        out.append(dense["lm"] @ rms(x, dense["final_norm"]))
    return np.array(out)


def test_decoder_with_attention_against_float64(oracle, gold, tiny):
    """The full stack, attention and RoPE included, against its float64
    definition (down_mode 1: FP32 activations into the ternary projection)."""
    cfg, model = tiny
    dense = synth.decoder_dense(cfg, model)
    ids = [int(t) for t in gold["ids"]]
    ref = np_decoder(cfg, dense, ids)
    dec = oracle.decoder(cfg, model)
    kc, vc = dec.new_cache()
    for pos, tok in enumerate(ids):
        got = dec.step(kc, vc, pos, tok, down_mode=1, threads=1).astype(np.float64)
        err = np.linalg.norm(got - ref[pos]) / np.linalg.norm(ref[pos])
        assert err < 1e-5, (pos, err)


def test_bf16_round_pins(oracle):
    """orc_bf16_round: round to the nearest bf16, ties to even, checked
    against an integer restatement and hand-picked ties and specials."""
    g = np.random.default_rng(3)
    x = np.concatenate([g.normal(0, 1, 4000), g.normal(0, 1e30, 50), [0.0, -0.0, np.inf, -np.inf, 3.0e38]])
    x = x.astype(np.float32)
    got = np.array([oracle.bf16_round(float(v)) for v in x], np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    want = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # ties: 1 + 2^-8 sits halfway between 1 and 1 + 2^-7 -> the even one (1);
    # 1 + 3*2^-8 halfway between 1 + 2^-7 and 1 + 2^-6 -> 1 + 2^-6
    assert oracle.bf16_round(1.0 + 2.0 ** -8) == 1.0
    assert oracle.bf16_round(1.0 + 3 * 2.0 ** -8) == 1.0 + 2.0 ** -6
    assert np.isnan(oracle.bf16_round(float("nan")))


def test_attn_half_position0_closed_form(oracle, tiny):
    """At position 0 the softmax has one entry, so attention returns V: the
    attention half is x + Wo (Wv rmsnorm(x)), checked in float64 with the
    dequantised weights.  It appends the rotated K and the V to the cache."""
    cfg, model = tiny
    dec = oracle.decoder(cfg, model)
    kc, vc = dec.new_cache()
    g = np.random.default_rng(4)
    x = g.normal(0, 1, cfg["hidden"]).astype(np.float32)
    ly = model["layers"][1]
    y = dec.attn_half(kc, vc, 1, 0, x, threads=1).astype(np.float64)
    xd = x.astype(np.float64)
    h = xd / np.sqrt(np.mean(xd * xd) + cfg["eps"]) * ly["attn_norm"]
    v = synth.dequant_oil8(ly["wv"], ly["cbv"]).astype(np.float64) @ h
    heads, kvh, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    att = np.concatenate([v[(hh % kvh) * D:(hh % kvh + 1) * D] for hh in range(heads)])
    want = xd + synth.dequant_oil8(ly["wo"], ly["cbo"]).astype(np.float64) @ att
    assert np.linalg.norm(y - want) / np.linalg.norm(want) < 1e-6
    assert np.allclose(vc[1, :, 0].ravel(), v, rtol=1e-5, atol=1e-6)
    assert not kc[0].any() and not kc[1, :, 1:].any()      # only layer 1, position 0 written


def test_kv_bf16_cache_holds_rounded_values(oracle, tiny):
    """kv_bf16: every cached K/V value is a bf16 value (low 16 bits zero) and
    equals the FP32 cache's value rounded; the logits move by that rounding."""
    cfg, model = tiny
    d32 = oracle.decoder(cfg, model)
    d16 = oracle.decoder(dict(cfg, kv_bf16=1), model)
    k32, v32 = d32.new_cache()
    k16, v16 = d16.new_cache()
    ids = synth.decoder_prompts(cfg, 1, 4, config=61)[0]
    for pos, tok in enumerate(ids):
        a = d32.step(k32, v32, pos, int(tok), threads=1).astype(np.float64)
        b = d16.step(k16, v16, pos, int(tok), threads=1).astype(np.float64)
        assert np.linalg.norm(a - b) / np.linalg.norm(a) < 2e-2
    assert not (k16.view(np.uint32) & 0xFFFF).any() and not (v16.view(np.uint32) & 0xFFFF).any()
    # position 0 of layer 0 sees the same input on both sides
    r = np.array([oracle.bf16_round(float(t)) for t in k32[0, :, 0].ravel()], np.float32)
    assert np.array_equal(r, k16[0, :, 0].ravel())


def test_i2s_gemv_rows_composition(oracle):
    """i2s_gemv_rows on quantize_per_token(x) is the fused i2s_gemv_f32, and
    its integer dot product matches an int64 closed form."""
    g = np.random.default_rng(8)
    M, K = 37, 256
    packed = g.integers(0, 256, M * K // 4, dtype=np.uint8)
    x = g.normal(0, 1, K).astype(np.float32)
    q, _, inv = oracle.quantize_per_token(x, 1, K)
    y = oracle.i2s_gemv_rows(packed, 0.5, q.ravel(), float(inv[0]), M, K)
    assert np.array_equal(y, oracle.i2s_gemv_f32(packed, 0.5, x, M, K, 1).ravel())
    codes = np.stack([(packed.reshape(M, K // 4) >> (2 * j)) & 3 for j in range(4)], -1).reshape(M, K)
    t = np.where(codes == 0, -1, np.where(codes == 1, 0, 1)).astype(np.int64)
    dot = t @ q.ravel().astype(np.int64)
    want = (dot.astype(np.float32) * np.float32(0.5)) * np.float32(inv[0])
    assert np.array_equal(y, want)
