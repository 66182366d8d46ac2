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
