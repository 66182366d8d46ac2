"""The benchmark input generator (synth.py over host/synth.cpp) draws from
MYTHOS.cpp's RNG: pinned against the reference's own outputs (golden rng
fixture) and the documented derivations of indices, ternary codes and
normals.  CPU only."""
import os

import numpy as np

import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_stream_matches_reference_rng():
    z = np.load(os.path.join(GOLD, "rng.npz"))
    for i, seed in enumerate(z["seeds"]):
        n = z["u64"].shape[1]
        assert np.array_equal(synth.Stream(int(seed)).u64(n), z["u64"][i])
        assert np.array_equal(synth.Stream(int(seed)).uniform_int(n, 0, 2).astype(np.int32), z["uint_0_2"][i])
        assert np.array_equal(synth.Stream(int(seed)).uniform_int(n, -5, 9).astype(np.int32), z["uint_m5_9"][i])


def test_draws_continue_one_stream():
    a = synth.Stream(0x5EED0002)
    first, second = a.u64(100), a.u64(50)
    assert np.array_equal(np.concatenate([first, second]), synth.Stream(0x5EED0002).u64(150))


def test_indices_are_top_bits():
    u = synth.Stream(7).u64(1000)
    assert np.array_equal(synth.Stream(7).bits(1000, 8), (u >> np.uint64(56)).astype(np.uint8))
    assert np.array_equal(synth.Stream(7).bits(1000, 4), (u >> np.uint64(60)).astype(np.uint8))


def test_normal_is_double_box_muller():
    u = synth.Stream(11).u64(2000)
    u1 = (u[0::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(np.maximum(u1, 2.0 ** -53)))
    want = np.empty(2000)
    want[0::2] = 0.5 + 2.0 * r * np.cos(2 * np.pi * u2)
    want[1::2] = 0.5 + 2.0 * r * np.sin(2 * np.pi * u2)
    got = synth.Stream(11).normal(2000, 0.5, 2.0)
    np.testing.assert_allclose(got, want.astype(np.float32), rtol=1e-6, atol=1e-6)
    big = synth.Stream(12).normal(200000)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1.0) < 0.01


def test_float_to_half_trunc_matches_oracle(oracle):
    g = np.random.default_rng(3)
    f = np.concatenate([g.normal(0, 0.02, 3000), g.normal(0, 1e4, 1000), g.normal(0, 1e-6, 1000),
                        [0.0, -0.0, np.inf, -np.inf, 65520.0, -70000.0]]).astype(np.float32)
    want = np.array([oracle.float_to_half_trunc(float(v)) for v in f], np.uint16)
    assert np.array_equal(synth.float_to_half_trunc(f), want)


def test_config_generators_shapes_and_ranges():
    idx, cb, x = synth.oil8(64, 256, 2)
    assert idx.shape == (64, 256) and cb.shape == (256,) and x.shape == (2, 256)
    assert np.all(np.diff(cb) >= 0)
    packed, cbs, x = synth.oil4(32, 256, 3, 128)
    assert packed.shape == (32, 128) and cbs.shape == (32 * 2 * 16,)
    pk, ws, x = synth.ternary(16, 64, 1)
    codes = np.stack([(pk >> (2 * j)) & 3 for j in range(4)], -1)
    assert codes.max() <= 2 and ws == np.float32(0.0159577)


def test_packed_draws_equal_unpacked():
    a, b = synth.Stream(21), synth.Stream(21)
    assert np.array_equal(a.nibbles(7, 64), synth.pack_nibbles(b.bits((7, 64), 4)))
    assert np.array_equal(a.ternary(5, 48), synth.pack_ternary(b.uniform_int((5, 48), 0, 2) - 1))
    assert np.array_equal(a.u64(10), b.u64(10))      # both streams advanced alike


def test_normal_f16_is_truncated_normal():
    a, b = synth.Stream(33), synth.Stream(33)
    for shape in ((1001,), (64, 16)):
        want = synth.float_to_half_trunc(b.normal(shape, 0.0, 0.02))
        assert np.array_equal(a.normal_f16(shape, 0.0, 0.02), want)
    f = np.concatenate([synth.Stream(34).normal(4000, 0, 1e4), synth.Stream(35).normal(4000, 0, 1e-6)])
    c = synth.Stream(36)
    assert np.array_equal(c.normal_f16(5, 0, 1e5), synth.float_to_half_trunc(synth.Stream(36).normal(5, 0, 1e5)))

