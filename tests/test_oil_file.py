"""The `.oil` reader of libmythos_host.so (include/mythos_oil_file.h) against a
model file written by the reference's own OILWriter and the reference's
OILReader::read_tensor of every tensor in it (tests/golden/oil_file.npz,
src/oil_format.cpp:287-462).  CPU only: parsing and repacking never touch the
device; the upload + GEMV half is in test_gpu_oil_file.py.

The repacked layouts are checked two ways: bit-exactly against the inputs the
fixture was written from, and by dequantising them with the reference's own
decode (the oracle's restatement of CodebookOIL4::half_to_float, pinned by the
fp16 fixture) and comparing bit for bit with the reference reader's FP32.
"""
import os
import struct

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLD, "oil_file.npz"))


@pytest.fixture(scope="module")
def of():
    import oil_file
    return oil_file


@pytest.fixture(scope="module")
def oil_path(gold, tmp_path_factory):
    p = tmp_path_factory.mktemp("oil") / "tiny.oil"
    gold["oil"].tofile(p)
    return str(p)


def pack_nibbles(v):
    v = np.asarray(v, np.uint8).reshape(-1)
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


def pack_codes(c):
    c = np.asarray(c, np.uint8).reshape(-1, 4)
    return (c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)).astype(np.uint8)


def write_oil(path, config: bytes, blocks, tensors):
    """Test-side writer of the container (src/oil_format.cpp OILWriter);
    test_writer_reproduces_reference_file pins it to the reference's bytes.
    blocks: [(format, num_weights, codebook bytes, index bytes)];
    tensors: [(name, block_start, num_blocks)]."""
    out = [b"OIL1", struct.pack("<III", 1 << 22, 0, len(config)), config, struct.pack("<I", len(blocks))]
    out += [struct.pack("<IBI", i, b[0], len(b[2])) for i, b in enumerate(blocks)]
    out.append(struct.pack("<I", len(tensors)))
    for name, start, n in tensors:
        nm = name.encode()
        out += [struct.pack("<H", len(nm)), nm, struct.pack("<II", start, n)]
    for fmt, nw, cb, idx in blocks:
        out += [struct.pack("<II", nw, len(cb)), bytes(cb), struct.pack("<I", len(idx)), bytes(idx)]
    with open(path, "wb") as f:
        f.write(b"".join(out))


def oil4_cb_bytes(cb16):
    return struct.pack("<I", 0x4F494C34) + np.asarray(cb16, "<u2").tobytes()


def oil8_cb_bytes(cb):
    return struct.pack("<I", 0x4F494C38) + np.asarray(cb, "<f4").tobytes()


def fixture_blocks(g):
    """The blocks and tensor table make_golden.py handed to the reference's
    OILWriter, rebuilt from the fixture's inputs."""
    blocks = []
    r, c = g["oil8_shape"]
    blocks.append((3, r * c, oil8_cb_bytes(g["oil8_cb"]), g["oil8_idx"].tobytes()))
    for b in range(3):
        blocks.append((3, 128, oil8_cb_bytes(g["oil8_cb"]), g["oil8m_idx"][b * 128:(b + 1) * 128].tobytes()))
    r, c, B = g["oil4_shape"]
    for b in range(r * c // B):
        blocks.append((2, B, oil4_cb_bytes(g["oil4_cbs"][b]), pack_nibbles(g["oil4_vals"][b * B:(b + 1) * B]).tobytes()))
    blocks.append((2, 96, oil4_cb_bytes(g["oil4s_cb"]), pack_nibbles(g["oil4s_vals"]).tobytes()))
    blocks.append((1, 320, np.array([-1, 0, 1], "<f4").tobytes(), pack_codes(g["tern_codes"]).tobytes()))
    blocks.append((5, 64, b"", g["fp32_vals"].tobytes()))
    tensors = [(str(n), int(s), int(k)) for n, s, k in zip(g["names"], g["block_start"], g["num_blocks"])]
    return blocks, tensors


def test_writer_reproduces_reference_file(gold, tmp_path):
    blocks, tensors = fixture_blocks(gold)
    p = tmp_path / "w.oil"
    write_oil(p, b'{"arch":"mythos","n_layers":2}', blocks, tensors)
    assert p.read_bytes() == gold["oil"].tobytes()


def test_names_info_and_config(of, gold, oil_path):
    with of.OILReader(oil_path) as r:
        assert r.valid()
        assert r.tensor_names() == [str(n) for n in gold["names"]]
        assert r.read_config() == b'{"arch":"mythos","n_layers":2}'
        want = {  # name: (format, weights, blocks, block length)
            "blk.0.attn_q.weight": (of.OIL8, 240, 1, 240),
            "blk.0.ffn_up.weight": (of.OIL8, 384, 3, 128),
            "blk.0.ffn_down.weight": (of.OIL4, 768, 6, 128),
            "output.weight": (of.OIL4, 96, 1, 96),
            "blk.1.attn_k.weight": (of.TERNARY, 320, 1, 320),
            "token_norm.weight": (of.FP32, 64, 1, 64),
        }
        for name, (fm, nw, nb, bw) in want.items():
            assert r.info(name) == {"format": fm, "num_weights": nw, "num_blocks": nb, "block_weights": bw}
            # the reference reader's tensor holds the same number of weights
            i = [str(n) for n in gold["names"]].index(name)
            assert gold[f"read_{i}"].size == nw


def test_oil8_repack_matches_reference_read(of, gold, oil_path):
    with of.OILReader(oil_path) as r:
        idx, cb, cbk = r.repack("blk.0.attn_q.weight", 6, 40)
        assert cbk == 0 and np.array_equal(idx.ravel(), gold["oil8_idx"])
        assert np.array_equal(cb.view(np.uint32), gold["oil8_cb"].view(np.uint32))
        assert np.array_equal(cb[idx].ravel().view(np.uint32), gold["read_0"].view(np.uint32))
        idx, cb, _ = r.repack("blk.0.ffn_up.weight", 4, 96)    # three blocks, one codebook
        assert np.array_equal(idx.ravel(), gold["oil8m_idx"])
        assert np.array_equal(cb[idx].ravel().view(np.uint32), gold["read_1"].view(np.uint32))


def test_oil4_blocked_repack_matches_reference_read(of, oracle, gold, oil_path):
    with of.OILReader(oil_path) as r:
        nib, cbs, cbk = r.repack("blk.0.ffn_down.weight", 3, 256)
    assert cbk == 128 and nib.shape == (3, 128) and cbs.shape == (6, 16)
    assert np.array_equal(nib.ravel(), pack_nibbles(gold["oil4_vals"]))
    assert np.array_equal(cbs, gold["oil4_cbs"])
    # dequantise as the kernels index it: row m, column k -> codebook m*(K/B) + k/B
    v = np.stack([nib & 15, nib >> 4], -1).reshape(3, 256)
    blk = np.arange(3)[:, None] * 2 + np.arange(256)[None, :] // 128
    h = cbs[blk, v]
    ref_decode = np.vectorize(oracle.half_to_float_codebook, otypes=[np.float32])(h)
    assert np.array_equal(ref_decode.ravel().view(np.uint32), gold["read_2"].view(np.uint32))
    # all entries are FP16 normals, where the reference's decode is the exact one
    assert np.array_equal(h.astype(np.uint16).view(np.float16).astype(np.float32).ravel(), gold["read_2"])


def test_oil4_single_codebook(of, oracle, gold, oil_path):
    with of.OILReader(oil_path) as r:
        nib, cbs, cbk = r.repack("output.weight", 2, 48)
    assert cbk == 0 and cbs.shape == (1, 16)
    v = np.stack([nib & 15, nib >> 4], -1).ravel()
    assert np.array_equal(v, gold["oil4s_vals"])
    got = np.array([oracle.half_to_float_codebook(int(cbs[0, i])) for i in v], np.float32)
    assert np.array_equal(got.view(np.uint32), gold["read_3"].view(np.uint32))


def test_ternary_repack(of, gold, oil_path):
    with of.OILReader(oil_path) as r:
        codes, cb, _ = r.repack("blk.1.attn_k.weight", 5, 64)
    assert np.array_equal(codes, pack_codes(gold["tern_codes"]))      # code q+1, I2_S bit order
    assert np.array_equal(cb, np.array([-1, 0, 1], np.float32))
    # The reference's read_tensor has no ternary branch and returns zeros
    # (src/oil_format.cpp:447-451); the repack keeps the codes instead.
    assert not gold["read_4"].any()


def test_fp32_repack(of, gold, oil_path):
    with of.OILReader(oil_path) as r:
        w, cb, _ = r.repack("token_norm.weight", 1, 64)
    assert cb is None and np.array_equal(w.ravel().view(np.uint32), gold["read_5"].view(np.uint32))


def test_every_truncation_is_an_error(of, gold, tmp_path):
    raw = gold["oil"].tobytes()
    p = tmp_path / "t.oil"
    for cut in list(range(0, 200)) + list(range(200, len(raw), 7)) + [len(raw) - 1]:
        p.write_bytes(raw[:cut])
        r = of.OILReader(str(p))
        assert not r.valid(), cut
        assert r.error, cut


def test_corrupt_files_rejected(of, gold, tmp_path):
    raw = bytearray(gold["oil"].tobytes())
    p = tmp_path / "c.oil"
    bad = bytearray(raw)
    bad[0:4] = b"OIL2"
    p.write_bytes(bytes(bad))
    r = of.OILReader(str(p))
    assert not r.valid() and "OIL1" in r.error
    bad = bytearray(raw)
    struct.pack_into("<I", bad, 12, 1 << 30)                   # config larger than the file
    p.write_bytes(bytes(bad))
    assert not of.OILReader(str(p)).valid()
    bad = bytearray(raw)
    struct.pack_into("<I", bad, 16 + 30, 1 << 28)              # format-table count past the end
    p.write_bytes(bytes(bad))
    assert not of.OILReader(str(p)).valid()
    # a tensor entry that points past the block table
    blocks, tensors = fixture_blocks(gold)
    tensors[0] = (tensors[0][0], 20, 1)
    write_oil(p, b"", blocks, tensors)
    r = of.OILReader(str(p))
    assert not r.valid() and "past the table" in r.error


def test_argument_errors(of, gold, oil_path, tmp_path):
    from mythos_oil import MythosError
    r = of.OILReader(oil_path)
    with pytest.raises(MythosError, match="no tensor"):
        r.info("missing.weight")
    with pytest.raises(MythosError, match="weights, not"):
        r.repack("blk.0.attn_q.weight", 5, 40)
    with pytest.raises(MythosError) as e:                      # 128-weight blocks do not tile rows of 64
        r.repack("blk.0.ffn_down.weight", 12, 64)
    assert e.value.code == of.EUNSUPPORTED
    # buffers smaller than the layout are refused, not overrun
    idx = np.zeros(8, np.uint8)
    cb = np.zeros(1024, np.uint8)
    rc = of.lib.mth_oil_repack(r._h, b"blk.0.attn_q.weight", 6, 40, 0, idx.ctypes.data, 8, cb.ctypes.data, 1024, None)
    assert rc == of.EINVAL and "index bytes" in of.last_error()
    rc = of.lib.mth_oil_repack(r._h, b"blk.0.ffn_down.weight", 3, 256, 0, np.zeros(384, np.uint8).ctypes.data, 384,
                               cb.ctypes.data, 100, None)
    assert rc == of.EINVAL and "codebook bytes" in of.last_error()
    # OIL8 blocks of one tensor with different codebooks
    blocks, tensors = fixture_blocks(gold)
    f, nw, cbb, ix = blocks[2]
    blocks[2] = (f, nw, oil8_cb_bytes(gold["oil8_cb"] * 2), ix)
    p = tmp_path / "m.oil"
    write_oil(p, b"", blocks, tensors)
    with pytest.raises(MythosError, match="different codebooks"):
        of.OILReader(str(p)).repack("blk.0.ffn_up.weight", 4, 96)
    r.close()
    with pytest.raises(MythosError):
        r.tensor_names()


# ---- Linear weights (input-major, as the reference's model holds them) ----
@pytest.fixture(scope="module")
def lin(tmp_path_factory):
    g = np.load(os.path.join(GOLD, "oil_linear.npz"))
    p = tmp_path_factory.mktemp("lin") / "linear.oil"
    g["oil"].tofile(p)
    return g, str(p)


def test_linear_orientation_matches_reference_forward(of, oracle, lin):
    """Repacked with in_major, W[m][k] @ x reproduces the reference's
    Linear::forward product scalar_gemm(x, W) for OIL8, OIL4 and FP32."""
    g, path = lin
    out_f, in_f, nt = (int(v) for v in g["shape"])
    x = g["x"].astype(np.float64)
    with of.OILReader(path) as r:
        idx, cb, _ = r.repack("layers.0.attention.q_proj.weight", out_f, in_f, in_major=True)
        nib, cb4, cbk = r.repack("layers.0.ffn.up_proj.weight", out_f, in_f, in_major=True)
        wf, _, _ = r.repack("layers.0.attention.o_proj.weight", out_f, in_f, in_major=True)
        # the same bytes read output-major are the transpose
        idx_t, _, _ = r.repack("layers.0.attention.q_proj.weight", in_f, out_f)
    assert np.array_equal(idx, idx_t.T)
    assert np.array_equal(idx.T.ravel(), g["idx8"])
    assert cbk == 0 and cb4.shape == (1, 16) and np.array_equal(cb4[0], g["cb4"])
    v = np.stack([nib & 15, nib >> 4], -1).reshape(out_f, in_f)
    assert np.array_equal(v.T.ravel(), g["vals4"])
    w8 = cb[idx]
    w4 = np.vectorize(oracle.half_to_float_codebook, otypes=[np.float32])(cb4[0][v])
    for i, w in enumerate((w8, w4, wf)):
        # the repacked weight is the reference reader's tensor, transposed
        assert np.array_equal(w.T.ravel().view(np.uint32), g[f"w_{i}"].view(np.uint32)), i
        y = (x @ w.astype(np.float64).T).ravel()
        absw = (np.abs(x) @ np.abs(w.astype(np.float64)).T).ravel()
        assert np.all(np.abs(y - g[f"y_{i}"]) <= 1e-6 * absw + 1e-30), i


def test_linear_oil4_needs_one_codebook(of, gold, oil_path):
    from mythos_oil import MythosError
    with of.OILReader(oil_path) as r:
        with pytest.raises(MythosError, match="input-major OIL4") as e:
            r.repack("blk.0.ffn_down.weight", 128, 6, in_major=True)
        assert e.value.code == of.EUNSUPPORTED
        # a single-codebook OIL4 tensor transposes element by element
        nib, _, _ = r.repack("output.weight", 48, 2, in_major=True)
    v = np.stack([nib & 15, nib >> 4], -1).reshape(48, 2)
    assert np.array_equal(v.T.ravel(), gold["oil4s_vals"])


def test_ternary_in_major(of, gold, tmp_path):
    c = gold["tern_codes"].reshape(16, 20)           # file order [in=16][out=20]
    p = tmp_path / "t.oil"
    write_oil(p, b"", [(1, 320, np.array([-1, 0, 1], "<f4").tobytes(), pack_codes(c).tobytes())],
              [("w", 0, 1)])
    with of.OILReader(str(p)) as r:
        codes, _, _ = r.repack("w", 20, 16, in_major=True)
    assert np.array_equal(codes, pack_codes(c.T))
