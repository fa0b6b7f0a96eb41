"""I2 (int8 absmax activations x 2-bit ternary) oracle, pinned by closed
forms, brute force and invariants (the format has no reference code)."""
import numpy as np
import pytest

from ouroboros_amd import quant


def rand_w(rng, out_len, in_len):
    return rng.integers(-1, 2, size=(out_len, in_len)).astype(np.int8)


def test_pack_known_bytes(orc):
    # row [-1, 0, 1, 1 | 0, 0, 0, 0]: codes 0,1,2,2 -> 0b10_10_01_00 = 0xA4; 1,1,1,1 -> 0x55
    w = np.array([[-1, 0, 1, 1, 0, 0, 0, 0]], np.int8)
    assert list(orc.i2_pack(w)[0]) == [0xA4, 0x55]
    assert list(quant.i2_pack(w)[0]) == [0xA4, 0x55]


def test_pack_unpack_roundtrip(orc):
    rng = np.random.default_rng(0)
    w = rand_w(rng, 33, 256)
    p = orc.i2_pack(w)
    assert np.array_equal(orc.i2_unpack(p, 33, 256), w)
    assert np.array_equal(quant.i2_pack(w), p)
    assert np.array_equal(quant.i2_unpack(p, 256), w)
    # every canonical byte (codes 0..2) survives unpack -> pack
    b = np.array([x for x in range(256) if all(((x >> (2 * f)) & 3) < 3 for f in range(4))], np.uint8)
    b = np.resize(b, 81 * 4).reshape(-1, 4)
    assert np.array_equal(orc.i2_pack(orc.i2_unpack(b, b.shape[0], 16)), b)


def test_pack_rejects_non_ternary(orc):
    with pytest.raises(ValueError):
        orc.i2_pack(np.array([[2, 0, 0, 0]], np.int8))
    with pytest.raises(ValueError):
        quant.i2_pack(np.array([[0, 0, -2, 0]], np.int8))


def test_act_quant_closed_form(orc):
    x = np.array([[0.0, 0.5, -1.0, 2.0, -2.0, 1.0 / 254.0]], np.float32)
    q, ds = orc.act_quant_i8(x)
    s = np.float32(127.0) / np.float32(2.0)
    assert list(q[0]) == [0, int(np.rint(np.float32(0.5) * s)), int(np.rint(np.float32(-1.0) * s)), 127, -127,
                          int(np.rint(np.float32(1 / 254) * s))]
    assert ds[0] == np.float32(2.0) / np.float32(127.0)
    # all-zero row: zero codes and zero scale
    q, ds = orc.act_quant_i8(np.zeros((1, 8), np.float32))
    assert not q.any() and ds[0] == 0.0
    # single outlier maps to +-127 exactly, ties round half to even
    q, _ = orc.act_quant_i8(np.array([[127.0, 0.5, 1.5, 2.5, -0.5]], np.float32))
    assert list(q[0]) == [127, 0, 2, 2, 0]


def test_act_quant_matches_numpy(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((7, 2560)).astype(np.float32)
    x[3] = 0
    q, ds = orc.act_quant_i8(x)
    amax = np.abs(x).max(axis=1)
    for r in range(7):
        if amax[r] == 0:
            assert not q[r].any() and ds[r] == 0
            continue
        s = np.float32(127.0) / amax[r]
        want = np.clip(np.rint(x[r] * s), -127, 127).astype(np.int8)
        assert np.array_equal(q[r], want)
        assert ds[r] == amax[r] / np.float32(127.0)


def test_gemm_brute_force_and_epilogue(orc):
    rng = np.random.default_rng(2)
    out_len, in_len, nc = 29, 512, 3
    w = rand_w(rng, out_len, in_len)
    x = rng.standard_normal((nc, in_len)).astype(np.float32)
    xq, ds = orc.act_quant_i8(x)
    w_scale = np.float32(1.37)
    acc, y = orc.gemm_i2(orc.i2_pack(w), out_len, in_len, xq, ds, w_scale)
    ref = (xq.astype(np.int64) @ w.astype(np.int64).T).reshape(-1)  # [nc][out]
    assert np.array_equal(acc, ref)
    want = ((ref.astype(np.float32) * np.repeat(ds, out_len)).astype(np.float32) * w_scale).astype(np.float32)
    assert np.array_equal(y, want)


def test_gemm_invariants(orc):
    rng = np.random.default_rng(3)
    out_len, in_len = 4, 256
    xq, ds = orc.act_quant_i8(rng.standard_normal((1, in_len)).astype(np.float32))
    ones = np.ones((out_len, in_len), np.int8)
    acc, _ = orc.gemm_i2(orc.i2_pack(ones), out_len, in_len, xq, ds, 1.0)
    assert (acc == xq.astype(np.int64).sum()).all()
    acc0, y0 = orc.gemm_i2(orc.i2_pack(np.zeros_like(ones)), out_len, in_len, xq, ds, 1.0)
    assert not acc0.any() and not y0.any()
    w = rand_w(rng, out_len, in_len)
    a1, _ = orc.gemm_i2(orc.i2_pack(w), out_len, in_len, xq, ds, 1.0)
    a2, _ = orc.gemm_i2(orc.i2_pack(-w), out_len, in_len, xq, ds, 1.0)
    assert np.array_equal(a1, -a2)


def kgroup(G, lane, g):
    """Canonical byte column of lane-local group g (chunks of 4, then 2, then 1 groups)."""
    sizes = [4] * (G // 4) + ([2] if G % 4 >= 2 else []) + ([1] if G % 2 else [])
    o = 0
    for s in sizes:
        if g < o + s:
            return 64 * o + s * lane + (g - o)
        o += s
    raise ValueError(g)


def test_kgroup_is_a_permutation():
    for G in range(1, 33):
        cols = sorted(kgroup(G, lane, g) for lane in range(64) for g in range(G))
        assert cols == list(range(64 * G))


def untile(tiled, out_len, in_len):
    """Inverse of the documented tiled layout (written from the layout text)."""
    G = in_len // 256
    R = 8
    U = 8 if G % 2 else 16
    W = U // 4
    rb = in_len // 4
    tiles = -(-out_len // R)
    canon = np.zeros((tiles * R, rb), np.uint8)
    words = tiled.view(np.uint32)
    for t in range(tiles):
        for lane in range(64):
            for d in range(2 * G):
                off = t * R * rb + (d // W) * 64 * U + lane * U + (d % W) * 4
                word = int(words[off // 4])
                for f in range(4):
                    gi = 4 * d + f
                    r, g = gi // G, gi % G
                    byte = 0
                    for b in range(4):
                        byte |= ((word >> (8 * b + 2 * f)) & 3) << (2 * b)
                    canon[t * R + r, kgroup(G, lane, g)] = byte
    return canon


@pytest.mark.parametrize("out_len,in_len", [(16, 256), (13, 512), (9, 2560), (20, 1024), (11, 768)])
def test_tile_roundtrip(orc, out_len, in_len):
    rng = np.random.default_rng(out_len)
    canon = orc.i2_pack(rand_w(rng, out_len, in_len))
    tiled = orc.i2_tile(canon, out_len, in_len)
    back = untile(tiled, out_len, in_len)
    assert np.array_equal(back[:out_len], canon)
    assert (back[out_len:] == 0x55).all()  # padding rows are w = 0


def untile_mfma(units, out_len, in_len):
    """Weights w = -v recovered from the documented MFMA layout (written from the layout text)."""
    nkb, tiles = in_len // 256, -(-out_len // 16)
    words = units.view(np.uint32).reshape(tiles, nkb, 64, 4)
    w = np.zeros((tiles * 16, in_len), np.int8)
    for rt in range(tiles):
        for kb in range(nkb):
            for lane in range(64):
                for s in range(4):
                    word = int(words[rt, kb, lane, s])
                    for j in range(4):
                        for i in range(4):
                            v = (word >> (8 * i + 2 * j)) & 3
                            v = v - 4 if v >= 2 else v  # 2-bit two's complement
                            w[rt * 16 + lane % 16, 256 * kb + 64 * s + 16 * (lane // 16) + 4 * j + i] = -v
    return w


@pytest.mark.parametrize("out_len,in_len", [(16, 256), (5, 512), (33, 768)])
def test_tile_mfma_roundtrip(orc, out_len, in_len):
    rng = np.random.default_rng(out_len + in_len)
    w = rand_w(rng, out_len, in_len)
    units = orc.i2_tile_mfma(orc.i2_pack(w), out_len, in_len)
    back = untile_mfma(units, out_len, in_len)
    assert np.array_equal(back[:out_len], w)
    assert (back[out_len:] == 0).all()  # padding rows are w = 0


def test_tile_mfma_keeps_code_3(orc):
    # code 3 (never produced by the packer) decodes to w = 2 (orc_i2_unpack); the
    # MFMA layout stores v = 1 - code = -2, which two bits still hold
    canon = np.full((1, 64), 0x55, np.uint8)
    canon[0, 0] = 0x57  # k = 0 has code 3
    back = untile_mfma(orc.i2_tile_mfma(canon, 1, 256), 1, 256)
    assert back[0, 0] == 2 and (back[0, 1:] == 0).all()
