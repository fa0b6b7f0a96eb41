"""The int8-activation x 2-bit ternary oracle: bitnet.cpp's I2_S tensor and
I8_S activation rules (microsoft/BitNet, src/ggml-bitnet-mad.cpp, the
reference's absent bitnet-cpp submodule), pinned by hand-computed bytes and
values, by int64 brute force and by invariants; and this library's canonical
and tiled repacks of the same codes, pinned by round trips.

These rules are this repository's transcription of the published bitnet.cpp
source: with the submodule empty there is no bitnet.cpp output or reference
fixture to compare with, so "bit-exact" elsewhere means bit-exact vs this
oracle."""
import numpy as np
import pytest

from ouroboros_amd import quant


def rand_w(rng, out_len, in_len):
    return rng.integers(-1, 2, size=(out_len, in_len)).astype(np.int8)


SCALE_1 = [0x00, 0x00, 0x80, 0x3F]  # 1.0f little-endian


def one_hot_row(n, j, v):
    w = np.zeros((1, n), np.int8)
    w[0, j] = v
    return w


@pytest.mark.parametrize("j,v,byte,value", [
    (0, +1, 0, 0x95),     # j = 0: byte 0, bits 6-7 (code 2 = 0b10 over 0b01 fill)
    (31, +1, 31, 0x95),   # j = 31: byte 31, bits 6-7
    (32, +1, 0, 0x65),    # j = 32: byte 0, bits 4-5
    (127, +1, 31, 0x56),  # j = 127: byte 31, bits 0-1
    (0, -1, 0, 0x15),     # code 0 for w = -1
    (95, -1, 31, 0x51),   # j = 95: byte 31, bits 2-3
])
def test_i2s_byte_positions(orc, j, v, byte, value):
    w = one_hot_row(128, j, v)
    want = np.full(64, 0x55, np.uint8)  # every other weight is 0 (code 1)
    want[byte] = value
    want[32:36] = SCALE_1
    want[36:] = 0
    assert list(orc.i2s_pack(w, 1.0)) == list(want)
    assert list(quant.i2s_pack(w, 1.0)) == list(want)
    assert orc.i2s_code(want, 128, 0, j) == v + 1


def test_i2s_blocks_span_the_flattened_tensor(orc):
    # 1 x 256: weight 128 is block 1, j = 0 -> byte 32 bits 6-7; weight 255 -> byte 63 bits 0-1
    w = np.zeros((1, 256), np.int8)
    w[0, 128], w[0, 255] = 1, -1
    b = orc.i2s_pack(w, 1.0)
    assert b[32] == 0x95 and b[63] == 0x54 and (np.delete(b[:64], [32, 63]) == 0x55).all()
    assert list(b[64:68]) == SCALE_1 and b.size == 64 + 32
    # 2 x 128: row 1, k = 0 is flat weight 128, the same byte 32
    w2 = np.zeros((2, 128), np.int8)
    w2[1, 0] = 1
    assert orc.i2s_pack(w2, 1.0)[32] == 0x95


def test_quantize_i2_s_from_floats(orc):
    # quantize_i2_s: scale = max|src| = 2; |v| < 1e-6 -> code 1; sign -> code 2 / 0
    src = np.zeros((1, 128), np.float32)
    src[0, :4] = [0.5, -0.25, 1e-7, -2.0]
    b = orc.quantize_i2_s(src)
    assert list(b[:4]) == [0x95, 0x15, 0x55, 0x15] and (b[4:32] == 0x55).all()
    assert list(b[32:36]) == [0x00, 0x00, 0x00, 0x40]  # 2.0f
    assert b.size == 64


def test_i2s_roundtrip_and_canonical(orc):
    rng = np.random.default_rng(0)
    for shape in [(3, 128), (5, 256), (33, 512)]:
        w = rand_w(rng, *shape)
        b = orc.i2s_pack(w, 0.75)
        assert np.array_equal(quant.i2s_pack(w, 0.75), b)
        back, sc = quant.i2s_unpack(b, *shape)
        assert np.array_equal(back, w) and sc == 0.75
        assert np.array_equal(orc.i2_unpack(orc.i2s_to_canonical(b, *shape), *shape), w)


def test_i8s_quantizer_ties_round_away_from_zero(orc):
    # max|x| = 127 -> s = 1 exactly, so x * s is exact and the halves are exact ties
    q, s, t = orc.quantize_row_i8_s([127.0, 0.5, 1.5, 2.5, -0.5, -2.5, 0.0, 0.49])
    assert s == 1.0
    assert list(q) == [127, 1, 2, 3, -1, -3, 0, 0]  # rint would give 0, 2, 2, -0, -2
    assert t == 129


def test_i8s_quantizer_amax_floor(orc):
    # all-zero row: max = 1e-5, s = (float)(127 / 1e-5) = 12700000.0f, q = 0
    q, s, t = orc.quantize_row_i8_s(np.zeros(8, np.float32))
    assert s == np.float32(12700000.0) and not q.any() and t == 0
    # a row below the floor still uses it: 1e-6f * 1.27e7f = 12.7 -> 13, -3e-6f * 1.27e7f = -38.1 -> -38
    q, s, _ = orc.quantize_row_i8_s([1e-6, -3e-6, 0.0, 0.0])
    assert s == np.float32(12700000.0) and list(q) == [13, -38, 0, 0]


def test_i8s_scale_is_the_double_division(orc):
    # s = (float)(127.0 / 3.0) = 42.333332f (0x42295555); row max 3.8379693f -> 33.090416f (0x42048596)
    _, s, _ = orc.quantize_row_i8_s([3.0, -1.0])
    assert np.float32(s).view(np.uint32) == 0x42295555
    _, s, _ = orc.quantize_row_i8_s([np.float32(3.8379693031311035), 0.25])
    assert np.float32(s).view(np.uint32) == 1107582102
    # the clamp: |x * s| never exceeds 127 by more than rounding, so a row's max maps to +-127
    q, _, _ = orc.quantize_row_i8_s([-3.0, 1.0, 3.0])
    assert list(q) == [-127, 42, 127]


def test_epilogue_operation_order(orc):
    # y = RN(RN(acc / s) * w_scale).  For acc = 1255, s = 0x42048596, w_scale = 0x3FA7E64D the
    # value is 0x4246FE9B; (acc * w) / s and acc * (w / s) give 0x4246FE9C, acc * (1/s) * w 0x4246FE9D.
    s = np.array([1107582102], np.uint32).view(np.float32)
    w_scale = float(np.array([1067968077], np.uint32).view(np.float32)[0])
    w = np.zeros((1, 128), np.int8)
    w[0, :10] = 1
    xq = np.zeros((1, 128), np.int8)
    xq[0, :10] = [127] * 9 + [1255 - 9 * 127]
    i2s = orc.i2s_pack(w, w_scale)
    acc, y = orc.gemm_i2s(i2s, 1, 128, xq, s)
    assert acc[0] == 1255 and y.view(np.uint32)[0] == 0x4246FE9B
    acc2, y2 = orc.gemm_i2(orc.i2s_to_canonical(i2s, 1, 128), 1, 128, xq, s, w_scale)
    assert acc2[0] == 1255 and y2.view(np.uint32)[0] == 0x4246FE9B
    # a KAT with an exact value: s = 63.5 from max|x| = 2 (x = 1 -> 63.5 -> 64), acc = 127 -> 2 * 1.5 = 3
    q, s2, _ = orc.quantize_row_i8_s(np.r_[2.0, 1.0, np.zeros(126)])
    assert s2 == 63.5 and list(q[:2]) == [127, 64]
    _, y3 = orc.gemm_i2s(orc.i2s_pack(one_hot_row(128, 0, 1), 1.5), 1, 128, q[None], [s2])
    assert y3[0] == 3.0


def decode_i2s(b, out_len, in_len):
    """Weights of an I2_S tensor, written from the layout text (independent of both packers)."""
    w = np.empty(out_len * in_len, np.int8)
    for e in range(out_len * in_len):
        w[e] = ((int(b[32 * (e // 128) + e % 32]) >> (6 - 2 * ((e % 128) // 32))) & 3) - 1
    return w.reshape(out_len, in_len)


def test_gemm_i2s_brute_force(orc):
    rng = np.random.default_rng(2)
    out_len, in_len, nc = 29, 512, 3
    w = rand_w(rng, out_len, in_len)
    x = rng.standard_normal((nc, in_len)).astype(np.float32)
    xq, s = orc.act_quant_i8(x)
    i2s = orc.i2s_pack(w, 1.37)
    assert np.array_equal(decode_i2s(i2s, out_len, in_len), w)
    acc, y = orc.gemm_i2s(i2s, out_len, in_len, xq, s)
    ref = (xq.astype(np.int64) @ w.astype(np.int64).T).reshape(-1)  # [nc][out]
    assert np.array_equal(acc, ref)
    # vec_dot sums codes (w + 1); the act_sum correction recovers sum w*q
    for r in (0, 7, 28):
        assert orc.vec_dot_i2_i8_s(i2s, in_len, r, xq[1]) == int(ref[out_len + r]) + int(xq[1].astype(np.int64).sum())
    # every output within half an ulp of the real-valued (acc / s) * w_scale, twice rounded
    exact = ref / np.repeat(s.astype(np.float64), out_len) * np.float64(np.float32(1.37))
    assert (np.abs(y - exact) <= 2 * np.abs(exact) * 2.0 ** -24 + 1e-30).all()
    # the canonical-code product is the same function
    acc2, y2 = orc.gemm_i2(orc.i2s_to_canonical(i2s, out_len, in_len), out_len, in_len, xq, s, np.float32(1.37))
    assert np.array_equal(acc2, acc) and np.array_equal(y2.view(np.uint32), y.view(np.uint32))


def test_gemm_invariants(orc):
    rng = np.random.default_rng(3)
    out_len, in_len = 4, 256
    xq, s = orc.act_quant_i8(rng.standard_normal((1, in_len)).astype(np.float32))
    ones = np.ones((out_len, in_len), np.int8)
    acc, _ = orc.gemm_i2s(orc.i2s_pack(ones, 1.0), out_len, in_len, xq, s)
    assert (acc == xq.astype(np.int64).sum()).all()
    z = orc.i2s_pack(np.zeros_like(ones), 1.0)
    assert np.array_equal(quant.i2s_pack(np.zeros_like(ones), 1.0), z) and orc.i2s_scale(z, out_len, in_len) == 0
    acc0, y0 = orc.gemm_i2s(z, out_len, in_len, xq, s)
    assert not acc0.any() and not y0.any()
    w = rand_w(rng, out_len, in_len)
    a1, _ = orc.gemm_i2s(orc.i2s_pack(w, 1.0), out_len, in_len, xq, s)
    a2, _ = orc.gemm_i2s(orc.i2s_pack(-w, 1.0), out_len, in_len, xq, s)
    assert np.array_equal(a1, -a2)


# ---- this library's canonical and tiled layouts of the same codes ----

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
    with pytest.raises(ValueError):
        orc.i2s_pack(np.full((1, 128), 2, np.int8), 1.0)
    with pytest.raises(ValueError):
        quant.i2s_pack(np.zeros((1, 100), np.int8), 1.0)


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
