"""Oracle decoders pinned by the reference's own KATs (dequant.rs tests),
restated here independently of the C oracle."""
import numpy as np
import pytest


def digit(byte, n, pow3):
    q = (byte * pow3[n]) & 0xFF
    return ((q * 3) >> 8) - 1


def test_f16_known_values(orc):  # dequant.rs:692-702
    assert orc.f16_to_f32(0x0000) == 0.0
    assert orc.f16_to_f32(0x3C00) == 1.0
    assert orc.f16_to_f32(0xBC00) == -1.0
    assert orc.f16_to_f32(0x3800) == 0.5
    assert orc.f16_to_f32(0x7C00) == float("inf")
    assert abs(np.float32(orc.f16_to_f32(0x3555)) - np.float32(0.33325195)) < 1e-9  # f32 literal
    assert abs(np.float32(orc.f16_to_f32(0x0001)) - np.float32(5.9604645e-8)) < 1e-12


def test_f16_matches_numpy_everywhere(orc):
    # Every non-NaN f16 bit pattern decodes as IEEE half (numpy) does.
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.isnan(got[~ok]).all()


def test_bf16_known_values(orc):  # dequant.rs:680-690
    assert orc.bf16_to_f32(0x0000) == 0.0
    assert orc.bf16_to_f32(0x3F80) == 1.0
    assert orc.bf16_to_f32(0xBF80) == -1.0
    assert orc.bf16_to_f32(0x7F80) == float("inf")
    assert orc.bf16_to_f32(0x4000) == 2.0
    assert abs(orc.bf16_to_f32(0x3EAA) - 0.33203125) < 1e-6


def test_tl1_group_matches_c_reference(orc):  # dequant.rs:563-603
    buf = np.zeros(28, np.uint8)
    for i in range(26):
        buf[i] = (i * 131 + 7) & 0xFF
    buf[26], buf[27] = 0x35, 0x3A
    fast = orc.tl1_group(buf)
    d = np.float32(np.array([0x3A35], np.uint16).view(np.float16)[0])
    pow3 = [1, 3, 9, 27, 81, 243]
    expect = np.zeros(128, np.float32)
    for n in range(5):
        for m in range(16):
            expect[n * 16 + m] = np.float32(digit(int(buf[m]), n, pow3)) * d
    for n in range(5):
        for m in range(8):
            expect[80 + n * 8 + m] = np.float32(digit(int(buf[16 + m]), n, pow3)) * d
    for n in range(4):
        for h in range(2):
            expect[120 + n * 2 + h] = np.float32(digit(int(buf[24 + h]), n, pow3)) * d
    assert np.array_equal(fast, expect)
    assert np.isfinite(fast).all()


def quantize_group_ref(x):  # the C quantizer transcribed in dequant.rs:609-640
    blk = np.zeros(28, np.uint8)
    blk[27] = 0x3C
    xi = [int(round(v)) + 1 for v in x]
    for m in range(16):
        q = 0
        for n in range(5):
            q = q * 3 + xi[m + n * 16]
        blk[m] = -(-(q * 256) // 243)
    for m in range(8):
        q = 0
        for n in range(5):
            q = q * 3 + xi[80 + m + n * 8]
        blk[16 + m] = -(-(q * 256) // 243)
    for h in range(2):
        q = 0
        for m in range(4):
            q = q * 3 + xi[120 + h + m * 2]
        q *= 3
        blk[24 + h] = -(-(q * 256) // 243)
    return blk


def test_ptq1_roundtrip_vs_c_quantizer(orc):  # dequant.rs:607-664
    lcg = 0x12345678
    for _ in range(64):
        x = np.zeros(128, np.float32)
        for i in range(128):
            lcg = (lcg * 1664525 + 1013904223) & 0xFFFFFFFF
            x[i] = (-1.0, 0.0, 1.0)[(lcg >> 16) % 3]
        out = orc.tl1_group(quantize_group_ref(x))
        assert np.array_equal(out, x), "roundtrip must be bit-exact"
    blk = quantize_group_ref(np.zeros(128))
    assert (orc.tl1_group(blk) == 0).all()


def test_tl1_group_trits_in_range(orc):  # dequant.rs:666-677
    buf = np.zeros(28, np.uint8)
    for i in range(26):
        buf[i] = ((i * 29) & 0xFF) ^ ((i * 7) & 0xFF)
    buf[26], buf[27] = 0x00, 0x3C
    out = orc.tl1_group(buf)
    assert np.isin(out, [-1.0, 0.0, 1.0]).all()


def test_tq1_values_are_ternary_scaled(orc):  # dequant.rs:704-713
    blk = np.zeros(54, np.uint8)
    blk[53] = 0x3C
    v = orc.tq1_block(blk)
    assert (v == -1.0).all()


def test_tq1_all_values_in_set(orc):  # dequant.rs:715-726
    blk = np.zeros(54, np.uint8)
    for i in range(52):
        blk[i] = (i * 7 + 3) & 0xFF
    blk[53] = 0x40
    v = orc.tq1_block(blk)
    assert np.isin(v, [-2.0, 0.0, 2.0]).all()


def test_tq1_block_element_order(orc):
    # dequant.rs:61-79: qs[0..32] -> n*32+m, qs[32..48] -> 160+n*16+m, qh -> 240+n*4+m
    rng = np.random.default_rng(3)
    blk = rng.integers(0, 256, 54, dtype=np.uint8)
    blk[52], blk[53] = 0x00, 0x3C
    v = orc.tq1_block(blk)
    pow3 = [1, 3, 9, 27, 81]
    exp = np.zeros(256, np.float32)
    for n in range(5):
        for m in range(32):
            exp[n * 32 + m] = digit(int(blk[m]), n, pow3)
        for m in range(16):
            exp[160 + n * 16 + m] = digit(int(blk[32 + m]), n, pow3)
    for n in range(4):
        for m in range(4):
            exp[240 + n * 4 + m] = digit(int(blk[48 + m]), n, pow3)
    assert np.array_equal(v, exp)


def test_quantkind_row_bytes(orc):  # dequant.rs:796-807
    assert orc.row_bytes(12, 5120) == 20 * 144
    assert orc.row_bytes(orc.KIND_TQ1_0, 2560) == 10 * 54
    assert orc.row_bytes(8, 512) == 16 * 34
    assert orc.row_bytes(13, 5120) == 20 * 176
    assert orc.row_bytes(11, 2560) == 10 * 110
    assert orc.row_bytes(orc.KIND_TL1, 2560) == 20 * 28
    assert orc.row_bytes(orc.KIND_I2, 2560) == 640
    from ouroboros_amd.quant import QuantKind
    for kind in QuantKind:
        for k in (256, 2560, 6912):
            assert QuantKind(kind).row_bytes(k) == orc.row_bytes(int(kind), k)
