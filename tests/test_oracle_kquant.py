"""Oracle pins for the Q8_0 and K-quant decoders (Q3_K, Q4_K, Q5_K, Q6_K) and
matvec_qblock over them (dequant.rs:218-310, 390-560; ops.rs:101-128).

The reference pins these decoders bit for bit against ggml's C
(bitnet-rs/tests/verify_infer.rs:84-158), which is not available here. What
pins the oracle instead:
  * the reference's own KATs (dequant.rs:756-795);
  * an independent decoder below, written element by element from the
    block layouts (for element e: which byte, which bits, which scale),
    where the oracle restates the reference's block loops; both use the
    reference's float operation order, so they must agree bit for bit;
  * byte-position probes: changing one payload byte changes exactly the
    elements the layout assigns to it;
  * closed forms on single blocks (all-equal codes, zero scales);
  * matvec_qblock against float64 dequant-then-dot.
Inputs use the reference's own generator (verify_infer.rs:11-17, the 64-bit
LCG with its f16 sanitising, 88-98).
"""
import numpy as np
import pytest

import oracle

Q8, Q3K, Q4K, Q5K, Q6K = 8, 11, 12, 13, 14
KINDS = [Q8, Q3K, Q4K, Q5K, Q6K]
# byte offsets of the f16 scales of each block (their high byte is sanitised)
F16_AT = {Q8: [0], Q3K: [108], Q4K: [0, 2], Q5K: [0, 2], Q6K: [208], 34: [52]}


def lcg_bytes(seed: int, n: int) -> np.ndarray:
    """verify_infer.rs:11-17: st = st * 6364136223846793005 + 1442695040888963407; byte = st >> 33."""
    out = np.empty(n, np.uint8)
    st = seed
    m = (1 << 64) - 1
    for i in range(n):
        st = (st * 6364136223846793005 + 1442695040888963407) & m
        out[i] = (st >> 33) & 0xFF
    return out


def payload(kind: int, nblk: int, seed: int) -> np.ndarray:
    bb, _ = oracle.QBLOCK[kind]
    rng = np.random.default_rng(seed)
    p = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    for o in F16_AT[kind]:
        p[:, o + 1] %= 0x78  # finite f16 (verify_infer.rs:91-97)
    return p.reshape(-1)


def f16(lo, hi) -> np.float32:
    return np.frombuffer(bytes([int(lo), int(hi)]), np.float16)[0].astype(np.float32)


def scale_min(j: int, sc: np.ndarray) -> tuple[int, int]:
    """The 6-bit (scale, min) pair of sub-block j of a Q4_K/Q5_K block: for
    j < 4 the low six bits of bytes j and j + 4; for j >= 4 the low/high
    nibble of byte j + 4 below the top two bits of bytes j - 4 / j."""
    sc = [int(v) for v in sc]
    if j < 4:
        return sc[j] & 63, sc[j + 4] & 63
    return (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4), (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)


def q3k_scale(k: int, sc: np.ndarray) -> int:
    """Scale k (0..15) of a Q3_K block: its low four bits are nibble k // 8 of
    byte k % 8, its high two bits field k // 4 of byte 8 + k % 4."""
    lo = (int(sc[k % 8]) >> (4 * (k // 8))) & 15
    hi = (int(sc[8 + k % 4]) >> (2 * (k // 4))) & 3
    return lo | (hi << 4)


def decode_block(kind: int, b: np.ndarray) -> np.ndarray:
    """Element-by-element decode of one block, in the reference's float order."""
    f = np.float32
    if kind == Q8:
        d = f16(b[0], b[1])
        return np.array([f(np.int8(b[2 + e].astype(np.int8))) * d for e in range(32)], np.float32)
    out = np.empty(256, np.float32)
    if kind in (Q4K, Q5K):
        d, dmin = f16(b[0], b[1]), f16(b[2], b[3])
        sc = b[4:16]
        qh, qs = (b[16:48], b[48:176]) if kind == Q5K else (None, b[16:144])
        for e in range(256):
            j, hi, l = e // 64, (e % 64) // 32, e % 32
            byte = int(qs[32 * j + l])
            q = (byte >> 4) if hi else (byte & 15)
            s, m = scale_min(2 * j + hi, sc)
            if kind == Q5K:
                qf = f(q) + (f(16) if (int(qh[l]) >> (2 * j + hi)) & 1 else f(0))
            else:
                qf = f(q)
            out[e] = (d * f(s)) * qf - dmin * f(m)
        return out
    if kind == Q6K:
        ql, qh, sc = b[0:128], b[128:192], b[192:208].astype(np.int8)
        d = f16(b[208], b[209])
        for e in range(256):
            n, r = e // 128, e % 128
            k, l = r // 32, r % 32
            byte = int(ql[64 * n + l + 32 * (k % 2)])
            nib = (byte >> 4) if k // 2 else (byte & 15)
            hb = (int(qh[32 * n + l]) >> (2 * k)) & 3
            q = (nib | (hb << 4)) - 32
            out[e] = (d * f(int(sc[8 * n + l // 16 + 2 * k]))) * f(q)
        return out
    if kind == Q3K:
        hm, qs, sc = b[0:32], b[32:96], b[96:108]
        d = f16(b[108], b[109])
        for e in range(256):
            n, r = e // 128, e % 128
            j, l = r // 32, r % 32
            qi = (int(qs[32 * n + l]) >> (2 * j)) & 3
            hb = (int(hm[l]) >> (4 * n + j)) & 1
            s = q3k_scale(8 * n + 2 * j + l // 16, sc)
            out[e] = (d * (f(s) - f(32))) * f(qi - (0 if hb else 4))
        return out
    raise ValueError(kind)


# ---- the reference's KATs (dequant.rs:756-795) --------------------------------


def test_q8_block_simple():  # dequant.rs:757-768
    blk = np.zeros(34, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:34] = np.arange(32)
    blk[33] = 0x80
    v = oracle.dequant_qblock(Q8, blk)
    assert v[0] == 0.0 and v[10] == 10.0 and v[31] == -128.0


def test_q4k_scale_nibble_math():  # dequant.rs:770-785
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[4], blk[5] = 30, 2
    blk[16:] = 0xF0
    v = oracle.dequant_qblock(Q4K, blk)
    assert np.all(v[0:32] == 0.0) and np.all(v[32:64] == 30.0) and np.all(v[64:] == 0.0)


def test_q4k_min_offsets():  # dequant.rs:787-796
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x2C]
    v = oracle.dequant_qblock(Q4K, blk)
    assert np.all(v == 0.0)


def test_quantkind_row_bytes_kquant():  # dequant.rs:798-809
    assert oracle.row_bytes(Q4K, 5120) == 20 * 144
    assert oracle.row_bytes(34, 2560) == 10 * 54
    assert oracle.row_bytes(Q8, 512) == 16 * 34
    assert oracle.row_bytes(Q5K, 5120) == 20 * 176
    assert oracle.row_bytes(Q3K, 2560) == 10 * 110
    assert oracle.row_bytes(Q6K, 2560) == 10 * 210
    for k in (8, 11, 12, 13, 14):
        assert oracle.lib().orc_kind_supported(k) == 1


# ---- independent element-wise decoder, bit for bit -----------------------------


@pytest.mark.parametrize("kind", KINDS)
def test_decoder_matches_elementwise_layout(kind):
    bb, be = oracle.QBLOCK[kind]
    nblk = 48
    raw = lcg_bytes(7777 if kind != Q8 else 42, nblk * bb).reshape(nblk, bb)
    for o in F16_AT[kind]:
        raw[:, o + 1] %= 0x78
    got = oracle.dequant_qblock(kind, raw.reshape(-1)).reshape(nblk, be)
    for i in range(nblk):
        want = decode_block(kind, raw[i])
        np.testing.assert_array_equal(got[i].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_byte_positions(kind):
    """Changing one byte changes exactly the elements the layout gives it."""
    bb, be = oracle.QBLOCK[kind]
    rng = np.random.default_rng(kind)
    # scales that decode to non-zero, distinct values, so every code byte matters
    base = payload(kind, 1, 100 + kind).copy()
    if kind in (Q4K, Q5K):
        base[0:4] = [0x00, 0x3C, 0x00, 0x38]  # d = 1, dmin = 0.5
        base[4:16] = rng.integers(1, 64, 12)  # 6-bit fields non-zero in every sub-block
    elif kind == Q6K:
        base[192:208] = rng.integers(1, 100, 16)
        base[208:210] = [0x00, 0x3C]
    elif kind == Q3K:
        base[96:108] = 0x11  # every scale 17: s - 32 = -15 != 0
        base[108:110] = [0x00, 0x3C]
    else:
        base[0:2] = [0x00, 0x3C]
    ref = oracle.dequant_qblock(kind, base)
    owners = {}
    for e in range(be):
        # bytes an element depends on, from the element-wise layout
        owners[e] = element_bytes(kind, e)
    code_bytes = set().union(*owners.values())
    for pos in sorted(code_bytes):
        b = base.copy()
        b[pos] ^= 0xFF
        changed = set(np.nonzero(oracle.dequant_qblock(kind, b) != ref)[0].tolist())
        expect = {e for e, s in owners.items() if pos in s}
        assert changed == expect, (kind, pos)


def element_bytes(kind: int, e: int) -> set:
    """Code bytes (not scales) element e of a block reads."""
    if kind == Q8:
        return {2 + e}
    if kind == Q4K:
        return {16 + 32 * (e // 64) + e % 32}
    if kind == Q5K:
        return {48 + 32 * (e // 64) + e % 32, 16 + e % 32}
    if kind == Q6K:
        n, r = e // 128, e % 128
        k, l = r // 32, r % 32
        return {64 * n + l + 32 * (k % 2), 128 + 32 * n + l}
    if kind == Q3K:
        n, l = e // 128, e % 32
        return {32 + 32 * n + l, l}
    raise ValueError(kind)


# ---- closed forms on single blocks ---------------------------------------------


def test_q6k_uniform_codes():
    b = np.zeros(210, np.uint8)
    b[0:128] = 0xFF  # nibbles 15
    b[128:192] = 0xFF  # high bits 3 -> q = 63 - 32 = 31
    b[192:208] = np.arange(-8, 8, dtype=np.int8).view(np.uint8)
    b[208:210] = [0x00, 0x38]  # d = 0.5
    v = oracle.dequant_qblock(Q6K, b)
    sc = np.arange(-8, 8)
    for e in range(256):
        n, r = e // 128, e % 128
        assert v[e] == 0.5 * sc[8 * n + (r % 32) // 16 + 2 * (r // 32)] * 31


def test_q3k_all_high_bits_clear():
    b = np.zeros(110, np.uint8)  # hmask 0: every code is qi - 4; scales 0 -> s - 32 = -32
    b[32:96] = 0xFF  # qi = 3
    b[108:110] = [0x00, 0x3C]
    v = oracle.dequant_qblock(Q3K, b)
    assert np.all(v == -32.0 * -1.0)


def test_q5k_high_bit_adds_sixteen():
    b = np.zeros(176, np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[4:8] = 1  # scales 0..3 = 1, mins 0
    b[16:48] = 0x55  # bits 0, 2, 4, 6: the low nibble of every pair
    v = oracle.dequant_qblock(Q5K, b)
    for e in range(128):  # sub-blocks 0..3 have scale 1
        assert v[e] == (16.0 if (e % 64) < 32 else 0.0)


# ---- matvec_qblock ------------------------------------------------------------


@pytest.mark.parametrize("kind", KINDS + [34])
def test_matvec_qblock_is_dequant_then_dot(kind):
    bb, be = oracle.QBLOCK[kind]
    out_len, in_len = 37, 768
    p = payload(kind, out_len * in_len // be, 5 + kind)
    x = np.random.default_rng(1).standard_normal(in_len).astype(np.float32)
    y = oracle.matvec_q(p, kind, out_len, in_len, x, nthreads=3)
    w = oracle.dequant_qblock(kind, p).reshape(out_len, in_len).astype(np.float64)
    want = w @ x.astype(np.float64)
    assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want))
    # the reference's own summation: dot() over the decoded row, in order
    row = oracle.dequant_qblock(kind, p[: bb * in_len // be])
    assert y[0] == oracle.lib().orc_dot(row.ctypes.data, x.ctypes.data, in_len)


def test_reference_q6k_deterministic_payload():
    """agent/src/gpu.rs:288-318: the reference's OpenCL parity matrix (d = 1,
    mixed-sign scales) and x; the oracle against float64."""
    out_len, in_len = 8, 512
    bpr = in_len // 256
    pl = np.empty(out_len * bpr * 210, np.uint8)
    for i in range(pl.size):
        b, off = i // 210, i % 210
        if 192 <= off <= 207:
            s = (off * 3 + b * 5) % 64
            pl[i] = 192 + s if ((b + off) & 1) == 1 else s
        elif off == 208:
            pl[i] = 0x00
        elif off == 209:
            pl[i] = 0x3C
        else:
            pl[i] = (i * 7 + 13) & 0xFF
    x = np.array([((i % 17) - 8.0) * 0.125 for i in range(in_len)], np.float32)
    y = oracle.matvec_q(pl, Q6K, out_len, in_len, x)
    w = oracle.dequant_qblock(Q6K, pl).reshape(out_len, in_len).astype(np.float64)
    want = w @ x.astype(np.float64)
    np.testing.assert_allclose(y, want, rtol=0, atol=1e-5 * np.max(np.abs(want)))
