"""Oracle matvec/matmul pinned by the reference equivalence tests (ops.rs)."""
import numpy as np


def tl1_payload(out_len, in_len, mul_shift, d_lo=0x10, d_hi=0x38):
    rb = in_len // 128 * 28
    i = np.arange(out_len * rb, dtype=np.uint64)
    p = ((i * (0x9B ^ (i >> mul_shift))) & 0xFF).astype(np.uint8)
    g = p.reshape(-1, 28)
    g[:, 26], g[:, 27] = d_lo, d_hi
    return p


def test_dot(orc):  # ops.rs:671-675
    a = np.array([1, 2], np.float32)
    b = np.array([5, 6], np.float32)
    assert orc.lib().orc_dot(a.ctypes.data, b.ctypes.data, 2) == 17.0


def test_matvec_tl1_fused_matches_reference(orc):  # ops.rs:800-838
    out_len, in_len = 37, 384
    p = tl1_payload(out_len, in_len, 7)
    x = ((np.arange(in_len) % 7) - 3.0).astype(np.float32) * 0.5
    for simd in (0, 1):
        fused = orc.matvec_tl1(p, out_len, in_len, x, simd=simd)
        rb = in_len // 128 * 28
        for row in range(out_len):
            flat = np.concatenate([orc.tl1_group(p[row * rb + g * 28: row * rb + (g + 1) * 28])
                                   for g in range(in_len // 128)])
            want = np.float32(0)
            for a, b in zip(flat, x):
                want = np.float32(want + np.float32(a * b))
            assert abs(fused[row] - want) / max(abs(want), 1e-9) < 1e-5


def test_matvec_tl1_scalar_order_is_sequential(orc):
    # tl1_rows_scalar (ops.rs:324-363) sums every term in element order of the
    # decode loops; rebuild that sum in float32 step by step.
    out_len, in_len = 5, 256
    p = tl1_payload(out_len, in_len, 7)
    x = np.random.default_rng(0).standard_normal(in_len).astype(np.float32)
    y = orc.matvec_tl1(p, out_len, in_len, x, simd=0)
    rb = in_len // 128 * 28
    order = ([n * 16 + m for n in range(5) for m in range(16)] +
             [80 + n * 8 + m for n in range(5) for m in range(8)] +
             [120 + n * 2 + m for n in range(4) for m in range(2)])
    for r in range(out_len):
        s = np.float32(0)
        for g in range(in_len // 128):
            w = orc.tl1_group(p[r * rb + g * 28: r * rb + (g + 1) * 28])
            for e in order:
                s = np.float32(s + np.float32(w[e] * x[g * 128 + e]))
        assert y[r] == s


def test_matmul_tl1_k_columns_matches_matvec(orc):  # ops.rs:720-750
    out_len, in_len, k = 97, 384, 4
    rb = in_len // 128 * 28
    i = np.arange(out_len * rb, dtype=np.uint64)
    p = ((i * (0x9B ^ (i >> 5))) & 0xFF).astype(np.uint8)
    g = p.reshape(-1, 28)
    g[:, 26], g[:, 27] = 0x10, 0x38
    x = (((np.arange(k * in_len) % 11) - 5.0) * 0.25).astype(np.float32)
    for simd in (0, 1):
        batched = orc.matmul_tl1(p, out_len, in_len, x, k, simd=simd)
        for c in range(k):
            want = orc.matvec_tl1(p, out_len, in_len, x[c * in_len:(c + 1) * in_len], simd=simd)
            got = batched[c * out_len:(c + 1) * out_len]
            assert (np.abs(got - want) <= 1e-3 * np.maximum(np.abs(want), 1.0)).all()
    # the scalar K path is the scalar matvec order exactly (ops.rs:244-286)
    sk = orc.matmul_tl1(p, out_len, in_len, x, k, simd=0)
    for c in range(k):
        assert np.array_equal(sk[c * out_len:(c + 1) * out_len],
                              orc.matvec_tl1(p, out_len, in_len, x[c * in_len:(c + 1) * in_len], simd=0))


def test_matmul_q_fallback_matches(orc):  # ops.rs:781-797
    out_len, in_len = 16, 32
    v = (((np.arange(out_len * in_len) % 17) - 8.0) * 0.25).astype(np.float32)
    payload = (v.view(np.uint32) & 0xFFFF).astype(np.uint16)  # low half bytes, as the test does
    payload = payload.view(np.uint8)
    x = ((np.arange(2 * in_len) % 7) * 0.5).astype(np.float32)
    y = orc.matmul_q(payload, orc.KIND_F16, out_len, in_len, x, 2)
    for c in range(2):
        want = orc.matvec_q(payload, orc.KIND_F16, out_len, in_len, x[c * in_len:(c + 1) * in_len])
        assert np.array_equal(y[c * out_len:(c + 1) * out_len], want)


def test_matvec_tq1_is_dequant_then_dot(orc):  # ops.rs:101-128
    rng = np.random.default_rng(5)
    out_len, in_len = 9, 512
    p = rng.integers(0, 256, out_len * (in_len // 256) * 54, dtype=np.uint8)
    blocks = p.reshape(-1, 54)
    blocks[:, 52], blocks[:, 53] = 0x00, 0x3A
    x = rng.standard_normal(in_len).astype(np.float32)
    y = orc.matvec_q(p, orc.KIND_TQ1_0, out_len, in_len, x)
    for r in range(out_len):
        row = orc.dequant_tq1_row(p, r, in_len)
        s = np.float32(0)
        for a, b in zip(row, x):
            s = np.float32(s + np.float32(a * b))
        assert y[r] == s


def test_dense_kinds_match_float64(orc):
    rng = np.random.default_rng(1)
    out_len, in_len = 7, 96
    w = rng.standard_normal((out_len, in_len)).astype(np.float32)
    x = rng.standard_normal(in_len).astype(np.float32)
    for kind, payload, wf in (
        (orc.KIND_F32, w.view(np.uint8), w),
        (orc.KIND_F16, w.astype(np.float16).view(np.uint8), w.astype(np.float16).astype(np.float32)),
        (orc.KIND_BF16, (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8),
         ((w.view(np.uint32) >> 16) << 16).view(np.float32)),
    ):
        y = orc.matvec_q(payload.reshape(-1), kind, out_len, in_len, x)
        ref = wf.astype(np.float64) @ x.astype(np.float64)
        assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_finite_argmax(orc):  # infer/mod.rs:70-83
    nan, inf = float("nan"), float("inf")
    assert orc.finite_argmax([1.0, 3.0, 2.0]) == 1
    assert orc.finite_argmax([nan, 1.0, nan, 5.0, nan]) == 3   # NaN skipped
    assert orc.finite_argmax([2.0, 7.0, 7.0, 1.0]) == 1        # strict >: first maximum wins
    assert orc.finite_argmax([nan, nan]) == 0                  # nothing found
    assert orc.finite_argmax([-0.0, 0.0]) == 0                 # -0 and +0 compare equal
    assert orc.finite_argmax([-inf, -inf]) == 0
    assert orc.finite_argmax([nan, -inf, -5.0]) == 2
    assert orc.finite_argmax([1.0, inf, nan, inf]) == 1
    rng = np.random.default_rng(3)
    for _ in range(20):  # against numpy's nanargmax (first occurrence) on NaN-sprinkled vectors
        x = rng.standard_normal(1000).astype(np.float32)
        x[rng.random(1000) < 0.1] = nan
        assert orc.finite_argmax(x) == int(np.nanargmax(x))
