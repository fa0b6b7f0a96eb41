"""ouro_matvec_q_noalloc (static per-device scratch, no allocation) against
ouro_matvec_q, bit for bit, on two calls in a row with the second smaller,
for both 2-bit kinds and for the TL1 / TQ1_0 lookup GEMVs (partial sums in
the static array); plus its size limits and a kind that uses no scratch."""
import numpy as np
import pytest

from ouroboros_amd import ops, quant
from ouroboros_amd._lib import KIND_F32, KIND_I2, KIND_I2_S, KIND_TL1, KIND_TQ1_0, OuroError, call
from ouroboros_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def run(entry, payload, kind, out_len, in_len, x):
    y = DeviceBuffer((out_len,), np.float32)
    call(entry, payload.ptr, kind, out_len, in_len, x.ptr, y.ptr, None)
    return y.download().view(np.uint32)


def test_noalloc_matches_matvec_q(gpu):
    rng = np.random.default_rng(77)
    for out_len, in_len in [(6912, 2560), (300, 1024)]:  # the second call is smaller
        w = rng.integers(-1, 2, size=(out_len, in_len)).astype(np.int8)
        i2s = DeviceBuffer.from_host(quant.i2s_pack(w, 1.3))
        tiled = ops.i2s_payload(i2s, out_len, in_len)
        x = DeviceBuffer.from_host(rng.standard_normal(in_len).astype(np.float32))
        for kind, p in ((KIND_I2_S, i2s), (KIND_I2, tiled)):
            want = run("ouro_matvec_q", p, kind, out_len, in_len, x)
            got = run("ouro_matvec_q_noalloc", p, kind, out_len, in_len, x)
            assert np.array_equal(got, want), (out_len, in_len, kind)


def test_noalloc_limit_and_other_kinds(gpu):
    buf = DeviceBuffer((4096,), np.uint8)
    with pytest.raises(OuroError) as e:
        call("ouro_matvec_q_noalloc", buf.ptr, KIND_I2_S, 8, 32768 + 256, buf.ptr, buf.ptr, None)
    assert e.value.code == 2
    rng = np.random.default_rng(5)
    w = DeviceBuffer.from_host(rng.standard_normal((16, 64)).astype(np.float32))
    x = DeviceBuffer.from_host(rng.standard_normal(64).astype(np.float32))
    assert np.array_equal(run("ouro_matvec_q_noalloc", w, KIND_F32, 16, 64, x),
                          run("ouro_matvec_q", w, KIND_F32, 16, 64, x))


def lut_payload(rng, kind, out_len, in_len):
    """Random TL1 (28 B per 128) or TQ1_0 (54 B per 256) bytes with small f16 scales."""
    gb, ge, d_at = (28, 128, 26) if kind == KIND_TL1 else (54, 256, 52)
    p = rng.integers(0, 256, out_len * (in_len // ge) * gb, dtype=np.uint8)
    g = p.reshape(-1, gb)
    d = rng.uniform(0.01, 0.1, g.shape[0]).astype(np.float16).view(np.uint16)
    g[:, d_at], g[:, d_at + 1] = d & 0xFF, d >> 8
    return p


@pytest.mark.parametrize("kind", [KIND_TL1, KIND_TQ1_0])
def test_noalloc_lookup_partials(gpu, kind):
    """The lm_head shape (9.9 MB of partial sums in the static array), then a
    smaller matrix: the same lookup kernels as ouro_matvec_q, so bit-equal."""
    rng = np.random.default_rng(31 + kind)
    for out_len, in_len in [(248320, 5120), (8192, 1024)]:
        w = DeviceBuffer.from_host(lut_payload(rng, kind, out_len, in_len))
        x = DeviceBuffer.from_host(rng.standard_normal(in_len).astype(np.float32))
        want = run("ouro_matvec_q", w, kind, out_len, in_len, x)
        got = run("ouro_matvec_q_noalloc", w, kind, out_len, in_len, x)
        assert np.array_equal(got, want), (kind, out_len, in_len)
        del w


@pytest.mark.parametrize("kind", [KIND_TL1, KIND_TQ1_0])
def test_noalloc_lookup_beyond_static_scratch(gpu, orc, kind):
    """Partial sums past 16 MiB (40960 x 65536: 128 x 40960 floats, 20 MiB)
    run the direct kernel: its first 256 rows within the dot product's fp32
    error bound of the float64 sums (|err| <= 1e-5 |y| + 2e-6 sum |w_i x_i|),
    all rows within 1e-5 normwise of ouro_matvec_q."""
    rng = np.random.default_rng(41 + kind)
    out_len, in_len = 40960, 65536
    ph = lut_payload(rng, kind, out_len, in_len)
    w = DeviceBuffer.from_host(ph)
    xh = rng.standard_normal(in_len).astype(np.float32)
    x = DeviceBuffer.from_host(xh)
    want = run("ouro_matvec_q", w, kind, out_len, in_len, x).view(np.float32)
    got = run("ouro_matvec_q_noalloc", w, kind, out_len, in_len, x).view(np.float32)
    assert np.linalg.norm(got - want) <= 1e-5 * np.linalg.norm(want)
    del w
    deq = orc.dequant_tl1_row if kind == KIND_TL1 else orc.dequant_tq1_row
    t = np.stack([deq(ph, r, in_len).astype(np.float64) for r in range(256)]) * xh.astype(np.float64)
    exact, mag = t.sum(axis=1), np.abs(t).sum(axis=1)
    for y in (got[:256], want[:256]):
        assert (np.abs(y - exact) <= 1e-5 * np.abs(exact) + 2e-6 * mag).all()
