"""ouro_matvec_q_noalloc (static per-device scratch, no allocation) against
ouro_matvec_q, bit for bit, on two calls in a row with the second smaller,
for both 2-bit kinds; plus its size limit and a kind that uses no scratch."""
import numpy as np
import pytest

from ouroboros_amd import ops, quant
from ouroboros_amd._lib import KIND_F32, KIND_I2, KIND_I2_S, OuroError, call
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
