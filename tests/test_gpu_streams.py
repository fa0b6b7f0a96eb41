"""Calls issued on two streams share no scratch: the library workspace (raw
TL1 matvec_q of >= 8192 rows keeps its partial sums there), a weight
handle's per-stream sets (TL1 lookup partials, I2 activation codes) and the
finite_argmax key slots are each kept per stream, so work queued on two
streams without any wait between them gives each stream's results exactly as
the same calls run alone."""
import numpy as np
import pytest

from ouroboros_amd import ops
from ouroboros_amd._lib import KIND_TL1, call
from ouroboros_amd.device import DeviceBuffer, Stream, synchronize
from ouroboros_amd.quant import QuantKind, i2_pack

pytestmark = pytest.mark.gpu


def tl1_payload(rng, out_len, in_len):
    p = rng.integers(0, 256, out_len * (in_len // 128) * 28, dtype=np.uint8)
    g = p.reshape(-1, 28)
    d = rng.uniform(0.01, 0.1, g.shape[0]).astype(np.float16).view(np.uint16)
    g[:, 26], g[:, 27] = d & 0xFF, d >> 8
    return p


def test_two_streams_raw_tl1_and_handles(gpu):
    rng = np.random.default_rng(5)
    out_len, in_len = 16384, 2048  # >= 8192 rows: the lookup kernel with workspace partials
    p = tl1_payload(rng, out_len, in_len)
    xs = [rng.standard_normal(in_len).astype(np.float32) for _ in range(2)]
    pd = DeviceBuffer.from_host(p)
    xd = [DeviceBuffer.from_host(x) for x in xs]
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len)
    # I2 handle (activation codes in the handle's scratch)
    w = rng.integers(-1, 2, size=(1024, 2560)).astype(np.int8)
    hi2 = ops.Weight(QuantKind.I2, i2_pack(w), 1024, 2560, w_scale=0.7, max_cols=2)
    xi = [DeviceBuffer.from_host(rng.standard_normal(2560).astype(np.float32)) for _ in range(2)]

    def run(stream, i, ys):
        call("ouro_matvec_q", pd.ptr, KIND_TL1, out_len, in_len, xd[i].ptr, ys[0].ptr, stream)
        call("ouro_weight_matvec", h.handle, xd[i].ptr, ys[1].ptr, stream)
        call("ouro_weight_matvec", hi2.handle, xi[i].ptr, ys[2].ptr, stream)
        call("ouro_finite_argmax", ys[0].ptr, out_len, ys[3].ptr, stream)

    def outs():
        return [DeviceBuffer((out_len,), np.float32), DeviceBuffer((out_len,), np.float32),
                DeviceBuffer((1024,), np.float32), DeviceBuffer((1,), np.int32)]

    # each stream's calls alone, on the null stream
    alone = []
    for i in range(2):
        ys = outs()
        run(None, i, ys)
        synchronize()
        alone.append([y.download() for y in ys])
    # both streams at once, several rounds queued back to back with no waits
    streams = [Stream(), Stream()]
    ys = [outs(), outs()]
    for _ in range(4):
        run(streams[0].handle, 0, ys[0])
        run(streams[1].handle, 1, ys[1])
    streams[0].synchronize()
    streams[1].synchronize()
    for i in range(2):
        for got, want in zip(ys[i], alone[i]):
            assert np.array_equal(got.download(), want)
    assert alone[0][3][0] == int(np.argmax(alone[0][0]))
    for s in streams:
        call("ouro_stream_destroy", s.handle)
        s.handle = None
