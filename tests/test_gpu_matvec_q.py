"""GPU matvec_q / matmul_q on the reference kinds (TL1 = PTQ1_0, TQ1_0,
F32/F16/BF16) against the oracle restatement of ops.rs, at the reference's
own fused-vs-scalar bar (rel 1e-5) for matvec and rel 1e-3 for matmul
(ops.rs:720-750)."""
import numpy as np
import pytest

from ouroboros_amd import ops
from ouroboros_amd.quant import QuantKind

pytestmark = pytest.mark.gpu


def tl1_payload(rng, out_len, in_len):
    p = rng.integers(0, 256, out_len * (in_len // 128) * 28, dtype=np.uint8)
    g = p.reshape(-1, 28)
    d = (rng.uniform(0.01, 0.1, g.shape[0]).astype(np.float16)).view(np.uint16)
    g[:, 26], g[:, 27] = d & 0xFF, d >> 8
    return p


def tq1_payload(rng, out_len, in_len):
    p = rng.integers(0, 256, out_len * (in_len // 256) * 54, dtype=np.uint8)
    g = p.reshape(-1, 54)
    d = (rng.uniform(0.01, 0.1, g.shape[0]).astype(np.float16)).view(np.uint16)
    g[:, 52], g[:, 53] = d & 0xFF, d >> 8
    return p


def close(got, want, rtol):
    # |got - want| <= rtol * max(|want|, scale): row dot products can cancel,
    # so the tolerance floor is the row's own magnitude scale.
    scale = np.abs(want).max()
    return np.abs(got - want) <= rtol * np.maximum(np.abs(want), 1e-2 * scale) + 1e-6 * scale


def test_reference_fixture_37x384(gpu, orc):  # ops.rs:800-838 inputs
    out_len, in_len = 37, 384
    rb = in_len // 128 * 28
    i = np.arange(out_len * rb, dtype=np.uint64)
    p = ((i * (0x9B ^ (i >> 7))) & 0xFF).astype(np.uint8)
    g = p.reshape(-1, 28)
    g[:, 26], g[:, 27] = 0x10, 0x38
    x = (((np.arange(in_len) % 7) - 3.0) * 0.5).astype(np.float32)
    want = orc.matvec_tl1(p, out_len, in_len, x, simd=0)
    got = ops.matvec_q(p, QuantKind.TL1, out_len, in_len, x)
    assert (np.abs(got - want) / np.maximum(np.abs(want), 1e-9) < 1e-5).all()


@pytest.mark.parametrize("out_len,in_len", [(6912, 2560), (2560, 6912), (97, 384), (5, 128)])
def test_tl1_matvec(gpu, orc, out_len, in_len):
    rng = np.random.default_rng(out_len)
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_tl1(p, out_len, in_len, x)
    got = ops.matvec_q(p, QuantKind.TL1, out_len, in_len, x)
    assert close(got, want, 1e-5).all()


# Raw payloads of >= 8192 rows run the table-lookup kernel on the reference
# bytes (a lane per (row, group)): row pitches of 4k, 4k+2 and odd group
# counts, partial last group blocks, partial 64-row tiles, and payloads 4 or
# 8 bytes past an aligned address.
@pytest.mark.parametrize("out_len,in_len,offset", [(8192, 512, 0), (8209, 2560, 0), (8195, 6912, 0),
                                                   (8250, 384, 0), (8500, 640, 0), (8257, 1024, 4),
                                                   (8192, 5120, 8)])
def test_tl1_matvec_raw_lookup(gpu, orc, out_len, in_len, offset):
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(out_len + in_len + offset)
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_tl1(p, out_len, in_len, x)
    buf = DeviceBuffer((p.size + 16,), np.uint8)
    from ouroboros_amd._lib import call
    call("ouro_memcpy_htod", buf.ptr + offset, p.ctypes.data, p.size)
    xd, y = DeviceBuffer.from_host(x), DeviceBuffer((out_len,), np.float32)
    call("ouro_matvec_q", buf.ptr + offset, int(QuantKind.TL1), out_len, in_len, xd.ptr, y.ptr, None)
    assert close(y.download(), want, 1e-5).all()
    # the allocation-free entry takes the direct kernel; same tolerance
    call("ouro_matvec_q_noalloc", buf.ptr + offset, int(QuantKind.TL1), out_len, in_len, xd.ptr, y.ptr, None)
    assert close(y.download(), want, 1e-5).all()


# TQ1_0 payloads of >= 8192 rows with an even block count per row on a
# 4-byte-aligned address run the table-lookup kernel (a lane per (row,
# block), odd blocks realigned by 2 bytes); odd block counts, a payload 2
# bytes past a dword and the allocation-free entry take the direct kernel.
@pytest.mark.parametrize("out_len,in_len,offset", [(8192, 512, 0), (8209, 5120, 0), (8257, 2560, 4),
                                                   (9001, 1024, 8), (8500, 768, 0), (8193, 1024, 2)])
def test_tq1_matvec_raw_lookup(gpu, orc, out_len, in_len, offset):
    from ouroboros_amd._lib import call
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(out_len + in_len + offset)
    p = tq1_payload(rng, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, orc.KIND_TQ1_0, out_len, in_len, x)
    buf = DeviceBuffer((p.size + 16,), np.uint8)
    call("ouro_memcpy_htod", buf.ptr + offset, p.ctypes.data, p.size)
    xd, y = DeviceBuffer.from_host(x), DeviceBuffer((out_len,), np.float32)
    for entry in ("ouro_matvec_q", "ouro_matvec_q_noalloc"):
        call(entry, buf.ptr + offset, int(QuantKind.TQ1_0), out_len, in_len, xd.ptr, y.ptr, None)
        assert close(y.download(), want, 1e-5).all(), entry


def test_tq1_handle_lookup_and_argmax(gpu, orc):
    # a resident TQ1_0 weight of >= 8192 rows: matvec, 3 columns and the greedy sample
    rng = np.random.default_rng(77)
    out_len, in_len = 9000, 2048
    p = tq1_payload(rng, out_len, in_len)
    h = ops.Weight(QuantKind.TQ1_0, p, out_len, in_len)
    x = rng.standard_normal(3 * in_len).astype(np.float32)
    want = np.concatenate([orc.matvec_q(p, orc.KIND_TQ1_0, out_len, in_len, x[c * in_len:(c + 1) * in_len])
                           for c in range(3)])
    assert close(h.matvec(x[:in_len]), want[:out_len], 1e-5).all()
    # 3 columns: one int8 MFMA pass (the handle holds max_cols = 8), the K-column bar (ops.rs:720-750)
    assert close(h.matmul(x, 3), want, 1e-3).all()
    idx = h.matvec_argmax(x[:in_len])
    best = orc.finite_argmax(want[:out_len])
    assert idx == best or abs(float(want[idx]) - float(want[best])) <= 1e-5 * abs(float(want[best]))
    h.free()


@pytest.mark.parametrize("k", [1, 3, 4, 8, 11])
def test_tl1_matmul_column_major(gpu, orc, k):
    rng = np.random.default_rng(k)
    out_len, in_len = 97, 384
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    want = orc.matmul_tl1(p, out_len, in_len, x, k)
    got = ops.matmul_q(p, QuantKind.TL1, out_len, in_len, x, k)
    assert got.shape == (k * out_len,)
    assert close(got, want, 1e-3).all()


@pytest.mark.parametrize("out_len,in_len", [(2560, 2560), (33, 512), (7, 256)])
def test_tq1_matvec(gpu, orc, out_len, in_len):
    rng = np.random.default_rng(in_len)
    p = tq1_payload(rng, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, orc.KIND_TQ1_0, out_len, in_len, x)
    got = ops.matvec_q(p, QuantKind.TQ1_0, out_len, in_len, x)
    assert close(got, want, 1e-5).all()
    got2 = ops.matmul_q(p, QuantKind.TQ1_0, out_len, in_len, np.concatenate([x, -x]), 2)
    assert close(got2[:out_len], want, 1e-5).all() and close(got2[out_len:], -want, 1e-5).all()


@pytest.mark.parametrize("kind", [QuantKind.F32, QuantKind.F16, QuantKind.BF16])
def test_dense_matvec(gpu, orc, kind):
    rng = np.random.default_rng(int(kind))
    out_len, in_len = 300, 1000
    w = rng.standard_normal((out_len, in_len)).astype(np.float32)
    if kind == QuantKind.F32:
        payload = w.view(np.uint8).reshape(-1)
    elif kind == QuantKind.F16:
        payload = w.astype(np.float16).view(np.uint8).reshape(-1)
    else:
        payload = (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(payload, int(kind), out_len, in_len, x)
    got = ops.matvec_q(payload, kind, out_len, in_len, x)
    assert close(got, want, 1e-4).all()


def test_weight_handle_tl1(gpu, orc):
    rng = np.random.default_rng(2)
    out_len, in_len = 512, 2560
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(3 * in_len).astype(np.float32)
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len)
    want = orc.matmul_tl1(p, out_len, in_len, x, 3)
    assert close(h.matmul(x, 3), want, 1e-3).all()
    h.free()


def test_kind_errors(gpu):
    from ouroboros_amd._lib import OuroError

    with pytest.raises(OuroError) as e:
        ops.matvec_q(np.zeros(64, np.uint8), 10, 1, 256, np.zeros(256, np.float32))  # Q2_K: not a reference kind
    assert e.value.code == 4
    with pytest.raises(OuroError) as e:
        ops.matvec_q(np.zeros(64, np.uint8), QuantKind.TL1, 1, 100, np.zeros(100, np.float32))
    assert e.value.code == 2
