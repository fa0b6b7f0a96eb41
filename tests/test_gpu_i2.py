"""GPU parity of the I2 path (int8 absmax activations x 2-bit ternary):
bit-exact against the oracle for tiling, quantisation, int32 sums and the
fp32 epilogue."""
import numpy as np
import pytest

from ouroboros_amd import ops, quant
from ouroboros_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def make_case(rng, out_len, in_len, ncols=1):
    w = rng.integers(-1, 2, size=(out_len, in_len)).astype(np.int8)
    x = rng.standard_normal((ncols, in_len)).astype(np.float32)
    w_scale = np.float32(rng.uniform(0.5, 2.0))
    return w, x, w_scale


@pytest.mark.parametrize("out_len,in_len", [(6912, 2560), (2560, 6912), (37, 256), (100, 512),
                                             (64, 1024), (33, 2048), (16, 4096), (24, 5120),
                                             (10, 3072), (8, 6144), (4, 8192)])
def test_tile_matches_oracle(gpu, orc, out_len, in_len):
    rng = np.random.default_rng(out_len + in_len)
    canon = orc.i2_pack(rng.integers(-1, 2, size=(out_len, in_len)).astype(np.int8))
    payload = ops.i2_payload(canon, out_len, in_len, 1.5)
    tb = ops.i2_tiled_bytes(out_len, in_len)
    got = payload.download()
    assert np.array_equal(got[:tb], orc.i2_tile(canon, out_len, in_len))
    assert got[tb:tb + 4].view(np.float32)[0] == np.float32(1.5)


@pytest.mark.parametrize("rows,n", [(1, 2560), (7, 2560), (512, 4096), (3, 6912), (2, 100)])
@pytest.mark.parametrize("bf16", [False, True])
def test_act_quant_matches_oracle(gpu, orc, rows, n, bf16):
    rng = np.random.default_rng(rows * n)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    x[0, : min(n, 8)] = [0.5, -0.5, 1.5, 2.5, 127.0, -3.0, 0.0, 1e-3][: min(n, 8)]  # ties, outlier
    if rows > 2:
        x[2] = 0.0  # all-zero row
    if bf16:
        xb = quant.f32_to_bf16_bits(x)
        x = quant.bf16_bits_to_f32(xb)
        xd = DeviceBuffer.from_host(xb)
    else:
        xd = DeviceBuffer.from_host(x)
    xq = DeviceBuffer((rows, n), np.int8)
    ds = DeviceBuffer((rows,), np.float32)
    ops.act_quant_i8(xd, rows, n, xq, ds)
    want_q, want_ds = orc.act_quant_i8(x)
    assert np.array_equal(xq.download(), want_q)
    assert np.array_equal(ds.download().view(np.uint32), want_ds.view(np.uint32))


@pytest.mark.parametrize("out_len,in_len,ncols", [(6912, 2560, 1), (2560, 6912, 1), (6912, 2560, 3),
                                                  (6912, 2560, 8), (37, 256, 1), (1000, 1024, 5),
                                                  (130, 5120, 2), (17, 6144, 1), (9, 8192, 4),
                                                  (251, 2048, 1), (3, 4096, 2)])
def test_gemm_i2_bit_exact(gpu, orc, out_len, in_len, ncols):
    rng = np.random.default_rng(out_len * 7 + in_len + ncols)
    w, x, w_scale = make_case(rng, out_len, in_len, ncols)
    canon = orc.i2_pack(w)
    xq_h, ds_h = orc.act_quant_i8(x)
    want_acc, want_y = orc.gemm_i2(canon, out_len, in_len, xq_h, ds_h, w_scale)
    payload = ops.i2_payload(canon, out_len, in_len, float(w_scale))
    xq = DeviceBuffer.from_host(xq_h)
    ds = DeviceBuffer.from_host(ds_h)
    y = DeviceBuffer((ncols * out_len,), np.float32)
    acc = DeviceBuffer((ncols * out_len,), np.int32)
    ops.gemm_i2(payload, out_len, in_len, xq, ds, ncols, y, acc)
    assert np.array_equal(acc.download(), want_acc)
    assert np.array_equal(y.download().view(np.uint32), want_y.view(np.uint32))


def test_gemm_extremes(gpu, orc):
    # All +1 weights with all +127 activations: the largest sums; all -1 too.
    out_len, in_len = 48, 6144
    for wv in (1, -1):
        w = np.full((out_len, in_len), wv, np.int8)
        xq_h = np.full((1, in_len), 127, np.int8)
        ds_h = np.array([1.0], np.float32)
        payload = ops.i2_payload(orc.i2_pack(w), out_len, in_len, 1.0)
        y = DeviceBuffer((out_len,), np.float32)
        acc = DeviceBuffer((out_len,), np.int32)
        ops.gemm_i2(payload, out_len, in_len, DeviceBuffer.from_host(xq_h), DeviceBuffer.from_host(ds_h), 1, y, acc)
        assert (acc.download() == wv * 127 * in_len).all()


# (4096, 1024, 8) and (40001, 256, 1) reach 4096 tiles, where in_len <= 1024
# takes two tiles per wavefront; 40001 rows end in a wavefront whose second
# tile lies past the last one.
@pytest.mark.parametrize("out_len,in_len,count", [(6912, 2560, 4), (2560, 6912, 3), (4096, 1024, 8),
                                                  (40001, 256, 1), (1000, 512, 2)])
def test_grouped_gemv_bit_exact(gpu, orc, out_len, in_len, count):
    from ouroboros_amd._lib import call

    rng = np.random.default_rng(5 + out_len + count)
    tb = ops.i2_tiled_bytes(out_len, in_len)
    stride = tb + 256
    wbuf = DeviceBuffer((count * stride,), np.uint8)
    scales = np.empty(count, np.float32)
    xs = np.empty((count, in_len), np.int8)
    dss = np.empty(count, np.float32)
    wants = []
    for m in range(count):
        w, x, sc = make_case(rng, out_len, in_len)
        canon = orc.i2_pack(w)
        p = ops.i2_payload(canon, out_len, in_len, float(sc))
        call("ouro_memcpy_dtod", wbuf.ptr + m * stride, p.ptr, tb, None)
        xq_h, ds_h = orc.act_quant_i8(x)
        xs[m], dss[m], scales[m] = xq_h[0], ds_h[0], sc
        wants.append(orc.gemm_i2(canon, out_len, in_len, xq_h, ds_h, sc)[1])
    y = DeviceBuffer((count, out_len), np.float32)
    # keep every buffer referenced until the kernel has finished
    sc_d, xs_d, ds_d = (DeviceBuffer.from_host(a) for a in (scales, xs, dss))
    call("ouro_gemv_i2_grouped", wbuf.ptr, stride, sc_d.ptr, xs_d.ptr, in_len, ds_d.ptr, y.ptr,
         out_len, out_len, in_len, count, None)
    got = y.download()
    for m in range(count):
        assert np.array_equal(got[m].view(np.uint32), wants[m].view(np.uint32))


def test_matvec_q_i2_and_weight_handle(gpu, orc):
    rng = np.random.default_rng(8)
    out_len, in_len = 6912, 2560
    w, x, sc = make_case(rng, out_len, in_len, 2)
    canon = orc.i2_pack(w)
    xq_h, ds_h = orc.act_quant_i8(x)
    want = orc.gemm_i2(canon, out_len, in_len, xq_h, ds_h, sc)[1]
    payload = ops.i2_payload(canon, out_len, in_len, float(sc))
    y1 = ops.matvec_q(payload, ops.QuantKind.I2, out_len, in_len, x[0])
    assert np.array_equal(y1, want[:out_len])
    y2 = ops.matmul_q(payload, ops.QuantKind.I2, out_len, in_len, x.reshape(-1), 2)
    assert np.array_equal(y2, want)
    h = ops.Weight(ops.QuantKind.I2, canon, out_len, in_len, float(sc), max_cols=2)
    assert np.array_equal(h.matmul(x.reshape(-1), 2), want)
    assert np.array_equal(h.matvec(x[1]), want[out_len:])
    h.free()


def test_shape_errors_are_status_codes(gpu):
    from ouroboros_amd._lib import OuroError, call

    buf = DeviceBuffer((1024,), np.uint8)
    with pytest.raises(OuroError) as e:
        call("ouro_gemm_i2", buf.ptr, 8, 300, buf.ptr, buf.ptr, buf.ptr, 1, buf.ptr, None, None)
    assert e.value.code == 2  # in_len % 256 != 0
    with pytest.raises(OuroError) as e:
        call("ouro_gemm_i2", buf.ptr + 1, 8, 256, buf.ptr, buf.ptr, buf.ptr, 1, buf.ptr, None, None)
    assert e.value.code == 3  # misaligned weights
    with pytest.raises(OuroError) as e:
        call("ouro_gemm_i2", buf.ptr, 8, 256, buf.ptr, buf.ptr + 4, buf.ptr, 1, buf.ptr, None, None)
    assert e.value.code == 3  # activations must be 16-byte aligned
