"""Ternary x int8 GEMM on int8 MFMA (ouro_gemm_i2_mfma): bit-exact against
the oracle's int32 GEMM for any column count, and identical to the GEMV."""
import numpy as np
import pytest

from ouroboros_amd import ops
from ouroboros_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def make_case(rng, out_len, in_len, ncols):
    w = rng.integers(-1, 2, size=(out_len, in_len)).astype(np.int8)
    x = rng.standard_normal((ncols, in_len)).astype(np.float32)
    return w, x, np.float32(rng.uniform(0.5, 2.0))


@pytest.mark.parametrize("out_len,in_len", [(6912, 2560), (2560, 6912), (37, 256), (100, 512), (17, 5120)])
def test_tile_mfma_matches_oracle(gpu, orc, out_len, in_len):
    rng = np.random.default_rng(out_len * 3 + in_len)
    canon = orc.i2_pack(rng.integers(-1, 2, size=(out_len, in_len)).astype(np.int8))
    payload = ops.i2_mfma_payload(canon, out_len, in_len, 1.25)
    tb = ops.i2_mfma_bytes(out_len, in_len)
    got = payload.download()
    assert np.array_equal(got[:tb], orc.i2_tile_mfma(canon, out_len, in_len))
    assert got[tb:tb + 4].view(np.float32)[0] == np.float32(1.25)


# Column counts cover every launch shape (<= 16, <= 32, > 32 columns; few
# columns on tall weights; 256 x 128 tiles) and partial column and row tiles.
@pytest.mark.parametrize("out_len,in_len,ncols", [(6912, 2560, 1), (6912, 2560, 16), (6912, 2560, 100),
                                                  (2560, 6912, 33), (37, 256, 5), (1000, 1024, 64),
                                                  (130, 5120, 17), (17, 768, 300), (4096, 4096, 256),
                                                  (8, 2048, 2), (4000, 256, 3000), (4002, 256, 3000),
                                                  (12000, 512, 40), (66000, 256, 20)])
def test_gemm_i2_mfma_bit_exact(gpu, orc, out_len, in_len, ncols):
    rng = np.random.default_rng(out_len * 5 + in_len + ncols)
    w, x, w_scale = make_case(rng, out_len, in_len, ncols)
    canon = orc.i2_pack(w)
    xq_h, ds_h = orc.act_quant_i8(x)
    want_acc, want_y = orc.gemm_i2(canon, out_len, in_len, xq_h, ds_h, w_scale)
    payload = ops.i2_mfma_payload(canon, out_len, in_len, float(w_scale))
    xq, ds = DeviceBuffer.from_host(xq_h), DeviceBuffer.from_host(ds_h)
    y = DeviceBuffer((ncols * out_len,), np.float32)
    acc = DeviceBuffer((ncols * out_len,), np.int32)
    ops.gemm_i2_mfma(payload, out_len, in_len, xq, ds, ncols, y, acc)
    assert np.array_equal(acc.download(), want_acc.reshape(-1))
    assert np.array_equal(y.download().view(np.uint32), want_y.reshape(-1).view(np.uint32))


@pytest.mark.parametrize("out_len,ncols", [(4000, 3000), (2560, 4096)])
def test_gemm_i2_mfma_large_no_acc(gpu, orc, out_len, ncols):
    # 256 x 128 workgroup tiles (partial row and column tiles in the first
    # case) storing y four rows at a time, which the int32 output turns off
    rng = np.random.default_rng(out_len + ncols)
    in_len = 512
    w, x, w_scale = make_case(rng, out_len, in_len, ncols)
    canon = orc.i2_pack(w)
    xq_h, ds_h = orc.act_quant_i8(x)
    _, want_y = orc.gemm_i2(canon, out_len, in_len, xq_h, ds_h, w_scale)
    payload = ops.i2_mfma_payload(canon, out_len, in_len, float(w_scale))
    y = DeviceBuffer((ncols * out_len,), np.float32)
    ops.gemm_i2_mfma(payload, out_len, in_len, DeviceBuffer.from_host(xq_h), DeviceBuffer.from_host(ds_h), ncols, y)
    assert np.array_equal(y.download().view(np.uint32), want_y.reshape(-1).view(np.uint32))


def test_gemm_i2_mfma_extremes(gpu, orc):
    # all +1 or all -1 weights against all-127 activations: |acc| = 127 * in_len
    out_len, in_len, ncols = 48, 6912, 20
    xq = DeviceBuffer.from_host(np.full((ncols, in_len), 127, np.int8))
    ds = DeviceBuffer.from_host(np.ones(ncols, np.float32))
    for wv in (1, -1):
        canon = orc.i2_pack(np.full((out_len, in_len), wv, np.int8))
        payload = ops.i2_mfma_payload(canon, out_len, in_len, 1.0)
        y = DeviceBuffer((ncols * out_len,), np.float32)
        acc = DeviceBuffer((ncols * out_len,), np.int32)
        ops.gemm_i2_mfma(payload, out_len, in_len, xq, ds, ncols, y, acc)
        assert (acc.download() == wv * 127 * in_len).all()


def test_gemm_i2_mfma_matches_gemv_path(gpu, orc):
    # the same columns through the tiled GEMV layout and the MFMA layout
    rng = np.random.default_rng(11)
    out_len, in_len, ncols = 2560, 2560, 8
    w, x, w_scale = make_case(rng, out_len, in_len, ncols)
    canon = orc.i2_pack(w)
    xq_h, ds_h = orc.act_quant_i8(x)
    xq, ds = DeviceBuffer.from_host(xq_h), DeviceBuffer.from_host(ds_h)
    y1 = DeviceBuffer((ncols * out_len,), np.float32)
    y2 = DeviceBuffer((ncols * out_len,), np.float32)
    ops.gemm_i2(ops.i2_payload(canon, out_len, in_len, float(w_scale)), out_len, in_len, xq, ds, ncols, y1)
    ops.gemm_i2_mfma(ops.i2_mfma_payload(canon, out_len, in_len, float(w_scale)), out_len, in_len, xq, ds, ncols,
                     y2)
    assert np.array_equal(y1.download().view(np.uint32), y2.download().view(np.uint32))


def test_gemm_i2_mfma_errors(gpu):
    from ouroboros_amd._lib import OuroError, call

    buf = DeviceBuffer((4096,), np.uint8)
    with pytest.raises(OuroError) as e:
        call("ouro_gemm_i2_mfma", buf.ptr, 8, 300, buf.ptr, buf.ptr, buf.ptr, 1, buf.ptr, None, None)
    assert e.value.code == 2  # in_len % 256 != 0
    with pytest.raises(OuroError) as e:
        call("ouro_gemm_i2_mfma", buf.ptr, 8, 256, buf.ptr, buf.ptr + 8, buf.ptr, 1, buf.ptr, None, None)
    assert e.value.code == 3  # activations must be 16-byte aligned
    with pytest.raises(OuroError) as e:
        call("ouro_gemm_i2_mfma", buf.ptr, 8, 256, buf.ptr, buf.ptr, buf.ptr, 0, buf.ptr, None, None)
    assert e.value.code == 1  # no columns


@pytest.mark.parametrize("k", [1, 7, 8, 40])
def test_weight_handle_matmul_uses_either_path_bit_exact(gpu, orc, k):
    # a handle uploaded for up to 64 columns: k < 8 runs the multi-column
    # GEMV, k >= 8 the MFMA GEMM; both match the oracle bit for bit
    rng = np.random.default_rng(k)
    out_len, in_len = 1000, 2560
    w, x, w_scale = make_case(rng, out_len, in_len, k)
    canon = orc.i2_pack(w)
    xq_h, ds_h = orc.act_quant_i8(x)
    want = orc.gemm_i2(canon, out_len, in_len, xq_h, ds_h, w_scale)[1].reshape(-1)
    h = ops.Weight(ops.QuantKind.I2, canon, out_len, in_len, float(w_scale), max_cols=64)
    got = h.matmul(x.reshape(-1), k)
    h.free()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
