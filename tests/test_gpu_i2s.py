"""bitnet.cpp's int8-activation x 2-bit ternary contract on the GPU: I2_S
tensors (raw, and repacked on upload) with I8_S activations, bit-exact vs
the oracle (quantisation, int32 sums and the fp32 epilogue), at the
6912x2560 / 2560x6912 layer shapes and at every raw-kernel shape class.

The oracle's I2_S / I8_S functions are this repository's transcription of
the published bitnet.cpp source (src/ggml-bitnet-mad.cpp); the reference's
bitnet-cpp submodule is empty, so no output of bitnet.cpp itself (and no
reference fixture) backs them.  Their rules are pinned by hand-made vectors
in tests/test_oracle_i2.py, not by bitnet.cpp runs."""
import numpy as np
import pytest

from ouroboros_amd import ops, quant
from ouroboros_amd._lib import OuroError
from ouroboros_amd.device import DeviceBuffer
from ouroboros_amd.quant import QuantKind

pytestmark = pytest.mark.gpu


def layer(rng, out_len, in_len, ncols=1):
    """Trits i.i.d. with p = 1/3 each, w_scale ~ U(0.5, 2), x ~ N(0, 1)."""
    w = rng.integers(-1, 2, size=(out_len, in_len)).astype(np.int8)
    w_scale = np.float32(rng.uniform(0.5, 2.0))
    x = rng.standard_normal((ncols, in_len)).astype(np.float32)
    return w, w_scale, x


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("out_len,in_len", [(6912, 2560), (2560, 6912), (37, 256), (17, 5120), (9, 8192)])
def test_i2s_repack_matches_oracle(gpu, orc, out_len, in_len):
    rng = np.random.default_rng(out_len + 3 * in_len)
    w, sc, _ = layer(rng, out_len, in_len)
    i2s = quant.i2s_pack(w, sc)
    assert np.array_equal(i2s, orc.i2s_pack(w, sc))
    canon = orc.i2s_to_canonical(i2s, out_len, in_len)
    tb = ops.i2_tiled_bytes(out_len, in_len)
    got = ops.i2s_payload(i2s, out_len, in_len).download()
    assert np.array_equal(got[:tb], orc.i2_tile(canon, out_len, in_len))
    assert got[tb:tb + 4].view(np.float32)[0] == sc
    mb = ops.i2_mfma_bytes(out_len, in_len)
    got = ops.i2s_mfma_payload(i2s, out_len, in_len).download()
    assert np.array_equal(got[:mb], orc.i2_tile_mfma(canon, out_len, in_len))
    assert got[mb:mb + 4].view(np.float32)[0] == sc


def test_act_quant_i8s_known_answers(gpu):
    rows = np.zeros((4, 256), np.float32)
    rows[0, :8] = [127.0, 0.5, 1.5, 2.5, -0.5, -2.5, 0.0, 0.49]  # s = 1: exact ties, away from zero
    rows[2, :2] = [1e-6, -3e-6]                                    # below the 1e-5 amax floor
    rows[3, :3] = [-3.0, 1.0, 3.0]                                 # s = (float)(127 / 3)
    xq = DeviceBuffer((4, 256), np.int8)
    s = DeviceBuffer((4,), np.float32)
    ops.act_quant_i8(DeviceBuffer.from_host(rows), 4, 256, xq, s)
    q, s = xq.download(), s.download()
    assert list(q[0, :8]) == [127, 1, 2, 3, -1, -3, 0, 0] and s[0] == 1.0
    assert not q[1].any() and s[1] == np.float32(12700000.0)
    assert list(q[2, :2]) == [13, -38] and s[2] == np.float32(12700000.0)
    assert list(q[3, :3]) == [-127, 42, 127] and bits(s[3:4])[0] == 0x42295555


@pytest.mark.parametrize("out_len,in_len", [(6912, 2560), (2560, 6912)])
def test_config_layer_bit_exact(gpu, orc, out_len, in_len):
    """The 6912x2560 layer (and its transpose) end to end: raw I2_S, resident handle, repack."""
    rng = np.random.default_rng(20261202 + in_len)
    w, sc, x = layer(rng, out_len, in_len, 2)
    i2s = quant.i2s_pack(w, sc)
    xq_h, s_h = orc.act_quant_i8(x)
    want_acc, want_y = orc.gemm_i2s(i2s, out_len, in_len, xq_h, s_h)
    # quantisation on the GPU
    xq, s = DeviceBuffer((2, in_len), np.int8), DeviceBuffer((2,), np.float32)
    ops.act_quant_i8(DeviceBuffer.from_host(x), 2, in_len, xq, s)
    assert np.array_equal(xq.download(), xq_h) and np.array_equal(bits(s.download()), bits(s_h))
    # raw tensor through matvec_q / matmul_q
    y = ops.matvec_q(i2s, QuantKind.I2_S, out_len, in_len, x[0])
    assert np.array_equal(bits(y), bits(want_y[:out_len]))
    y = ops.matmul_q(i2s, QuantKind.I2_S, out_len, in_len, x.reshape(-1), 2)
    assert np.array_equal(bits(y), bits(want_y))
    # repacked payload: exact sums and outputs
    p = ops.i2s_payload(i2s, out_len, in_len)
    yd, acc = DeviceBuffer((2 * out_len,), np.float32), DeviceBuffer((2 * out_len,), np.int32)
    ops.gemm_i2(p, out_len, in_len, xq, s, 2, yd, acc)
    assert np.array_equal(acc.download(), want_acc)
    assert np.array_equal(bits(yd.download()), bits(want_y))
    # resident handle (GEMV and, with max_cols >= 8, the MFMA GEMM)
    h = ops.Weight(QuantKind.I2_S, i2s, out_len, in_len, max_cols=16)
    assert np.array_equal(bits(h.matvec(x[0])), bits(want_y[:out_len]))
    x16 = rng.standard_normal((16, in_len)).astype(np.float32)
    q16, s16 = orc.act_quant_i8(x16)
    assert np.array_equal(bits(h.matmul(x16.reshape(-1), 16)), bits(orc.gemm_i2s(i2s, out_len, in_len, q16, s16)[1]))
    h.free()


# in_len sets the raw kernel's chunk sets per lane (1..8) and its rows per
# wavefront (8, 4, 2); odd row counts leave partial wavefronts.
@pytest.mark.parametrize("out_len,in_len,ncols", [(37, 256, 1), (100, 2560, 2), (33, 4096, 1), (21, 5120, 3),
                                                  (13, 8192, 1), (11, 12288, 2), (9, 16384, 1), (7, 20480, 1),
                                                  (5, 24576, 2), (6, 28672, 1), (3, 32768, 1), (4097, 1024, 1)])
def test_raw_i2s_shapes(gpu, orc, out_len, in_len, ncols):
    rng = np.random.default_rng(out_len * 31 + in_len + ncols)
    w, sc, x = layer(rng, out_len, in_len, ncols)
    i2s = quant.i2s_pack(w, sc)
    xq_h, s_h = orc.act_quant_i8(x)
    want = orc.gemm_i2s(i2s, out_len, in_len, xq_h, s_h)[1]
    got = ops.matmul_q(i2s, QuantKind.I2_S, out_len, in_len, x.reshape(-1), ncols)
    assert np.array_equal(bits(got), bits(want))


def test_raw_i2s_extremes(gpu, orc):
    # all codes 2 (or 0) against q = 127: the largest sums, exact in int32
    out_len, in_len = 16, 16384
    x = np.full((1, in_len), 3.0, np.float32)  # s = 127 / 3, q = 127
    for wv in (1, -1):
        i2s = quant.i2s_pack(np.full((out_len, in_len), wv, np.int8), 1.0)
        xq_h, s_h = orc.act_quant_i8(x)
        acc, want = orc.gemm_i2s(i2s, out_len, in_len, xq_h, s_h)
        assert (acc == wv * 127 * in_len).all()
        got = ops.matvec_q(i2s, QuantKind.I2_S, out_len, in_len, x[0])
        assert np.array_equal(bits(got), bits(want))


def test_i2s_upload_sizes(gpu):
    w = np.zeros((8, 256), np.int8)
    b = quant.i2s_pack(w, 1.0)  # 512 code bytes + 32
    for n in (512 + 4, 512 + 32):
        ops.Weight(QuantKind.I2_S, b[:n], 8, 256).free()
    for n in (512 + 3, 512 + 33):
        with pytest.raises(OuroError) as e:
            ops.Weight(QuantKind.I2_S, np.resize(b, n), 8, 256)
        assert e.value.code == 2
    with pytest.raises(OuroError) as e:
        ops.matvec_q(np.zeros(64 * 300 // 4 + 32, np.uint8), QuantKind.I2_S, 64, 300, np.zeros(300, np.float32))
    assert e.value.code == 2  # in_len % 256 != 0
