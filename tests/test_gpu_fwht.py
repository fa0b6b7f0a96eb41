"""GPU parity of the Walsh-Hadamard rotation: bit-identical fp32 to the
oracle (same butterfly stages in the same order), bf16 outputs equal after
round-to-nearest-even, fused quantisation equal to the separate path."""
import numpy as np
import pytest

from ouroboros_amd import hadamard, ops, quant
from ouroboros_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def config2_input(rng, rows=512, n=4096):
    x = rng.standard_normal((rows, n)).astype(np.float32)
    mask = rng.random((rows, n)) < 0.01
    x[mask] *= 50.0
    return x


def test_config2_bf16_bit_exact(gpu, orc):
    rng = np.random.default_rng(0)
    xb = quant.f32_to_bf16_bits(config2_input(rng))
    x32 = quant.bf16_bits_to_f32(xb)
    want = x32.copy()
    orc.rotate_rows(want, None, 4096)
    xd = DeviceBuffer.from_host(xb)
    y32 = DeviceBuffer((512, 4096), np.float32)
    hadamard.fwht_rows(xd, y32, 512, 4096, 4096)
    assert np.array_equal(y32.download().view(np.uint32), want.view(np.uint32))
    y16 = DeviceBuffer((512, 4096), np.uint16)
    hadamard.fwht_rows(xd, y16, 512, 4096, 4096)
    assert np.array_equal(y16.download(), quant.f32_to_bf16_bits(want))
    # relative error of the bf16 output vs the fp32 result: within one bf16 ulp
    rel = np.abs(quant.bf16_bits_to_f32(y16.download()) - want) / np.maximum(np.abs(want), 1e-30)
    assert rel.max() <= 2.0 ** -8


@pytest.mark.parametrize("n,block", [(16, 16), (32, 16), (64, 64), (128, 64), (192, 64), (256, 2),
                                     (512, 8), (1024, 1024), (5120, 1024), (6144, 1024),
                                     (17408, 1024), (2048, 2048), (8192, 8192), (2560, 512),
                                     (6912, 256), (4096, 32), (4096, 4096), (8192, 4096), (12288, 4096)])
@pytest.mark.parametrize("inverse", [False, True])
def test_f32_bit_exact_with_signs(gpu, orc, n, block, inverse):
    rng = np.random.default_rng(n + block)
    rows = 3
    x = rng.standard_normal((rows, n)).astype(np.float32)
    s = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    want = x.copy()
    orc.rotate_rows(want, s, block, inverse=inverse)
    xd = DeviceBuffer.from_host(x)
    yd = DeviceBuffer((rows, n), np.float32)
    hadamard.fwht_rows(xd, yd, rows, n, block, signs=DeviceBuffer.from_host(s), inverse=inverse)
    assert np.array_equal(yd.download().view(np.uint32), want.view(np.uint32))


def test_rotate_mirrors_in_place(gpu, orc):
    rng = np.random.default_rng(3)
    n, block = 5120, 1024
    x = rng.standard_normal(n).astype(np.float32)
    s = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    for fwd in (True, False):
        want = x.copy()
        (orc.rotate_fwd if fwd else orc.rotate_inv)(want, s, block)
        got = x.copy()
        (hadamard.rotate_fwd if fwd else hadamard.rotate_inv)(got, s, block)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_roundtrip_on_device(gpu):
    rng = np.random.default_rng(4)
    n, block = 2048, 1024
    x = rng.standard_normal(n).astype(np.float32)
    s = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    xd = DeviceBuffer.from_host(x)
    sd = DeviceBuffer.from_host(s)
    hadamard.rotate_inv(xd, sd, block)
    hadamard.rotate_fwd(xd, sd, block)
    assert np.abs(xd.download() - x).max() < 1e-5


@pytest.mark.parametrize("ydt", [np.uint16, np.float32])
def test_fused_quant_equals_separate(gpu, orc, ydt):
    rng = np.random.default_rng(5)
    rows, n = 64, 4096
    xb = quant.f32_to_bf16_bits(config2_input(rng, rows, n))
    xd = DeviceBuffer.from_host(xb)
    y = DeviceBuffer((rows, n), ydt)
    xq = DeviceBuffer((rows, n), np.int8)
    ds = DeviceBuffer((rows,), np.float32)
    hadamard.fwht_rows(xd, y, rows, n, 4096, xq=xq, act_scale=ds)
    stored = y.download()
    as_f32 = quant.bf16_bits_to_f32(stored) if ydt == np.uint16 else stored
    want_q, want_ds = orc.act_quant_i8(as_f32)
    assert np.array_equal(xq.download(), want_q)
    assert np.array_equal(ds.download(), want_ds)
    # quantise-only (no stored output) gives the same codes
    xq2 = DeviceBuffer((rows, n), np.int8)
    ds2 = DeviceBuffer((rows,), np.float32)
    from ouroboros_amd._lib import DT_BF16, DT_F32, call
    call("ouro_fwht_rows", xd.ptr, DT_BF16, None, DT_BF16 if ydt == np.uint16 else DT_F32, rows, n,
         4096, None, 0, xq2.ptr, ds2.ptr, None)
    assert np.array_equal(xq2.download(), want_q)


def test_check_args_errors(gpu):
    from ouroboros_amd._lib import OuroError

    xd = DeviceBuffer((24,), np.float32)
    sd = DeviceBuffer((24,), np.float32)
    with pytest.raises(OuroError) as e:
        hadamard.rotate_fwd(xd, sd, 16)  # len not a multiple of block (hadamard.rs:36)
    assert e.value.code == 2
    with pytest.raises(OuroError):
        hadamard.rotate_fwd(xd, sd, 12)  # not a power of two (hadamard.rs:35)
