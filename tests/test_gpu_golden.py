"""The HIP path against the committed golden fixtures: bit-exact where the
path is exact (I2_S / I8_S, FWHT), within the stated tolerances elsewhere."""
from pathlib import Path

import numpy as np
import pytest

from ouroboros_amd import hadamard, ops, qwen35
from ouroboros_amd.device import DeviceBuffer
from ouroboros_amd.quant import QuantKind

pytestmark = pytest.mark.gpu
G = Path(__file__).resolve().parent / "golden"


def test_tl1_golden(gpu):
    f = np.load(G / "tl1_matvec_37x384.npz")
    y = ops.matvec_q(f["payload"], QuantKind.TL1, int(f["out_len"]), int(f["in_len"]), f["x"])
    assert (np.abs(y - f["y_scalar"]) / np.maximum(np.abs(f["y_scalar"]), 1e-9) < 1e-5).all()


def test_i2s_golden(gpu):
    f = np.load(G / "i2s_gemm_40x512x3.npz")
    p = ops.i2s_payload(f["i2s"], 40, 512)
    assert np.array_equal(p.download()[: f["tiled"].size], f["tiled"])
    xd = DeviceBuffer.from_host(f["x"])
    xq = DeviceBuffer((3, 512), np.int8)
    s = DeviceBuffer((3,), np.float32)
    ops.act_quant_i8(xd, 3, 512, xq, s)
    y = DeviceBuffer((3 * 40,), np.float32)
    acc = DeviceBuffer((3 * 40,), np.int32)
    ops.gemm_i2(p, 40, 512, xq, s, 3, y, acc)
    assert np.array_equal(xq.download(), f["xq"])
    assert np.array_equal(s.download().view(np.uint32), f["act_scale"].view(np.uint32))
    assert np.array_equal(acc.download(), f["acc"])
    assert np.array_equal(y.download().view(np.uint32), f["y"].view(np.uint32))
    # the raw I2_S tensor through matmul_q gives the same bits
    y2 = ops.matmul_q(f["i2s"], QuantKind.I2_S, 40, 512, f["x"], 3)
    assert np.array_equal(y2.view(np.uint32), f["y"].view(np.uint32))


def test_hadamard_golden(gpu):
    f = np.load(G / "hadamard.npz")
    a = f["fwd_x"].copy()
    hadamard.rotate_fwd(a, f["fwd_signs"], 16)
    assert np.array_equal(a.view(np.uint32), f["fwd_y"].view(np.uint32))
    b = f["inv_x"].copy()
    hadamard.rotate_inv(b, f["inv_signs"], 16)
    assert np.array_equal(b.view(np.uint32), f["inv_y"].view(np.uint32))
    xd = DeviceBuffer.from_host(f["rows_x_bf16"])
    y16 = DeviceBuffer((2, 4096), np.uint16)
    hadamard.fwht_rows(xd, y16, 2, 4096, 4096)
    assert np.array_equal(y16.download(), f["rows_y_bf16"])


def rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


def test_gdn_golden(gpu):
    f = np.load(G / "gdn_decode_b1.npz")
    sd = DeviceBuffer.from_host(f["state"])
    out = DeviceBuffer((1, 2, 128), np.float32)
    qwen35.gdn_decode(sd, *(DeviceBuffer.from_host(f[n]) for n in ("q", "k", "v", "gate", "beta")), out, 1, 1, 2)
    assert rel(out.download(), f["out"]) < 1e-3 and rel(sd.download(), f["state_out"]) < 1e-3
    f = np.load(G / "gdn_prefill_t70.npz")
    sd = DeviceBuffer.from_host(f["state"][None])
    out = DeviceBuffer((70, 2, 128), np.float32)
    qwen35.gdn_chunk_prefill(sd, *(DeviceBuffer.from_host(f[n]) for n in ("q", "k", "v", "gate", "beta")), out,
                             None, 70, 1, 2)
    assert rel(out.download(), f["out"]) < 1e-3 and rel(sd.download()[0], f["state_out"]) < 1e-3
