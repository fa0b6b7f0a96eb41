"""GPU TL1 (PTQ1_0) resident-weight GEMV (table-lookup kernel, repacked on
upload) against the oracle's matvec_tl1 at the reference's rel 1e-5 bar
(ops.rs:800-838), and finite_argmax (infer/mod.rs:70-83) alone and fused
after the GEMV (Qwen35Stage::sample, qwen35.rs:746-757)."""
import numpy as np
import pytest

from ouroboros_amd import ops
from ouroboros_amd.device import DeviceBuffer
from ouroboros_amd.quant import QuantKind

pytestmark = pytest.mark.gpu


def tl1_payload(rng, out_len, in_len):
    p = rng.integers(0, 256, out_len * (in_len // 128) * 28, dtype=np.uint8)
    g = p.reshape(-1, 28)
    d = (rng.uniform(0.01, 0.1, g.shape[0]).astype(np.float16)).view(np.uint16)
    g[:, 26], g[:, 27] = d & 0xFF, d >> 8
    return p


def close(got, want, rtol):
    scale = np.abs(want).max()
    return np.abs(got - want) <= rtol * np.maximum(np.abs(want), 1e-2 * scale) + 1e-6 * scale


@pytest.mark.parametrize("shape", [(37, 384), (64, 512), (130, 640), (1000, 5120), (97, 128)])
def test_tl1_handle_matvec(gpu, orc, shape):
    # in_len 640 = 5 groups (one block of 4 + a block of 1); 384 = 3 groups; ragged row tiles
    out_len, in_len = shape
    rng = np.random.default_rng(out_len + in_len)
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len)
    want = orc.matvec_tl1(p, out_len, in_len, x)
    assert close(h.matvec(x), want, 1e-5).all()
    h.free()


def test_tl1_reference_fixture(gpu, orc):  # ops.rs:800-838 payload bytes and scales
    out_len, in_len = 37, 384
    rb = in_len // 128 * 28
    i = np.arange(out_len * rb, dtype=np.uint64)
    p = ((i * (0x9B ^ (i >> 7))) & 0xFF).astype(np.uint8)
    g = p.reshape(-1, 28)
    g[:, 26], g[:, 27] = 0x10, 0x38
    x = ((np.arange(in_len) % 17) - 8).astype(np.float32) * 0.05
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len)
    assert close(h.matvec(x), orc.matvec_tl1(p, out_len, in_len, x), 1e-5).all()
    h.free()


def test_tl1_handle_matmul_columns(gpu, orc):
    rng = np.random.default_rng(5)
    out_len, in_len, k = 300, 1024, 3
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len)
    want = orc.matmul_tl1(p, out_len, in_len, x, k)  # column-major y[c*out + r]
    # several columns run the MFMA pass (rel 1e-3, the reference's K-column bar, ops.rs:720-750)
    assert close(h.matmul(x, k), want, 1e-3).all()
    h.free()


def test_finite_argmax_edge_cases(gpu, orc):
    nan, inf = float("nan"), float("inf")
    for v in ([1.0, 3.0, 2.0], [nan, 1.0, nan, 5.0, nan], [2.0, 7.0, 7.0, 1.0], [nan, nan], [-0.0, 0.0],
              [0.0, -0.0, -1.0], [-inf, -inf], [nan, -inf, -5.0], [1.0, inf, nan, inf], [5.0]):
        a = np.array(v, np.float32)
        assert ops.finite_argmax(a) == orc.finite_argmax(a), v


def test_finite_argmax_large(gpu, orc):
    rng = np.random.default_rng(8)
    for n in (248320, 1000, 257):
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.random(n) < 0.05] = np.nan
        x[rng.integers(0, n, 3)] = np.float32(9.5)  # a tie of the maximum: the first index wins
        assert ops.finite_argmax(x) == orc.finite_argmax(x)


def test_matvec_argmax_tl1_handle(gpu, orc):
    rng = np.random.default_rng(13)
    out_len, in_len = 20000, 1280
    p = tl1_payload(rng, out_len, in_len)
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len)
    for call in range(3):  # repeated calls reuse the handle's argmax scratch
        x = rng.standard_normal(in_len).astype(np.float32)
        want = orc.matvec_tl1(p, out_len, in_len, x)
        y = DeviceBuffer((out_len,), np.float32)
        idx = h.matvec_argmax(x, y)
        yv = y.download()
        assert idx == orc.finite_argmax(yv)  # exactly the argmax of the logits it returns
        best = orc.finite_argmax(want)
        # and the oracle's argmax, unless the two logits tie within the matvec tolerance
        assert idx == best or abs(float(want[idx]) - float(want[best])) <= 1e-5 * abs(float(want[best])), call
        assert h.matvec_argmax(x) == idx  # without a caller y
    h.free()


def test_lm_head_full_size(gpu, orc):
    # The reference's lm_head shape, 248320 x 5120 TL1 (docs/BONSAI_PTQ1.md:30;
    # the head of Qwen35Stage::sample, qwen35.rs:746-757): the resident
    # table-lookup GEMV with the fused finite_argmax, and the raw-payload
    # matvec_q, against the oracle's matvec_tl1 and finite_argmax.
    rng = np.random.default_rng(248320)
    out_len, in_len = 248320, 5120
    p = tl1_payload(rng, out_len, in_len)
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len)
    try:
        for call in range(2):
            x = rng.standard_normal(in_len).astype(np.float32)
            want = orc.matvec_tl1(p, out_len, in_len, x)
            y = DeviceBuffer((out_len,), np.float32)
            idx = h.matvec_argmax(x, y)
            yv = y.download()
            ok = close(yv, want, 1e-5)
            assert ok.all(), (call, int((~ok).sum()))
            assert idx == orc.finite_argmax(yv)
            best = orc.finite_argmax(want)
            assert idx == best or abs(float(want[idx]) - float(want[best])) <= 1e-5 * abs(float(want[best])), call
        raw = ops.matvec_q(p, QuantKind.TL1, out_len, in_len, x)
        assert close(raw, want, 1e-5).all()
    finally:
        h.free()
