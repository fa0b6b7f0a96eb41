"""K-column TL1 (PTQ1_0) matmul of a resident weight in one pass over its
trits (matmul_tl1, ops.rs:156-286): trits on int8 MFMA, x as exact int8
digit planes per group, the f16 group scales applied per group.  Checked
against the oracle's matmul_tl1 at the reference's K-column bar, rel 1e-3
(ops.rs:720-750), on the reference's own K-column inputs, on the ternary
layer and lm_head shapes, on rows of 128 (not 256) elements and on more
columns than one launch takes (16).  TQ1_0 handles take the same pass (their
trits tiled from the 54-byte blocks, each block's d for both 128-groups),
checked against the oracle's matmul_q (ops.rs:219-230)."""
import numpy as np
import pytest

from ouroboros_amd import ops
from ouroboros_amd.quant import QuantKind

pytestmark = pytest.mark.gpu


def tl1_payload(rng, out_len, in_len):
    p = rng.integers(0, 256, out_len * (in_len // 128) * 28, dtype=np.uint8)
    g = p.reshape(-1, 28)
    d = rng.uniform(0.01, 0.1, g.shape[0]).astype(np.float16).view(np.uint16)
    g[:, 26], g[:, 27] = d & 0xFF, d >> 8
    return p


def close(got, want, rtol):
    scale = np.abs(want).max()
    return np.abs(got - want) <= rtol * np.maximum(np.abs(want), 1e-2 * scale) + 1e-6 * scale


def test_reference_k_columns_inputs(gpu, orc):
    """ops.rs:720-750: 97 x 384, K = 4, bytes i * (0x9B ^ (i >> 5)), d bytes
    0x10 0x38, x[i] = ((i % 11) - 5) / 4; each column against matvec_tl1 at
    |got - want| <= 1e-3 max(|want|, 1)."""
    out_len, in_len, k = 97, 384, 4
    i = np.arange(out_len * in_len // 128 * 28, dtype=np.uint64)
    p = ((i * (0x9B ^ (i >> 5))) & 0xFF).astype(np.uint8)
    g = p.reshape(-1, 28)
    g[:, 26], g[:, 27] = 0x10, 0x38
    x = (((np.arange(k * in_len) % 11) - 5.0) * 0.25).astype(np.float32)
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len, max_cols=k)
    got = h.matmul(x, k)
    for c in range(k):
        want = orc.matvec_tl1(p, out_len, in_len, x[c * in_len:(c + 1) * in_len])
        assert (np.abs(got[c * out_len:(c + 1) * out_len] - want) <= 1e-3 * np.maximum(np.abs(want), 1.0)).all()
    h.free()


@pytest.mark.parametrize("out_len,in_len,k", [(6912, 2560, 2), (6912, 2560, 4), (6912, 2560, 8), (2560, 6912, 8),
                                              (97, 384, 3), (97, 384, 6), (37, 128, 5), (300, 1024, 11),
                                              (300, 1024, 16), (300, 1024, 17), (129, 640, 33)])
def test_tl1_handle_matmul_mfma(gpu, orc, margin, out_len, in_len, k):
    rng = np.random.default_rng(out_len + in_len + k)
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    x[3] = 40.0  # an outlier in a group of column 0
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len, max_cols=k)
    want = orc.matmul_tl1(p, out_len, in_len, x, k)
    got = h.matmul(x, k)
    margin(f"TL1 {out_len}x{in_len} k={k}", got, want, 1e-3)
    assert close(got, want, 1e-3).all()
    # the first column through the table-lookup matvec of the same handle
    y0 = h.matvec(x[:in_len])
    assert close(y0, want[:out_len], 1e-5).all()
    h.free()


def test_tl1_handle_matmul_lm_head(gpu, orc, margin):
    """The reference's lm_head probe shape, 248320 x 5120, at 8 columns."""
    out_len, in_len, k = 248320, 5120, 8
    rng = np.random.default_rng(9)
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len, max_cols=k)
    got = h.matmul(x, k)
    h.free()
    want = orc.matmul_tl1(p, out_len, in_len, x, k)
    margin("TL1 248320x5120 k=8", got, want, 1e-3)
    assert close(got, want, 1e-3).all()


@pytest.mark.parametrize("out_len,in_len,k", [(6912, 2560, 8), (97, 384, 4), (37, 128, 3), (300, 1024, 17)])
def test_tl1_raw_matmul_q_mfma(gpu, orc, margin, out_len, in_len, k):
    """ouro_matmul_q on a raw device payload: the digits decoded in registers
    for the int8 MFMA pass (rows of one group, 128-element rows past a
    256-deep block, more than one launch's 16 columns)."""
    rng = np.random.default_rng(out_len * 7 + k)
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    want = orc.matmul_tl1(p, out_len, in_len, x, k)
    got = ops.matmul_q(p, QuantKind.TL1, out_len, in_len, x, k)
    margin(f"raw TL1 {out_len}x{in_len} k={k}", got, want, 1e-3)
    assert close(got, want, 1e-3).all()


def test_tl1_raw_matmul_q_lm_head(gpu, orc, margin):
    out_len, in_len, k = 248320, 5120, 8
    rng = np.random.default_rng(10)
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    got = ops.matmul_q(p, QuantKind.TL1, out_len, in_len, x, k)
    want = orc.matmul_tl1(p, out_len, in_len, x, k)
    margin("raw TL1 248320x5120 k=8", got, want, 1e-3)
    assert close(got, want, 1e-3).all()


def test_tl1_handle_single_column_layout_keeps_lookups(gpu, orc):
    """A handle for one column holds no MFMA layout; its matmuls are one
    lookup pass per column (rel 1e-5 per column)."""
    rng = np.random.default_rng(4)
    out_len, in_len, k = 300, 1024, 3
    p = tl1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    h = ops.Weight(QuantKind.TL1, p, out_len, in_len, max_cols=1)
    want = orc.matmul_tl1(p, out_len, in_len, x, k)
    assert close(h.matmul(x, k), want, 1e-5).all()
    h.free()


def tq1_payload(rng, out_len, in_len):
    p = rng.integers(0, 256, out_len * (in_len // 256) * 54, dtype=np.uint8)
    g = p.reshape(-1, 54)
    d = rng.uniform(0.01, 0.1, g.shape[0]).astype(np.float16).view(np.uint16)
    g[:, 52], g[:, 53] = d & 0xFF, d >> 8
    return p


@pytest.mark.parametrize("out_len,in_len,k", [(6912, 2560, 2), (6912, 2560, 8), (2560, 6912, 4), (37, 256, 5),
                                              (300, 1024, 17), (129, 768, 33), (9000, 2048, 3)])
def test_tq1_handle_matmul_mfma(gpu, orc, margin, out_len, in_len, k):
    rng = np.random.default_rng(out_len * 3 + in_len + k)
    p = tq1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    x[5] = -30.0  # an outlier in a group of column 0
    h = ops.Weight(QuantKind.TQ1_0, p, out_len, in_len, max_cols=k)
    want = orc.matmul_q(p, orc.KIND_TQ1_0, out_len, in_len, x, k)
    got = h.matmul(x, k)
    margin(f"TQ1_0 {out_len}x{in_len} k={k}", got, want, 1e-3)
    assert close(got, want, 1e-3).all()
    assert close(h.matvec(x[:in_len]), want[:out_len], 1e-5).all()  # the matvec keeps its own kernels
    h.free()


def test_tq1_handle_matmul_lm_head(gpu, orc, margin):
    out_len, in_len, k = 248320, 5120, 8
    rng = np.random.default_rng(12)
    p = tq1_payload(rng, out_len, in_len)
    x = rng.standard_normal(k * in_len).astype(np.float32)
    h = ops.Weight(QuantKind.TQ1_0, p, out_len, in_len, max_cols=k)
    got = h.matmul(x, k)
    h.free()
    want = orc.matmul_q(p, orc.KIND_TQ1_0, out_len, in_len, x, k)
    margin("TQ1_0 248320x5120 k=8", got, want, 1e-3)
    assert close(got, want, 1e-3).all()


def test_upload_rejects_partial_blocks(gpu):
    from ouroboros_amd._lib import OuroError
    for kind, in_len, nb in ((QuantKind.TQ1_0, 384, 54), (QuantKind.TL1, 192, 28), (QuantKind.Q4K, 384, 144)):
        with pytest.raises(OuroError) as e:
            ops.Weight(kind, np.zeros(4 * nb, np.uint8), 4, in_len, max_cols=4)
        assert e.value.code == 2
