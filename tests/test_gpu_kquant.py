"""GPU matvec_q / matmul_q on the block-quantised kinds Q8_0, Q3_K, Q4_K,
Q5_K, Q6_K (matvec_qblock, ops.rs:101-128) against the oracle's restatement
of the reference decoders (dequant.rs:218-310, 390-560).  Bars: max|err| /
max|y| <= 1e-5 (the reference's fused-vs-scalar rel 1e-5, ops.rs:800-838;
rel 1e-3 for matmul, ops.rs:720-750), and per row
|err| <= 1e-5 |y| + 2e-6 sum_i |w_i x_i| (see close()).  Shapes: the ternary
layer 6912x2560 and the lm_head probe 248320x5120; misaligned payloads; the
>512-task and >1024-task rows; each tiling of the matrix-core kernels."""
import ctypes as C

import numpy as np
import pytest

from ouroboros_amd import ops
from ouroboros_amd._lib import OuroError, call
from ouroboros_amd.device import DeviceBuffer
from ouroboros_amd.quant import QuantKind

pytestmark = pytest.mark.gpu

KINDS = [QuantKind.Q8_0, QuantKind.Q3K, QuantKind.Q4K, QuantKind.Q5K, QuantKind.Q6K]
F16_AT = {QuantKind.Q8_0: [0], QuantKind.Q3K: [108], QuantKind.Q4K: [0, 2], QuantKind.Q5K: [0, 2],
          QuantKind.Q6K: [208]}


def kq_payload(rng, kind, out_len, in_len):
    """Random codes and scale bytes; the f16 super-scales drawn in a model's range."""
    bb, be = kind.block_bytes(), kind.block_elems()
    nblk = out_len * (in_len // be)
    p = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    for o in F16_AT[kind]:
        d = rng.uniform(0.002, 0.02, nblk).astype(np.float16).view(np.uint16)
        p[:, o], p[:, o + 1] = d & 0xFF, d >> 8
    return p.reshape(-1)


def abs_dot(orc, p, kind, out_len, in_len, x, chunk=8192):
    """sum_i |w_ri x_i| per row, from the oracle's decoded weights (row chunks)."""
    rb = kind.row_bytes(in_len)
    ax = np.abs(x.astype(np.float64))
    out = np.empty(out_len)
    for r0 in range(0, out_len, chunk):
        r1 = min(out_len, r0 + chunk)
        w = orc.dequant_qblock(int(kind), p[r0 * rb:r1 * rb]).reshape(r1 - r0, in_len)
        out[r0:r1] = np.abs(w) @ ax
    return out


def close(got, want, rtol, absdot):
    """The floating-point dot product's componentwise error model: two fp32
    sums of the same terms in different orders differ by a few ulps of
    sum|w x|.  The reference's own sums (the oracle) stay within 2.4e-7 of
    sum|w x| of the exact product at 2560x6912 (float64 check), but reach
    5e-5 relative on rows whose terms cancel, so a bar relative to |y| alone
    would fail the reference itself."""
    return np.abs(got - want) <= rtol * np.abs(want) + 2e-6 * absdot


def check(orc, margin, label, got, want, p, kind, out_len, in_len, x, rtol):
    norm, _ = margin(label, got, want, rtol)
    assert norm <= rtol  # max|err| / max|want|
    assert close(got, want, rtol, abs_dot(orc, p, kind, out_len, in_len, x)).all()


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: k.name)
@pytest.mark.parametrize("out_len,in_len", [(6912, 2560), (2560, 6912), (37, 256), (1, 512)])
def test_kquant_matvec(gpu, orc, margin, kind, out_len, in_len):
    rng = np.random.default_rng(out_len + int(kind))
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, int(kind), out_len, in_len, x)
    got = ops.matvec_q(p, kind, out_len, in_len, x)
    check(orc, margin, f"{kind.name} {out_len}x{in_len}", got, want, p, kind, out_len, in_len, x, 1e-5)


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: k.name)
def test_kquant_lm_head_shape(gpu, orc, margin, kind):
    """The reference's lm_head probe shape, 248320 x 5120 (ops.rs:694-717)."""
    out_len, in_len = 248320, 5120
    rng = np.random.default_rng(int(kind))
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, int(kind), out_len, in_len, x)
    got = ops.matvec_q(p, kind, out_len, in_len, x)
    check(orc, margin, f"{kind.name} 248320x5120", got, want, p, kind, out_len, in_len, x, 1e-5)


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: k.name)
@pytest.mark.parametrize("offset", [1, 2, 3, 4, 6, 16])
@pytest.mark.parametrize("in_len", [768, 1024])
def test_kquant_misaligned_payload(gpu, orc, margin, kind, offset, in_len):
    """The payload at any byte offset (the reference takes &[u8]); rows of
    an odd and an even number of blocks (Q6_K rows of an even number of
    blocks are dword-aligned when the payload is)."""
    out_len = 97
    rng = np.random.default_rng(offset + in_len)
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, int(kind), out_len, in_len, x)
    buf = DeviceBuffer((p.size + 32,), np.uint8)
    host = np.zeros(p.size + 32, np.uint8)
    host[offset:offset + p.size] = p
    buf.upload(host)
    xb = DeviceBuffer.from_host(x)
    y = DeviceBuffer((out_len,), np.float32)
    call("ouro_matvec_q", buf.ptr + offset, int(kind), out_len, in_len, xb.ptr, y.ptr, None)
    check(orc, margin, f"{kind.name} +{offset}", y.download(), want, p, kind, out_len, in_len, x, 1e-5)


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: k.name)
@pytest.mark.parametrize("in_len", [20480, 40960])
def test_kquant_long_rows(gpu, orc, margin, kind, in_len):
    """Rows of 640 tasks (one 1024-thread task set) and of 1280 (the per-row kernel)."""
    out_len = 45
    rng = np.random.default_rng(in_len)
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, int(kind), out_len, in_len, x)
    got = ops.matvec_q(p, kind, out_len, in_len, x)
    check(orc, margin, f"{kind.name} in {in_len}", got, want, p, kind, out_len, in_len, x, 1e-5)


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: k.name)
@pytest.mark.parametrize("out_len,in_len", [(2049, 512), (2100, 768), (3001, 1280), (4100, 4096), (8200, 8192),
                                             (16399, 512), (16399, 768)])
def test_kquant_tilings(gpu, orc, margin, kind, out_len, in_len):
    """Each tiling of the matrix-core kernels: the shared 16-row tiles
    (2048 <= rows < 64 per CU) with ragged last tiles and rows of 2, 3, 5
    and 16 blocks (with fewer than four steps some wavefronts have none;
    5 splits unevenly; 8192-element rows of 16 and 32 steps), and Q3_K's
    64-row tiles (16399 rows; rows of 3 blocks are not dword-aligned: the
    unstaged kernel)."""
    rng = np.random.default_rng(out_len * 7 + in_len + int(kind))
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, int(kind), out_len, in_len, x)
    got = ops.matvec_q(p, kind, out_len, in_len, x)
    check(orc, margin, f"{kind.name} {out_len}x{in_len}", got, want, p, kind, out_len, in_len, x, 1e-5)


def test_q8_0_rows_not_whole_chunks(gpu, orc, margin):
    """Q8_0 rows of 25 blocks (800 elements: not whole 256-element chunks)
    on a matrix of the matrix-core row counts: the task kernel; and the same
    rows with one chunk more (1056 elements: 33 blocks, still not 8k)."""
    for in_len in (800, 1056):
        out_len = 2100
        rng = np.random.default_rng(in_len)
        p = kq_payload(rng, QuantKind.Q8_0, out_len, in_len)
        x = rng.standard_normal(in_len).astype(np.float32)
        want = orc.matvec_q(p, int(QuantKind.Q8_0), out_len, in_len, x)
        got = ops.matvec_q(p, QuantKind.Q8_0, out_len, in_len, x)
        check(orc, margin, f"Q8_0 {out_len}x{in_len}", got, want, p, QuantKind.Q8_0, out_len, in_len, x, 1e-5)


def test_kquant_64_row_tiles(gpu, orc, margin):
    """Q6_K rows of 42 blocks on a tall matrix: the shared 16-row tiles do
    not fit in LDS there, the 64-row tiles do (for Q4_K and Q5_K no row
    length fits the one and not the other)."""
    kind, out_len, in_len = QuantKind.Q6K, 16399, 10752
    rng = np.random.default_rng(in_len)
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, int(kind), out_len, in_len, x)
    got = ops.matvec_q(p, kind, out_len, in_len, x)
    check(orc, margin, f"{kind.name} {out_len}x{in_len}", got, want, p, kind, out_len, in_len, x, 1e-5)


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: k.name)
@pytest.mark.parametrize("offset", [2, 4])
def test_kquant_misaligned_tall(gpu, orc, margin, kind, offset):
    """Payload offsets on a matrix of the shared 16-row tiles: 4 keeps Q3_K
    and Q6_K rows dword-aligned (staged), 2 does not."""
    out_len, in_len = 2100, 1024
    rng = np.random.default_rng(offset + 99)
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    want = orc.matvec_q(p, int(kind), out_len, in_len, x)
    buf = DeviceBuffer((p.size + 32,), np.uint8)
    host = np.zeros(p.size + 32, np.uint8)
    host[offset:offset + p.size] = p
    buf.upload(host)
    xb = DeviceBuffer.from_host(x)
    y = DeviceBuffer((out_len,), np.float32)
    call("ouro_matvec_q", buf.ptr + offset, int(kind), out_len, in_len, xb.ptr, y.ptr, None)
    check(orc, margin, f"{kind.name} tall +{offset}", y.download(), want, p, kind, out_len, in_len, x, 1e-5)


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: k.name)
@pytest.mark.parametrize("out_len", [300, 2100])
def test_kquant_matmul_columns(gpu, orc, kind, out_len):
    in_len, k = 1024, 5
    rng = np.random.default_rng(7)
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal((k, in_len)).astype(np.float32)
    want = orc.matmul_q(p, int(kind), out_len, in_len, x.reshape(-1), k)
    got = ops.matmul_q(p, kind, out_len, in_len, x.reshape(-1), k)
    for c in range(k):
        ad = abs_dot(orc, p, kind, out_len, in_len, x[c])
        sl = slice(c * out_len, (c + 1) * out_len)
        assert close(got[sl], want[sl], 1e-3, ad).all()
    # each column is exactly the matvec of that column (column-major y)
    y0 = ops.matvec_q(p, kind, out_len, in_len, x[2])
    assert np.array_equal(got[2 * out_len:3 * out_len], y0)


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: k.name)
def test_kquant_weight_handle(gpu, kind):
    """A resident handle of the raw bytes gives matvec_q's result bit for bit."""
    out_len, in_len = 513, 512
    rng = np.random.default_rng(3)
    p = kq_payload(rng, kind, out_len, in_len)
    x = rng.standard_normal(in_len).astype(np.float32)
    w = ops.Weight(kind, p, out_len, in_len)
    assert np.array_equal(w.matvec(x), ops.matvec_q(p, kind, out_len, in_len, x))


def test_reference_q6k_opencl_matrix(gpu, orc):
    """agent/src/gpu.rs:288-318: the reference's GPU parity matrix and x
    (8 x 512, d = 1, mixed-sign scales); its gate is cos > 0.9999 (gpu.rs:12-15),
    this one the rel 1e-5 bar."""
    out_len, in_len = 8, 512
    i = np.arange(out_len * (in_len // 256) * 210)
    b, off = i // 210, i % 210
    s = (off * 3 + b * 5) % 64
    pl = np.where(((b + off) & 1) == 1, 192 + s, s)
    pl = np.where((off >= 192) & (off <= 207), pl, (i * 7 + 13) & 0xFF)
    pl[off == 208], pl[off == 209] = 0x00, 0x3C
    pl = pl.astype(np.uint8)
    x = (((np.arange(in_len) % 17) - 8.0) * 0.125).astype(np.float32)
    want = orc.matvec_q(pl, int(QuantKind.Q6K), out_len, in_len, x)
    got = ops.matvec_q(pl, QuantKind.Q6K, out_len, in_len, x)
    cos = float(np.dot(got, want) / (np.linalg.norm(got) * np.linalg.norm(want)))
    assert cos > 0.9999
    assert close(got, want, 1e-5, abs_dot(orc, pl, QuantKind.Q6K, out_len, in_len, x)).all()


def test_kquant_shape_errors(gpu):
    p = DeviceBuffer((4096,), np.uint8)
    x = DeviceBuffer((1024,), np.float32)
    y = DeviceBuffer((16,), np.float32)
    with pytest.raises(OuroError):  # in_len not a multiple of 256
        call("ouro_matvec_q", p.ptr, int(QuantKind.Q4K), 4, 300, x.ptr, y.ptr, None)
    with pytest.raises(OuroError):  # in_len not a multiple of 32
        call("ouro_matvec_q", p.ptr, int(QuantKind.Q8_0), 4, 48, x.ptr, y.ptr, None)
    with pytest.raises(OuroError):  # x misaligned
        call("ouro_matvec_q", p.ptr, int(QuantKind.Q6K), 4, 256, x.ptr + 2, y.ptr, None)
