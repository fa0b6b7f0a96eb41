"""GPU chunked prefill vs the token-by-token recurrence (the reference's own
prefill), within 1e-3 relative, on the config-4 shape and ragged varlen
batches."""
import numpy as np
import pytest

from ouroboros_amd import quant, qwen35
from ouroboros_amd._lib import GDN_KHEAD_DIV, GDN_L2NORM_QK, GDN_SCALE_Q, OuroError
from ouroboros_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
D = 128
TOL = 1e-3


def rel(got, want):
    scale = max(float(np.abs(want).max()), 1e-30)
    return float(np.abs(got - want).max()) / scale


def inputs(rng, T, Hk, Hv, N):
    q = quant.f32_to_bf16_bits(rng.standard_normal((T, Hk, D)).astype(np.float32))
    k = quant.f32_to_bf16_bits(rng.standard_normal((T, Hk, D)).astype(np.float32))
    v = quant.f32_to_bf16_bits(rng.standard_normal((T, Hv, D)).astype(np.float32))
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, Hv))))).astype(np.float32)
    gate = (-np.log1p(np.exp(rng.standard_normal((T, Hv))))).astype(np.float32)
    state = (0.02 * rng.standard_normal((N, Hv, D * D))).astype(np.float32)
    return q, k, v, gate, beta, state


def run_both(orc, cu, Hk, Hv, flags, seed=0, workspace=False):
    rng = np.random.default_rng(seed)
    T = int(cu[-1])
    N = len(cu) - 1
    q, k, v, gate, beta, state = inputs(rng, T, Hk, Hv, N)
    qf, kf, vf = (quant.bf16_bits_to_f32(a) for a in (q, k, v))
    want_state = state.copy()
    want_out = np.zeros((T, Hv, D), np.float32)
    for s in range(N):
        a, b = int(cu[s]), int(cu[s + 1])
        if b > a:
            st = np.ascontiguousarray(want_state[s])
            want_out[a:b] = orc.gdn_prefill_tokens(st, qf[a:b], kf[a:b], vf[a:b], gate[a:b], beta[a:b],
                                                   b - a, Hk, Hv, D, flags, 1e-6)
            want_state[s] = st
    sd = DeviceBuffer.from_host(state)
    out = DeviceBuffer((max(T, 1), Hv, D), np.float32, zero=True)
    ws = None
    if workspace:
        ws = DeviceBuffer((qwen35.chunk_workspace_bytes(T, N, Hv),), np.uint8)
    qwen35.gdn_chunk_prefill(sd, DeviceBuffer.from_host(q), DeviceBuffer.from_host(k), DeviceBuffer.from_host(v),
                             DeviceBuffer.from_host(gate), DeviceBuffer.from_host(beta), out,
                             np.asarray(cu, np.int32), T, Hk, Hv, flags=flags, eps=1e-6, workspace=ws)
    return out.download()[:T], want_out, sd.download(), want_state


def test_single_chunk_small(gpu, orc):
    got, want, gs, ws = run_both(orc, [0, 64], 1, 2, GDN_L2NORM_QK | GDN_SCALE_Q)
    assert rel(got, want) < TOL and rel(gs, ws) < TOL, (rel(got, want), rel(gs, ws))


@pytest.mark.parametrize("cu", [[0, 1], [0, 63], [0, 65], [0, 130, 130, 131, 300], [0, 0, 64, 200]])
def test_ragged_varlen(gpu, orc, margin, cu):
    got, want, gs, ws = run_both(orc, cu, 2, 4, GDN_L2NORM_QK | GDN_SCALE_Q, seed=len(cu))
    assert margin("out", got, want, TOL)[0] < TOL, rel(got, want)
    assert margin("state", gs, ws, TOL)[0] < TOL, rel(gs, ws)


@pytest.mark.parametrize("flags", [GDN_L2NORM_QK | GDN_SCALE_Q | GDN_KHEAD_DIV, GDN_L2NORM_QK])
def test_flags(gpu, orc, flags):
    got, want, gs, ws = run_both(orc, [0, 200, 333], 2, 4, flags, seed=3)
    assert rel(got, want) < TOL and rel(gs, ws) < TOL


def test_many_sequences_caller_workspace(gpu, orc, margin):
    # 300 ragged sequences (two launch slices of up to 256), caller-owned
    # workspace of exactly chunk_workspace_bytes, empty sequences included.
    rng = np.random.default_rng(21)
    lens = rng.integers(0, 140, 300)
    lens[[0, 17, 255, 256]] = 0
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    got, want, gs, ws = run_both(orc, cu, 1, 2, GDN_L2NORM_QK | GDN_SCALE_Q, seed=22, workspace=True)
    assert margin("out", got, want, TOL)[0] < TOL and margin("state", gs, ws, TOL)[0] < TOL


def test_config4_shape(gpu, orc, margin):
    # 4 sequences x 4096 tokens, Hk=16, Hv=32, chunk 64: the full workload.
    cu = [0, 4096, 8192, 12288, 16384]
    got, want, gs, ws = run_both(orc, cu, 16, 32, GDN_L2NORM_QK | GDN_SCALE_Q, seed=4)
    e_out, l2 = margin("out", got, want, TOL)
    e_state, l2s = margin("state", gs, ws, TOL)
    assert e_out < TOL and e_state < TOL and l2 < TOL and l2s < TOL, (e_out, e_state, l2, l2s)


def test_prefill_then_decode_matches_tokens(gpu, orc, margin):
    # chunked prefill of 100 tokens, then one decode step, equals 101 token steps.
    rng = np.random.default_rng(9)
    Hk, Hv, T = 2, 4, 101
    q, k, v, gate, beta, state = inputs(rng, T, Hk, Hv, 1)
    qf, kf, vf = (quant.bf16_bits_to_f32(a) for a in (q, k, v))
    fl = GDN_L2NORM_QK | GDN_SCALE_Q
    ref = state[0].copy()  # the oracle updates its state in place
    want = orc.gdn_prefill_tokens(ref, qf, kf, vf, gate, beta, T, Hk, Hv, D, fl, 1e-6)
    sd = DeviceBuffer.from_host(state)
    out = DeviceBuffer((T - 1, Hv, D), np.float32)
    qwen35.gdn_chunk_prefill(sd, *(DeviceBuffer.from_host(a[:T - 1]) for a in (q, k, v, gate, beta)), out,
                             None, T - 1, Hk, Hv)
    o1 = DeviceBuffer((1, Hv, D), np.float32)
    qwen35.gdn_decode(sd, *(DeviceBuffer.from_host(np.ascontiguousarray(a[T - 1:])) for a in (q, k, v, gate, beta)),
                      o1, 1, Hk, Hv)
    assert margin("out", o1.download()[0], want[T - 1], TOL)[0] < TOL
    assert margin("state", sd.download()[0], ref, TOL)[0] < TOL


def test_bad_offsets_rejected(gpu):
    buf = DeviceBuffer((4096,), np.float32)
    with pytest.raises(OuroError) as e:
        qwen35.gdn_chunk_prefill(buf, buf, buf, buf, buf, buf, buf, np.array([0, 5, 3], np.int32), 3, 1, 1)
    assert e.value.code == 2
