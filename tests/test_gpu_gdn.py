"""GPU parity of the gated delta-net decode step against the oracle
(delta_head_dim per head, run_delta preprocessing), within 1e-3 relative."""
import numpy as np
import pytest

from ouroboros_amd import qwen35, quant
from ouroboros_amd._lib import GDN_KHEAD_DIV, GDN_L2NORM_QK, GDN_SCALE_Q
from ouroboros_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
S = 128
TOL = 1e-3  # relative, as stated for the fp32 delta-net outputs


def rel_err(got, want):
    """Max abs error relative to the tensor's max magnitude, and the L2 ratio."""
    scale = max(float(np.abs(want).max()), 1e-30)
    return float(np.abs(got - want).max()) / scale, float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def config3_inputs(rng, B=32, Hk=16, Hv=32, d=S):
    state = (0.02 * rng.standard_normal((B, Hv, d * d))).astype(np.float32)
    q = quant.f32_to_bf16_bits(rng.standard_normal((B, Hk, d)).astype(np.float32))
    k = quant.f32_to_bf16_bits(rng.standard_normal((B, Hk, d)).astype(np.float32))
    v = quant.f32_to_bf16_bits(rng.standard_normal((B, Hv, d)).astype(np.float32))
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, Hv))))).astype(np.float32)
    # decay g = exp(-softplus(N(0,1)))  ->  gate (log-decay) = -softplus(N(0,1))
    gate = (-np.log1p(np.exp(rng.standard_normal((B, Hv))))).astype(np.float32)
    return state, q, k, v, gate, beta


@pytest.mark.parametrize("flags", [GDN_L2NORM_QK | GDN_SCALE_Q, GDN_L2NORM_QK | GDN_SCALE_Q | GDN_KHEAD_DIV])
def test_config3_decode_steps(gpu, orc, margin, flags):
    rng = np.random.default_rng(0)
    B, Hk, Hv, d, eps = 32, 16, 32, S, 1e-6
    state, q, k, v, gate, beta = config3_inputs(rng, B, Hk, Hv, d)
    sd = DeviceBuffer.from_host(state)
    ref_state = state.copy()
    out = DeviceBuffer((B, Hv, d), np.float32)
    for step in range(3):  # state carried across steps on both sides
        if step:
            _, q, k, v, gate, beta = config3_inputs(np.random.default_rng(step), B, Hk, Hv, d)
        want = orc.gdn_decode(ref_state, quant.bf16_bits_to_f32(q), quant.bf16_bits_to_f32(k),
                              quant.bf16_bits_to_f32(v), gate, beta, B, Hk, Hv, d, flags, eps)
        qwen35.gdn_decode(sd, DeviceBuffer.from_host(q), DeviceBuffer.from_host(k), DeviceBuffer.from_host(v),
                          DeviceBuffer.from_host(gate), DeviceBuffer.from_host(beta), out, B, Hk, Hv, d,
                          flags=flags, eps=eps)
        eo = margin(f"out step {step}", out.download(), want, TOL)
        es = margin(f"state step {step}", sd.download(), ref_state, TOL)
        assert eo[0] < TOL and eo[1] < TOL, (step, eo)
        assert es[0] < TOL and es[1] < TOL, (step, es)


def test_f32_inputs_unnormalised(gpu, orc, margin):
    rng = np.random.default_rng(1)
    B, Hk, Hv, d = 2, 2, 4, S
    state = rng.standard_normal((B, Hv, d * d)).astype(np.float32)
    q = rng.standard_normal((B, Hk, d)).astype(np.float32) * 0.1
    k = rng.standard_normal((B, Hk, d)).astype(np.float32) * 0.1
    v = rng.standard_normal((B, Hv, d)).astype(np.float32)
    gate = -rng.random((B, Hv)).astype(np.float32)
    beta = rng.random((B, Hv)).astype(np.float32)
    ref = state.copy()
    want = orc.gdn_decode(ref, q, k, v, gate, beta, B, Hk, Hv, d, 0, 0.0)
    sd = DeviceBuffer.from_host(state)
    out = DeviceBuffer((B, Hv, d), np.float32)
    qwen35.gdn_decode(sd, *(DeviceBuffer.from_host(a) for a in (q, k, v, gate, beta)), out, B, Hk, Hv, d, flags=0)
    assert margin("out", out.download(), want, TOL)[0] < TOL
    assert margin("state", sd.download(), ref, TOL)[0] < TOL


def test_delta_head_dim_kats_on_gpu(gpu):
    # qwen35.rs:241-259 through the single-head mirror.
    state = np.zeros(S * S, np.float32)
    q = np.zeros(S, np.float32)
    q[5] = qwen35.delta_q_scale()
    k = np.zeros(S, np.float32)
    k[5], k[9] = 2.0, 1.0
    v = np.zeros(S, np.float32)
    v[7] = 4.0
    out = np.zeros(S, np.float32)
    qwen35.delta_head_dim(state, S, q, k, v, qwen35.DeltaStep(gate=0.0, beta=1.0), out)
    assert abs(state[5 + 7 * S] - 8.0) < 1e-6 and abs(state[9 + 7 * S] - 4.0) < 1e-6
    assert abs(out[7] - 4.0 * qwen35.delta_q_scale() * 2.0) < 1e-6
    assert np.abs(np.delete(out, 7)).max() < 1e-6
    # qwen35.rs:225-239: beta = 0 is pure decay
    state = np.full(S * S, 0.5, np.float32)
    out = np.zeros(S, np.float32)
    qwen35.delta_head_dim(state, S, np.full(S, 0.1, np.float32), np.full(S, 0.2, np.float32),
                          np.full(S, 0.3, np.float32), qwen35.DeltaStep(gate=-0.25, beta=0.0), out)
    expect = np.float32(0.5) * np.exp(np.float32(-0.25))
    assert np.abs(state - expect).max() < 1e-6
    assert np.abs(out - np.float32(0.1 * S) * expect).max() < 1e-4


@pytest.mark.parametrize("sdim", [1, 16, 64, 100, 192, 256])
def test_delta_head_dim_runtime_sdim(gpu, orc, margin, sdim):
    # delta_head_dim is the reference's runtime-dim variant (qwen35.rs:26-27)
    rng = np.random.default_rng(sdim)
    state = (0.1 * rng.standard_normal(sdim * sdim)).astype(np.float32)
    q, k, v = (rng.standard_normal(sdim).astype(np.float32) for _ in range(3))
    step = qwen35.DeltaStep(gate=-0.3, beta=0.7)
    ref, want = state.copy(), np.zeros(sdim, np.float32)
    orc.delta_head_dim(ref, sdim, q, k, v, step.gate, step.beta, want)
    got = np.zeros(sdim, np.float32)
    qwen35.delta_head_dim(state, sdim, q, k, v, step, got)
    assert margin("out", got, want, TOL)[0] < TOL and margin("state", state, ref, TOL)[0] < TOL


@pytest.mark.parametrize("d,dt", [(64, "bf16"), (96, "f32"), (256, "bf16")])
def test_decode_other_head_dims(gpu, orc, margin, d, dt):
    rng = np.random.default_rng(d)
    B, Hk, Hv, flags = 3, 2, 4, GDN_L2NORM_QK | GDN_SCALE_Q
    state, q, k, v, gate, beta = config3_inputs(rng, B, Hk, Hv, d)
    if dt == "f32":
        q, k, v = (quant.bf16_bits_to_f32(a) for a in (q, k, v))
    ref = state.copy()
    f32 = lambda a: quant.bf16_bits_to_f32(a) if a.dtype == np.uint16 else a  # noqa: E731
    want = orc.gdn_decode(ref, f32(q), f32(k), f32(v), gate, beta, B, Hk, Hv, d, flags, 1e-6)
    sd = DeviceBuffer.from_host(state)
    out = DeviceBuffer((B, Hv, d), np.float32)
    qwen35.gdn_decode(sd, *(DeviceBuffer.from_host(a) for a in (q, k, v, gate, beta)), out, B, Hk, Hv, d,
                      flags=flags, eps=1e-6)
    assert margin("out", out.download(), want, TOL)[0] < TOL and margin("state", sd.download(), ref, TOL)[0] < TOL


def test_bad_shapes_rejected(gpu):
    from ouroboros_amd._lib import OuroError

    st = DeviceBuffer((257 * 257,), np.float32)
    v = DeviceBuffer((257,), np.float32)
    with pytest.raises(OuroError) as e:
        qwen35.delta_head_dim(st, 257, v, v, v, qwen35.DeltaStep(0.0, 1.0), v)
    assert e.value.code == 2
