"""GPU delta-net layer block (run_delta's gates, conv + SiLU, normed
recurrence, gated RMS norm, V-grouped order) against the oracle."""
import numpy as np
import pytest

from ouroboros_amd import qwen35
from ouroboros_amd._lib import GDN_KHEAD_DIV, GDN_V_GROUPED, OuroError
from ouroboros_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu
D = 128
TOL = 1e-3
NAMES = ("qkv", "z", "beta_raw", "alpha_raw", "dt_bias", "a_log", "conv_w", "norm_w")


def rel(got, want):
    return float(np.abs(got - want).max()) / max(float(np.abs(want).max()), 1e-30)


def inputs(rng, B, Hk, Hv):
    ch = 2 * Hk * D + Hv * D
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    return dict(qkv=f(B, ch), z=f(B, Hv * D), beta_raw=f(B, Hv), alpha_raw=f(B, Hv), dt_bias=f(Hv),
                a_log=(-np.exp(f(Hv))).astype(np.float32), conv_w=(0.5 * f(ch, 4)).astype(np.float32),
                norm_w=f(D), conv=f(B, ch, 3), state=(0.02 * f(B, Hv, D * D)).astype(np.float32))


def run(orc, B, Hk, Hv, flags, steps=1, seed=0, workspace=False, margin=None):
    rng = np.random.default_rng(seed)
    x = inputs(rng, B, Hk, Hv)
    conv_ref, st_ref = x["conv"].copy(), x["state"].copy()
    dconv, dst = DeviceBuffer.from_host(x["conv"]), DeviceBuffer.from_host(x["state"])
    # a caller workspace is accepted and ignored (the block needs none)
    ws = DeviceBuffer((256,), np.uint8) if workspace else None
    for s in range(steps):
        if s:  # fresh token inputs for the next step, same weights
            x["qkv"], x["z"] = inputs(rng, B, Hk, Hv)["qkv"], inputs(rng, B, Hk, Hv)["z"]
        want = orc.gdn_layer_decode(*(x[n] for n in NAMES), conv_ref, st_ref, B, Hk, Hv, D, flags, 1e-6)
        out = DeviceBuffer((B, Hv * D), np.float32)
        qwen35.gdn_layer_decode(*(DeviceBuffer.from_host(x[n]) for n in NAMES), dconv, dst, out, B, Hk, Hv,
                                flags=flags, eps=1e-6, workspace=ws)
        got = out.download()
        if margin:
            margin(f"out step {s}", got, want, TOL)
        assert rel(got, want) < TOL, (s, rel(got, want))
    assert np.array_equal(dconv.download(), conv_ref)  # the ring update is a pure shift
    if margin:
        margin("state", dst.download(), st_ref, TOL)
    assert rel(dst.download(), st_ref) < TOL


@pytest.mark.parametrize("flags", [0, GDN_KHEAD_DIV, GDN_V_GROUPED, GDN_KHEAD_DIV | GDN_V_GROUPED])
def test_layer_block_matches_oracle(gpu, orc, margin, flags):
    run(orc, 3, 2, 4, flags, seed=flags, margin=margin)


def test_layer_block_three_steps_carry_conv_and_state(gpu, orc):
    run(orc, 2, 2, 6, GDN_V_GROUPED, steps=3, seed=11, workspace=True)


@pytest.mark.parametrize("B,Hk,Hv,flags", [(5, 3, 3, 0), (4, 2, 8, GDN_KHEAD_DIV | GDN_V_GROUPED),
                                           (3, 1, 8, GDN_V_GROUPED), (2, 2, 32, GDN_KHEAD_DIV)])
def test_layer_block_heads_per_khead(gpu, orc, B, Hk, Hv, flags):
    # one workgroup per (sequence, k-head) walks the g = Hv / Hk v-heads:
    # g = 1, 4, 8 and 16 (more column groups than wavefronts), two steps so
    # the ring shift of every channel is checked too
    run(orc, B, Hk, Hv, flags, steps=2, seed=B * 100 + Hv)


def test_layer_block_config3_shape(gpu, orc, margin):
    # B=32 sequences, Hk=16, Hv=32, d=128 (the decode workload's shape)
    run(orc, 32, 16, 32, GDN_V_GROUPED, seed=12, margin=margin)


def test_layer_block_rejects_bad_flags(gpu):
    b = DeviceBuffer((1 << 16,), np.float32)
    with pytest.raises(OuroError) as e:
        qwen35.gdn_layer_decode(*([b] * 11), 1, 1, 1, flags=1)
    assert e.value.code == 1  # OURO_ERR_INVALID_ARG
