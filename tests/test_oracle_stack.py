"""The stack oracle's pieces (oracle/stack_oracle.py), pinned by the
reference's own tests of them (ops.rs:628-696, qwen35.rs:312-320), closed
forms, and the C oracle's delta-net layer block."""
import numpy as np
import pytest

from oracle import stack_oracle as so


def test_rmsnorm_basic():  # ops.rs:629-638
    y = so.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 1e-5)
    inv = 1.0 / np.sqrt((1 + 4 + 9 + 16) / 4.0 + 1e-5)
    assert abs(y[0] - inv) < 1e-6 and abs(y[3] - 4 * inv) < 1e-6


def test_rmsnorm_weight_scale():  # ops.rs:640-648
    y = so.rmsnorm(np.array([3, 3], np.float32), np.array([2.0, 0.5], np.float32), 0.0)
    assert abs(y[0] - 2.0) < 1e-6 and abs(y[1] - 0.5) < 1e-6


def test_rope_preserves_norm_and_moves():  # ops.rs:650-659 (rot = the whole vector)
    v0 = (0.1 * np.arange(8) + 0.05).astype(np.float32)
    v = so.rope_partial_neox(v0, 5, 8, 500000.0)
    assert abs(float((v0 * v0).sum() - (v * v).sum())) < 1e-4
    assert not np.array_equal(v, v0)


def test_rope_position_zero_is_identity():  # ops.rs:661-669
    v0 = (0.25 * np.arange(8)).astype(np.float32)
    assert np.abs(so.rope_partial_neox(v0, 0, 8, 500000.0) - v0).max() < 1e-5


def test_rope_partial_keeps_tail():  # qwen35.rs:312-320
    v0 = np.arange(256, dtype=np.float32)
    v = so.rope_partial_neox(v0, 7, 64, 1e7)
    assert np.array_equal(v[64:], v0[64:])
    assert np.abs(v[:64] - v0[:64]).max() > 1e-4


def test_rope_first_pair_closed_form():
    # pair 0 has theta = 1: (a, b) -> (a cos t - b sin t, b cos t + a sin t), split-half pairing
    v = np.zeros(8, np.float32)
    v[0], v[4] = 1.0, 2.0
    r = so.rope_partial_neox(v, 3, 8, 1e4)
    assert abs(r[0] - (np.cos(3.0) - 2 * np.sin(3.0))) < 1e-5
    assert abs(r[4] - (2 * np.cos(3.0) + np.sin(3.0))) < 1e-5
    assert r[1] == 0 and r[5] == 0


def test_rope_relative_position():
    # <rope(q, m), rope(k, n)> depends only on m - n
    rng = np.random.default_rng(0)
    q, k = rng.standard_normal(128).astype(np.float32), rng.standard_normal(128).astype(np.float32)
    d1 = float(so.rope_partial_neox(q, 10, 64, 1e7) @ so.rope_partial_neox(k, 7, 64, 1e7))
    d2 = float(so.rope_partial_neox(q, 103, 64, 1e7) @ so.rope_partial_neox(k, 100, 64, 1e7))
    assert abs(d1 - d2) < 1e-3 * max(1.0, abs(d1))


def test_softmax_and_silu():  # ops.rs:677-695
    p = so.softmax(np.array([1.0, 2.0, 3.0, -10.0], np.float32))
    assert abs(float(p.sum()) - 1.0) < 1e-6 and p[3] < 1e-4 and p[2] > p[0]
    s = so.silu(np.array([0.0, 10.0, -10.0], np.float32))
    assert abs(s[0]) < 1e-9 and abs(s[1] - 10.0) < 1e-3 and abs(s[2]) < 1e-3


def test_mix3_matches_integer_restatement():
    def mix(seed, tensor, idx):
        m = 0xFFFFFFFF
        x = seed ^ ((tensor * 0x9E3779B9) & m) ^ ((idx * 0x85EBCA6B) & m)
        x ^= x >> 16
        x = (x * 0x7FEB352D) & m
        x ^= x >> 15
        x = (x * 0x846CA68B) & m
        return x ^ (x >> 16)

    idx = np.array([0, 1, 2, 12345, 2**31 - 1, 2**32 - 1], np.uint64).astype(np.uint32)
    for seed, tensor in [(0, 0), (7, 5), (0xDEADBEEF, 0x100006)]:
        got = so.mix3(seed, tensor, idx)
        assert [int(g) for g in got] == [mix(seed, tensor, int(i)) for i in idx]


def test_generators_ranges():
    f = so.gen_floats(7, 12, 20000, -2.0, 1.9)
    assert f.dtype == np.float32 and f.min() >= -2.0 and f.max() < -0.1
    s = so.gen_floats(7, 13, 20000, 0.0, 0.0)
    assert set(np.unique(s)) == {-1.0, 1.0} and abs(float(s.mean())) < 0.05
    t = so.gen_ternary(7, 14, 64, 512)
    counts = np.bincount((t + 1).reshape(-1), minlength=3) / t.size
    assert set(np.unique(t)) == {-1, 0, 1} and np.abs(counts - 1 / 3).max() < 0.02


def test_bf16_round_matches_c_rne(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(4000).astype(np.float32) * np.float32(3.0)
    ties = (np.arange(1, 50, dtype=np.uint32) << 16 | 0x8000).view(np.float32)  # exact halfway cases
    x = np.concatenate([x, ties, -ties, np.array([0.0, 1.0, -1.0, 65504.0], np.float32)])
    want = np.array([orc.bf16_to_f32(orc.lib().orc_f32_to_bf16_rne(float(v))) for v in x], np.float32)
    assert np.array_equal(so.bf16_round(x), want)


@pytest.mark.parametrize("Hk,Hv", [(1, 2), (2, 4), (2, 6)])
def test_delta_block_composite_equals_c_block(Hk, Hv):
    # the composed block (used for bf16 prompt tokens) against orc_gdn_layer_decode, three tokens
    rng = np.random.default_rng(Hk * 10 + Hv)
    ch = 2 * Hk * 128 + Hv * 128
    L = dict(conv_w=(0.5 * rng.standard_normal(4 * ch)).astype(np.float32),
             a_log=(-np.exp(rng.standard_normal(Hv))).astype(np.float32),
             dt_bias=rng.standard_normal(Hv).astype(np.float32), ssm_norm=rng.standard_normal(128).astype(np.float32))
    s1 = dict(ring=rng.standard_normal((1, ch, 3)).astype(np.float32),
              state=(0.02 * rng.standard_normal((1, Hv, 128 * 128))).astype(np.float32))
    s2 = {k: v.copy() for k, v in s1.items()}
    for _ in range(3):
        qkv, z = rng.standard_normal(ch).astype(np.float32), rng.standard_normal(Hv * 128).astype(np.float32)
        br, ar = rng.standard_normal(Hv).astype(np.float32), rng.standard_normal(Hv).astype(np.float32)
        a = so.delta_block(L, s1, qkv, z, br, ar, Hk, Hv, 1e-6, composite=True)
        b = so.delta_block(L, s2, qkv, z, br, ar, Hk, Hv, 1e-6)
        assert np.abs(a - b).max() <= 1e-5 * np.abs(b).max()
        assert np.array_equal(s1["ring"], s2["ring"])
        assert np.abs(s1["state"] - s2["state"]).max() < 1e-6


def test_delta_block_bf16_moves_only_by_rounding():
    rng = np.random.default_rng(5)
    Hk, Hv = 1, 2
    ch = 2 * Hk * 128 + Hv * 128
    L = dict(conv_w=(0.5 * rng.standard_normal(4 * ch)).astype(np.float32),
             a_log=(-np.exp(rng.standard_normal(Hv))).astype(np.float32),
             dt_bias=rng.standard_normal(Hv).astype(np.float32), ssm_norm=np.ones(128, np.float32))
    fresh = lambda: dict(ring=np.zeros((1, ch, 3), np.float32), state=np.zeros((1, Hv, 128 * 128), np.float32))  # noqa: E731
    qkv, z = rng.standard_normal(ch).astype(np.float32), rng.standard_normal(Hv * 128).astype(np.float32)
    br, ar = rng.standard_normal(Hv).astype(np.float32), rng.standard_normal(Hv).astype(np.float32)
    a = so.delta_block(L, fresh(), qkv, z, br, ar, Hk, Hv, 1e-6, bf16_qkv=True)
    b = so.delta_block(L, fresh(), qkv, z, br, ar, Hk, Hv, 1e-6)
    err = np.abs(a - b).max() / np.abs(b).max()
    assert 0 < err < 2e-2  # bf16 keeps 8 bits of mantissa


SMALL = dict(n_layer=2, n_embd=256, n_ff=256, n_vocab=64, full_attention_interval=2, n_head=2, n_head_kv=1,
             n_rot=64, ssm_n_k_heads=1, ssm_n_v_heads=2, eps=1e-6, rope_base=1e7)


def test_rq_leaves_its_input_alone():
    from ouroboros_amd.stack import Card

    o = so.StackOracle(Card(**SMALL), seed=3)
    h = np.linspace(-1, 1, 256).astype(np.float32)
    keep = h.copy()
    o._rq(h, o.sign_e)
    assert np.array_equal(h, keep)


def test_run_with_own_tokens_fed_is_greedy_run():
    from ouroboros_amd.stack import Card

    card = Card(**SMALL)
    la, ta = so.StackOracle(card, seed=3).run([[1, 2, 3], [4]], 2)
    lb, tb = so.StackOracle(card, seed=3).run([[1, 2, 3], [4]], 2, feed=ta[:-1])
    assert ta == tb and all(np.array_equal(x, y) for x, y in zip(la, lb))
