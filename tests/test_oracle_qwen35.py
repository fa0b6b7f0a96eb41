"""Oracle delta-net pinned by the qwen35.rs KATs and a float64 brute force."""
import numpy as np
import pytest

S = 128


def test_delta_head_decay_only_when_beta_zero(orc):  # qwen35.rs:225-239
    state = np.full(S * S, 0.5, np.float32)
    q = np.full(S, 0.1, np.float32)
    k = np.full(S, 0.2, np.float32)
    v = np.full(S, 0.3, np.float32)
    out = np.zeros(S, np.float32)
    gate = np.float32(-0.25)
    orc.delta_head_dim(state, S, q, k, v, gate, 0.0, out)
    expect = np.float32(0.5) * np.exp(gate)
    assert (np.abs(state - expect) < 1e-6).all()
    dot_q = np.float32(q.sum()) * expect
    assert (np.abs(out - dot_q) < 1e-4).all()


def test_delta_head_single_write_read(orc):  # qwen35.rs:241-259
    state = np.zeros(S * S, np.float32)
    q = np.zeros(S, np.float32)
    q[5] = orc.delta_q_scale(S)
    k = np.zeros(S, np.float32)
    k[5], k[9] = 2.0, 1.0
    v = np.zeros(S, np.float32)
    v[7] = 4.0
    out = np.zeros(S, np.float32)
    orc.delta_head_dim(state, S, q, k, v, 0.0, 1.0, out)
    assert abs(state[5 + 7 * S] - 8.0) < 1e-6
    assert abs(state[9 + 7 * S] - 4.0) < 1e-6
    for j in range(S):
        if j == 7:
            assert abs(out[j] - 4.0 * orc.delta_q_scale(S) * 2.0) < 1e-6
        else:
            assert abs(out[j]) < 1e-6


def test_delta_head_is_deterministic(orc):  # qwen35.rs:261-274
    q = np.array([((i * 7) % 13) * 0.1 for i in range(S)], np.float32)
    k = np.array([((i * 5) % 11) * 0.1 for i in range(S)], np.float32)
    v = np.array([((i * 3) % 17) * 0.1 for i in range(S)], np.float32)
    s1 = np.full(S * S, 0.3, np.float32)
    s2 = s1.copy()
    o1 = np.zeros(S, np.float32)
    o2 = np.zeros(S, np.float32)
    orc.delta_head_dim(s1, S, q, k, v, -0.1, 0.7, o1)
    orc.delta_head_dim(s2, S, q, k, v, -0.1, 0.7, o2)
    assert np.array_equal(s1, s2) and np.array_equal(o1, o2)


def delta_f64(state, q, k, v, gate, beta):
    """The recurrence in float64, written as matrix algebra: S(i,j) at i + j*d."""
    d = q.size
    Sm = state.astype(np.float64).reshape(d, d).T  # Sm[i, j]
    decay = np.exp(np.float64(gate))
    sk = decay * (Sm.T @ k)
    dv = beta * (v - sk)
    Sm = decay * Sm + np.outer(k, dv)
    return Sm.T.reshape(-1).copy(), Sm.T @ q


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_delta_head_matches_float64(orc, seed):
    rng = np.random.default_rng(seed)
    state = (0.02 * rng.standard_normal(S * S)).astype(np.float32)
    q, k, v = (rng.standard_normal(S).astype(np.float32) for _ in range(3))
    k /= np.linalg.norm(k)
    gate, beta = np.float32(-0.7), np.float32(0.6)
    st = state.copy()
    out = np.zeros(S, np.float32)
    orc.delta_head_dim(st, S, q, k, v, gate, beta, out)
    s64, o64 = delta_f64(state, q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), gate, beta)
    assert np.abs(st - s64).max() < 1e-5 * np.abs(s64).max() + 1e-6
    assert np.abs(out - o64).max() < 1e-5 * np.abs(o64).max() + 1e-6


def test_orientation_column_j_only_touches_column_j(orc):
    # Perturbing column j of S changes only out[j] and column j of S'.
    rng = np.random.default_rng(4)
    state = rng.standard_normal(S * S).astype(np.float32)
    q, k, v = (rng.standard_normal(S).astype(np.float32) for _ in range(3))
    a = state.copy()
    oa = np.zeros(S, np.float32)
    orc.delta_head_dim(a, S, q, k, v, -0.2, 0.5, oa)
    b = state.copy()
    b[3 + 11 * S] += 1.0
    ob = np.zeros(S, np.float32)
    orc.delta_head_dim(b, S, q, k, v, -0.2, 0.5, ob)
    diff_cols = np.nonzero(np.any(a.reshape(S, S) != b.reshape(S, S), axis=1))[0]
    assert list(diff_cols) == [11]
    assert list(np.nonzero(oa != ob)[0]) == [11]


def test_l2_norm_unit_length(orc):  # qwen35.rs:293-299
    v = np.array([3.0, 4.0, 0.0, 0.0], np.float32)
    orc.l2_norm(v, 1e-12)
    assert abs(v[0] - 0.6) < 1e-6 and abs(v[1] - 0.8) < 1e-6


def test_gated_norm_rms(orc):  # qwen35.rs:301-311
    x = np.ones(4, np.float32)
    w = np.ones(4, np.float32)
    y = orc.gated_norm_rms(x, w, np.zeros(4, np.float32), 1e-5)
    assert (np.abs(y) < 1e-6).all()
    y2 = orc.gated_norm_rms(x, w, np.full(4, 10.0, np.float32), 1e-5)
    assert abs(y2[0] - 10.0) < 0.1


def test_conv_step(orc):  # qwen35.rs:276-291
    ring = np.array([3.0, 3.0, 3.0], np.float32)
    assert abs(orc.conv_step(ring, [0.25] * 4, 3.0) - 3.0) < 1e-6
    assert list(ring) == [3.0, 3.0, 3.0]
    ring = np.array([1.0, 2.0, 3.0], np.float32)
    assert abs(orc.conv_step(ring, [0, 0, 0, 1.0], 9.0) - 9.0) < 1e-6
    assert list(ring) == [2.0, 3.0, 9.0]


def test_softplus_and_sigmoid(orc):  # qwen35.rs:1241-1243, 1067
    assert orc.softplus(25.0) == 25.0
    assert abs(orc.softplus(0.0) - np.log(2.0)) < 1e-6
    assert abs(orc.sigmoid(0.0) - 0.5) < 1e-7
    assert abs(orc.silu(10.0) - 10.0) < 1e-3


def test_gdn_decode_is_per_head_loop(orc):
    # orc_gdn_decode == run_delta's per-head loop (qwen35.rs:1096-1112) built
    # here from the single-head pieces: l2_norm, q scale, k-head = v % Hk.
    rng = np.random.default_rng(9)
    B, Hk, Hv, d, eps = 2, 2, 4, S, 1e-6
    state = (0.02 * rng.standard_normal((B, Hv, d * d))).astype(np.float32)
    q = rng.standard_normal((B, Hk, d)).astype(np.float32)
    k = rng.standard_normal((B, Hk, d)).astype(np.float32)
    v = rng.standard_normal((B, Hv, d)).astype(np.float32)
    gate = -np.log1p(np.exp(rng.standard_normal((B, Hv)))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, Hv))))).astype(np.float32)
    st = state.copy()
    out = orc.gdn_decode(st, q, k, v, gate, beta, B, Hk, Hv, d, orc.L2NORM_QK | orc.SCALE_Q, eps, 2)
    for b in range(B):
        for h in range(Hv):
            kh = h % Hk
            qq, kk = q[b, kh].copy(), k[b, kh].copy()
            orc.l2_norm(qq, eps)
            orc.l2_norm(kk, eps)
            qq = (qq * np.float32(orc.delta_q_scale(d))).astype(np.float32)
            s1 = state[b, h].copy()
            o1 = np.zeros(d, np.float32)
            orc.delta_head_dim(s1, d, qq, kk, v[b, h], gate[b, h], beta[b, h], o1)
            assert np.array_equal(s1, st[b, h]) and np.array_equal(o1, out[b, h])


def test_prefill_tokens_equals_repeated_decode(orc):
    rng = np.random.default_rng(10)
    T, Hk, Hv, d = 5, 1, 2, S
    state = (0.02 * rng.standard_normal((Hv, d * d))).astype(np.float32)
    q = rng.standard_normal((T, Hk, d)).astype(np.float32)
    k = rng.standard_normal((T, Hk, d)).astype(np.float32)
    v = rng.standard_normal((T, Hv, d)).astype(np.float32)
    gate = -np.abs(rng.standard_normal((T, Hv))).astype(np.float32)
    beta = rng.random((T, Hv)).astype(np.float32)
    fl = orc.L2NORM_QK | orc.SCALE_Q
    a = state.copy()
    out = orc.gdn_prefill_tokens(a, q, k, v, gate, beta, T, Hk, Hv, d, fl, 1e-6)
    b = state.copy()[None]
    for t in range(T):
        o = orc.gdn_decode(b, q[t:t + 1], k[t:t + 1], v[t:t + 1], gate[t:t + 1], beta[t:t + 1], 1, Hk, Hv, d, fl, 1e-6)
        assert np.array_equal(o[0], out[t])
    assert np.array_equal(a, b[0])


def layer_inputs(rng, B, Hk, Hv, d=S):
    ch = 2 * Hk * d + Hv * d
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    return dict(qkv=f(B, ch), z=f(B, Hv * d), beta_raw=f(B, Hv), alpha_raw=f(B, Hv), dt_bias=f(Hv),
                a_log=(-np.exp(f(Hv))).astype(np.float32), conv_w=(0.5 * f(ch, 4)).astype(np.float32),
                norm_w=f(d), conv=f(B, ch, 3), state=(0.02 * f(B, Hv, d * d)).astype(np.float32))


def layer_f64(x, B, Hk, Hv, d, flags, eps):
    """run_delta's block in float64 numpy: conv over the ring, matrix-form
    recurrence per head, gated RMS norm, optional V-grouped permutation."""
    qkv, ring = x["qkv"].astype(np.float64), x["conv"].astype(np.float64)
    w = x["conv_w"].astype(np.float64)
    y = (ring * w[None, :, :3]).sum(-1) + w[None, :, 3] * qkv
    co = y / (1 + np.exp(-y))
    new_ring = np.concatenate([ring[:, :, 1:], qkv[:, :, None]], axis=2)
    beta = 1 / (1 + np.exp(-x["beta_raw"].astype(np.float64)))
    sp = x["alpha_raw"].astype(np.float64) + x["dt_bias"].astype(np.float64)
    sp = np.where(sp > 20, sp, np.log1p(np.exp(np.minimum(sp, 20))))
    gate = x["a_log"].astype(np.float64) * sp
    di = Hk * d
    st = x["state"].astype(np.float64).reshape(B, Hv, d, d)  # [b][h][j][i]: S(i, j) at i + j d
    out = np.zeros((B, Hv * d))
    for b in range(B):
        for h in range(Hv):
            kh = h // (Hv // Hk) if flags & 4 else h % Hk
            q = co[b, kh * d:(kh + 1) * d]
            k = co[b, di + kh * d:di + (kh + 1) * d]
            v = co[b, 2 * di + h * d:2 * di + (h + 1) * d]
            q = q / (np.sqrt((q * q).sum()) + eps) / np.sqrt(d)
            k = k / (np.sqrt((k * k).sum()) + eps)
            Sm = st[b, h].T  # Sm[i][j]
            dec = np.exp(gate[b, h])
            dv = beta[b, h] * (v - dec * Sm.T @ k)
            Sm = dec * Sm + np.outer(k, dv)
            st[b, h] = Sm.T
            o = Sm.T @ q
            zz = x["z"][b, h * d:(h + 1) * d].astype(np.float64)
            g = o / np.sqrt((o * o).mean() + eps) * x["norm_w"] * (zz / (1 + np.exp(-zz)))
            dst = (h % Hk) * (Hv // Hk) + h // Hk if flags & 8 else h
            out[b, dst * d:(dst + 1) * d] = g
    return out, new_ring, st.reshape(B, Hv, d * d)


@pytest.mark.parametrize("flags", [0, 4, 8, 12])
def test_layer_block_matches_float64(orc, flags):
    rng = np.random.default_rng(40 + flags)
    B, Hk, Hv = 2, 2, 4
    x = layer_inputs(rng, B, Hk, Hv)
    want, ring, st = layer_f64(x, B, Hk, Hv, S, flags, 1e-6)
    conv, state = x["conv"].copy(), x["state"].copy()
    got = orc.gdn_layer_decode(x["qkv"], x["z"], x["beta_raw"], x["alpha_raw"], x["dt_bias"], x["a_log"],
                               x["conv_w"], x["norm_w"], conv, state, B, Hk, Hv, S, flags, 1e-6)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5
    assert np.array_equal(conv, ring.astype(np.float32))  # the ring shifts exactly
    assert np.abs(state - st).max() / np.abs(st).max() < 1e-5


def test_layer_block_v_grouped_is_a_head_permutation(orc):
    # qwen35.rs:1126-1135: v-head r*nk + k lands at k*rep + r.
    rng = np.random.default_rng(7)
    B, Hk, Hv = 1, 2, 6
    x = layer_inputs(rng, B, Hk, Hv)
    args = lambda: [x[n] for n in ("qkv", "z", "beta_raw", "alpha_raw", "dt_bias", "a_log", "conv_w", "norm_w")]  # noqa: E731
    plain = orc.gdn_layer_decode(*args(), x["conv"].copy(), x["state"].copy(), B, Hk, Hv, S, 0, 1e-6)
    grouped = orc.gdn_layer_decode(*args(), x["conv"].copy(), x["state"].copy(), B, Hk, Hv, S,
                                   orc.GDN_V_GROUPED, 1e-6)
    rep = Hv // Hk
    for k in range(Hk):
        for r in range(rep):
            src, dst = (r * Hk + k) * S, (k * rep + r) * S
            assert np.array_equal(grouped[0, dst:dst + S], plain[0, src:src + S])
