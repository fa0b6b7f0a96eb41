"""CPU oracle of the hybrid decoder stack (test infrastructure only).

Restates the reference's per-token stage, one sequence and one token at a
time, with the ternary products on the I2 oracle (int8 absmax activations,
Hadamard-rotated where the reference rotates):
  forward / run_layer      cluster/src/infer/qwen35.rs:730-795
  run_ffn                  qwen35.rs:798-805
  run_delta                qwen35.rs:1048-1158 (delta_block = orc_gdn_layer_decode)
  run_attn, attn_head      qwen35.rs:1160-1240
  rope_partial_neox        qwen35.rs:96-106
  rmsnorm, silu, softmax   ops.rs:12-48
  sample / finite_argmax   qwen35.rs:746-757, infer/mod.rs:70-83
and regenerates the synthetic weights of include/ouro_stack.h from the seed.
Only for small cards: everything is numpy or scalar C.
"""
from __future__ import annotations

import numpy as np

import oracle as orc

# tensor ids (ouroboros_amd/csrc/stack.hip)
(T_ATTN_NORM, T_POST_NORM, T_UP, T_GATE, T_DOWN, T_QKV, T_Z, T_BETA, T_ALPHA, T_OUT, T_CONV, T_DT, T_ALOG,
 T_SSM_NORM, T_Q, T_K, T_V, T_O, T_QN, T_KN) = range(20)
(G_EMBD, G_OUT_NORM, G_LM, G_SIGN_E, G_SIGN_FF, G_SIGN_DI, G_SIGN_Q) = range(7)
GLOBAL = 0x100000
HD = 128
GDN_L2NORM_QK, GDN_SCALE_Q = 1, 2  # orc_gdn_decode flags


def mix3(seed: int, tensor: int, idx: np.ndarray) -> np.ndarray:
    """The stack's 32-bit weight hash of (seed, tensor, index)."""
    idx = np.asarray(idx, dtype=np.uint32)
    with np.errstate(over="ignore"):
        x = np.uint32(seed) ^ np.uint32((tensor * 0x9E3779B9) & 0xFFFFFFFF) ^ (idx * np.uint32(0x85EBCA6B))
        x = x ^ (x >> np.uint32(16))
        x = x * np.uint32(0x7FEB352D)
        x = x ^ (x >> np.uint32(15))
        x = x * np.uint32(0x846CA68B)
        x = x ^ (x >> np.uint32(16))
    return x.astype(np.uint32)


def gen_ternary(seed, tensor, rows, cols):
    codes = (mix3(seed, tensor, np.arange(rows * cols, dtype=np.uint64).astype(np.uint32)) % np.uint32(3))
    return (codes.astype(np.int8) - 1).reshape(rows, cols)


def gen_floats(seed, tensor, n, lo, span):
    h = mix3(seed, tensor, np.arange(n, dtype=np.uint32))
    if span == 0.0:
        return np.where(h & np.uint32(1), np.float32(1.0), np.float32(-1.0)).astype(np.float32)
    u = (h >> np.uint32(8)).astype(np.float32) * np.float32(5.9604644775390625e-8)
    return (np.float32(lo) + np.float32(span) * u).astype(np.float32)


def rot_block(n: int) -> int:
    b = 1
    while b < 4096 and n % (2 * b) == 0:
        b *= 2
    return b


class Lin:
    def __init__(self, seed, tensor, out, inp):
        self.out, self.inp = out, inp
        self.canon = orc.i2_pack(gen_ternary(seed, tensor, out, inp))
        self.scale = np.float32(1.0 / np.sqrt(inp * 2.0 / 3.0))

    def __call__(self, xq, ds):
        # small products run on the calling thread (thread start-up would dominate)
        nt = 1 if self.out * self.inp < (1 << 22) else 0
        return orc.gemm_i2(self.canon, self.out, self.inp, xq, ds, self.scale, nthreads=nt)[1]


def rmsnorm(x, w, eps):
    x = np.asarray(x, np.float32)
    # sequential f32 sum, as ops.rs:14 (np.add.accumulate adds in order, in float32)
    ms = np.add.accumulate((x * x).astype(np.float32), dtype=np.float32)[-1]
    ms = np.float32(ms / np.float32(x.size))
    inv = np.float32(1.0) / np.float32(np.sqrt(np.float32(ms + np.float32(eps))))
    return (x * inv * w).astype(np.float32)


def silu(x):
    x = np.asarray(x, np.float32)
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def rope_partial_neox(v, t, rot, base):
    v = np.array(v, np.float32, copy=True)
    half = rot // 2
    i = np.arange(half, dtype=np.float32)
    theta = (np.float32(1.0) / np.power(np.float32(base), (np.float32(2) * i) / np.float32(rot))).astype(np.float32)
    ang = (np.float32(t) * theta).astype(np.float32)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    a, b = v[:half].copy(), v[half:rot].copy()
    v[:half] = a * c - b * s
    v[half:rot] = b * c + a * s
    return v


def softmax(x):
    m = np.max(x)
    e = np.exp(x - m).astype(np.float32)
    return (e / np.sum(e, dtype=np.float32)).astype(np.float32)


def bf16_round(x):
    """fp32 -> nearest bf16 (ties to even) -> fp32, for finite x."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def delta_block(L, s, qkv, z, braw, araw, Hk, Hv, eps, bf16_qkv=False, composite=None):
    """run_delta between its input and output projections for one token
    (qwen35.rs:1066-1140) on the sequence state s (ring, state; updated).

    Without bf16_qkv this is orc_gdn_layer_decode.  With it, the same block
    is composed here so that the conv outputs can be rounded to bf16 before
    the recurrence (the operands of the chunked prefill): conv_step + SiLU
    per channel (numpy, ring updated), beta and gate per v-head, the
    l2-normed recurrence (orc_gdn_decode), gated RMS norm per head in the
    V-grouped order.  composite=True takes this path without the rounding."""
    if composite is None:
        composite = bf16_qkv
    if not composite:
        return orc.gdn_layer_decode(qkv[None], z[None], braw[None], araw[None], L["dt_bias"], L["a_log"],
                                    L["conv_w"], L["ssm_norm"], s["ring"], s["state"], 1, Hk, Hv, HD,
                                    orc.GDN_V_GROUPED, eps)[0]
    ch, di = qkv.size, Hk * HD
    ring = s["ring"].reshape(ch, 3)
    w = L["conv_w"].reshape(ch, 4)
    x = np.asarray(qkv, np.float32)
    y = (w[:, 0] * ring[:, 0] + w[:, 1] * ring[:, 1] + w[:, 2] * ring[:, 2] + w[:, 3] * x).astype(np.float32)
    ring[:, 0], ring[:, 1], ring[:, 2] = ring[:, 1].copy(), ring[:, 2].copy(), x
    co = (y / (np.float32(1.0) + np.exp(-y))).astype(np.float32)
    if bf16_qkv:
        co = bf16_round(co)
    beta = np.array([orc.sigmoid(float(b)) for b in braw], np.float32)
    gate = np.array([np.float32(L["a_log"][h]) * np.float32(orc.softplus(float(np.float32(araw[h] + L["dt_bias"][h]))))
                     for h in range(Hv)], np.float32)
    o = orc.gdn_decode(s["state"], co[None, :di], co[None, di:2 * di], co[None, 2 * di:], gate[None], beta[None],
                       1, Hk, Hv, HD, GDN_L2NORM_QK | GDN_SCALE_Q, eps)[0]
    out = np.empty(Hv * HD, np.float32)
    rep = Hv // Hk
    for h in range(Hv):
        dst = (h % Hk) * rep + h // Hk
        out[dst * HD:(dst + 1) * HD] = orc.gated_norm_rms(o[h], L["ssm_norm"], z[h * HD:(h + 1) * HD], eps)
    return out


class StackOracle:
    def __init__(self, card, seed: int, bf16_prefill: bool = False):
        self.c, self.seed = card, seed
        self.bf16_prefill = bf16_prefill
        c = card
        self.E, self.F, self.V = c.n_embd, c.n_ff, c.n_vocab
        self.di = c.ssm_n_k_heads * HD
        self.dv = c.ssm_n_v_heads * HD
        self.ch = 2 * self.di + self.dv
        self.qdim, self.kvdim = c.n_head * HD, c.n_head_kv * HD
        g = lambda t: GLOBAL + t  # noqa: E731
        self.embd = gen_floats(seed, g(G_EMBD), self.V * self.E, -1.0, 2.0).reshape(self.V, self.E)
        self.out_norm = gen_floats(seed, g(G_OUT_NORM), self.E, 0.8, 0.4)
        self.lm = Lin(seed, g(G_LM), self.V, self.E)
        self.sign_e = gen_floats(seed, g(G_SIGN_E), self.E, 0.0, 0.0)
        self.sign_ff = gen_floats(seed, g(G_SIGN_FF), self.F, 0.0, 0.0)
        self.sign_di = gen_floats(seed, g(G_SIGN_DI), self.dv, 0.0, 0.0)
        self.sign_q = gen_floats(seed, g(G_SIGN_Q), self.qdim, 0.0, 0.0)
        self.layers = []
        for il in range(c.n_layer):
            t = lambda k: il * 64 + k  # noqa: E731
            L = {"delta": (il + 1) % c.full_attention_interval != 0,
                 "attn_norm": gen_floats(seed, t(T_ATTN_NORM), self.E, 0.8, 0.4),
                 "post_norm": gen_floats(seed, t(T_POST_NORM), self.E, 0.8, 0.4),
                 "up": Lin(seed, t(T_UP), self.F, self.E), "gate": Lin(seed, t(T_GATE), self.F, self.E),
                 "down": Lin(seed, t(T_DOWN), self.E, self.F)}
            if L["delta"]:
                hv = c.ssm_n_v_heads
                L.update(qkv=Lin(seed, t(T_QKV), self.ch, self.E), z=Lin(seed, t(T_Z), self.dv, self.E),
                         beta=Lin(seed, t(T_BETA), hv, self.E), alpha=Lin(seed, t(T_ALPHA), hv, self.E),
                         out=Lin(seed, t(T_OUT), self.E, self.dv),
                         conv_w=gen_floats(seed, t(T_CONV), 4 * self.ch, -0.5, 1.0),
                         dt_bias=gen_floats(seed, t(T_DT), hv, -1.0, 2.0),
                         a_log=gen_floats(seed, t(T_ALOG), hv, -2.0, 1.9),
                         ssm_norm=gen_floats(seed, t(T_SSM_NORM), HD, 0.8, 0.4))
            else:
                L.update(q=Lin(seed, t(T_Q), 2 * self.qdim, self.E), k=Lin(seed, t(T_K), self.kvdim, self.E),
                         v=Lin(seed, t(T_V), self.kvdim, self.E), o=Lin(seed, t(T_O), self.E, self.qdim),
                         qn=gen_floats(seed, t(T_QN), HD, 0.8, 0.4), kn=gen_floats(seed, t(T_KN), HD, 0.8, 0.4))
            self.layers.append(L)

    def new_sequence(self):
        c = self.c
        st = []
        for L in self.layers:
            if L["delta"]:
                st.append({"state": np.zeros((1, c.ssm_n_v_heads, HD * HD), np.float32),
                           "ring": np.zeros((1, self.ch, 3), np.float32)})
            else:
                st.append({"k": [], "v": []})
        return st

    def _rq(self, x, signs):
        """wh then int8 absmax (the rotated-activation input of a ternary product)."""
        # a copy: rotate_rows works in place and the caller may reuse x
        # (run_delta feeds the unrotated h to beta and alpha)
        r = np.array(x, dtype=np.float32, copy=True).reshape(1, -1)
        orc.rotate_rows(r, signs, rot_block(r.shape[1]))
        return orc.act_quant_i8(r)

    def forward(self, st, x, pos, prompt=False):
        """One token through every layer (Qwen35Stage::forward), returns the
        final hidden after output_norm.  prompt: the token is part of a
        prompt (rounds the delta-net q, k, v to bf16 when bf16_prefill)."""
        c = self.c
        x = np.asarray(x, np.float32)
        for L, s in zip(self.layers, st):
            h = rmsnorm(x, L["attn_norm"], c.eps)
            if L["delta"]:
                xq, ds = self._rq(h, self.sign_e)
                qkv, z = L["qkv"](xq, ds), L["z"](xq, ds)
                hq, hds = orc.act_quant_i8(h)
                braw, araw = L["beta"](hq, hds), L["alpha"](hq, hds)
                g = delta_block(L, s, qkv, z, braw, araw, c.ssm_n_k_heads, c.ssm_n_v_heads, c.eps,
                                bf16_qkv=prompt and self.bf16_prefill)
                gq, gds = self._rq(g, self.sign_di)
                o = L["out"](gq, gds)
            else:
                xq, ds = self._rq(h, self.sign_e)
                qf, k, v = L["q"](xq, ds), L["k"](xq, ds), L["v"](xq, ds)
                nh, nkv = c.n_head, c.n_head_kv
                q = np.empty(self.qdim, np.float32)
                gate = np.empty(self.qdim, np.float32)
                for hi in range(nh):
                    qh = rmsnorm(qf[hi * 2 * HD:hi * 2 * HD + HD], L["qn"], c.eps)
                    q[hi * HD:(hi + 1) * HD] = rope_partial_neox(qh, pos, c.n_rot, c.rope_base)
                    gate[hi * HD:(hi + 1) * HD] = qf[hi * 2 * HD + HD:(hi + 1) * 2 * HD]
                kk = np.empty(self.kvdim, np.float32)
                for hi in range(nkv):
                    kh = rmsnorm(k[hi * HD:(hi + 1) * HD], L["kn"], c.eps)
                    kk[hi * HD:(hi + 1) * HD] = rope_partial_neox(kh, pos, c.n_rot, c.rope_base)
                s["k"].append(kk)
                s["v"].append(v.astype(np.float32))
                K, Vv = np.stack(s["k"]), np.stack(s["v"])
                scale = np.float32(1.0 / np.sqrt(np.float32(HD)))
                o_att = np.zeros(self.qdim, np.float32)
                for hi in range(nh):
                    kvh = hi // (nh // nkv)
                    sc = (K[:, kvh * HD:(kvh + 1) * HD] @ q[hi * HD:(hi + 1) * HD]).astype(np.float32) * scale
                    w = softmax(sc)
                    o_att[hi * HD:(hi + 1) * HD] = (w @ Vv[:, kvh * HD:(kvh + 1) * HD]).astype(np.float32)
                o_att = (o_att * (np.float32(1.0) / (np.float32(1.0) + np.exp(-gate)))).astype(np.float32)
                oq, ods = self._rq(o_att, self.sign_q)
                o = L["o"](oq, ods)
            pre = (x + o).astype(np.float32)
            f = rmsnorm(pre, L["post_norm"], c.eps)
            fq, fds = self._rq(f, self.sign_e)
            up, gt = L["up"](fq, fds), L["gate"](fq, fds)
            act = (silu(gt) * up).astype(np.float32)
            aq, ads = self._rq(act, self.sign_ff)
            x = (pre + L["down"](aq, ads)).astype(np.float32)
        return rmsnorm(x, self.out_norm, c.eps)

    def logits(self, hfin):
        xq, ds = self._rq(hfin, self.sign_e)
        return self.lm(xq, ds)

    def run(self, prompts, steps, feed=None):
        """Greedy prefill of every prompt then `steps` decode steps; returns
        the logits after each prompt and after each step ([steps+1][N][V])
        and the greedy tokens ([steps+1][N]).  Decode step i is fed feed[i]
        when given (teacher forcing), else the previous greedy tokens."""
        out_logits, tokens = [], []
        states = [self.new_sequence() for _ in prompts]
        lg_step = []
        for st, p in zip(states, prompts):
            for pos, tok in enumerate(p):
                hfin = self.forward(st, self.embd[tok], pos, prompt=True)
            lg_step.append(self.logits(hfin))
        out_logits.append(np.stack(lg_step))
        tokens.append([orc.finite_argmax(lg) for lg in lg_step])
        for step in range(steps):
            cur = feed[step] if feed is not None else tokens[-1]
            lg_step = []
            for i, (st, p) in enumerate(zip(states, prompts)):
                hfin = self.forward(st, self.embd[cur[i]], len(p) + step)
                lg_step.append(self.logits(hfin))
            out_logits.append(np.stack(lg_step))
            tokens.append([orc.finite_argmax(lg) for lg in lg_step])
        return out_logits, tokens
