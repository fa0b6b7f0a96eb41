"""One layer of the hybrid stack at the config-5 widths (hidden 2560, FFN
6912, 16 query / 4 KV heads of 128 with a 64-dim partial rope, 16 k / 32 v
delta-net heads of 128), against the CPU oracle of the reference's
per-token stage (oracle/stack_oracle.py; qwen35.rs:730-805, 1048-1239),
with a small vocabulary so the oracle runs in seconds: a ragged prefill of
three prompts, then two decode steps fed the oracle's greedy tokens.

The full 24-layer card can only be held to a loose bar: every ternary
product requantises its input to int8, and the flips that a last-bit change
causes grow through the layers (the oracle differs from itself by 5-6 %
after 4 layers and 13-18 % relative L2 after 24 when the RMS-norm epsilon
moves by 1e-7).  One layer keeps those flips few, so each layer kind is
held here to a bar set from its own noise floor, measured on the CPU:

- attention layer: a change that flips only a few int8 roundings (the
  epsilon moved by 1e-6) moves the oracle's logits by 0.9-1.3 % of the
  largest and 0.7 % in relative L2 (one flipped activation moves some
  logits by about one int8 step of a product), so the GPU (fp32 MFMA
  attention in another summation order) is held to 5 % max-abs and 3 % L2;
- delta-net layer: the epsilon moved by 1e-7 moves the oracle by 2.0-2.7 %
  of the largest logit, and the bf16 q/k/v of the GPU's chunked prefill by
  1.4-1.6 %, so the GPU is held to 5 % of the bf16-prefill oracle and 10 % of
  the fp32 one (the bars of the small-card tests), a wiring mistake moving
  the logits by tens of percent."""
import dataclasses

import numpy as np
import pytest

from ouroboros_amd.device import DeviceBuffer
from ouroboros_amd.stack import Card, Stack

pytestmark = pytest.mark.gpu

VOCAB = 2048
ATTN1 = dataclasses.replace(Card(), n_layer=1, n_vocab=VOCAB, full_attention_interval=1)
DELTA1 = dataclasses.replace(Card(), n_layer=1, n_vocab=VOCAB)  # layer 0 of the 3:1 pattern is a delta-net layer


def prompts():
    rng = np.random.default_rng(3)
    return [rng.integers(0, VOCAB, n).astype(np.int32) for n in (9, 3, 1)]


def rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


def gpu_run(card, ps, feed, max_ctx=32):
    N = len(ps)
    st = Stack(card, 7, max_seqs=N, max_tokens=int(sum(len(p) for p in ps)), max_ctx=max_ctx)
    try:
        cu = np.concatenate([[0], np.cumsum([len(p) for p in ps])]).astype(np.int32)
        toks = DeviceBuffer.from_host(np.concatenate(ps).astype(np.int32))
        nxt = DeviceBuffer((N,), np.int32)
        lg = DeviceBuffer((N * card.n_vocab,), np.float32)
        st.prefill(toks, cu, nxt, lg)
        logits, tokens = [lg.download().reshape(N, card.n_vocab)], [nxt.download()]
        for f in feed:
            st.decode(DeviceBuffer.from_host(np.asarray(f, np.int32)), nxt, lg)
            logits.append(lg.download().reshape(N, card.n_vocab))
            tokens.append(nxt.download())
    finally:
        st.free()
    return logits, tokens


def test_full_width_attention_layer(gpu, margin):
    from oracle.stack_oracle import StackOracle

    ps = prompts()
    want, wtok = StackOracle(ATTN1, seed=7).run(ps, 2)
    got, gtok = gpu_run(ATTN1, ps, wtok[:-1])
    errs = [rel(g, w) for g, w in zip(got, want)]
    l2s = [float(np.linalg.norm(g - w) / np.linalg.norm(w)) for g, w in zip(got, want)]
    for i, (g, w) in enumerate(zip(got, want)):
        margin(f"attention layer 2560 wide, step {i}", g, w, 5e-2)
    print("attention layer vs fp32 oracle: max-abs", errs, "L2", l2s)
    assert max(errs) < 5e-2, errs
    assert max(l2s) < 3e-2, l2s
    # greedy tokens agree wherever the oracle's top two logits are apart
    for g, w, lg in zip(gtok, wtok, want):
        top2 = np.sort(lg, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 0.1 * np.abs(lg).max(axis=1)
        assert np.array_equal(np.asarray(g)[clear], np.asarray(w)[clear])


def test_full_width_delta_layer(gpu, margin):
    from oracle.stack_oracle import StackOracle

    ps = prompts()
    l32, t32 = StackOracle(DELTA1, seed=7).run(ps, 2)
    l16, _ = StackOracle(DELTA1, seed=7, bf16_prefill=True).run(ps, 2, feed=t32[:-1])
    got, _ = gpu_run(DELTA1, ps, t32[:-1])
    e16 = [rel(g, w) for g, w in zip(got, l16)]
    e32 = [rel(g, w) for g, w in zip(got, l32)]
    for i, (g, w) in enumerate(zip(got, l16)):
        margin(f"delta-net layer 2560 wide, step {i}", g, w, 5e-2)
    print("delta-net layer vs bf16-prefill oracle:", e16, "vs fp32 oracle:", e32)
    assert max(e16) < 5e-2, e16
    assert max(e32) < 0.1, e32


def long_prompts():
    rng = np.random.default_rng(5)
    return [rng.integers(0, VOCAB, n).astype(np.int32) for n in (300, 131)]


def test_full_width_layers_long_prefill(gpu, margin):
    """The same layers over 431 prompt tokens: enough columns that the
    projections run on the 32x32x32 ternary GEMM (its row-major and SwiGLU
    epilogues) and the attention covers five 64-key pages of one prompt,
    against the same oracles at the same bars (one decode step after)."""
    from oracle.stack_oracle import StackOracle

    ps = long_prompts()
    want, wtok = StackOracle(ATTN1, seed=7).run(ps, 1)
    got, _ = gpu_run(ATTN1, ps, wtok[:-1], max_ctx=320)
    ea = [rel(g, w) for g, w in zip(got, want)]
    for i, (g, w) in enumerate(zip(got, want)):
        margin(f"attention layer, 431 tokens, step {i}", g, w, 5e-2)
    l32, t32 = StackOracle(DELTA1, seed=7).run(ps, 1)
    l16, _ = StackOracle(DELTA1, seed=7, bf16_prefill=True).run(ps, 1, feed=t32[:-1])
    gd, _ = gpu_run(DELTA1, ps, t32[:-1], max_ctx=320)
    e16 = [rel(g, w) for g, w in zip(gd, l16)]
    for i, (g, w) in enumerate(zip(gd, l16)):
        margin(f"delta-net layer, 431 tokens, step {i}", g, w, 5e-2)
    print("431-token prefill: attention", ea, "delta-net vs bf16 oracle", e16)
    assert max(ea) < 5e-2, ea
    assert max(e16) < 5e-2, e16

