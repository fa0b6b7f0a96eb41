"""The hybrid stack at its full size on the GPU: 24 layers (18 gated
delta-net, 6 full attention), hidden 2560, FFN 6912, vocab 248320, ternary
I2 projections on Hadamard-rotated int8 activations (the reference's stage,
cluster/src/infer/qwen35.rs:730-805 forward / run_layer / run_ffn and
1160-1239 run_attn, for a continuous batch).

Checks the mathematics fixes, at this size (and at the config-5 workload
itself: 64 prompts of 16..2048 tokens, then 128 greedy decode steps):
  (i)   a sequence's logits are bit-identical alone and inside a ragged
        batch of 16..2048-token prompts, prefill and decode: the ternary
        products accumulate exact int32 sums and every other operation is
        per row or per sequence;
  (ii)  a prefill of P tokens then one decode step gives the logits of a
        prefill of P + 1 tokens, up to the arithmetic's noise (the prefill
        feeds the recurrence bf16 q, k, v; decode keeps fp32);
  (iii) every logit is finite;
  (iv)  two 3-token prompts with one fed decode step, and three one-token
        prompts, against the CPU oracle of the per-token stage (committed
        fixture tests/golden/stack_full_3tok.npz, written by
        tests/golden/make_stack_full.py).

Why (ii) and (iv) are noise bars and not 1e-3: every product requantises
its input to int8, so an ulp-sized difference anywhere (a reduction order)
flips a few roundings, which grow through 24 layers.  The fixture records
that floor: the oracle against itself with the RMS-norm epsilon moved by
1e-7 differs by NOISE_SINGLE / NOISE_3TOK (relative L2) -- and the oracle
with fp32 delta-net prefill operands differs from the bf16 one by ~10-14 %.
The bars are a small multiple of that floor; a wiring mistake (another
sequence's logits, a wrong head) lands at relative L2 ~1.4 and correlation
~0."""
from pathlib import Path

import numpy as np
import pytest

from ouroboros_amd.device import DeviceBuffer
from ouroboros_amd.stack import Card, Stack

pytestmark = pytest.mark.gpu
G = Path(__file__).resolve().parent / "golden"
CARD = Card()
V = CARD.n_vocab


def l2(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def run(prompts, feeds, seed=1234):
    N = len(prompts)
    lens = [len(p) for p in prompts]
    st = Stack(CARD, seed, max_seqs=N, max_tokens=int(sum(lens)), max_ctx=max(lens) + len(feeds) + 1)
    try:
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        toks = DeviceBuffer.from_host(np.concatenate(prompts).astype(np.int32))
        nxt = DeviceBuffer((N,), np.int32)
        lg = DeviceBuffer((N * V,), np.float32)
        st.prefill(toks, cu, nxt, lg)
        out, tok = [lg.download().reshape(N, V)], [nxt.download()]
        for f in feeds:
            st.decode(DeviceBuffer.from_host(np.asarray(f, np.int32)), nxt, lg)
            out.append(lg.download().reshape(N, V))
            tok.append(nxt.download())
        return out, tok
    finally:
        st.free()


# 40 sequences: the decode step's tall products (the qkv/z/beta/alpha group,
# up/gate) run on the k-split 16x16 MFMA kernel over fragment-ordered int8
# activations (3 column tiles, the last one partial), a sequence decoded
# alone on the one-tile kernel
@pytest.fixture(scope="module")
def batch():
    rng = np.random.default_rng(11)
    lens = rng.integers(16, 2049, 40)
    lens[3], lens[9] = 2048, 16
    prompts = [rng.integers(0, V, int(n)).astype(np.int32) for n in lens]
    feeds = [rng.integers(0, V, 40) for _ in range(2)]
    logits, toks = run(prompts, feeds)
    return prompts, feeds, logits, toks


def test_full_card_logits_finite_and_greedy(gpu, batch):
    _, _, logits, toks = batch
    for lg, tk in zip(logits, toks):
        assert np.isfinite(lg).all()
        assert np.array_equal(tk, lg.argmax(axis=1))  # finite_argmax: first index of the largest


@pytest.mark.parametrize("seq", [3, 9, 0])
def test_full_card_batch_invariance(gpu, batch, seq):
    prompts, feeds, logits, _ = batch
    alone, _ = run([prompts[seq]], [[f[seq]] for f in feeds])
    for i in range(len(alone)):
        assert np.array_equal(alone[i][0].view(np.uint32), logits[i][seq].view(np.uint32)), (seq, i)


@pytest.mark.parametrize("seq,P", [(3, 700), (0, 64), (9, 15)])
def test_full_card_prefill_then_decode(gpu, batch, seq, P):
    prompts = batch[0]
    full, ftok = run([prompts[seq][:P + 1]], [])
    step, stok = run([prompts[seq][:P]], [[prompts[seq][P]]])
    e, c = l2(step[1][0], full[0][0]), float(np.corrcoef(step[1][0], full[0][0])[0, 1])
    print(f"seq {seq} P={P}: relative L2 {e:.4f}, correlation {c:.5f}")
    assert e < BAR_L2 and c > BAR_CORR, (e, c)
    top2 = np.sort(full[0][0])[-2:]
    if top2[1] - top2[0] > 0.05 * np.abs(full[0][0]).max():
        assert stok[1][0] == ftok[0][0]


def test_full_card_against_oracle(gpu):
    f = np.load(G / "stack_full_3tok.npz")
    assert int(f["seed"]) == 1234
    got, toks = run([p for p in f["prompts"]], [list(x) for x in f["feed"]])
    errs = []
    for p in range(2):
        for s in range(2):
            g = got[p][s][f["idx"][p, s]]
            errs.append(l2(g, f["bf16"][p, s]))
            assert toks[p][s] == f["bf16_argmax"][p][s] or abs(
                got[p][s][toks[p][s]] - got[p][s][f["bf16_argmax"][p][s]]) < 0.05 * np.abs(got[p][s]).max()
    one, otoks = run([p for p in f["single"]], [])
    for i in range(len(f["single"])):
        errs.append(l2(one[0][i][f["single_idx"][i]], f["single_bf16"][i]))
    floor = float(max(f["noise_single_l2"].max(), f["noise_3tok_l2"].max()))
    print(f"relative L2 against the bf16-prefill oracle: {np.round(errs, 4).tolist()}; noise floor {floor:.4f}")
    assert floor < BAR_L2  # the committed fixture still carries the floor the bar is set from
    assert max(errs) < BAR_L2, errs


# ---- the config-5 workload: 64 ragged prompts of 16..2048 tokens packed
# varlen, then 128 greedy decode steps of all 64 sequences (four full column
# tiles in every decode product; every sequence crosses at least one 64-token
# KV page boundary while decoding) ----
C5_SEQS, C5_STEPS = 64, 128
C5_KEEP_STEPS = (0, 64, 128)  # prefill's sample, a middle step, the last step
C5_KEEP_SEQS = (0, 2, 4)      # the 2048-token prompt, one 1 short of a page, one 1 short of two pages


def run_greedy(prompts, steps, feeds=None, keep_seqs=(), keep_steps=()):
    """Prefill, then `steps` decode steps fed with the previous step's greedy
    tokens (or with `feeds[t]`).  Checks every step's logits are finite and
    its tokens their argmax; returns the tokens of every step and the kept
    logits {(step, seq): row}."""
    N = len(prompts)
    lens = [len(p) for p in prompts]
    st = Stack(CARD, 1234, max_seqs=N, max_tokens=int(sum(lens)), max_ctx=max(lens) + steps + 1)
    try:
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        toks = DeviceBuffer.from_host(np.concatenate(prompts).astype(np.int32))
        nxt = DeviceBuffer((N,), np.int32)
        lg = DeviceBuffer((N * V,), np.float32)
        st.prefill(toks, cu, nxt, lg)
        kept, all_toks = {}, []
        for t in range(steps + 1):
            if t:
                feed = nxt if feeds is None else DeviceBuffer.from_host(np.asarray(feeds[t - 1], np.int32))
                out = DeviceBuffer((N,), np.int32)
                st.decode(feed, out, lg)
                nxt = out
            logits = lg.download().reshape(N, V)
            tk = nxt.download()
            assert np.isfinite(logits).all(), f"step {t}: non-finite logits"
            assert np.array_equal(tk, logits.argmax(axis=1)), f"step {t}: token is not the argmax"
            all_toks.append(tk)
            if t in keep_steps:
                for sq in keep_seqs:
                    kept[(t, sq)] = logits[sq].copy()
        return all_toks, kept
    finally:
        st.free()


@pytest.fixture(scope="module")
def config5():
    rng = np.random.default_rng(55)
    lens = rng.integers(16, 2049, C5_SEQS)
    lens[0], lens[1], lens[2], lens[3], lens[4], lens[5] = 2048, 62, 63, 126, 127, 16
    prompts = [rng.integers(0, V, int(n)).astype(np.int32) for n in lens]
    toks, kept = run_greedy(prompts, C5_STEPS, keep_seqs=C5_KEEP_SEQS, keep_steps=C5_KEEP_STEPS)
    return prompts, toks, kept


def test_config5_workload_finite_and_greedy(gpu, config5):
    """Every one of the 129 samples (prefill + 128 steps) of all 64 sequences
    has finite logits and is their argmax (checked inside run_greedy)."""
    prompts, toks, _ = config5
    assert len(prompts) == C5_SEQS and len(toks) == C5_STEPS + 1
    assert max(len(p) for p in prompts) == 2048 and min(len(p) for p in prompts) >= 16


@pytest.mark.parametrize("seq", C5_KEEP_SEQS)
def test_config5_workload_batch_invariance(gpu, config5, seq):
    """A sequence run alone along the batch's own greedy path gives the
    batch's logits bit for bit at the first, a middle and the last step."""
    prompts, toks, kept = config5
    feeds = [[toks[t][seq]] for t in range(C5_STEPS)]
    atoks, akept = run_greedy([prompts[seq]], C5_STEPS, feeds=feeds, keep_seqs=(0,), keep_steps=C5_KEEP_STEPS)
    for t in C5_KEEP_STEPS:
        assert np.array_equal(akept[(t, 0)].view(np.uint32), kept[(t, seq)].view(np.uint32)), (seq, t)
    assert all(atoks[t][0] == toks[t][seq] for t in range(C5_STEPS + 1))


@pytest.mark.parametrize("n", [17, 33, 47, 62, 63])
def test_short_prompt_alone_matches_batch(gpu, n):
    """A stack sized for one prompt of n <= 64 tokens (n not a multiple of 16)
    runs its prefill on the few-row path, whose int8 activations are laid out
    in whole 16-row tiles; the buffers hold the padded rows (a prompt of 62
    tokens once wrote 2 rows past them).  Its logits equal the batch's, where
    the same prompt runs on the many-row path, for the prefill and two decode
    steps."""
    rng = np.random.default_rng(n)
    prompts = [rng.integers(0, V, 700).astype(np.int32), rng.integers(0, V, n).astype(np.int32)]
    feeds = [rng.integers(0, V, 2) for _ in range(2)]
    batch, _ = run(prompts, feeds)
    alone, _ = run([prompts[1]], [[f[1]] for f in feeds])
    for i in range(len(alone)):
        assert np.array_equal(alone[i][0].view(np.uint32), batch[i][1].view(np.uint32)), (n, i)


# From the fixture's noise floor: the oracle against itself with the epsilon
# moved by 1e-7 differs by 0.13-0.18 relative L2 (noise_single_l2,
# noise_3tok_l2); unrelated logits differ by ~1.4 with correlation ~0.
BAR_L2 = 0.3
BAR_CORR = 0.95
