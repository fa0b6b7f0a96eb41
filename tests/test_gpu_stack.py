"""Hybrid decoder stack (include/ouro_stack.h) against the CPU oracle of the
reference's per-token stage (oracle/stack_oracle.py) on small cards: a
ragged packed prefill of several prompts, then decode steps fed the fp32
oracle's greedy tokens (teacher forcing, so every step compares the same
history).

Every ternary product requantises its input to int8, so a perturbation of
any size flips a few roundings and moves the logits by about one int8 step:
on these cards a relative change of 1e-6 in the delta-net conv outputs
already moves the logits by up to 1.5% of their largest magnitude (two
oracle runs on the CPU).  The GPU prefill feeds the delta-net recurrence
bf16 q, k, v (the MFMA operands of the chunked prefill) and computes the
chunk algebra to ~16 bits; the oracle run with the same bf16 rounding
(bf16_prefill=True) is matched to TOL_BF16, a few int8 steps, and the fp32
token-by-token oracle (the reference's own arithmetic; bf16 alone moves the
logits by up to ~5%) to TOL_F32.  A wiring mistake (a wrong operand, head
order or state hand-off) moves them by tens of percent."""
import numpy as np
import pytest

from ouroboros_amd._lib import OuroError
from ouroboros_amd.device import DeviceBuffer
from ouroboros_amd.stack import Card, Stack

pytestmark = pytest.mark.gpu

TOL_BF16 = 5e-2
TOL_F32 = 0.1

SMALL = Card(n_layer=4, n_embd=256, n_ff=512, n_vocab=512, full_attention_interval=2, n_head=2, n_head_kv=1,
             n_rot=64, ssm_n_k_heads=1, ssm_n_v_heads=2, eps=1e-6, rope_base=1e7)
# wider heads: GQA 4:2, Hk=2 Hv=4 (V-grouped order matters), 3 delta + 1 attention layer
WIDE = Card(n_layer=4, n_embd=512, n_ff=768, n_vocab=1000, full_attention_interval=4, n_head=4, n_head_kv=2,
            n_rot=32, ssm_n_k_heads=2, ssm_n_v_heads=4, eps=1e-6, rope_base=1e6)


def rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


def oracle_runs(card, prompts, steps):
    from oracle.stack_oracle import StackOracle

    l32, t32 = StackOracle(card, seed=7).run(prompts, steps)
    l16, t16 = StackOracle(card, seed=7, bf16_prefill=True).run(prompts, steps, feed=t32[:-1])
    return l32, t32, l16, t16


def gpu_run(card, prompts, feed, max_seqs=4, max_tokens=64, max_ctx=32):
    N, V = len(prompts), card.n_vocab
    st = Stack(card, 7, max_seqs=max_seqs, max_tokens=max_tokens, max_ctx=max_ctx)
    try:
        cu = np.concatenate([[0], np.cumsum([len(p) for p in prompts])]).astype(np.int32)
        toks = DeviceBuffer.from_host(np.concatenate(prompts).astype(np.int32))
        nxt = DeviceBuffer((N,), np.int32)
        lg = DeviceBuffer((N * V,), np.float32)
        st.prefill(toks, cu, nxt, lg)
        logits, tokens = [lg.download().reshape(N, V)], [nxt.download()]
        for f in feed:
            st.decode(DeviceBuffer.from_host(np.array(f, np.int32)), nxt, lg)
            logits.append(lg.download().reshape(N, V))
            tokens.append(nxt.download())
    finally:
        st.free()
    return logits, tokens


def check(card, prompts, steps, **kw):
    l32, t32, l16, t16 = oracle_runs(card, prompts, steps)
    got, gtok = gpu_run(card, prompts, t32[:-1], **kw)
    e16 = [rel(g, w) for g, w in zip(got, l16)]
    e32 = [rel(g, w) for g, w in zip(got, l32)]
    print("vs bf16-prefill oracle", e16, "vs fp32 oracle", e32)
    assert max(e16) < TOL_BF16, e16
    assert max(e32) < TOL_F32, e32
    # greedy tokens agree with the matching oracle wherever its top two logits are apart
    for g, w, lg in zip(gtok, t16, l16):
        top2 = np.sort(lg, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2 * TOL_BF16 * np.abs(lg).max(axis=1)
        assert np.array_equal(np.asarray(g)[clear], np.asarray(w)[clear])


def test_stack_matches_oracle(gpu):
    rng = np.random.default_rng(3)
    prompts = [list(rng.integers(0, SMALL.n_vocab, n)) for n in (5, 9, 2)]
    check(SMALL, prompts, 3)


def test_stack_single_token_prompts(gpu):
    check(SMALL, [[5], [511], [0]], 2)


def test_stack_attention_only_single_token_matches_oracle_closely(gpu):
    # no delta layers (no bf16 anywhere) and one key per sequence: everything
    # from the synthetic weights to the head runs the oracle's arithmetic
    # up to summation order, so the logits agree far inside one int8 step
    from oracle.stack_oracle import StackOracle

    card = Card(n_layer=2, n_embd=256, n_ff=512, n_vocab=512, full_attention_interval=1, n_head=2, n_head_kv=1,
                n_rot=64, ssm_n_k_heads=1, ssm_n_v_heads=2, eps=1e-6, rope_base=1e7)
    prompts = [[5], [17], [300]]
    want, _ = StackOracle(card, seed=7).run(prompts, 0)
    got, _ = gpu_run(card, prompts, [])
    assert rel(got[0], want[0]) < 1e-4, rel(got[0], want[0])


def test_stack_long_ragged_prompts_wide_heads(gpu):
    # prompts across the 64-token chunk and attention-tile edges, one of length 1
    rng = np.random.default_rng(4)
    prompts = [list(rng.integers(0, WIDE.n_vocab, n)) for n in (70, 1, 64, 129)]
    check(WIDE, prompts, 2, max_seqs=4, max_tokens=300, max_ctx=160)


def test_stack_decode_over_several_splits(gpu):
    # decode attention splits the keys in runs of 256 (plus a combine pass):
    # contexts of 301 and 521 keys cover full, partial and single-page splits
    rng = np.random.default_rng(8)
    prompts = [list(rng.integers(0, SMALL.n_vocab, n)) for n in (300, 5, 520)]
    check(SMALL, prompts, 2, max_seqs=4, max_tokens=900, max_ctx=600)


# a wide FFN: its up/gate pair (10752 rows) is tall enough for the 16x16
# MFMA kernel at more than 32 columns
FFN_TALL = Card(n_layer=2, n_embd=256, n_ff=5376, n_vocab=512, full_attention_interval=2, n_head=2, n_head_kv=1,
                n_rot=64, ssm_n_k_heads=1, ssm_n_v_heads=2, eps=1e-6, rope_base=1e7)


def test_stack_wide_ffn_long_prefill(gpu):
    # 825 prompt tokens through the wide FFN: the prefill's interleaved
    # up/gate product runs on the 256 x 128 tile kernel and writes
    # silu(gate) * up from its epilogue
    rng = np.random.default_rng(9)
    prompts = [list(rng.integers(0, FFN_TALL.n_vocab, n)) for n in (300, 5, 520)]
    check(FFN_TALL, prompts, 2, max_seqs=4, max_tokens=900, max_ctx=600)


# many delta-net heads: the decode step's qkv/z/beta/alpha group (12352
# rows) runs on the 16x16 MFMA kernel with the conv and gates in its epilogue
DELTA_WIDE = Card(n_layer=2, n_embd=256, n_ff=256, n_vocab=512, full_attention_interval=2, n_head=2, n_head_kv=1,
                  n_rot=64, ssm_n_k_heads=16, ssm_n_v_heads=32, eps=1e-6, rope_base=1e7)


@pytest.mark.parametrize("card,nseq", [(SMALL, 64), (FFN_TALL, 40), (FFN_TALL, 64), (DELTA_WIDE, 40)])
def test_stack_many_sequences(gpu, card, nseq):
    # more than 32 sequences: the decode step's int8 activations go out in
    # fragment order over 3 or 4 column tiles (the last one partial for 40);
    # the short products split k over the waves, the wide FFN's up/gate pair
    # runs on the grouped 16x16 MFMA kernel (64 sequences is the
    # configuration of the 64-sequence benchmark)
    rng = np.random.default_rng(6)
    prompts = [list(rng.integers(0, card.n_vocab, int(n))) for n in rng.integers(1, 4, nseq)]
    check(card, prompts, 2, max_seqs=64, max_tokens=256, max_ctx=16)


# two layers (one delta-net, one attention) keep the oracle quick for many sequences
MANY = Card(n_layer=2, n_embd=256, n_ff=512, n_vocab=512, full_attention_interval=2, n_head=2, n_head_kv=1,
            n_rot=64, ssm_n_k_heads=1, ssm_n_v_heads=2, eps=1e-6, rope_base=1e7)


def test_stack_more_than_64_sequences(gpu):
    # 72 sequences: decode steps take the path for more than 64 sequences
    # (conv and gates in their own kernel, one launch per product, row-major
    # activations), and the 66 prompts of exactly 64 tokens all enter a new
    # KV page on the first decode step, more assignments than one batch (64)
    from oracle.stack_oracle import StackOracle

    rng = np.random.default_rng(12)
    lens = [64] * 66 + [1, 2, 3, 5, 9, 17]
    prompts = [list(rng.integers(0, MANY.n_vocab, n)) for n in lens]
    steps = 2
    l16, t16 = StackOracle(MANY, seed=7, bf16_prefill=True).run(prompts, steps)
    got, gtok = gpu_run(MANY, prompts, t16[:-1], max_seqs=72, max_tokens=sum(lens), max_ctx=64 + steps + 1)
    e16 = [rel(g, w) for g, w in zip(got, l16)]
    print("72 sequences vs bf16-prefill oracle", e16)
    assert max(e16) < TOL_BF16, e16
    for g, w, lg in zip(gtok, t16, l16):
        top2 = np.sort(lg, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2 * TOL_BF16 * np.abs(lg).max(axis=1)
        assert np.array_equal(np.asarray(g)[clear], np.asarray(w)[clear])


def test_stack_rejects_bad_calls(gpu):
    st = Stack(SMALL, 7, max_seqs=2, max_tokens=10, max_ctx=8)
    try:
        nxt = DeviceBuffer((4,), np.int32)
        toks = DeviceBuffer.from_host(np.zeros(32, np.int32))
        with pytest.raises(OuroError):  # decode before any prefill
            st.decode(toks, nxt)
        for cu in ([0, 1, 2, 3], [0, 8], [0, 0, 3], [1, 3], [0, 6, 12]):
            # too many sequences, prompt >= max_ctx, empty prompt, bad start, > max_tokens
            with pytest.raises(OuroError):
                st.prefill(toks, np.array(cu, np.int32), nxt)
        st.prefill(toks, np.array([0, 7], np.int32), nxt)  # 7 tokens fill max_ctx - 1
        st.decode(toks, nxt)  # 8th position
        with pytest.raises(OuroError):  # the context is full
            st.decode(toks, nxt)
    finally:
        st.free()


def test_stack_kv_page_pool(gpu):
    # 64-token pages: two 64-token prompts take 2 pages; their first decode
    # step enters a new page each, so a pool of 3 runs dry, a pool of 4 does not
    rng = np.random.default_rng(5)
    prompts = [list(rng.integers(0, SMALL.n_vocab, 64)), list(rng.integers(0, SMALL.n_vocab, 64))]
    cu = np.array([0, 64, 128], np.int32)
    toks = DeviceBuffer.from_host(np.concatenate(prompts).astype(np.int32))
    nxt = DeviceBuffer((2,), np.int32)
    small = Stack(SMALL, 7, max_seqs=2, max_tokens=128, max_ctx=200, kv_pages=1)
    try:
        with pytest.raises(OuroError):  # the prompts alone need 2 pages
            small.prefill(toks, cu, nxt)
    finally:
        small.free()
    st = Stack(SMALL, 7, max_seqs=2, max_tokens=128, max_ctx=200, kv_pages=3)
    try:
        st.prefill(toks, cu, nxt)
        with pytest.raises(OuroError):
            st.decode(nxt, nxt)
    finally:
        st.free()
    got = []
    for pages in (4, 0):  # exactly enough, and the default max_seqs * ceil(max_ctx / 64)
        st = Stack(SMALL, 7, max_seqs=2, max_tokens=128, max_ctx=200, kv_pages=pages)
        try:
            lg = DeviceBuffer((2 * SMALL.n_vocab,), np.float32)
            st.prefill(toks, cu, nxt, lg)
            fed = DeviceBuffer.from_host(np.array([3, 4], np.int32))
            for _ in range(3):
                st.decode(fed, nxt, lg)
            got.append(lg.download())
        finally:
            st.free()
    assert np.array_equal(got[0], got[1])
