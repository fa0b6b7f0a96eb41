/*
 * ouro_stack.h - a Qwen3.5-style hybrid decoder stack on one MI355X, built
 * from the hot-path kernels of ouro_hip.h: gated delta-net layers with
 * full-attention layers every `full_attention_interval`, ternary (I2)
 * projections and FFN on Hadamard-rotated int8 activations, a packed
 * varlen prefill of many prompts followed by batched greedy decode steps.
 *
 * It restates the reference's single-sequence stage (Qwen35Stage::forward,
 * run_layer, run_delta, run_attn, run_ffn, sample:
 * cluster/src/infer/qwen35.rs:730-805, 1048-1240) for a continuous batch;
 * the reference itself runs one sequence at a time (qwen35.rs:1258-1264).
 * Weights are synthetic: generated on the device from `seed` (ternary codes
 * code = mix3(seed, tensor, k) % 3, per-tensor scale 1/sqrt(2/3 in_len),
 * float vectors from the same mix), so a host restatement can rebuild them.
 *
 * All pointers are device pointers unless named *_host; every call after
 * create is asynchronous on `stream` (NULL = default) and allocates nothing.
 */
#ifndef OURO_STACK_H
#define OURO_STACK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t n_layer;                 /* decoder layers */
    int32_t n_embd;                  /* hidden width, a multiple of 256, <= 6144 */
    int32_t n_ff;                    /* FFN width, a multiple of 256, <= 12288 */
    int32_t n_vocab;
    int32_t full_attention_interval; /* layer il is attention iff (il+1) % interval == 0 (qwen35.rs:421-423) */
    int32_t n_head, n_head_kv;       /* attention heads (n_head even, 1..8 x n_head_kv) */
    int32_t head_dim;                /* 128 */
    int32_t n_rot;                   /* rotated dims of rope_partial_neox, a multiple of 4, <= 128 */
    int32_t ssm_n_k_heads, ssm_n_v_heads, ssm_d_state; /* delta-net heads (n_v_heads even, <= 96); d_state 128 */
    float eps, rope_base;
} ouro_stack_card;

typedef struct ouro_stack *ouro_stack_t;

/* Build a stack with synthetic weights.  max_seqs sequences of at most
 * max_ctx tokens each (prompt + generated), at most max_tokens prompt
 * tokens per prefill call.  The attention layers' KV cache is a pool of
 * kv_pages pages of 64 tokens shared by all sequences through a page table
 * (0 = max_seqs * ceil(max_ctx / 64), enough for every sequence at
 * max_ctx); a sequence takes a page when it enters one.  Allocates
 * everything the calls need. */
int ouro_stack_create(const ouro_stack_card *card, uint32_t seed, size_t max_seqs,
                      size_t max_tokens, size_t max_ctx, size_t kv_pages, ouro_stack_t *out);
int ouro_stack_free(ouro_stack_t s);
/* Device bytes the stack holds (weights, caches, activations). */
size_t ouro_stack_device_bytes(ouro_stack_t s);
/* Prefill N prompts packed into tokens[T] (T = cu_seqlens_host[N]), which
 * starts N fresh sequences (state, conv rings reset, every KV page back in
 * the pool), each prompt token by token in the reference's sense (forward,
 * qwen35.rs:730).  next_tokens[N] receives the greedy token after each
 * prompt (sample, qwen35.rs:746-757); logits_or_null[N][n_vocab] its
 * logits.  Synchronises `stream` before it rewrites its pinned index
 * staging; fails (before launching anything) when the prompts need more
 * KV pages than the pool holds. */
int ouro_stack_prefill(ouro_stack_t s, const int32_t *tokens, const int32_t *cu_seqlens_host,
                       size_t N, int32_t *next_tokens, float *logits_or_null, void *stream);
/* One decode step of the N sequences of the last prefill: tokens[N] in,
 * next_tokens[N] (and logits_or_null[N][n_vocab]) out.  Fails, before
 * launching anything, when a sequence would pass max_ctx or the KV page
 * pool is exhausted. */
int ouro_stack_decode(ouro_stack_t s, const int32_t *tokens, int32_t *next_tokens,
                      float *logits_or_null, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OURO_STACK_H */
