// stack.hip - the hybrid decoder stack runner (ouro_stack.h): the
// reference's per-token stage (Qwen35Stage::forward / run_layer,
// qwen35.rs:730-805) restated for a continuous batch on one GPU.  Host code
// only: every step is a launch of a hot-path kernel (ternary MFMA GEMM on
// Hadamard-rotated int8 activations, delta-net chunked prefill and decode
// layer block) or of stack_ops.hip, all on the caller's stream, into
// buffers sized at creation.
#include "common.hpp"

#include "../../include/ouro_stack.h"

#include <algorithm>
#include <cmath>
#include <initializer_list>
#include <new>
#include <vector>

namespace ouro {
// hot-path kernels
size_t i2_mfma_bytes(size_t out_len, size_t in_len);
int i2_tile_mfma(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *dst, const float *w_scale,
                 void *stream, int src_i2s);
int i2_gemm_mfma(const uint8_t *w_mfma, size_t out_len, size_t in_len, const float *w_scale, const int8_t *xq,
                 const float *act_scale, size_t ncols, float *y, int32_t *acc, void *stream, int x_tiled, int swiglu = 0,
                 const GemmEpilogue *epi = nullptr);
size_t gdn_chunk_ws_bytes(size_t T, size_t N, size_t Hv);
int gdn_chunk_prefill(float *state, const void *q, const void *k, const void *v, const float *gate,
                      const float *beta, float *out, const int32_t *cu_host, size_t N, size_t T, size_t Hk,
                      size_t Hv, size_t d, size_t chunk, unsigned flags, float eps, void *workspace, void *stream);
size_t gdn_layer_ws_bytes(size_t B, size_t Hk, size_t Hv);
int gdn_decode(float *state, const void *q, const void *k, int qk_dtype, const void *v, int v_dtype,
               const float *gate, const float *beta, float gate_s, float beta_s, float *out,
               size_t B, size_t Hk, size_t Hv, size_t d, unsigned flags, float eps, void *stream,
               size_t qk_bs, size_t v_bs);
int gdn_decode_core(const float *qkv, const float *beta_raw, const float *alpha_raw, const float *dt_bias,
                    const float *a_log, const float *conv_w, float *conv, float *state, float *o, size_t B, size_t Hk,
                    size_t Hv, unsigned flags, float eps, void *workspace, void *stream);
int row_rotate_quant(int pro, const float *a, const float *b, const float *w, float *sum_out, size_t rows,
                     size_t n, size_t block, const float *signs, int8_t *xq, float *ds, int8_t *xq2, float *ds2,
                     int tiles, int Hk, int Hv, unsigned flags, float eps, void *stream);
enum { RQ_COPY = 0, RQ_NORM = 1, RQ_SWIGLU = 2, RQ_GNORM = 3 };  // row_rotate_quant prologues (fwht.hip)
// stack_ops.hip
int fill_zero(float *p, size_t n, void *stream);
int lens_step(int32_t *lens, int32_t *pos, int32_t *klen, size_t B, int32_t *pages, const PageAssign &pa,
              void *stream);
int gen_codes(uint32_t seed, uint32_t tensor, size_t rows, size_t cols, uint8_t *dst, void *stream);
int gen_floats(uint32_t seed, uint32_t tensor, size_t n, float lo, float span, float *dst, void *stream);
int embed_rows(const int32_t *tokens, const float *table, float *x, size_t n_tok, size_t n_vocab, size_t n_embd,
               void *stream);
int gather_rows(const float *src, const int32_t *rows_idx, float *dst, size_t n, size_t width, void *stream);
int attn_prep(const float *qfull, const float *k, const float *v, const float *qn, const float *kn,
              const int32_t *pos, const int32_t *seq, const int32_t *pages, int maxp, float *q_out, float *gate_out,
              float *kc, float *vc, size_t T, int nh, int nkv, int n_rot, float rope_base, float eps, void *stream);
int attn_prefill(const float *q, const float *gate, const float *kc, const float *vc, const int32_t *pages, int maxp,
                 const int32_t *cu, const int32_t *tile_seq, const int32_t *tile_p0, size_t n_tiles, float *out,
                 int nh, int nkv, void *stream);
size_t attn_decode_ws_bytes(size_t B, int nh, size_t max_ctx);
int attn_decode(const float *q, const float *gate, const float *kc, const float *vc, const int32_t *pages, int maxp,
                const int32_t *lens, size_t B, int max_len, float *out, int nh, int nkv, float *part, void *stream);
int prefill_conv_gate(const float *qkv, const float *ring, const float *conv_w, const int32_t *seq,
                      const int32_t *pos, const float *beta_raw, const float *alpha_raw, const float *dt_bias,
                      const float *a_log, uint16_t *qb, uint16_t *kb, uint16_t *vb, float *beta, float *gate,
                      size_t T, int ch, int di, int Hv, void *stream);
int ring_update(const float *qkv, float *ring, const int32_t *cu, size_t N, int ch, void *stream);
size_t argmax_rows_ws_bytes(size_t rows, size_t n);
int argmax_rows(const float *y, size_t rows, size_t n, int32_t *idx, unsigned long long *keys, void *stream);
}  // namespace ouro

using namespace ouro;

namespace {

constexpr int kHd = 128;

// Tensor ids of the synthetic weights: 64 per layer, globals after them.
enum LayerTensor {
    T_ATTN_NORM = 0, T_POST_NORM, T_UP, T_GATE, T_DOWN,
    T_QKV, T_Z, T_BETA, T_ALPHA, T_OUT, T_CONV, T_DT, T_ALOG, T_SSM_NORM,
    T_Q, T_K, T_V, T_O, T_QN, T_KN,
};
enum GlobalTensor { G_EMBD = 0, G_OUT_NORM, G_LM, G_SIGN_E, G_SIGN_FF, G_SIGN_DI, G_SIGN_Q };
constexpr uint32_t kGlobalBase = 0x100000u;
uint32_t tid_layer(int il, int t) { return static_cast<uint32_t>(il) * 64u + static_cast<uint32_t>(t); }

// Rotation block of a width: the largest power of two dividing it, <= 4096.
size_t rot_block(size_t n) {
    size_t b = 1;
    while (b < 4096 && n % (2 * b) == 0) b *= 2;
    return b;
}

struct Lin {
    uint8_t *w = nullptr;  // MFMA-tiled codes followed by the fp32 scale
    float *scale = nullptr;
    size_t out = 0, in = 0;
};

struct Layer {
    bool delta = false;
    float *attn_norm = nullptr, *post_norm = nullptr;
    Lin upgate, down;  // upgate: the up and gate rows interleaved; its GEMM writes silu(gate) * up
    // delta-net
    Lin qkv, z, beta, alpha, out;
    float *conv_w = nullptr, *dt_bias = nullptr, *a_log = nullptr, *ssm_norm = nullptr;
    float *state = nullptr, *ring = nullptr;
    // attention
    Lin q, k, v, o;
    float *qn = nullptr, *kn = nullptr, *kc = nullptr, *vc = nullptr;
};

}  // namespace

struct ouro_stack {
    ouro_stack_card c{};
    uint32_t seed = 0;
    size_t max_seqs = 0, max_tokens = 0, max_ctx = 0;
    size_t E = 0, F = 0, V = 0, ch = 0, di = 0, dv = 0, qdim = 0, kvdim = 0;
    std::vector<Layer> layers;
    float *embd = nullptr, *out_norm = nullptr;
    Lin lm;
    float *sign_e = nullptr, *sign_ff = nullptr, *sign_di = nullptr, *sign_q = nullptr;
    // activations, rows = max(max_tokens, max_seqs)
    float *x = nullptr, *pre = nullptr;  // residual stream: x (layer input), pre (after the mixer)
    float *big = nullptr, *zb = nullptr, *braw = nullptr, *araw = nullptr;
    float *o = nullptr, *g = nullptr, *qbuf = nullptr, *gbuf = nullptr, *kbuf = nullptr, *vbuf = nullptr;
    float *attn_o = nullptr, *attn_part = nullptr, *lp = nullptr, *logits = nullptr;
    int8_t *xq = nullptr, *xq2 = nullptr;  // rotated activations; unrotated h for beta / alpha
    size_t qrows = 0;                       // rows of xq / xq2 / ds / ds2
    float *ds = nullptr, *ds2 = nullptr;
    uint16_t *qb = nullptr, *kb = nullptr, *vb = nullptr;
    float *beta = nullptr, *gate = nullptr;
    int32_t *pos = nullptr, *seqid = nullptr, *cu = nullptr, *tile_seq = nullptr, *tile_p0 = nullptr;
    int32_t *lens = nullptr, *klen = nullptr, *last_rows = nullptr, *dec_seq = nullptr;
    int32_t *pages = nullptr;  // KV page table [max_seqs][maxp]
    unsigned long long *arg_keys = nullptr;  // argmax chunk keys of the head rows
    void *ws = nullptr;
    // host staging (pinned) for the per-prefill index arrays
    int32_t *host_i32 = nullptr;
    size_t host_i32_n = 0;
    std::vector<void *> allocs;
    size_t bytes = 0;
    size_t n_seqs = 0;
    int max_len = 0;  // longest sequence (keys) so far
    // paged KV cache: kv_pages pages of kPage rows, handed out on the host
    size_t kv_pages = 0;
    int maxp = 0;                         // page-table entries per sequence
    std::vector<int32_t> free_pages;      // stack of unused pages
    std::vector<int32_t> lens_host;       // tokens held per sequence
};

namespace {

void release(ouro_stack *s) {
    if (!s) return;
    for (void *p : s->allocs) (void)hipFree(p);
    if (s->host_i32) (void)hipHostFree(s->host_i32);
    delete s;
}

template <typename T>
int dalloc(ouro_stack *s, T **p, size_t count) {
    void *q = nullptr;
    const size_t b = (count * sizeof(T) + 255) & ~static_cast<size_t>(255);
    if (hipMalloc(&q, b ? b : 256) != hipSuccess) return fail(OURO_ERR_HIP, "ouro_stack_create: out of device memory (%zu B)", b);
    s->allocs.push_back(q);
    s->bytes += b;
    *p = static_cast<T *>(q);
    return OURO_OK;
}

int make_lin(ouro_stack *s, Lin &L, uint32_t tensor, size_t out, size_t in, uint8_t *canon_scratch) {
    L.out = out;
    L.in = in;
    const size_t tb = i2_mfma_bytes(out, in);
    int st = dalloc(s, &L.w, tb + 16);
    if (st) return st;
    L.scale = reinterpret_cast<float *>(L.w + tb);
    if ((st = gen_codes(s->seed, tensor, out, in, canon_scratch, nullptr))) return st;
    if ((st = i2_tile_mfma(canon_scratch, out, in, L.w, nullptr, nullptr, 0))) return st;
    const float sc = static_cast<float>(1.0 / std::sqrt(static_cast<double>(in) * 2.0 / 3.0));
    if (hipMemcpy(L.scale, &sc, 4, hipMemcpyHostToDevice) != hipSuccess) return fail(OURO_ERR_HIP, "stack: scale copy");
    return hipDeviceSynchronize() == hipSuccess ? OURO_OK : fail(OURO_ERR_HIP, "stack: weight generation");
}

// The codes make_lin would give the up and gate tensors, rows interleaved
// (up row i -> row 2i, gate row i -> row 2i + 1); both have the same scale.
// The canonical scratch holds up, gate and the interleaved rows (4 out rows).
int make_lin_pair(ouro_stack *s, Lin &L, uint32_t t_up, uint32_t t_gate, size_t out, size_t in, uint8_t *canon_scratch) {
    L.out = 2 * out;
    L.in = in;
    const size_t tb = i2_mfma_bytes(2 * out, in), rb = in / 4;
    int st = dalloc(s, &L.w, tb + 16);
    if (st) return st;
    L.scale = reinterpret_cast<float *>(L.w + tb);
    uint8_t *up = canon_scratch, *gate = up + out * rb, *pair = gate + out * rb;
    if ((st = gen_codes(s->seed, t_up, out, in, up, nullptr)) || (st = gen_codes(s->seed, t_gate, out, in, gate, nullptr)))
        return st;
    if (hipMemcpy2D(pair, 2 * rb, up, rb, rb, out, hipMemcpyDeviceToDevice) != hipSuccess ||
        hipMemcpy2D(pair + rb, 2 * rb, gate, rb, rb, out, hipMemcpyDeviceToDevice) != hipSuccess)
        return fail(OURO_ERR_HIP, "stack: interleaving up and gate");
    if ((st = i2_tile_mfma(pair, 2 * out, in, L.w, nullptr, nullptr, 0))) return st;
    const float sc = static_cast<float>(1.0 / std::sqrt(static_cast<double>(in) * 2.0 / 3.0));
    if (hipMemcpy(L.scale, &sc, 4, hipMemcpyHostToDevice) != hipSuccess) return fail(OURO_ERR_HIP, "stack: scale copy");
    return hipDeviceSynchronize() == hipSuccess ? OURO_OK : fail(OURO_ERR_HIP, "stack: weight generation");
}

int make_vec(ouro_stack *s, float **p, uint32_t tensor, size_t n, float lo, float span) {
    int st = dalloc(s, p, n);
    if (st) return st;
    return gen_floats(s->seed, tensor, n, lo, span, *p, nullptr);
}

#define TRY(expr)              \
    do {                       \
        const int st_ = (expr); \
        if (st_) return st_;   \
    } while (0)

// Launches of at most this many activation rows (decode steps, heads of a
// few sequences) pass the int8 activations in the few-column GEMM's
// fragment order; longer ones row-major.
constexpr size_t kFragRows = 64;
constexpr int kPage = 64;  // tokens per KV cache page (stack_ops.hip)
int frag_tiles(size_t rows) { return rows <= kFragRows ? static_cast<int>((rows + 15) / 16) : 0; }

// y[cols][L.out] = L x (int8 activations xq/ds of `cols` rows, as produced
// for the same row count).
int lin(const Lin &L, size_t cols, const int8_t *xq, const float *ds, float *y, void *stream) {
    return i2_gemm_mfma(L.w, L.out, L.in, L.scale, xq, ds, cols, y, nullptr, stream, frag_tiles(cols) ? 1 : 0);
}
// y = res + L x: a block's output projection with the residual add in the
// GEMM's epilogue (y and res are different buffers)
int lin_res(const Lin &L, size_t cols, const int8_t *xq, const float *ds, const float *res, float *y, void *stream) {
    const GemmEpilogue add{EPI_RESID, nullptr, nullptr, res, nullptr};
    return i2_gemm_mfma(L.w, L.out, L.in, L.scale, xq, ds, cols, y, nullptr, stream, frag_tiles(cols) ? 1 : 0, 0,
                        &add);
}

// Several projections of the same activation rows: one grouped launch for
// a few rows, else one launch each.
struct LinOp {
    const Lin *L;
    const int8_t *xq;
    const float *ds;
    float *y;
    GemmEpilogue epi;  // few-column launches only
    int swiglu;        // few-column launches only: interleaved (up, gate) rows -> silu(gate) * up
};
int lin_group(std::initializer_list<LinOp> ops, size_t cols, void *stream) {
    if (!frag_tiles(cols)) {
        for (const LinOp &o : ops) TRY(lin(*o.L, cols, o.xq, o.ds, o.y, stream));
        return OURO_OK;
    }
    GemmProblem p[4];
    int np = 0;
    for (const LinOp &o : ops)
        p[np++] = GemmProblem{o.L->w, o.L->out, o.L->scale, o.xq, o.ds, o.y, nullptr, o.epi, o.swiglu};
    return i2_gemm_skinny_group(p, np, ops.begin()->L->in, cols, 1, stream);
}

// Prologue + Hadamard rotation (signs of width n) + int8 absmax into s->xq / s->ds.
int rq(ouro_stack *s, int pro, const float *a, const float *b, const float *w, float *sum_out, size_t rows, size_t n,
       const float *signs, void *stream, bool also_plain = false) {
    const ouro_stack_card &c = s->c;
    const size_t laid = frag_tiles(rows) ? static_cast<size_t>(frag_tiles(rows)) * 16 : rows;
    if (laid > s->qrows)
        return fail(OURO_ERR_SHAPE, "ouro_stack: %zu activation rows (%zu laid out) exceed the %zu allocated", rows,
                    laid, s->qrows);
    return row_rotate_quant(pro, a, b, w, sum_out, rows, n, rot_block(n), signs, s->xq, s->ds,
                            also_plain ? s->xq2 : nullptr, also_plain ? s->ds2 : nullptr, frag_tiles(rows),
                            c.ssm_n_k_heads, c.ssm_n_v_heads, OURO_GDN_V_GROUPED, c.eps, stream);
}


// Mixer + FFN of one layer over `rows` token rows; x is the layer input (the
// residual stream), and the layer leaves its output (pre + FFN) in x.
int run_layer(ouro_stack *s, int il, size_t rows, bool prefill, const int32_t *cu_host, size_t N, size_t n_tiles,
              void *stream) {
    Layer &L = s->layers[il];
    const ouro_stack_card &c = s->c;
    const size_t Hk = c.ssm_n_k_heads, Hv = c.ssm_n_v_heads;
    // h = rmsnorm(x) * attn_norm, where x (the residual stream) = pre + the
    // previous layer's FFN output, added in its down projection's epilogue;
    // rotated and quantised; delta layers also quantise h itself for the
    // beta and alpha projections (qwen35.rs:1058-1065)
    TRY(rq(s, RQ_NORM, s->x, nullptr, L.attn_norm, nullptr, rows, s->E, s->sign_e, stream, L.delta));
    if (L.delta) {
        if (!prefill && frag_tiles(rows)) {
            // decode: the conv + SiLU (ring shifted in place) and the gates run
            // in the projections' epilogue; the recurrence reads them directly
            const GemmEpilogue conv{EPI_CONV, L.conv_w, L.ring, nullptr, nullptr};
            const GemmEpilogue sig{EPI_SIGMOID, nullptr, nullptr, nullptr, nullptr};
            const GemmEpilogue gat{EPI_GATE, nullptr, nullptr, L.dt_bias, L.a_log};
            TRY(lin_group({{&L.qkv, s->xq, s->ds, s->big, conv}, {&L.z, s->xq, s->ds, s->zb, {}},
                           {&L.beta, s->xq2, s->ds2, s->braw, sig}, {&L.alpha, s->xq2, s->ds2, s->araw, gat}},
                          rows, stream));
            const size_t di = Hk * kHd;
            TRY(gdn_decode(L.state, s->big, s->big + di, OURO_DT_F32, s->big + 2 * di, OURO_DT_F32, s->araw, s->braw,
                           0.f, 0.f, s->o, rows, Hk, Hv, kHd, OURO_GDN_L2NORM_QK | OURO_GDN_SCALE_Q, c.eps, stream,
                           s->ch, s->ch));
        } else {
            TRY(lin_group({{&L.qkv, s->xq, s->ds, s->big}, {&L.z, s->xq, s->ds, s->zb},
                           {&L.beta, s->xq2, s->ds2, s->braw}, {&L.alpha, s->xq2, s->ds2, s->araw}},
                          rows, stream));
            if (prefill) {
                TRY(prefill_conv_gate(s->big, L.ring, L.conv_w, s->seqid, s->pos, s->braw, s->araw, L.dt_bias, L.a_log,
                                      s->qb, s->kb, s->vb, s->beta, s->gate, rows, static_cast<int>(s->ch),
                                      static_cast<int>(s->di), static_cast<int>(Hv), stream));
                TRY(ring_update(s->big, L.ring, s->cu, N, static_cast<int>(s->ch), stream));
                TRY(gdn_chunk_prefill(L.state, s->qb, s->kb, s->vb, s->gate, s->beta, s->o, cu_host, N, rows, Hk, Hv,
                                      kHd, 64, OURO_GDN_L2NORM_QK | OURO_GDN_SCALE_Q, c.eps, s->ws, stream));
            } else {
                TRY(gdn_decode_core(s->big, s->braw, s->araw, L.dt_bias, L.a_log, L.conv_w, L.ring, L.state, s->o,
                                    rows, Hk, Hv, 0u, c.eps, s->ws, stream));
            }
        }
        // gated RMS norm per head in the V-grouped order, rotated, quantised
        TRY(rq(s, RQ_GNORM, s->o, s->zb, L.ssm_norm, nullptr, rows, s->dv, s->sign_di, stream));
        TRY(lin_res(L.out, rows, s->xq, s->ds, s->x, s->pre, stream));  // pre = x + mixer
    } else {
        TRY(lin_group({{&L.q, s->xq, s->ds, s->big}, {&L.k, s->xq, s->ds, s->kbuf}, {&L.v, s->xq, s->ds, s->vbuf}},
                      rows, stream));
        TRY(attn_prep(s->big, s->kbuf, s->vbuf, L.qn, L.kn, s->pos, prefill ? s->seqid : s->dec_seq, s->pages, s->maxp,
                      s->qbuf, s->gbuf, L.kc, L.vc, rows, c.n_head, c.n_head_kv, c.n_rot, c.rope_base, c.eps,
                      stream));
        if (prefill)
            TRY(attn_prefill(s->qbuf, s->gbuf, L.kc, L.vc, s->pages, s->maxp, s->cu, s->tile_seq, s->tile_p0, n_tiles,
                             s->attn_o, c.n_head, c.n_head_kv, stream));
        else
            TRY(attn_decode(s->qbuf, s->gbuf, L.kc, L.vc, s->pages, s->maxp, s->klen, rows, s->max_len, s->attn_o, c.n_head,
                            c.n_head_kv, s->attn_part, stream));
        TRY(rq(s, RQ_COPY, s->attn_o, nullptr, nullptr, nullptr, rows, s->qdim, s->sign_q, stream));
        TRY(lin_res(L.o, rows, s->xq, s->ds, s->x, s->pre, stream));  // pre = x + mixer
    }
    // f = rmsnorm(pre) * post_norm; x = pre + down(silu(gate f) * up f)
    TRY(rq(s, RQ_NORM, s->pre, nullptr, L.post_norm, nullptr, rows, s->E, s->sign_e, stream));
    // the interleaved up/gate product writes silu(gate) * up (few rows: the
    // fragment-ordered launch; more: the row-major one)
    if (frag_tiles(rows))
        TRY(lin_group({{&L.upgate, s->xq, s->ds, s->big, {}, 1}}, rows, stream));
    else
        TRY(i2_gemm_mfma(L.upgate.w, L.upgate.out, L.upgate.in, L.upgate.scale, s->xq, s->ds, rows, s->big, nullptr,
                         stream, 0, 1));
    TRY(rq(s, RQ_COPY, s->big, nullptr, nullptr, nullptr, rows, s->F, s->sign_ff, stream));
    TRY(lin_res(L.down, rows, s->xq, s->ds, s->pre, s->x, stream));  // x = pre + FFN
    return OURO_OK;
}

// Final norm of the chosen rows of the residual stream, lm_head, greedy token.
int head(ouro_stack *s, const int32_t *rows_idx, size_t n, int32_t *next, float *logits_out, void *stream) {
    TRY(gather_rows(s->x, rows_idx, s->lp, n, s->E, stream));
    TRY(rq(s, RQ_NORM, s->lp, nullptr, s->out_norm, nullptr, n, s->E, s->sign_e, stream));
    float *lg = logits_out ? logits_out : s->logits;
    TRY(lin(s->lm, n, s->xq, s->ds, lg, stream));
    return argmax_rows(lg, n, s->V, next, s->arg_keys, stream);
}

int check_card(const ouro_stack_card &c) {
    if (c.n_layer < 1 || c.n_embd < 256 || c.n_embd % 256 || c.n_embd > 6144 || c.n_ff < 256 || c.n_ff % 256 ||
        c.n_ff > 12288 || c.n_vocab < 1 || c.full_attention_interval < 1)
        return fail(OURO_ERR_SHAPE, "ouro_stack: bad sizes (n_embd <= 6144 and n_ff <= 12288, multiples of 256)");
    if (c.head_dim != kHd || c.ssm_d_state != kHd) return fail(OURO_ERR_SHAPE, "ouro_stack: head_dim and d_state must be 128");
    if (c.n_head < 2 || c.n_head % 2 || c.n_head_kv < 1 || c.n_head % c.n_head_kv || c.n_head / c.n_head_kv > 8)
        return fail(OURO_ERR_SHAPE, "ouro_stack: n_head even, a multiple of n_head_kv, at most 8 per kv head");
    if (c.n_rot < 0 || c.n_rot > kHd || c.n_rot % 4) return fail(OURO_ERR_SHAPE, "ouro_stack: n_rot");
    if (c.ssm_n_k_heads < 1 || c.ssm_n_v_heads % 2 || c.ssm_n_v_heads % c.ssm_n_k_heads || c.ssm_n_v_heads > 96 ||
        c.n_head > 96)
        return fail(OURO_ERR_SHAPE, "ouro_stack: ssm heads (n_v_heads even, a multiple of n_k_heads)");
    if (static_cast<size_t>(c.n_vocab) * c.n_embd >= (1ull << 32)) return fail(OURO_ERR_SHAPE, "ouro_stack: vocab too large");
    return OURO_OK;
}

}  // namespace

extern "C" {

int ouro_stack_create(const ouro_stack_card *card, uint32_t seed, size_t max_seqs, size_t max_tokens,
                      size_t max_ctx, size_t kv_pages, ouro_stack_t *out) {
    OURO_REQUIRE_INIT();
    if (!card || !out) return fail(OURO_ERR_INVALID_ARG, "ouro_stack_create: NULL argument");
    *out = nullptr;
    int st = check_card(*card);
    if (st) return st;
    if (!max_seqs || !max_tokens || max_ctx < 2 || max_ctx > 16384 || max_tokens > (1u << 20) || max_seqs > 4096 ||
        kv_pages > (1u << 24))
        return fail(OURO_ERR_SHAPE, "ouro_stack_create: max_seqs, max_tokens, max_ctx (<= 16384), kv_pages out of range");
    ouro_stack *s = new (std::nothrow) ouro_stack;
    if (!s) return fail(OURO_ERR_INVALID_ARG, "ouro_stack_create: out of host memory");
    s->c = *card;
    s->seed = seed;
    s->max_seqs = max_seqs;
    s->max_tokens = max_tokens;
    s->max_ctx = max_ctx;
    s->maxp = static_cast<int>((max_ctx + kPage - 1) / kPage);
    s->kv_pages = kv_pages ? kv_pages : max_seqs * static_cast<size_t>(s->maxp);
    s->lens_host.assign(max_seqs, 0);
    const ouro_stack_card &c = s->c;
    s->E = c.n_embd;
    s->F = c.n_ff;
    s->V = c.n_vocab;
    s->di = static_cast<size_t>(c.ssm_n_k_heads) * kHd;
    s->dv = static_cast<size_t>(c.ssm_n_v_heads) * kHd;
    s->ch = 2 * s->di + s->dv;
    s->qdim = static_cast<size_t>(c.n_head) * kHd;
    s->kvdim = static_cast<size_t>(c.n_head_kv) * kHd;
    const size_t E = s->E, F = s->F, V = s->V;
    const size_t rows = max_tokens > max_seqs ? max_tokens : max_seqs;
    const size_t wide = std::max({s->ch, 2 * s->qdim, F});
    // scratch for canonical codes of the largest tensor
    uint8_t *canon = nullptr;
    const size_t canon_bytes = std::max({V * E, 4 * F * E, s->ch * E, 2 * s->qdim * E}) / 4;
    if (hipMalloc(reinterpret_cast<void **>(&canon), canon_bytes) != hipSuccess) {
        release(s);
        return fail(OURO_ERR_HIP, "ouro_stack_create: out of device memory");
    }
    auto done = [&](int code) {
        (void)hipFree(canon);
        if (code) release(s);
        return code;
    };
    s->layers.resize(c.n_layer);
    for (int il = 0; il < c.n_layer; ++il) {
        Layer &L = s->layers[il];
        L.delta = (il + 1) % c.full_attention_interval != 0;
        if ((st = make_vec(s, &L.attn_norm, tid_layer(il, T_ATTN_NORM), E, 0.8f, 0.4f)) ||
            (st = make_vec(s, &L.post_norm, tid_layer(il, T_POST_NORM), E, 0.8f, 0.4f)) ||
            (st = make_lin_pair(s, L.upgate, tid_layer(il, T_UP), tid_layer(il, T_GATE), F, E, canon)) ||
            (st = make_lin(s, L.down, tid_layer(il, T_DOWN), E, F, canon)))
            return done(st);
        if (L.delta) {
            const size_t Hv = c.ssm_n_v_heads;
            if ((st = make_lin(s, L.qkv, tid_layer(il, T_QKV), s->ch, E, canon)) ||
                (st = make_lin(s, L.z, tid_layer(il, T_Z), s->dv, E, canon)) ||
                (st = make_lin(s, L.beta, tid_layer(il, T_BETA), Hv, E, canon)) ||
                (st = make_lin(s, L.alpha, tid_layer(il, T_ALPHA), Hv, E, canon)) ||
                (st = make_lin(s, L.out, tid_layer(il, T_OUT), E, s->dv, canon)) ||
                (st = make_vec(s, &L.conv_w, tid_layer(il, T_CONV), 4 * s->ch, -0.5f, 1.0f)) ||
                (st = make_vec(s, &L.dt_bias, tid_layer(il, T_DT), Hv, -1.0f, 2.0f)) ||
                (st = make_vec(s, &L.a_log, tid_layer(il, T_ALOG), Hv, -2.0f, 1.9f)) ||
                (st = make_vec(s, &L.ssm_norm, tid_layer(il, T_SSM_NORM), kHd, 0.8f, 0.4f)) ||
                (st = dalloc(s, &L.state, max_seqs * Hv * kHd * kHd)) ||
                (st = dalloc(s, &L.ring, max_seqs * s->ch * 3)))
                return done(st);
        } else {
            if ((st = make_lin(s, L.q, tid_layer(il, T_Q), 2 * s->qdim, E, canon)) ||
                (st = make_lin(s, L.k, tid_layer(il, T_K), s->kvdim, E, canon)) ||
                (st = make_lin(s, L.v, tid_layer(il, T_V), s->kvdim, E, canon)) ||
                (st = make_lin(s, L.o, tid_layer(il, T_O), E, s->qdim, canon)) ||
                (st = make_vec(s, &L.qn, tid_layer(il, T_QN), kHd, 0.8f, 0.4f)) ||
                (st = make_vec(s, &L.kn, tid_layer(il, T_KN), kHd, 0.8f, 0.4f)) ||
                (st = dalloc(s, &L.kc, s->kv_pages * kPage * s->kvdim)) ||
                (st = dalloc(s, &L.vc, s->kv_pages * kPage * s->kvdim)))
                return done(st);
        }
    }
    if ((st = make_vec(s, &s->embd, kGlobalBase + G_EMBD, V * E, -1.0f, 2.0f)) ||
        (st = make_vec(s, &s->out_norm, kGlobalBase + G_OUT_NORM, E, 0.8f, 0.4f)) ||
        (st = make_lin(s, s->lm, kGlobalBase + G_LM, V, E, canon)) ||
        (st = make_vec(s, &s->sign_e, kGlobalBase + G_SIGN_E, E, 0.f, 0.f)) ||
        (st = make_vec(s, &s->sign_ff, kGlobalBase + G_SIGN_FF, F, 0.f, 0.f)) ||
        (st = make_vec(s, &s->sign_di, kGlobalBase + G_SIGN_DI, s->dv, 0.f, 0.f)) ||
        (st = make_vec(s, &s->sign_q, kGlobalBase + G_SIGN_Q, s->qdim, 0.f, 0.f)))
        return done(st);
    const size_t xw = std::max({E, F, s->dv, s->qdim});
    const size_t tiles = max_tokens / 64 + max_seqs + 1;
    // int8 activations of a few-row launch (any launch of <= 64 rows: decode
    // steps, and prefills of <= 64 tokens) are laid out in whole 16-row
    // tiles, whose chunks interleave every row across the padded layout, so
    // the buffers hold round_up(rows, 16) rows
    const size_t qrows = (rows + 15) / 16 * 16;
    s->qrows = qrows;
    if ((st = dalloc(s, &s->x, rows * E)) || (st = dalloc(s, &s->pre, rows * E)) ||
        (st = dalloc(s, &s->big, rows * wide)) ||
        (st = dalloc(s, &s->zb, rows * s->dv)) || (st = dalloc(s, &s->braw, rows * c.ssm_n_v_heads)) ||
        (st = dalloc(s, &s->araw, rows * c.ssm_n_v_heads)) || (st = dalloc(s, &s->o, rows * s->dv)) ||
        (st = dalloc(s, &s->g, rows * s->dv)) || (st = dalloc(s, &s->qbuf, rows * s->qdim)) ||
        (st = dalloc(s, &s->gbuf, rows * s->qdim)) || (st = dalloc(s, &s->kbuf, rows * s->kvdim)) ||
        (st = dalloc(s, &s->vbuf, rows * s->kvdim)) || (st = dalloc(s, &s->attn_o, rows * s->qdim)) ||
        (st = dalloc(s, &s->lp, max_seqs * E)) ||
        (st = dalloc(s, &s->logits, max_seqs * V)) || (st = dalloc(s, &s->xq, qrows * xw)) ||
        (st = dalloc(s, &s->ds, qrows)) || (st = dalloc(s, &s->xq2, qrows * E)) || (st = dalloc(s, &s->ds2, qrows)) ||
        (st = dalloc(s, &s->qb, rows * s->di)) || (st = dalloc(s, &s->kb, rows * s->di)) ||
        (st = dalloc(s, &s->vb, rows * s->dv)) || (st = dalloc(s, &s->beta, rows * c.ssm_n_v_heads)) ||
        (st = dalloc(s, &s->gate, rows * c.ssm_n_v_heads)) || (st = dalloc(s, &s->pos, rows)) ||
        (st = dalloc(s, &s->seqid, rows)) || (st = dalloc(s, &s->cu, max_seqs + 1)) ||
        (st = dalloc(s, &s->tile_seq, tiles)) || (st = dalloc(s, &s->tile_p0, tiles)) ||
        (st = dalloc(s, &s->lens, max_seqs)) || (st = dalloc(s, &s->klen, max_seqs)) ||
        (st = dalloc(s, &s->last_rows, max_seqs)) || (st = dalloc(s, &s->dec_seq, max_seqs)) ||
        (st = dalloc(s, &s->pages, max_seqs * static_cast<size_t>(s->maxp))))
        return done(st);
    const size_t wsb = std::max(gdn_chunk_ws_bytes(max_tokens, max_seqs, c.ssm_n_v_heads),
                                gdn_layer_ws_bytes(max_seqs, c.ssm_n_k_heads, c.ssm_n_v_heads));
    if ((st = dalloc(s, reinterpret_cast<uint8_t **>(&s->ws), wsb)) ||
        (st = dalloc(s, reinterpret_cast<uint8_t **>(&s->attn_part), attn_decode_ws_bytes(max_seqs, c.n_head, max_ctx))) ||
        (st = dalloc(s, reinterpret_cast<uint8_t **>(&s->arg_keys), argmax_rows_ws_bytes(max_seqs, V))))
        return done(st);
    // pinned staging of the per-prefill index arrays and page table; the
    // decode row -> sequence map is constant
    s->host_i32_n = 3 * rows + 2 * tiles + 4 * max_seqs + max_seqs * static_cast<size_t>(s->maxp) + 8;
    if (hipHostMalloc(reinterpret_cast<void **>(&s->host_i32), s->host_i32_n * 4, hipHostMallocDefault) != hipSuccess)
        return done(fail(OURO_ERR_HIP, "ouro_stack_create: pinned host allocation failed"));
    std::vector<int32_t> ids(max_seqs);
    for (size_t i = 0; i < max_seqs; ++i) ids[i] = static_cast<int32_t>(i);
    if (hipMemcpy(s->dec_seq, ids.data(), max_seqs * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess)
        return done(fail(OURO_ERR_HIP, "ouro_stack_create: setup copy failed"));
    *out = s;
    return done(OURO_OK);
}

int ouro_stack_free(ouro_stack_t s) {
    OURO_REQUIRE_INIT();
    if (s) {
        (void)hipDeviceSynchronize();
        release(s);
    }
    return OURO_OK;
}

size_t ouro_stack_device_bytes(ouro_stack_t s) { return s ? s->bytes : 0; }

int ouro_stack_prefill(ouro_stack_t s, const int32_t *tokens, const int32_t *cu_host, size_t N, int32_t *next_tokens,
                       float *logits_or_null, void *stream) {
    OURO_REQUIRE_INIT();
    if (!s || !tokens || !cu_host || !next_tokens) return fail(OURO_ERR_INVALID_ARG, "ouro_stack_prefill: NULL argument");
    if (!N || N > s->max_seqs) return fail(OURO_ERR_SHAPE, "ouro_stack_prefill: %zu sequences (max %zu)", N, s->max_seqs);
    if (cu_host[0] != 0) return fail(OURO_ERR_SHAPE, "ouro_stack_prefill: cu_seqlens[0] != 0");
    int max_len = 0;
    for (size_t i = 0; i < N; ++i) {
        const int L = cu_host[i + 1] - cu_host[i];
        if (L < 1 || static_cast<size_t>(L) >= s->max_ctx)
            return fail(OURO_ERR_SHAPE, "ouro_stack_prefill: sequence %zu has %d tokens (1 .. max_ctx - 1)", i, L);
        max_len = L > max_len ? L : max_len;
    }
    const size_t T = cu_host[N];
    if (T > s->max_tokens) return fail(OURO_ERR_SHAPE, "ouro_stack_prefill: %zu tokens (max %zu)", T, s->max_tokens);
    // index arrays: pos[T], seq[T], cu[N+1], tiles, last rows, lens -> one pinned staging copy each
    int32_t *hp = s->host_i32;
    int32_t *h_pos = hp, *h_seq = h_pos + T, *h_cu = h_seq + T, *h_ts = h_cu + N + 1;
    size_t n_tiles = 0;
    for (size_t i = 0; i < N; ++i)
        for (int p0 = 0; p0 < cu_host[i + 1] - cu_host[i]; p0 += 64) ++n_tiles;
    int32_t *h_tp = h_ts + n_tiles, *h_last = h_tp + n_tiles, *h_lens = h_last + N, *h_pt = h_lens + N;
    const size_t n_pt = N * static_cast<size_t>(s->maxp);
    if (static_cast<size_t>(h_pt + n_pt - hp) > s->host_i32_n) return fail(OURO_ERR_SHAPE, "ouro_stack_prefill: index staging");
    // fresh sequences: every KV page returns to the pool, each prompt takes ceil(L / kPage)
    size_t need = 0;
    for (size_t i = 0; i < N; ++i) need += (cu_host[i + 1] - cu_host[i] + kPage - 1) / kPage;
    if (need > s->kv_pages)
        return fail(OURO_ERR_SHAPE, "ouro_stack_prefill: prompts need %zu KV pages of %d tokens (pool %zu)", need, kPage,
                    s->kv_pages);
    hipStream_t st = as_stream(stream);
    // the staging buffer is rewritten: earlier copies from it must be done
    if (hipStreamSynchronize(st) != hipSuccess) return fail(OURO_ERR_HIP, "ouro_stack_prefill: stream sync");
    // query tiles, the longest first (a tile at p0 reads p0 / 64 + 1 key
    // tiles): workgroups start in launch order, so the heavy tiles of long
    // prompts start early and the short ones fill in at the end
    size_t k = 0;
    for (int p0 = (max_len - 1) / 64 * 64; p0 >= 0; p0 -= 64)
        for (size_t i = 0; i < N; ++i)
            if (p0 < cu_host[i + 1] - cu_host[i]) {
                h_ts[k] = static_cast<int32_t>(i);
                h_tp[k] = p0;
                ++k;
            }
    for (size_t i = 0; i < N; ++i) {
        const int t0 = cu_host[i], L = cu_host[i + 1] - t0;
        for (int p = 0; p < L; ++p) {
            h_pos[t0 + p] = p;
            h_seq[t0 + p] = static_cast<int32_t>(i);
        }
        h_last[i] = t0 + L - 1;
        h_lens[i] = L;
    }
    for (size_t i = 0; i <= N; ++i) h_cu[i] = cu_host[i];
    s->free_pages.resize(s->kv_pages);
    for (size_t i = 0; i < s->kv_pages; ++i) s->free_pages[i] = static_cast<int32_t>(s->kv_pages - 1 - i);
    std::fill(h_pt, h_pt + n_pt, 0);
    std::fill(s->lens_host.begin(), s->lens_host.end(), 0);
    for (size_t i = 0; i < N; ++i) {
        const int L = cu_host[i + 1] - cu_host[i];
        for (int p = 0; p * kPage < L; ++p) {
            h_pt[i * s->maxp + p] = s->free_pages.back();
            s->free_pages.pop_back();
        }
        s->lens_host[i] = L;
    }
    if (hipMemcpyAsync(s->pos, h_pos, T * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s->seqid, h_seq, T * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s->cu, h_cu, (N + 1) * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s->tile_seq, h_ts, n_tiles * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s->tile_p0, h_tp, n_tiles * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s->last_rows, h_last, N * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s->lens, h_lens, N * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(s->pages, h_pt, n_pt * 4, hipMemcpyHostToDevice, st) != hipSuccess)
        return fail(OURO_ERR_HIP, "ouro_stack_prefill: index upload");
    // fresh sequences: zero recurrent state and conv rings
    for (auto &L : s->layers)
        if (L.delta) {
            TRY(fill_zero(L.state, N * s->c.ssm_n_v_heads * kHd * kHd, stream));
            TRY(fill_zero(L.ring, N * s->ch * 3, stream));
        }
    s->n_seqs = N;
    s->max_len = max_len;
    TRY(embed_rows(tokens, s->embd, s->x, T, s->V, s->E, stream));
    for (int il = 0; il < s->c.n_layer; ++il) TRY(run_layer(s, il, T, true, cu_host, N, n_tiles, stream));
    return head(s, s->last_rows, N, next_tokens, logits_or_null, stream);
}

int ouro_stack_decode(ouro_stack_t s, const int32_t *tokens, int32_t *next_tokens, float *logits_or_null,
                      void *stream) {
    OURO_REQUIRE_INIT();
    if (!s || !tokens || !next_tokens) return fail(OURO_ERR_INVALID_ARG, "ouro_stack_decode: NULL argument");
    const size_t B = s->n_seqs;
    if (!B) return fail(OURO_ERR_SHAPE, "ouro_stack_decode: no sequences (prefill first)");
    if (static_cast<size_t>(s->max_len) + 1 > s->max_ctx)
        return fail(OURO_ERR_SHAPE, "ouro_stack_decode: a sequence reached max_ctx = %zu", s->max_ctx);
    // a sequence whose new token starts a page takes one from the pool
    size_t need = 0;
    for (size_t b = 0; b < B; ++b) need += s->lens_host[b] % kPage == 0;
    if (need > s->free_pages.size())
        return fail(OURO_ERR_SHAPE, "ouro_stack_decode: KV page pool (%zu pages) exhausted", s->kv_pages);
    PageAssign pa{};
    for (size_t b = 0; b < B; ++b) {
        const int l = s->lens_host[b]++;
        if (l % kPage) continue;
        if (pa.n == kMaxPageAssign) {  // more than one launch's worth: flush first
            TRY(lens_step(s->lens, s->pos, s->klen, 0, s->pages, pa, stream));
            pa.n = 0;
        }
        pa.slot[pa.n] = static_cast<int>(b) * s->maxp + l / kPage;
        pa.page[pa.n++] = s->free_pages.back();
        s->free_pages.pop_back();
    }
    TRY(lens_step(s->lens, s->pos, s->klen, B, s->pages, pa, stream));
    s->max_len += 1;
    TRY(embed_rows(tokens, s->embd, s->x, B, s->V, s->E, stream));
    for (int il = 0; il < s->c.n_layer; ++il) TRY(run_layer(s, il, B, false, nullptr, B, 0, stream));
    return head(s, s->dec_seq, B, next_tokens, logits_or_null, stream);
}

}  // extern "C"
