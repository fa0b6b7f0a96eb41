/*
 * ouro_oracle.h - CPU oracle for the quantized-inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * CPU arithmetic (Rust, cluster/src/infer/{dequant,ops,hadamard,qwen35}.rs)
 * used as the parity checker by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py.  The shipped product (libouro_hip.so) never
 * links, loads or calls anything in this directory.
 *
 * Every function cites the reference file:line it follows.  The
 * int8-activation x 2-bit ternary functions restate a third-party
 * dependency instead: microsoft/BitNet, the reference's `bitnet-cpp`
 * submodule (.gitmodules; bitnet-rs/build.rs:10), file
 * src/ggml-bitnet-mad.cpp (quantize_i2_s, quantize_row_i8_s,
 * ggml_vec_dot_i2_i8_s) and the I2_S branch of its ggml fork's mul_mat.
 * The submodule is empty in the reference checkout, so its pinned commit
 * cannot be recovered; the restatement follows the published source.  The
 * reference's own plan names this format as its portable ternary baseline
 * and its GPU route ("I2_S repack", PLAN.md:465,1277).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; Rust never contracts
 * a*b+c, so neither may the oracle).
 */
#ifndef OURO_ORACLE_H
#define OURO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- dequant.rs ------------------------------------------------------- */

/* Quant kinds, same set and ggml dtype ids as QuantKind (dequant.rs:315-348). */
enum {
    ORC_KIND_F32 = 0,
    ORC_KIND_F16 = 1,
    ORC_KIND_BF16 = 30,
    ORC_KIND_Q8_0 = 8,
    ORC_KIND_Q3K = 11,
    ORC_KIND_Q4K = 12,
    ORC_KIND_Q5K = 13,
    ORC_KIND_Q6K = 14,
    ORC_KIND_TQ1_0 = 34,
    ORC_KIND_TL1 = 143,
    /* GGML_TYPE_I2_S of BitNet's ggml fork: bitnet.cpp's 2-bit ternary
     * tensor (codes + one fp32 per-tensor scale) */
    ORC_KIND_I2_S = 36,
    /* the library's canonical row-major 2-bit codes (no reference kind) */
    ORC_KIND_I2 = 0x4932,
};

float orc_f16_to_f32(uint16_t bits);                  /* dequant.rs:21-47 */
float orc_bf16_to_f32(uint16_t bits);                 /* dequant.rs:197-199 */
uint16_t orc_f32_to_bf16_rne(float x);                /* round-to-nearest-even */
void orc_tl1_group(const uint8_t *g28, float *out128); /* dequant.rs:146-171 */
void orc_dequant_tl1_row(const uint8_t *payload, size_t row, size_t row_elems,
                         float *out);                  /* dequant.rs:185-195 */
void orc_tq1_block(const uint8_t *b54, float *out256); /* dequant.rs:50-80 */
void orc_dequant_tq1_row(const uint8_t *payload, size_t row, size_t row_bytes,
                         float *out);                  /* dequant.rs:96-105 */
/* The Q8_0 and K-quant blocks (ggml's layouts, as dequant.rs decodes them):
 *   Q8_0 34 B / 32: d f16, qs int8[32]                    (dequant.rs:225-231)
 *   Q4_K 144 B / 256: d, dmin f16, scales[12], qs[128]     (dequant.rs:257-282)
 *   Q3_K 110 B / 256: hmask[32], qs[64], scales[12], d     (dequant.rs:398-451)
 *   Q5_K 176 B / 256: d, dmin, scales[12], qh[32], qs[128] (dequant.rs:454-481)
 *   Q6_K 210 B / 256: ql[128], qh[64], scales int8[16], d  (dequant.rs:484-510) */
void orc_q8_block(const uint8_t *b34, float *out32);
void orc_q4k_block(const uint8_t *b144, float *out256);
void orc_q3k_block(const uint8_t *b110, float *out256);
void orc_q5k_block(const uint8_t *b176, float *out256);
void orc_q6k_block(const uint8_t *b210, float *out256);
/* dequant_{tq1,q8,q3k,q4k,q5k,q6k}_row (dequant.rs:96-105,285-310,532-560):
 * the whole blocks of row `row` (row_bytes / block bytes of them) into out.
 * -1 for a kind that is not block-quantised. */
int orc_dequant_qblock_row(int kind, const uint8_t *payload, size_t row,
                           size_t row_bytes, float *out);
/* QuantKind::row_bytes (dequant.rs:376-387); 0 for an unknown kind. */
size_t orc_row_bytes(int kind, size_t k);
/* QuantKind::from_dtype (dequant.rs:334-348): 1 if supported, else 0. */
int orc_kind_supported(uint32_t dtype);

/* ---- ops.rs ------------------------------------------------------------ */

float orc_dot(const float *a, const float *b, size_t n); /* ops.rs:53-60 */

/* matvec_tl1 (ops.rs:294-321).  simd=0 follows tl1_rows_scalar
 * (ops.rs:324-363), simd=1 follows the SSE4.1 tl1_rows_avx2 summation order
 * (ops.rs:499-584).  nthreads<=0 means OURO_N_THREADS or all cores
 * (mt_threads, ops.rs:62-73). */
void orc_matvec_tl1(const uint8_t *payload, size_t out_len, size_t in_len,
                    const float *x, float *y, int simd, int nthreads);
/* matmul_tl1 (ops.rs:162-215): x row-major [k][in_len], y column-major
 * y[c*out_len + r].  simd selects tl1_rows_scalar_k (ops.rs:244-286) or
 * tl1_rows_avx2_k (ops.rs:381-473). */
void orc_matmul_tl1(const uint8_t *payload, size_t out_len, size_t in_len,
                    const float *x, size_t k, float *y, int simd, int nthreads);
/* matvec_qblock (ops.rs:101-128) for TQ1_0, Q8_0, Q3_K..Q6_K: each row
 * decoded into a zeroed row of in_len floats, then dot with x.  -1 for
 * another kind. */
int orc_matvec_qblock(const uint8_t *payload, int kind, size_t out_len,
                      size_t in_len, const float *x, float *y, int nthreads);
/* matvec_qblock for TQ1_0 (ops.rs:101-128): dequant row, then dot. */
void orc_matvec_tq1(const uint8_t *payload, size_t out_len, size_t in_len,
                    const float *x, float *y, int nthreads);
/* matvec_f32raw / matvec_f16 / matvec_bf16 (ops.rs:87-98,131-154,600-623). */
void orc_matvec_dense(const uint8_t *payload, int kind, size_t out_len,
                      size_t in_len, const float *x, float *y);
/* matvec_q dispatch (ops.rs:76-84) over the kinds above.  Returns 0, or -1
 * for a kind this oracle does not restate. */
int orc_matvec_q(const uint8_t *payload, int kind, size_t out_len,
                 size_t in_len, const float *x, float *y, int nthreads);
/* matmul_q (ops.rs:219-230): TL1 fused K-column, else K matvecs. */
int orc_matmul_q(const uint8_t *payload, int kind, size_t out_len,
                 size_t in_len, const float *x, size_t k, float *y,
                 int nthreads);

/* ---- I2_S / I8_S: int8 per-token absmax activations x 2-bit ternary ----
 *
 * bitnet.cpp's format (src/ggml-bitnet-mad.cpp), as restated here:
 *  I2_S tensor of nrow x n_per_row weights, n = nrow*n_per_row, n % 128 == 0:
 *    the flattened weights in blocks of 128; weight j of block i sits in
 *    byte 32*i + j%32 at bits 6 - 2*(j/32) .. 7 - 2*(j/32) as code w + 1
 *    (0 = -1, 1 = 0, 2 = +1); one fp32 scale at byte n/4; the tensor is
 *    n/4 + 32 bytes (the scale, then alignment padding).
 *  quantize_i2_s(src): max = max|src| (double); code = 1 where
 *    |src| < 1e-6, else 2 where src * max > 0, else 0; scale = max.
 *  quantize_row_i8_s(x): max = max(1e-5, max|x|) (double);
 *    s = (float)(127 / max); q = clamp(round((double)(x*s)), -128, 127)
 *    with round() half away from zero; act_sum = sum of q.
 *  vec_dot_i2_i8_s: sumi = sum of code * q (integer).
 *  mul_mat epilogue: y = (((float)sumi - act_sum) / s) * scale.
 */
size_t orc_i2s_bytes(size_t nrow, size_t n_per_row);          /* n/4 + 32 */
/* quantize_i2_s; dst holds orc_i2s_bytes() bytes (padding zeroed).
 * Returns -1 if n % 128 != 0. */
int orc_quantize_i2_s(const float *src, size_t nrow, size_t n_per_row,
                      uint8_t *dst);
/* Ternary weights w (values in {-1,0,1}) with per-tensor scale: the I2_S
 * bytes quantize_i2_s makes of w * w_scale (w_scale > 0).  -1 on a bad
 * weight or n % 128 != 0. */
int orc_i2s_pack(const int8_t *w, size_t nrow, size_t n_per_row,
                 float w_scale, uint8_t *dst);
/* Code of weight (r, k) of an I2_S tensor (0, 1, 2; 3 never produced). */
int orc_i2s_code(const uint8_t *i2s, size_t n_per_row, size_t r, size_t k);
float orc_i2s_scale(const uint8_t *i2s, size_t nrow, size_t n_per_row);
/* quantize_row_i8_s for one row of n floats. */
void orc_quantize_row_i8_s(const float *x, size_t n, int8_t *q,
                           float *act_scale, int32_t *act_sum);
/* Rows of the above: act_scale[r] = s of row r. */
void orc_act_quant_i8(const float *x, size_t rows, size_t n, int8_t *q,
                      float *act_scale);
/* ggml_vec_dot_i2_i8_s on row r: sum of code * q over the row. */
int32_t orc_vec_dot_i2_i8_s(const uint8_t *i2s, size_t n_per_row, size_t r,
                            const int8_t *q);
/* bitnet.cpp's mul_mat over I2_S for ncols activation rows (xq
 * [ncols][in_len], act_scale [ncols]): y[c*out_len + r] =
 * (((float)sumi - (float)act_sum[c]) / act_scale[c]) * scale, with
 * acc[c*out_len + r] = sumi - act_sum[c] (= sum_k w*q) when acc != NULL. */
void orc_gemm_i2s(const uint8_t *i2s, size_t out_len, size_t in_len,
                  const int8_t *xq, const float *act_scale, size_t ncols,
                  int32_t *acc, float *y, int nthreads);

/* ---- the library's I2 layouts (device repacks of I2_S) -------------------
 *
 * Canonical I2 packing: row r is in_len/4 bytes; element k sits in byte k/4
 * at bits 2*(k%4)..2*(k%4)+1 as code = w + 1.  w in {-1,0,1}.
 * Returns -1 if a weight is outside {-1,0,1} or in_len % 4 != 0. */
int orc_i2_pack(const int8_t *w, size_t out_len, size_t in_len, uint8_t *packed);
/* Decode: w = code - 1 (code 3, never produced by the packer, decodes to 2). */
void orc_i2_unpack(const uint8_t *packed, size_t out_len, size_t in_len,
                   int8_t *w);
/* I2_S codes -> canonical codes (the same code for every weight). */
int orc_i2s_to_canonical(const uint8_t *i2s, size_t out_len, size_t in_len,
                         uint8_t *canonical);
/* Device-tiled I2 layout (ouro_hip.h): G = in_len/256, 8-row tiles,
 * tiles = ceil(out_len/8), lane-local group g of lane l is canonical byte
 * column 64*o + s*l + (g - o) (chunks of 4, 2, 1 groups), a lane's share
 * stored in 16-byte units (G even) or 8-byte units (G odd); padding rows
 * hold code 1.  Returns the byte count written (0 if in_len % 256 != 0).
 * `tiled` must hold that many bytes. */
size_t orc_i2_tiled_bytes(size_t out_len, size_t in_len);
size_t orc_i2_tile(const uint8_t *canonical, size_t out_len, size_t in_len,
                   uint8_t *tiled);
/* MFMA-tiled I2 layout (ouro_hip.h): 1 KiB unit per (16-row tile, 256-k
 * block); lane l's word s holds row 16*rt + l%16, k = 256*kb + 64*s +
 * 16*(l/16) + 4j + i at bits 8i + 2j as the 2-bit two's complement of
 * 1 - code.  Padding rows hold code 1 (w = 0).  Returns the byte count. */
size_t orc_i2_mfma_bytes(size_t out_len, size_t in_len);
size_t orc_i2_tile_mfma(const uint8_t *canonical, size_t out_len, size_t in_len,
                        uint8_t *dst);
/* The product on canonical codes with bitnet.cpp's epilogue:
 * y[c*out_len + r] = ((float)acc / act_scale[c]) * w_scale,
 * acc = sum_k w[r][k] * xq[c][k] (exact int32).  acc may be NULL.  Equal to
 * orc_gemm_i2s on the same weights while |sumi| and |act_sum| < 2^24 (they
 * are then exact in float), i.e. for every in_len <= 66051. */
void orc_gemm_i2(const uint8_t *packed, size_t out_len, size_t in_len,
                 const int8_t *xq, const float *act_scale, size_t ncols,
                 float w_scale, int32_t *acc, float *y, int nthreads);

/* ---- hadamard.rs ------------------------------------------------------- */

void orc_wht_inplace(float *x, size_t n);              /* hadamard.rs:15-31 */
/* rotate_fwd / rotate_inv (hadamard.rs:41-66); check_args (33-37) failures
 * return -1 instead of panicking. */
int orc_rotate_fwd(float *x, const float *signs, size_t n, size_t block);
int orc_rotate_inv(float *x, const float *signs, size_t n, size_t block);
/* rows x n helper, rows split across threads (one rotate call per row). */
int orc_rotate_rows(float *x, const float *signs, size_t rows, size_t n,
                    size_t block, int inverse, int nthreads);

/* ---- qwen35.rs --------------------------------------------------------- */

/* delta_head_dim (qwen35.rs:27-57); state element (i,j) at i + j*sdim. */
void orc_delta_head_dim(float *state, size_t sdim, const float *q,
                        const float *k, const float *v, float gate, float beta,
                        float *out);
void orc_l2_norm(float *v, size_t n, float eps);       /* qwen35.rs:73-79 */
float orc_softplus(float x);                           /* qwen35.rs:1241-1243 */
float orc_sigmoid(float x);                            /* qwen35.rs:1067 */
float orc_silu(float x);                               /* ops.rs:34-36 */
float orc_conv_step(float ring[3], const float w[4], float x); /* qwen35.rs:64-70 */
void orc_gated_norm_rms(const float *x, const float *w, const float *gate,
                        size_t n, float eps, float *y); /* qwen35.rs:82-92 */
float orc_delta_q_scale(size_t d);                     /* qwen35.rs:108-110 */

/* Flags shared with ouro_hip.h (same values). */
#define ORC_GDN_L2NORM_QK   1u  /* l2_norm q and k per head (qwen35.rs:1101-1102) */
#define ORC_GDN_SCALE_Q     2u  /* q *= 1/sqrt(d) after the norm (qwen35.rs:1107) */
#define ORC_GDN_KHEAD_DIV   4u  /* k-head = v / (Hv/Hk) instead of v % Hk (qwen35.rs:1098) */

/* Batched decode step: the per-v-head loop of run_delta
 * (qwen35.rs:1096-1112) over B sequences.  Layouts:
 *   q,k [B][Hk][d] f32 (raw, e.g. bf16-decoded); v [B][Hv][d];
 *   gate, beta [B][Hv] (gate is the log-decay: decay = exp(gate));
 *   state [B][Hv][d*d] (element (i,j) at i + j*d); out [B][Hv][d]. */
void orc_gdn_decode(float *state, const float *q, const float *k,
                    const float *v, const float *gate, const float *beta,
                    float *out, size_t B, size_t Hk, size_t Hv, size_t d,
                    unsigned flags, float eps, int nthreads);
/* Token-by-token prefill (the reference prefill, shell/src/bonsai.rs:48-52
 * driving run_delta): T tokens of one sequence, q,k [T][Hk][d], v [T][Hv][d],
 * gate, beta [T][Hv], out [T][Hv][d]; state [Hv][d*d] updated in place. */
void orc_gdn_prefill_tokens(float *state, const float *q, const float *k,
                            const float *v, const float *gate,
                            const float *beta, float *out, size_t T,
                            size_t Hk, size_t Hv, size_t d, unsigned flags,
                            float eps, int nthreads);
/* N sequences packed varlen (cu_seqlens[0..N], state [N][Hv][d*d]), each
 * token by token as orc_gdn_prefill_tokens, threads over (sequence, head). */
void orc_gdn_prefill_varlen(float *state, const float *q, const float *k,
                            const float *v, const float *gate,
                            const float *beta, float *out,
                            const int32_t *cu_seqlens, size_t N, size_t Hk,
                            size_t Hv, size_t d, unsigned flags, float eps,
                            int nthreads);

#define ORC_GDN_V_GROUPED   8u  /* gated output in V-grouped order (qwen35.rs:1122-1138) */

/* The delta-net layer block of run_delta (qwen35.rs:1066-1140) for B
 * sequences, one token each: beta = sigmoid(beta_raw), gate =
 * a_log * softplus(alpha_raw + dt_bias); causal conv step + SiLU on every
 * channel; per v-head l2-normed q, k (q scaled by 1/sqrt(d)) through
 * delta_head_dim; gated_norm_rms(o, norm_w, z) per head; with
 * ORC_GDN_V_GROUPED the heads are written in the grouped order (v-head
 * r*Hk + k to position k*(Hv/Hk) + r).  flags: ORC_GDN_KHEAD_DIV,
 * ORC_GDN_V_GROUPED.  Layouts:
 *   qkv [B][ch], ch = 2*Hk*d + Hv*d (q | k | v); z [B][Hv*d];
 *   beta_raw, alpha_raw [B][Hv]; dt_bias, a_log [Hv]; conv_w [ch][4];
 *   norm_w [d]; conv [B][ch][3] and state [B][Hv][d*d] updated in place;
 *   out [B][Hv*d]. */
void orc_gdn_layer_decode(const float *qkv, const float *z,
                          const float *beta_raw, const float *alpha_raw,
                          const float *dt_bias, const float *a_log,
                          const float *conv_w, const float *norm_w,
                          float *conv, float *state, float *out, size_t B,
                          size_t Hk, size_t Hv, size_t d, unsigned flags,
                          float eps, int nthreads);

/* finite_argmax (infer/mod.rs:70-83): first index of the largest non-NaN
 * value under `>`, 0 when every value is NaN. */
size_t orc_finite_argmax(const float *l, size_t n);

/* OURO_N_THREADS or all logical cores (ops.rs:62-73). */
int orc_mt_threads(void);

#ifdef __cplusplus
}
#endif
#endif
