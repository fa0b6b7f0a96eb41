/*
 * ouro_hip.h - C ABI of the MI355X (gfx950) quantized-inference hot path.
 *
 * This is the drop-in boundary for the kernel-call surface of OuroborOS's
 * Rust engine (cluster/src/infer/).  Every entry point below names the
 * reference function it replaces (file:line in the reference tree).  All
 * compute entry points work on DEVICE buffers owned by the caller, are
 * stream-ordered (asynchronous w.r.t. the host) and never allocate device
 * memory, except the documented workspace users, which take memory from a
 * library workspace kept per (device, stream), grown on first use (after a
 * synchronise of that stream) and kept until ouro_stream_destroy() of the
 * stream or ouro_shutdown():
 *   - ouro_matvec_q / ouro_matmul_q on the 2-bit kinds (the int8
 *     activations of x);
 *   - ouro_matvec_q on a raw TL1 or TQ1_0 payload of 8192 rows or more
 *     (k == 1): the lookup kernels' per-block partial sums;
 *   - ouro_matmul_q on a raw TL1 payload for k >= 2 columns: x as int8
 *     digit planes for the MFMA pass;
 *   - ouro_gdn_chunk_prefill with a NULL workspace.
 * A weight handle (ouro_weight_upload) or ouro_matvec_q_noalloc avoids them.
 *
 * Conventions
 *  - Scratch is per stream: the library workspace, the ouro_finite_argmax
 *    key slots (the null stream's made by ouro_init, another stream's on its
 *    first call) and each weight handle's scratch (the null stream's made at
 *    upload, another stream's on the handle's first call there) are kept
 *    per (device, stream), so calls on different streams never share any;
 *    calls on one stream are ordered by it.  The first call on a new stream
 *    allocates that stream's share (hipMalloc) and is not capturable.  The
 *    one exception is the static array of ouro_matvec_q_noalloc: one per
 *    device, shared by every stream (overlapping calls race).
 *    Entry points given caller buffers share nothing.
 *  - Return value: OURO_OK (0) or an ouro_status code.  The failing call's
 *    message is kept in a thread-local buffer, read with ouro_last_error().
 *    No entry point aborts the process (the reference's assert!/bail! paths,
 *    e.g. infer/mod.rs:139-145, hadamard.rs:33-37, become status codes).
 *  - `stream` is a hipStream_t passed as void*; NULL is the null stream.
 *  - Shapes are checked on the host before any launch; a kernel is never
 *    launched on a shape it does not handle.
 *  - Element (i, j) of a delta-net state head is at i + j*d, i.e. the k
 *    dimension is contiguous (qwen35.rs:19-20).
 *  - Matrices are row-major W[out_len][in_len], y = W x (ops.rs:1-4).
 */
#ifndef OURO_HIP_H
#define OURO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OURO_ABI_VERSION 2

typedef enum ouro_status {
    OURO_OK = 0,
    OURO_ERR_INVALID_ARG = 1, /* NULL pointer, zero size, bad flag */
    OURO_ERR_SHAPE = 2,       /* shape the entry point does not support */
    OURO_ERR_ALIGN = 3,       /* pointer not aligned as documented */
    OURO_ERR_KIND = 4,        /* quant kind not supported by this entry */
    OURO_ERR_NO_DEVICE = 5,   /* no HIP device, or init failed */
    OURO_ERR_HIP = 6,         /* a HIP runtime call failed */
    OURO_ERR_NOT_INIT = 7,    /* ouro_init() was not called */
} ouro_status;

/* Quant kinds.  The ggml dtype ids of QuantKind::from_dtype
 * (dequant.rs:334-348) are kept as the numeric values. */
enum {
    OURO_KIND_F32 = 0,
    OURO_KIND_F16 = 1,
    OURO_KIND_BF16 = 30,
    OURO_KIND_Q8_0 = 8,    /* 34 B / 32: d f16, qs int8[32] (dequant.rs:225-231) */
    OURO_KIND_Q3K = 11,    /* 110 B / 256: hmask, qs, scales[12], d (dequant.rs:398-451) */
    OURO_KIND_Q4K = 12,    /* 144 B / 256: d, dmin, scales[12], qs (dequant.rs:257-282) */
    OURO_KIND_Q5K = 13,    /* 176 B / 256: d, dmin, scales[12], qh, qs (dequant.rs:454-481) */
    OURO_KIND_Q6K = 14,    /* 210 B / 256: ql, qh, scales int8[16], d (dequant.rs:484-510) */
    OURO_KIND_TQ1_0 = 34,  /* 54 B / 256 weights, base-3 (dequant.rs:49-105) */
    OURO_KIND_TL1 = 143,   /* PTQ1_0, 28 B / 128 weights (dequant.rs:124-195) */
    /* bitnet.cpp's I2_S tensor (GGML_TYPE_I2_S of microsoft/BitNet's ggml
     * fork, the reference's bitnet-cpp submodule, .gitmodules): 2-bit codes
     * in 128-weight blocks, then one fp32 per-tensor scale (layout below).
     * The reference names it its portable ternary baseline and GPU route
     * (PLAN.md:465,1277). */
    OURO_KIND_I2_S = 36,
    /* This library's resident layout of the same codes: the device-tiled
     * layout below followed by the fp32 per-tensor scale. */
    OURO_KIND_I2 = 0x4932,
};

/* Element dtypes for activation buffers. */
enum { OURO_DT_F32 = 0, OURO_DT_BF16 = 1 };

/* ------------------------------------------------------------------ */
/* Runtime                                                             */
/* ------------------------------------------------------------------ */

/* Select and initialise a device.  device < 0 picks OURO_GPU_INDEX from the
 * environment, else 0 (the reference's GPU pick, ouro-wgpu/src/lib.rs:219-248).
 * Safe to call again; it re-selects the device. */
int ouro_init(int device);
/* Releases the library workspaces.  Caller buffers are never touched. */
int ouro_shutdown(void);
const char *ouro_last_error(void);
int ouro_abi_version(void);
int ouro_device_count(int *count);
/* Device name of the initialised device (e.g. "gfx950"). */
int ouro_device_arch(char *buf, size_t len);

/* Device memory and stream plumbing for callers that have no other HIP
 * runtime at hand (tests, benches, FFI hosts).  Thin wrappers over HIP. */
int ouro_malloc(void **ptr, size_t bytes);
int ouro_free(void *ptr);
int ouro_memcpy_htod(void *dst, const void *src, size_t bytes);
int ouro_memcpy_dtoh(void *dst, const void *src, size_t bytes);
int ouro_memcpy_dtod(void *dst, const void *src, size_t bytes, void *stream);
int ouro_memset(void *dst, int value, size_t bytes, void *stream);
int ouro_stream_create(void **stream);
int ouro_stream_destroy(void *stream);
int ouro_stream_synchronize(void *stream);
int ouro_device_synchronize(void);
int ouro_event_create(void **event);
int ouro_event_destroy(void *event);
int ouro_event_record(void *event, void *stream);
int ouro_event_elapsed_ms(float *ms, void *start, void *stop);

/* ------------------------------------------------------------------ */
/* Ternary GEMV / GEMM: int8 per-token-absmax activations x 2-bit      */
/* ternary weights, exact int32 accumulation (bitnet.cpp's I2_S/I8_S). */
/* ------------------------------------------------------------------ */
/*
 * The contract is bitnet.cpp's (microsoft/BitNet, src/ggml-bitnet-mad.cpp;
 * its pinned commit is not recoverable from the reference checkout, whose
 * bitnet-cpp submodule is empty, so the rules follow the published source):
 *
 * I2_S tensor [out_len][in_len] (quantize_i2_s), n = out_len*in_len: the
 *   flattened weights in blocks of 128; weight j of block b sits in byte
 *   32*b + j%32 at bits 6-2*(j/32) .. 7-2*(j/32) as code = w + 1
 *   (0 = -1, 1 = 0, 2 = +1); one little-endian fp32 scale at byte n/4; the
 *   tensor is n/4 + 32 bytes (scale, then alignment padding).  With
 *   in_len % 256 == 0 (required here) row r is bytes r*in_len/4 ..
 *
 * Activation quantisation per row of n values (quantize_row_i8_s):
 *   s = (float)(127 / max(max|x|, 1e-5)) (in double), act_scale = s;
 *   q = clamp(round(x * s), -128, 127), x * s a float product, round()
 *   half away from zero.
 * Output (the I2_S branch of the fork's mul_mat):
 *   y = ((float)acc / act_scale) * w_scale, acc = sum_k w*q (exact int32),
 *   the division and the product rounded separately.  bitnet.cpp forms
 *   acc as sum(code*q) - sum(q) in float, which is the same value while
 *   both sums stay below 2^24 (in_len <= 66051).
 *
 * Canonical I2 bytes (this library's interchange form, e.g. for the
 * tilers): row r is in_len/4 bytes; weight k of the row sits in byte k/4 at
 * bits 2*(k%4)..2*(k%4)+1 as code = w + 1.  Decoding is w = code - 1.
 *
 * Device-tiled I2 (what the GEMV reads; ouro_i2s_tile() / ouro_i2_tile()
 * produce it):
 *   G = in_len / 256 four-weight groups per lane per row (in_len % 256 == 0),
 *   R = 8 rows per tile, tiles = ceil(out_len / 8) (rows past out_len hold
 *   code 1, i.e. w = 0, and are never written out).  Tile t starts at byte
 *   t * 8 * in_len / 4.  Inside a tile, lane l (0..63) owns G k-groups
 *   (four weights each) of all 8 rows: lane-local group g (0..G-1) is the
 *   canonical byte column
 *     kg(l, g) = 64*o + s*l + (g - o),
 *   where the G local groups are cut into chunks of s = 4 groups, then one
 *   of s = 2 (if G % 4 >= 2), then one of s = 1 (if G is odd), and o is the
 *   first local group of g's chunk; so each chunk's activations are one
 *   contiguous segment (4*s bytes per lane, lanes in order).  A lane's 2*G
 *   32-bit words are stored in units of U = 16 bytes (G even) or U = 8 bytes
 *   (G odd), W = U/4 words each; its word d (0 .. 2*G - 1) sits at byte
 *   (d/W)*64*U + l*U + (d%W)*4, so every U-byte load of a 64-lane wavefront
 *   is one contiguous 64*U-byte segment.  Word d carries four groups
 *   gi = 4d + f (f = 0..3); group gi is row r = gi / G, local group
 *   g = gi % G, i.e. weights k = 4*kg(l, g) + b (b = 0..3), whose codes sit
 *   at bits 8*b + 2*f of the word.
 */

/* Size in bytes of the device-tiled codes (without the trailing scale). */
size_t ouro_i2_tiled_bytes(size_t out_len, size_t in_len);
/* canonical (device) -> tiled (device).  in_len % 256 == 0.  When
 * w_scale_or_null is given, the fp32 scale is written right after the
 * tiled codes, making `tiled` a complete OURO_KIND_I2 payload. */
int ouro_i2_tile(const uint8_t *canonical, size_t out_len, size_t in_len,
                 uint8_t *tiled, const float *w_scale_or_null, void *stream);
/* I2_S tensor (device) -> complete OURO_KIND_I2 payload (tiled codes, then
 * the tensor's scale).  in_len % 256 == 0, tiled 16-byte aligned with
 * ouro_i2_tiled_bytes() + 4 bytes.  The device-side repack that the
 * reference's resident-weight upload does on the host
 * (ouro-wgpu/src/lib.rs:256-263); no counterpart in bitnet.cpp. */
int ouro_i2s_tile(const uint8_t *i2s, size_t out_len, size_t in_len,
                  uint8_t *tiled, void *stream);
/* quantize_row_i8_s (bitnet.cpp) of rows x n activations (f32 or bf16):
 * int8 rows xq [rows][n] and act_scale[rows] (s of each row, above). */
int ouro_act_quant_i8(const void *x, int x_dtype, size_t rows, size_t n,
                      int8_t *xq, float *act_scale, void *stream);
/* y[c*out_len + r] for ncols activation columns (xq row-major [ncols][in]),
 * column-major output like matmul_q (ops.rs:160-161).  acc_or_null, when
 * given, receives the exact int32 accumulators in the same layout.
 * w_scale is read from the device (4 bytes), e.g. the payload tail.
 * w_tiled and xq need 16-byte alignment. */
int ouro_gemm_i2(const uint8_t *w_tiled, size_t out_len, size_t in_len,
                 const float *w_scale, const int8_t *xq, const float *act_scale,
                 size_t ncols, float *y, int32_t *acc_or_null, void *stream);
/* Grouped launch over `count` independent (weight, activation, output)
 * triples of one shape, laid out at fixed strides (bytes / elements):
 * matrix m uses w_tiled + m*w_stride, w_scale[m], xq + m*x_stride,
 * act_scale[m], y + m*y_stride (w_stride and x_stride multiples of 16, both
 * bases 16-byte aligned).  One column each.  This is the shape of the
 * projections that share a step but not a matrix (e.g. all layers' weight
 * streams of one decode step handed to the GPU at once). */
int ouro_gemv_i2_grouped(const uint8_t *w_tiled, size_t w_stride,
                         const float *w_scale, const int8_t *xq,
                         size_t x_stride, const float *act_scale, float *y,
                         size_t y_stride, size_t out_len, size_t in_len,
                         size_t count, void *stream);

/*
 * Ternary x int8 GEMM on int8 MFMA for many activation columns: the
 * K-column product of matmul_q / matmul_tl1 (ops.rs:156-230; col-major
 * output as ops.rs:160-161), which decodes the weights once for all K
 * columns; for batched verify and prefill projections.
 *
 * MFMA-tiled I2 (ouro_i2_tile_mfma() produces it): 1 KiB units, one per
 * (row tile rt of 16 rows, k block kb of 256), unit at byte
 * (rt * in_len/256 + kb) * 1024; tiles = ceil(out_len / 16), rows past
 * out_len hold w = 0.  Lane l (0..63) of a unit has 16 bytes; its 32-bit
 * word s (0..3) holds row 16*rt + l%16, weights
 * k = 256*kb + 64*s + 16*(l/16) + 4*j + i (i, j = 0..3) at bits
 * 8*i + 2*j, each as the 2-bit two's complement of v = 1 - code (= -w).
 * Results are bit-identical to ouro_gemm_i2 for any ncols.
 */
size_t ouro_i2_mfma_bytes(size_t out_len, size_t in_len);
/* canonical (device) -> MFMA-tiled (device); in_len % 256 == 0, dst 16-byte
 * aligned.  When w_scale_or_null is given, the fp32 scale is written right
 * after the codes. */
int ouro_i2_tile_mfma(const uint8_t *canonical, size_t out_len, size_t in_len,
                      uint8_t *dst, const float *w_scale_or_null, void *stream);
/* I2_S tensor (device) -> MFMA-tiled codes followed by the tensor's scale
 * (dst: ouro_i2_mfma_bytes() + 4 bytes, 16-byte aligned). */
int ouro_i2s_tile_mfma(const uint8_t *i2s, size_t out_len, size_t in_len,
                       uint8_t *dst, void *stream);
/* y[c*out_len + r] = (acc / act_scale[c]) * w_scale for ncols int8 columns
 * (xq row-major [ncols][in_len], 16-byte aligned); acc_or_null receives
 * the exact int32 sums.  Same semantics as ouro_gemm_i2. */
int ouro_gemm_i2_mfma(const uint8_t *w_mfma, size_t out_len, size_t in_len,
                      const float *w_scale, const int8_t *xq,
                      const float *act_scale, size_t ncols, float *y,
                      int32_t *acc_or_null, void *stream);

/* ------------------------------------------------------------------ */
/* Reference matvec surface                                             */
/* ------------------------------------------------------------------ */

/* matvec_q (ops.rs:76-84): y = W x, x f32[in_len], y f32[out_len], W the
 * device payload of `kind`:
 *   OURO_KIND_TL1   - PTQ1_0 groups (fused decode + dot, ops.rs:294-363)
 *   OURO_KIND_TQ1_0 - TQ1_0 blocks (matvec_qblock, ops.rs:101-128)
 *   OURO_KIND_Q8_0, OURO_KIND_Q3K, OURO_KIND_Q4K, OURO_KIND_Q5K,
 *   OURO_KIND_Q6K   - ggml blocks as they are, any byte alignment
 *                     (matvec_qblock, ops.rs:101-128; in_len a multiple of
 *                     the block's 32 / 256 elements, x 4-byte aligned);
 *                     decode and dot fused in one pass, no scratch
 *   OURO_KIND_F32 / F16 / BF16 - dense rows (ops.rs:87-98,131-154,600-623)
 *   OURO_KIND_I2_S  - a bitnet.cpp I2_S tensor as it is (16-byte aligned,
 *                     in_len % 256 == 0, in_len <= 32768)
 *   OURO_KIND_I2    - tiled I2 + scale
 *   For both ternary 2-bit kinds x is quantised per call (quantize_row_i8_s,
 *   above) into the library workspace.  TL1 and TQ1_0 payloads of 8192 rows
 *   or more run the table-lookup kernels, whose per-block partial sums also
 *   live in the library workspace (per stream; ouro_matvec_q_noalloc or a
 *   weight handle keeps these calls allocation-free).
 * Floating-point sums are not in the reference's order; results agree to
 * float32 rounding (the reference's own fused-vs-scalar bar is rel 1e-5,
 * ops.rs:800-838). */
int ouro_matvec_q(const void *payload, int kind, size_t out_len,
                  size_t in_len, const float *x, float *y, void *stream);
/* matmul_q (ops.rs:219-230): x row-major [k][in_len], y column-major
 * y[c*out_len + r] (ops.rs:160-161). */
int ouro_matmul_q(const void *payload, int kind, size_t out_len,
                  size_t in_len, const float *x, size_t k, float *y,
                  void *stream);
/* ouro_matvec_q that allocates nothing, for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation).  No counterpart in the reference.  It uses a
 * static per-device scratch array of 16 MiB that each device holds until
 * the process ends.  For the 2-bit kinds (OURO_KIND_I2_S, OURO_KIND_I2) x
 * is quantised into its first 32 KiB + 256 B, so in_len <= 32768
 * (OURO_ERR_SHAPE beyond).  TL1 and TQ1_0 payloads of 8192 rows or more
 * keep the table-lookup kernels' per-block partial sums there when they fit
 * (TL1: ceil(in_len/512) * out_len floats, TQ1_0: in_len/512 * out_len,
 * at most 16 MiB: the 248320x5120 lm_head takes 9.9 MB); larger ones run
 * the direct decode kernel, which needs no scratch (slower; within rel
 * 1e-5 of ouro_matvec_q).  The other kinds use no scratch.  Wherever the
 * same kernels run, results equal ouro_matvec_q's bit for bit.  All calls on
 * one device share the scratch: calls that overlap on one device (e.g. on
 * two streams) race. */
int ouro_matvec_q_noalloc(const void *payload, int kind, size_t out_len,
                          size_t in_len, const float *x, float *y,
                          void *stream);

/* ------------------------------------------------------------------ */
/* Walsh-Hadamard rotation                                              */
/* ------------------------------------------------------------------ */

#define OURO_FWHT_INVERSE 1u /* rotate_inv: h = s o (H z)/sqrt(N) */

/* Row-batched rotate_fwd / rotate_inv (hadamard.rs:41-66): each of `rows`
 * rows of n elements is rotated in blocks of `block` (power of two,
 * 2..8192, n % block == 0).  signs: NULL (all +1) or f32[n], +-1 each.
 * The fp32 result is bit-identical to the reference: same butterfly stages
 * in the same order (hadamard.rs:15-31), same scale 1/sqrtf(block).
 * x and y may alias.  Either dtype on either side; bf16 output is rounded
 * to nearest-even.  When xq/act_scale are non-NULL, each row of the output
 * (as stored, i.e. after bf16 rounding) is also int8-absmax-quantised as
 * ouro_act_quant_i8 does (the fused FWHT -> quantisation epilogue);
 * y may then be NULL to skip storing the rotated activations. */
int ouro_fwht_rows(const void *x, int x_dtype, void *y, int y_dtype,
                   size_t rows, size_t n, size_t block, const float *signs,
                   unsigned flags, int8_t *xq, float *act_scale, void *stream);
/* Exact mirrors of hadamard::rotate_fwd / rotate_inv (hadamard.rs:41,57)
 * on one f32 device vector, in place. */
int ouro_rotate_fwd(float *x, const float *signs, size_t n, size_t block,
                    void *stream);
int ouro_rotate_inv(float *x, const float *signs, size_t n, size_t block,
                    void *stream);

/* ------------------------------------------------------------------ */
/* Gated delta-net                                                      */
/* ------------------------------------------------------------------ */

#define OURO_GDN_L2NORM_QK 1u /* l2_norm q,k per head (qwen35.rs:73-79,1101-1102) */
#define OURO_GDN_SCALE_Q   2u /* q *= 1/sqrt(d) after the norm (qwen35.rs:1095,1107) */
#define OURO_GDN_KHEAD_DIV 4u /* k-head = v/(Hv/Hk); default v % Hk (qwen35.rs:1098) */
#define OURO_GDN_V_GROUPED 8u /* layer output in V-grouped head order (qwen35.rs:1122-1138) */

/* delta_head_dim (qwen35.rs:27-57) for one head, in place on the device:
 * decay = exp(gate); sk = decay * S^T k; dv = beta (v - sk);
 * S = decay S + k dv^T; out = S^T q.  Like the reference's runtime-dim
 * variant any sdim works, here 1..256 (128 runs the tuned decode kernel);
 * q is pre-scaled. */
int ouro_delta_head_dim(float *state, size_t sdim, const float *q,
                        const float *k, const float *v, float gate,
                        float beta, float *out, void *stream);

/* One decode step for B sequences x Hv v-heads (run_delta's per-head loop,
 * qwen35.rs:1096-1112, with the recurrence of qwen35.rs:27-57).
 *   q, k   : [B][Hk][d], dtype qk_dtype (raw; normalised per flags)
 *   v      : [B][Hv][d], dtype v_dtype
 *   gate   : [B][Hv] f32 log-decay (decay = exp(gate)); beta: [B][Hv] f32
 *   state  : [B][Hv][d][d] f32, element (i,j) of a head at i + j*d; updated
 *   out    : [B][Hv][d] f32
 * d in 1..256 (d == 128, the qwen35 family's d_state, runs the tuned
 * kernel; OURO_GDN_SCALE_Q scales q by 1/sqrt(d)), Hv % Hk == 0.  eps is the
 * l2_norm epsilon (outside the sqrt). */
int ouro_gdn_decode(float *state, const void *q, const void *k, int qk_dtype,
                    const void *v, int v_dtype, const float *gate,
                    const float *beta, float *out, size_t B, size_t Hk,
                    size_t Hv, size_t d, unsigned flags, float eps,
                    void *stream);

/* Chunked prefill of N sequences packed into one varlen buffer of T tokens
 * (cu_seqlens_host[0..N] on the HOST, [0] = 0, [N] = T; NULL means one
 * sequence of T tokens).  Same head layout and flags as ouro_gdn_decode,
 * with a token axis in place of the batch axis:
 *   q, k [T][Hk][d] bf16; v [T][Hv][d] bf16; gate, beta [T][Hv] f32;
 *   state [N][Hv][d][d] f32 (initial state in, final state out);
 *   out [T][Hv][d] f32.
 * The result equals running the decode recurrence token by token (the
 * reference prefill, shell/src/bonsai.rs:48-52 driving run_delta,
 * qwen35.rs:1048-1158); inside each chunk of `chunk` (64) tokens it uses the
 * WY/UT form with bf16 MFMA contractions and fp32 accumulation.  d == 128.
 * A state-independent pass over all chunks writes per-chunk records into
 * `workspace` (device memory of ouro_gdn_chunk_workspace_bytes(T, N, Hv, d,
 * chunk) bytes, 16-byte aligned; NULL = the library's per-device workspace,
 * grown on demand).  Sequences are launched in slices of 256, offsets as
 * kernel arguments. */
size_t ouro_gdn_chunk_workspace_bytes(size_t T, size_t N, size_t Hv, size_t d,
                                      size_t chunk);
int ouro_gdn_chunk_prefill(float *state, const void *q, const void *k,
                           const void *v, const float *gate,
                           const float *beta, float *out,
                           const int32_t *cu_seqlens_host, size_t N,
                           size_t T, size_t Hk, size_t Hv, size_t d,
                           size_t chunk, unsigned flags, float eps,
                           void *workspace, void *stream);

/* The delta-net layer block of one decode step, replacing the middle of
 * Qwen35Stage::run_delta (qwen35.rs:1066-1140) between its input
 * projections and ssm_out, for B sequences:
 *   beta = sigmoid(beta_raw), gate = a_log * softplus(alpha_raw + dt_bias)
 *     (qwen35.rs:1066-1070, 1241-1243);
 *   conv_out = silu(conv_step(ring, conv_w, qkv)) per channel, ring updated
 *     (qwen35.rs:1080-1088, 64-70);
 *   per v-head: q, k of its k-head l2-normed, q scaled by 1/sqrt(d), one
 *     delta_head_dim step on its state (qwen35.rs:1096-1112);
 *   out = gated_norm_rms(o, norm_w, z) per head (qwen35.rs:1119-1121,
 *     82-92), in V-grouped head order with OURO_GDN_V_GROUPED.
 * Layouts (f32): qkv [B][ch] with ch = 2*Hk*d + Hv*d (q | k | v), z
 * [B][Hv*d], beta_raw/alpha_raw [B][Hv], dt_bias/a_log [Hv], conv_w
 * [ch][4], norm_w [d], conv_state [B][ch][3] (oldest first) and state
 * [B][Hv][d][d] updated in place, out [B][Hv*d].  d == 128; flags:
 * OURO_GDN_KHEAD_DIV, OURO_GDN_V_GROUPED.  One launch that needs no
 * scratch: `workspace` is ignored (pass NULL) and
 * ouro_gdn_layer_workspace_bytes returns 0; both stay for callers written
 * against a workspace-taking form. */
size_t ouro_gdn_layer_workspace_bytes(size_t B, size_t Hk, size_t Hv, size_t d);
int ouro_gdn_layer_decode(const float *qkv, const float *z, const float *beta_raw,
                          const float *alpha_raw, const float *dt_bias,
                          const float *a_log, const float *conv_w,
                          const float *norm_w, float *conv_state, float *state,
                          float *out, size_t B, size_t Hk, size_t Hv, size_t d,
                          unsigned flags, float eps, void *workspace,
                          void *stream);

/* ------------------------------------------------------------------ */
/* Resident weights (GpuPool::upload_q6k / matvec, ouro-wgpu/src/lib.rs:   */
/* 251-356): upload once, repacking on upload, then matvec by handle.    */
/* ------------------------------------------------------------------ */

typedef struct ouro_weight *ouro_weight_t;

/* Upload `bytes` host bytes of a `kind` tensor [out_len][in_len].  For
 * OURO_KIND_I2_S, `host` is a bitnet.cpp I2_S tensor (out_len*in_len/4
 * code bytes, its fp32 scale, up to 28 padding bytes: 4..32 bytes past the
 * codes) and w_scale is ignored.  For OURO_KIND_I2, `host` holds canonical
 * I2 codes (out_len*in_len/4 bytes) and w_scale is the per-tensor scale.
 * Both are tiled on upload and held as an OURO_KIND_I2 payload.  For the
 * other kinds host holds the reference payload (row_bytes*out_len bytes)
 * and w_scale is ignored.  In_len must be a whole number of the kind's
 * blocks (OURO_ERR_SHAPE otherwise).  max_cols sizes the handle's own
 * activation scratch (for matmul up to max_cols columns); an I2 handle with
 * max_cols >= 8 also keeps the codes in the MFMA layout, and its matmuls
 * of 8 or more columns run on the int8 MFMA GEMM (same results).  A TL1 or
 * TQ1_0 handle with max_cols >= 2 also keeps its trits in that layout with
 * the f16 scale of every 128-group (0.266 bytes per weight, built on the
 * device at upload): its matmuls of 2 or more columns are one int8 MFMA
 * pass for all of them (matmul_tl1's K-column amortisation, ops.rs:156-286;
 * within the reference's K-column bar, rel 1e-3), its matvec stays on the
 * table lookups. */
int ouro_weight_upload(int kind, const void *host, size_t bytes,
                       size_t out_len, size_t in_len, float w_scale,
                       size_t max_cols, ouro_weight_t *out);
int ouro_weight_free(ouro_weight_t w);
/* Device payload of a handle (what ouro_matvec_q takes for its kind; I2
 * and I2_S handles hold an OURO_KIND_I2 payload); NULL for OURO_KIND_TL1,
 * whose handle holds the payload repacked for the table-lookup GEMV
 * (ouro_weight_matvec/matmul) instead of the raw groups. */
const void *ouro_weight_payload(ouro_weight_t w);
int ouro_weight_matvec(ouro_weight_t w, const float *x, float *y,
                       void *stream);
int ouro_weight_matmul(ouro_weight_t w, const float *x, size_t k, float *y,
                       void *stream);
/* Greedy token of a head (Qwen35Stage::sample, qwen35.rs:746-757:
 * finite_argmax(W x)): y = W x for one column, then *idx = finite_argmax(y)
 * as a device int32.  y may be NULL (the handle's own logits scratch is
 * used).  Nothing is allocated. */
int ouro_weight_matvec_argmax(ouro_weight_t w, const float *x, float *y,
                              int32_t *idx, void *stream);
/* finite_argmax (infer/mod.rs:70-83) of n device floats: the first index of
 * the largest non-NaN value (-0 and +0 compare equal), 0 if every value is
 * NaN; *idx is a device int32.  Uses 8 KiB of per-device scratch that
 * ouro_init allocates; the call allocates nothing. */
int ouro_finite_argmax(const float *y, size_t n, int32_t *idx, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* OURO_HIP_H */
