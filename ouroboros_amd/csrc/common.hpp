// common.hpp - shared host/device helpers of libouro_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>

#include "../../include/ouro_hip.h"

namespace ouro {

// ---------------------------------------------------------------- errors --

// Records a formatted message as the calling thread's last error and
// returns `code`, so call sites read `return fail(OURO_ERR_SHAPE, "...")`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
bool initialised();
int current_device();

#define OURO_HIP_TRY(expr)                                                     \
    do {                                                                       \
        hipError_t e_ = (expr);                                                \
        if (e_ != hipSuccess)                                                  \
            return ::ouro::fail(OURO_ERR_HIP, "%s failed: %s", #expr,          \
                                hipGetErrorString(e_));                        \
    } while (0)

#define OURO_REQUIRE_INIT()                                                    \
    do {                                                                       \
        if (!::ouro::initialised())                                            \
            return ::ouro::fail(OURO_ERR_NOT_INIT, "ouro_init() not called");  \
    } while (0)

// Checks the launch that was just enqueued.
int check_launch(const char *what);

// Library scratch per (device, stream, purpose): grown on demand (after a
// synchronise of that stream), freed by ouro_stream_destroy of the stream or
// ouro_shutdown.  Calls on different streams never share a block.  Returns
// nullptr and sets the error on failure.
enum { SCRATCH_WORKSPACE = 0, SCRATCH_ARGMAX = 1 };
void *stream_scratch(int kind, size_t bytes, void *stream, size_t min_bytes);
// The workspace of matvec_q / matmul_q and the chunked prefill (at least 1 MiB).
void *workspace(size_t bytes, void *stream);

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------ device helpers --

// bf16 <-> f32 with round-to-nearest-even (bf16 -> f32 is exact).
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// gfx950 converts with v_cvt_pk_bf16_f32 (round to nearest even).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}

// ---- bitnet.cpp's int8 activation format (I8_S, quantize_row_i8_s in
// src/ggml-bitnet-mad.cpp) and its I2_S mul_mat epilogue.
// Scale of a row with largest magnitude amax: s = 127 / max(amax, 1e-5),
// divided in double and rounded once to float, as the C source does.
__device__ __forceinline__ float i8s_scale(float amax) {
    const double m = fmax(1e-5, static_cast<double>(amax));
    return static_cast<float>(127.0 / m);
}
// q = clamp(round(x * s), -128, 127); the product is a float product and
// round() takes halves away from zero.
__device__ __forceinline__ int i8s_quant(float x, float s) {
    float t = roundf(x * s);
    t = fminf(fmaxf(t, -128.f), 127.f);
    return static_cast<int>(t);
}
// y = (acc / s) * w_scale: the integer sum divided by the activation scale
// (an IEEE division), then times the per-tensor weight scale.
__device__ __forceinline__ float i8s_out(int acc, float s, float w_scale) {
    const float t = static_cast<float>(acc) / s;
    return t * w_scale;
}
// The same value from a per-row reciprocal: for s >= 2^-76, inv = RN(1 / s)
// (one IEEE division per activation row); q = RN(acc inv) is within an ulp
// of acc / s, the residual r = acc - q s is exact in one fma, and
// RN(q + r inv) is the correctly rounded quotient (Markstein's theorem,
// which holds without overflow or underflow: |acc| < 2^24 keeps
// |q| < 2^100, and s <= 127 / 1e-5 keeps it normal).  Three instructions
// instead of the ~10 of a correctly rounded division.  A smaller scale
// (amax past ~1e24) is taken as s 2^64 and the quotient scaled back by 2^64,
// exact since scaling by a power of two commutes with rounding and
// overflows to inf exactly where the quotient does; s = 0 (amax = inf)
// gives acc * (1 / 0), which is acc / 0 (+-inf, or NaN for 0).
// tests/cpp/i8s_quotient_check.c compares this with the division on the host
// for every integer |acc| <= 2^20 against a spread of scales.
struct I8sInv {
    float s, inv, post;
    bool zero;
};
__device__ __forceinline__ I8sInv i8s_inv(float s) {
    I8sInv r;
    const bool small = s < 0x1p-76f;
    r.s = small ? s * 0x1p64f : s;
    r.inv = 1.0f / r.s;
    r.post = small ? 0x1p64f : 1.0f;
    r.zero = s == 0.0f;
    return r;
}
__device__ __forceinline__ float i8s_out_inv(int acc, const I8sInv &d, float w_scale) {
    const float a = static_cast<float>(acc);
    const float q = a * d.inv;
    const float r = __builtin_fmaf(-q, d.s, a);
    const float t = d.zero ? q : __builtin_fmaf(r, d.inv, q) * d.post;
    return t * w_scale;
}

// Canonical byte (codes of weights 4*kg .. 4*kg+3 at bits 2*i) of row `row`
// of an I2_S tensor: the flattened weights in 128-blocks, weight j of block
// b in byte 32*b + j%32 at bits 6 - 2*(j/32) (quantize_i2_s).  The four
// weights share one block and one bit field, in four consecutive bytes.
__device__ __forceinline__ uint32_t i2s_canon_byte(const uint8_t *i2s, long long row, int in_len, int kg) {
    const long long e = row * in_len + 4LL * kg;
    const int j = static_cast<int>(e & 127);
    const uint8_t *p = i2s + (e >> 7) * 32 + (j & 31);
    const int sh = 6 - 2 * (j >> 5);
    uint32_t byte = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) byte |= ((static_cast<uint32_t>(p[i]) >> sh) & 3u) << (2 * i);
    return byte;
}

// Lane exchange across the 64-wide wavefront (ds_bpermute based).
__device__ __forceinline__ float xor_shfl(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}
__device__ __forceinline__ int xor_shfl(int v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// Reduce-scatter of N per-lane values over the lanes of a group of `Lanes`
// consecutive lanes (Lanes a power of two, N a power of two <= Lanes).
// On return, v[0] of lane L holds the group-wide sum of value index
//   idx(L) = sum over the first log2(N) halving stages of the bit of L that
//            was used in that stage, i.e. idx = (L % Lanes) / (Lanes / N).
// Stage offsets run Lanes/2, Lanes/4, ...; the first log2(N) stages halve
// the value count, the rest are a plain butterfly.
template <int N, int Lanes, typename T>
__device__ __forceinline__ T reduce_scatter(T (&v)[N], int lane) {
    static_assert((N & (N - 1)) == 0 && (Lanes & (Lanes - 1)) == 0, "pow2");
    static_assert(N <= Lanes, "N <= Lanes");
    int n = N;
#pragma unroll
    for (int off = Lanes / 2; off >= 1; off >>= 1) {
        if (n > 1) {
            const bool upper = (lane & off) != 0;
            const int h = n / 2;
#pragma unroll
            for (int i = 0; i < N / 2; ++i) {
                if (i < h) {
                    T keep = upper ? v[i + h] : v[i];
                    T send = upper ? v[i] : v[i + h];
                    v[i] = keep + xor_shfl(send, off);
                }
            }
            n = h;
        } else {
            v[0] += xor_shfl(v[0], off);
        }
    }
    return v[0];
}

// Most workgroups of an argmax (slots of 64-bit keys in its scratch).
constexpr int kArgmaxBlocks = 1024;
int argmax_final(const unsigned long long *keys, int nk, int32_t *idx, void *stream);

// One ternary x int8 product of a grouped few-column launch (i2_gemm.hip):
// MFMA-tiled weights w with out_len rows, activations xq/act_scale, y[ncols][out_len].
// Optional element-wise epilogue of a product (the delta-net's conv and gates
// of one decode step, run where the projection outputs are produced):
//   EPI_CONV     y <- silu(conv4(ring[n][row], y)), ring[n][row] shifted in
//                (conv_step, qwen35.rs:64-70; w = conv weights [rows][4])
//   EPI_SIGMOID  y <- 1 / (1 + e^-y)  (beta, qwen35.rs:1066-1067)
//   EPI_GATE     y <- c[row] * softplus(y + b[row])  (qwen35.rs:1068-1070,
//                1241-1243; b = dt_bias, c = a_log)
//   EPI_RESID    y <- b[n][row] + y  (the residual add after a block's
//                output projection; b has y's layout and is not y)
enum { EPI_NONE = 0, EPI_CONV = 1, EPI_SIGMOID = 2, EPI_GATE = 3, EPI_RESID = 4 };
struct GemmEpilogue {
    int op;
    const float *w;  // EPI_CONV
    float *ring;     // EPI_CONV: [ncols][rows][3]
    const float *b, *c;  // EPI_GATE
};
struct GemmProblem {
    const uint8_t *w;
    size_t out_len;
    const float *w_scale;
    const int8_t *xq;
    const float *act_scale;
    float *y;
    int32_t *acc;  // optional exact int32 sums
    GemmEpilogue epi;
    int swiglu;    // rows are interleaved (up, gate) pairs: y[ncols][out_len / 2] = silu(gate) * up
};

// The epilogue's element-wise step for output (column n, row) of a product
// with `rows` rows; the arithmetic of gdn_conv_gate_kernel.
__device__ __forceinline__ float gemm_epilogue(const GemmEpilogue &e, float y, long long n, int row, int rows) {
#pragma clang fp contract(off)
    if (e.op == EPI_CONV) {
        float *r = e.ring + (n * rows + row) * 3;
        const float4 w = *reinterpret_cast<const float4 *>(e.w + 4LL * row);
        const float r0 = r[0], r1 = r[1], r2 = r[2];
        const float v = w.x * r0 + w.y * r1 + w.z * r2 + w.w * y;
        r[0] = r1;
        r[1] = r2;
        r[2] = y;
        return v / (1.0f + expf(-v));
    }
    if (e.op == EPI_SIGMOID) return 1.0f / (1.0f + expf(-y));
    if (e.op == EPI_GATE) {
        const float x = y + e.b[row];
        return e.c[row] * (x > 20.0f ? x : logf(1.0f + expf(x)));
    }
    if (e.op == EPI_RESID) return e.b[n * rows + row] + y;
    return y;
}
// gemm_epilogue on rows row .. row+3 of column n (row and rows multiples of
// 4; y, ring, w and b 16-byte aligned), the operands moved as 16-byte
// pieces; the same arithmetic per element.  Row i's ring is floats 3i .. 3i+2
// of the three pieces.
__device__ __forceinline__ float4 gemm_epilogue4(const GemmEpilogue &e, float4 y, long long n, int row, int rows) {
#pragma clang fp contract(off)
    if (e.op == EPI_CONV) {
        float4 *r = reinterpret_cast<float4 *>(e.ring + (n * rows + row) * 3);
        const float4 R0 = r[0], R1 = r[1], R2 = r[2];
        const float4 *wp = reinterpret_cast<const float4 *>(e.w + 4LL * row);
        const float4 w0 = wp[0], w1 = wp[1], w2 = wp[2], w3 = wp[3];
        const float c0 = w0.x * R0.x + w0.y * R0.y + w0.z * R0.z + w0.w * y.x;
        const float c1 = w1.x * R0.w + w1.y * R1.x + w1.z * R1.y + w1.w * y.y;
        const float c2 = w2.x * R1.z + w2.y * R1.w + w2.z * R2.x + w2.w * y.z;
        const float c3 = w3.x * R2.y + w3.y * R2.z + w3.z * R2.w + w3.w * y.w;
        r[0] = make_float4(R0.y, R0.z, y.x, R1.x);
        r[1] = make_float4(R1.y, y.y, R1.w, R2.x);
        r[2] = make_float4(y.z, R2.z, R2.w, y.w);
        return make_float4(c0 / (1.0f + expf(-c0)), c1 / (1.0f + expf(-c1)), c2 / (1.0f + expf(-c2)),
                           c3 / (1.0f + expf(-c3)));
    }
    if (e.op == EPI_RESID) {
        const float4 b = *reinterpret_cast<const float4 *>(e.b + n * rows + row);
        return make_float4(b.x + y.x, b.y + y.y, b.z + y.z, b.w + y.w);
    }
    return make_float4(gemm_epilogue(e, y.x, n, row, rows), gemm_epilogue(e, y.y, n, row + 1, rows),
                       gemm_epilogue(e, y.z, n, row + 2, rows), gemm_epilogue(e, y.w, n, row + 3, rows));
}
int i2_gemm_skinny_group(const GemmProblem *probs, int np, size_t in_len, size_t ncols, int x_tiled, void *stream);

// KV-cache pages handed out by the host for one decode step of the hybrid
// stack: page_table[slot[i]] = page[i] (stack.hip, stack_ops.hip).
constexpr int kMaxPageAssign = 64;
struct PageAssign {
    int n;
    int slot[kMaxPageAssign];
    int page[kMaxPageAssign];
};
static_assert(sizeof(PageAssign) == 516, "PageAssign: kernel argument layout");

// finite_argmax keys (infer/mod.rs:70-83): the value's bits in an
// order-preserving form (-0 taken as +0, as `>` does) in the high word, the
// complement of the index in the low word (the lowest index wins a tie), 0
// for NaN, so the largest key is the answer and key 0 means "nothing found".
__device__ __forceinline__ unsigned long long argmax_key(float v, unsigned i) {
    if (v != v) return 0ull;
    uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(u) << 32) | (0xffffffffu - i);
}

__device__ __forceinline__ unsigned long long argmax_key_max(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

// Reduce a thread's key over the workgroup (blockDim.x a multiple of 64, at
// most 1024 threads); thread 0 gets the workgroup's key.
__device__ __forceinline__ unsigned long long argmax_block_key(unsigned long long k) {
    __shared__ unsigned long long part[16];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(k), off, 64);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(k >> 32), off, 64);
        k = argmax_key_max(k, (static_cast<unsigned long long>(hi) << 32) | lo);
    }
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0)
        for (unsigned w = 1; w < blockDim.x / 64; ++w) k = argmax_key_max(k, part[w]);
    return k;
}

// The key of an argmax over per-workgroup keys, as the index it stands for.
__device__ __forceinline__ int32_t argmax_index(unsigned long long best) {
    return best ? static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(best)) : 0;
}

}  // namespace ouro
