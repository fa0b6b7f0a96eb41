// stack_ops.hip - the device operations of a Qwen3.5-style hybrid decoder
// stack that the hot-path kernels do not already cover: the attention
// block's per-head norm + partial NEOX rope + KV append, causal attention
// over a packed varlen batch (prefill) and over each sequence's cache
// (decode), the delta-net block's causal conv + gates over a packed varlen
// batch, embedding lookup, per-row finite_argmax and the seeded synthetic
// weights.  (RMS norm, SwiGLU and the gated norm run fused ahead of the
// activation rotation, fwht.hip.)
//
// Reference semantics followed: run_layer (qwen35.rs:776-795), run_ffn
// (798-805), run_attn (1160-1215) with attn_head (1227-1240), run_delta's
// conv and gates (1066-1088), silu/softmax (ops.rs:34-48),
// rope_partial_neox (qwen35.rs:96-106).
#include "common.hpp"

#include <atomic>

#pragma clang fp contract(off)

namespace ouro {
namespace {
typedef float nt4 __attribute__((ext_vector_type(4)));  // 16-byte vector for non-temporal loads

constexpr int kHd = 128;  // attention head dim and delta-net d handled here
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kPage = 64;  // tokens per KV cache page

// Cache row of (sequence, position): the KV cache is a pool of pages of
// kPage rows; pages[seq * maxp + pos / kPage] names the page holding pos.
__device__ __forceinline__ long long kv_row(const int32_t *pages, int maxp, int seq, int pos) {
    return static_cast<long long>(pages[static_cast<long long>(seq) * maxp + pos / kPage]) * kPage + pos % kPage;
}

// ------------------------------------------------------- synthetic weights --

// 32-bit mix of (seed, tensor, index); the same arithmetic is restated in
// the oracle so synthetic weights are reproducible on the host.
__device__ __forceinline__ uint32_t mix3(uint32_t seed, uint32_t tensor, uint32_t idx) {
    uint32_t x = seed ^ (tensor * 0x9E3779B9u) ^ (idx * 0x85EBCA6Bu);
    x ^= x >> 16;
    x *= 0x7FEB352Du;
    x ^= x >> 15;
    x *= 0x846CA68Bu;
    x ^= x >> 16;
    return x;
}

// Canonical I2 bytes of a rows x cols ternary tensor: code(k) = mix3 % 3.
__global__ void gen_codes_kernel(uint32_t seed, uint32_t tensor, long long rows, int cols, uint8_t *dst) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const long long bytes = rows * (cols / 4);
    if (i >= bytes) return;
    const long long row = i / (cols / 4);
    const int j = static_cast<int>(i % (cols / 4));
    uint32_t b = 0;
#pragma unroll
    for (int f = 0; f < 4; ++f) {
        const uint32_t idx = static_cast<uint32_t>(row * cols + 4 * j + f);
        b |= (mix3(seed, tensor, idx) % 3u) << (2 * f);
    }
    dst[i] = static_cast<uint8_t>(b);
}

// dst[i] = lo + span * u, u = (mix3 >> 8) * 2^-24 in [0, 1); signs (span
// == 0): +1 or -1 from the low bit.
__global__ void gen_floats_kernel(uint32_t seed, uint32_t tensor, long long n, float lo, float span, float *dst) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t h = mix3(seed, tensor, static_cast<uint32_t>(i));
    if (span == 0.f) {
        dst[i] = (h & 1u) ? 1.0f : -1.0f;
        return;
    }
    const float u = static_cast<float>(h >> 8) * 5.9604644775390625e-8f;
    dst[i] = lo + span * u;
}

// -------------------------------------------------------------- embedding --

// Token rows -> embedding rows (ids clamped into the table).
__global__ void embed_kernel(const int32_t *tokens, const float *table, float *x, int n_tok, int n_vocab, int n_embd) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long long>(n_tok) * n_embd) return;
    const int t = static_cast<int>(i / n_embd), c = static_cast<int>(i % n_embd);
    int id = tokens[t];
    id = id < 0 ? 0 : (id >= n_vocab ? n_vocab - 1 : id);
    x[i] = table[static_cast<long long>(id) * n_embd + c];
}

// Rows src_rows[i] of src -> row i of dst (the last token of each sequence).
__global__ void gather_rows_kernel(const float *src, const int32_t *src_rows, float *dst, int n, int width) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long long>(n) * width) return;
    const int r = static_cast<int>(i / width), c = static_cast<int>(i % width);
    dst[i] = src[static_cast<long long>(src_rows[r]) * width + c];
}

// --------------------------------------------------------- attention prep --

struct AttnPrepArgs {
    const float *qfull;       // [T][nh][2*hd]: q | gate per head (qwen35.rs:1174)
    const float *k, *v;       // [T][nkv][hd]
    const float *qn, *kn;     // [hd] head-norm gains
    const int32_t *pos;       // [T] position of the token in its sequence
    const int32_t *seq;       // [T] sequence of the token
    const int32_t *pages;     // [N][maxp] page table
    float *q_out, *gate_out;  // [T][nh][hd]
    float *kc, *vc;           // cache pages [pages * kPage][nkv][hd]
    int T, nh, nkv, n_rot, maxp;
    float rope_base, eps;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (128 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(AttnPrepArgs) == 128, "AttnPrepArgs: kernel argument layout");

// Workgroup (token, y) of gridDim.y per token; wavefront w takes heads
// 4 y + w, then every 4 gridDim.y-th (q heads, then k heads); lane l holds
// dims 2l, 2l+1.  The rope's angles depend on the position and the dim
// only, so each wavefront computes its lanes' cos / sin once and uses them
// for all its heads (a long prefill: one workgroup per token; a decode
// step: one head per wavefront, for parallelism).
__global__ __launch_bounds__(256) void attn_prep_kernel(AttnPrepArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = static_cast<int>(blockIdx.x);
    if (t >= a.T) return;  // whole workgroup
    const int heads = a.nh + a.nkv;
    // rope_partial_neox on the first n_rot dims: pair (i, i + n_rot/2)
    const int half = a.n_rot / 2;
    const int p = a.pos[t];
    const int partner = lane < half / 2 ? lane + half / 2 : lane - half / 2;
    const bool rot = 2 * lane < a.n_rot;
    float cs[2] = {1.f, 1.f}, sn[2] = {0.f, 0.f};
    if (rot) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int d = 2 * lane + e;
            const int i = d < half ? d : d - half;
            const float theta = 1.0f / powf(a.rope_base, static_cast<float>(2 * i) / static_cast<float>(a.n_rot));
            const float ang = static_cast<float>(p) * theta;
            cs[e] = cosf(ang);
            sn[e] = sinf(ang);
        }
    }
    const long long krow = kv_row(a.pages, a.maxp, a.seq[t], p);  // the token's cache row
    for (int hh = 4 * static_cast<int>(blockIdx.y) + wave; hh < heads; hh += 4 * static_cast<int>(gridDim.y)) {
        const bool isq = hh < a.nh;
        const int h = isq ? hh : hh - a.nh;
        const float *src = isq ? a.qfull + (static_cast<long long>(t) * a.nh + h) * (2 * kHd)
                               : a.k + (static_cast<long long>(t) * a.nkv + h) * kHd;
        float2 x = *reinterpret_cast<const float2 *>(src + 2 * lane);
        // rmsnorm_head (qwen35.rs:1246-1248)
        float ss = x.x * x.x + x.y * x.y;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss += xor_shfl(ss, off);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(kHd) + a.eps);
        const float2 g = *reinterpret_cast<const float2 *>((isq ? a.qn : a.kn) + 2 * lane);
        x.x = x.x * inv * g.x;
        x.y = x.y * inv * g.y;
        const float px = __shfl(x.x, partner, 64), py = __shfl(x.y, partner, 64);
        if (rot) {
            float r[2] = {x.x, x.y};
            const float pr[2] = {px, py};
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int d = 2 * lane + e;
                r[e] = d < half ? r[e] * cs[e] - pr[e] * sn[e] : r[e] * cs[e] + pr[e] * sn[e];
            }
            x.x = r[0];
            x.y = r[1];
        }
        if (isq) {
            const long long o = (static_cast<long long>(t) * a.nh + h) * kHd + 2 * lane;
            *reinterpret_cast<float2 *>(a.q_out + o) = x;
            *reinterpret_cast<float2 *>(a.gate_out + o) = *reinterpret_cast<const float2 *>(src + kHd + 2 * lane);
        } else {
            const long long o = (krow * a.nkv + h) * kHd + 2 * lane;
            *reinterpret_cast<float2 *>(a.kc + o) = x;
            *reinterpret_cast<float2 *>(a.vc + o) =
                *reinterpret_cast<const float2 *>(a.v + (static_cast<long long>(t) * a.nkv + h) * kHd + 2 * lane);
        }
    }
}

// ---------------------------------------------------- attention (prefill) --

constexpr int kQT = 64;  // query rows per tile
constexpr int kKT = 64;  // keys per tile (one KV page)

struct AttnArgs {
    const float *q, *gate;    // [T][nh][hd]
    const float *kc, *vc;     // cache pages [pages * kPage][nkv][hd]
    const int32_t *pages;     // [N][maxp] page table
    const int32_t *cu;        // [N+1] token offsets (prefill); NULL for decode
    const int32_t *lens;      // [N] keys per sequence (decode)
    const int32_t *tile_seq, *tile_p0;  // prefill query tiles
    float *out;               // [T][nh][hd]
    int nh, nkv, maxp;
    float scale;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (96 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(AttnArgs) == 96, "AttnArgs: kernel argument layout");

__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
    return v;
}

// Causal attention over a packed varlen batch on bf16 MFMA with every fp32
// operand split as x = hi + lo (hi = bf16(x), lo = bf16(x - hi)) and each
// product taken as hi*hi + hi*lo + lo*hi (v_mfma_f32_16x16x32_bf16, fp32
// sums): products to about 2^-16 of their size, well inside the 1e-3
// relative bar on the attention output, at about five times the fp32 MFMA
// rate.  One workgroup per (query tile of 64 tokens of one sequence, q
// head); wavefront w owns query rows 16w..16w+15 as the 16 columns of its
// products, with their Q (hi, lo) in registers as B operands.  Per key tile
// of 64 (one KV page), staged in LDS as split operand fragments:
// S^T = K Q^T (4 tiles of 16 keys, k = 128 dims), the online softmax per
// query (a lane holds one query: in-lane maxima and sums, then the three
// other lanes of that query), then O^T += V^T P^T with P^T taken straight
// from the score registers as the B operand (keys 32q + 4g + 0..3 and
// 32q + 16 + 4g + 0..3 of lane group g, the order the V^T fragments are
// staged in), so P never goes through LDS.  The sigmoid output gate is
// applied at the end, and a lane stores four consecutive dims of its query.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4_t mfma_bf16(const bf16x8_t &a, const bf16x8_t &b, const f32x4_t &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// (a, b) = hi + lo as bf16 pairs (round to nearest even; x - hi is exact)
__device__ __forceinline__ void split_pair(float a, float b, uint32_t &hi, uint32_t &lo) {
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
    hi = h;
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                          f32x2_t{a - __uint_as_float(h << 16), b - __uint_as_float(h & 0xffff0000u)},
                                          bf16x2_t));
}
// eight values (x0[0..3], x1[0..3]) as hi and lo operands
__device__ __forceinline__ void split_op(const f32x4_t &x0, const f32x4_t &x1, bf16x8_t &hi, bf16x8_t &lo) {
    uint4 h, l;
    split_pair(x0[0], x0[1], h.x, l.x);
    split_pair(x0[2], x0[3], h.y, l.y);
    split_pair(x1[0], x1[1], h.z, l.z);
    split_pair(x1[2], x1[3], h.w, l.w);
    hi = __builtin_bit_cast(bf16x8_t, h);
    lo = __builtin_bit_cast(bf16x8_t, l);
}

// LDS operand fragments: a block is one 16 x 32 bf16 operand (64 lanes x
// 16 B), lane r + 16 g at 272 g + 16 r, so a wavefront's 16-byte operand
// read is 16 contiguous lanes per group (conflict-free) and the 16 B of
// padding per group spread the staging writes over the banks.
constexpr int kFragGrp = 272;
constexpr int kFragBlk = 4 * kFragGrp;
__device__ __forceinline__ int frag_off(int blk, int lane) { return blk * kFragBlk + (lane >> 4) * kFragGrp + (lane & 15) * 16; }
// K tile: block (4 t + j) * 2 + hl holds keys 16 t + r, dims 32 j + 8 g + 0..7
// at lane r + 16 g (hl: 0 hi, 1 lo).  V^T tile: block kVtBlk + (2 t + q) * 2 +
// hl holds dims 16 t + r over keys 32 q + 4 g + 0..3 and 32 q + 16 + 4 g + 0..3.
constexpr int kVtBlk = 32;
constexpr int kAttnLds = 64 * kFragBlk;  // 68 KiB: two workgroups per CU

__global__ __launch_bounds__(256) void attn_prefill_kernel(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char alds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int s = a.tile_seq[blockIdx.x], p0 = a.tile_p0[blockIdx.x];
    const int h = blockIdx.y;
    const int kvh = h / (a.nh / a.nkv);
    const int t0 = a.cu[s], L = a.cu[s + 1] - t0;
    const int qp = p0 + 16 * wave + lr;  // this lane's query position

    // Q row qp, dims 32 j + 8 g .. +7: the B operand of k-step j
    bf16x8_t qh[4], ql[4];
    {
        const float *qr = a.q + ((static_cast<long long>(t0) + min(qp, L - 1)) * a.nh + h) * kHd + 8 * lg;
#pragma unroll
        for (int j = 0; j < 4; ++j)  // rows past the end: any valid row, never stored
            split_op(*reinterpret_cast<const f32x4_t *>(qr + 32 * j), *reinterpret_cast<const f32x4_t *>(qr + 32 * j + 4),
                     qh[j], ql[j]);
    }
    f32x4_t o[8];  // o[t][e] = O[qp][16 t + 4 g + e] (unnormalised)
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    const float sl2 = a.scale * 1.4426950408889634f;  // scale * log2(e)
    const int last = min(p0 + kQT, L) - 1;  // last query position of the tile
    // Staging units u = tid + 256 i: keys 2 p, 2 p + 1 (p = u / 32), dims
    // 4 c .. 4 c + 3 (c = u % 32); the next tile's K and V are loaded into
    // registers while the current one is used (rows past L read the page's
    // unused rows and are zeroed)
    f32x4_t kpre[4][2], vpre[4][2];
    auto load_kv = [&](int k0) {
        const long long row0 = kv_row(a.pages, a.maxp, s, k0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = tid + 256 * i, pr = u >> 5, c4 = u & 31;
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const long long off = ((row0 + 2 * pr + w) * a.nkv + kvh) * kHd + 4 * c4;
                kpre[i][w] = *reinterpret_cast<const f32x4_t *>(a.kc + off);
                vpre[i][w] = *reinterpret_cast<const f32x4_t *>(a.vc + off);
            }
        }
    };
    load_kv(0);
    for (int k0 = 0; k0 <= last; k0 += kKT) {
        __syncthreads();  // the previous tile's fragments are consumed
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = tid + 256 * i, pr = u >> 5, c4 = u & 31;
            const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
            f32x4_t kv[2], vv[2];
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const bool live = k0 + 2 * pr + w < L;
                kv[w] = live ? kpre[i][w] : z;
                vv[w] = live ? vpre[i][w] : z;
            }
            // K: key kk = 2 pr + w, dims 4 c4 .. +3 -> 8 bytes of lane r + 16 g of block (4 t + j) * 2 + hl
            const int j = c4 >> 3, g = (c4 >> 1) & 3, half = c4 & 1;
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const int kk = 2 * pr + w, t = kk >> 4, r = kk & 15;
                uint2 hi, lo;
                split_pair(kv[w][0], kv[w][1], hi.x, lo.x);
                split_pair(kv[w][2], kv[w][3], hi.y, lo.y);
                const int blk = (4 * t + j) * 2;
                *reinterpret_cast<uint2 *>(alds + frag_off(blk, r + 16 * g) + 8 * half) = hi;
                *reinterpret_cast<uint2 *>(alds + frag_off(blk + 1, r + 16 * g) + 8 * half) = lo;
            }
            // V^T: dim d = 4 c4 + e, keys kk, kk + 1 (kk = 2 pr even) -> one bf16 pair at
            // position (kk & 3) + 4 ((kk & 31) >> 4) of lane (d & 15) + 16 ((kk & 15) >> 2)
            const int kk = 2 * pr, q = kk >> 5, pos = (kk & 3) + 4 * ((kk & 31) >> 4), gv = (kk & 15) >> 2;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = 4 * c4 + e, t = d >> 4;
                uint32_t hi, lo;
                split_pair(vv[0][e], vv[1][e], hi, lo);
                const int blk = kVtBlk + (2 * t + q) * 2;
                *reinterpret_cast<uint32_t *>(alds + frag_off(blk, (d & 15) + 16 * gv) + 2 * pos) = hi;
                *reinterpret_cast<uint32_t *>(alds + frag_off(blk + 1, (d & 15) + 16 * gv) + 2 * pos) = lo;
            }
        }
        __syncthreads();
        if (k0 + kKT <= last) load_kv(k0 + kKT);
        // S^T: sc[t][e] = S[qp][k0 + 16 t + 4 g + e]
        f32x4_t sc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int blk = (4 * t + j) * 2;
                const bf16x8_t kh = *reinterpret_cast<const bf16x8_t *>(alds + frag_off(blk, lane));
                const bf16x8_t kl = *reinterpret_cast<const bf16x8_t *>(alds + frag_off(blk + 1, lane));
                sc[t] = mfma_bf16(kh, qh[j], sc[t]);
                sc[t] = mfma_bf16(kh, ql[j], sc[t]);
                sc[t] = mfma_bf16(kl, qh[j], sc[t]);
            }
        }
        // online softmax of query qp (its keys are spread over lanes lr + 16 g),
        // in base 2: scores scaled by scale * log2(e), p = 2^(s - m)
        float mx = -INFINITY;
        if (k0 + kKT - 1 <= p0 + 16 * wave && k0 + kKT <= L) {  // every key visible to every row of the wave
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sc[t][e] *= sl2;
                    mx = fmaxf(mx, sc[t][e]);
                }
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int kp = k0 + 16 * t + 4 * lg + e;
                    sc[t][e] = (kp <= qp && kp < L) ? sc[t][e] * sl2 : -INFINITY;
                    mx = fmaxf(mx, sc[t][e]);
                }
        }
        {
            const auto x32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(x32[0]), __uint_as_float(x32[1]));
            const auto x16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(x16[0]), __uint_as_float(x16[1]));
        }
        const float mn = fmaxf(m, mx);
        // a query with no visible key yet keeps m = -inf; use 0 to avoid inf - inf
        const float mref = mn == -INFINITY ? 0.f : mn;
        const float corr = __builtin_amdgcn_exp2f(m - mref);
        float ps = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc[t][e] = __builtin_amdgcn_exp2f(sc[t][e] - mref);
                ps += sc[t][e];
            }
        {
            const auto x32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
            ps = __uint_as_float(x32[0]) + __uint_as_float(x32[1]);
            const auto x16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
            ps = __uint_as_float(x16[0]) + __uint_as_float(x16[1]);
        }
        l = l * corr + ps;
        m = mn;
        if (!__all(corr == 1.0f)) {  // the running maxima moved
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) o[t][e] *= corr;
        }
        // P^T as B operands: slab q = score tiles 2 q, 2 q + 1
        bf16x8_t ph[2], pl[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) split_op(sc[2 * q], sc[2 * q + 1], ph[q], pl[q]);
        // O^T += V^T P^T
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int blk = kVtBlk + (2 * t + q) * 2;
                const bf16x8_t vh = *reinterpret_cast<const bf16x8_t *>(alds + frag_off(blk, lane));
                const bf16x8_t vl = *reinterpret_cast<const bf16x8_t *>(alds + frag_off(blk + 1, lane));
                o[t] = mfma_bf16(vh, ph[q], o[t]);
                o[t] = mfma_bf16(vh, pl[q], o[t]);
                o[t] = mfma_bf16(vl, ph[q], o[t]);
            }
    }
    // o / l, times sigmoid(gate) (qwen35.rs:1208-1210): dims 16 t + 4 g .. +3 of query qp
    if (qp < L) {
        const long long base = ((static_cast<long long>(t0) + qp) * a.nh + h) * kHd + 4 * lg;
        const float il = 1.0f / l;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const f32x4_t g = *reinterpret_cast<const f32x4_t *>(a.gate + base + 16 * t);
            f32x4_t r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = (o[t][e] * il) * (1.0f / (1.0f + expf(-g[e])));
            *reinterpret_cast<f32x4_t *>(a.out + base + 16 * t) = r;
        }
    }
}

// ----------------------------------------------------- attention (decode) --


// Decode attention, split over the context (flash-decoding): workgroup
// (sequence b, kv head, split sp) takes keys sp*kDecKeys .. +kDecKeys of b
// for all G = nh/nkv query heads of that kv head, so each K and V row is
// read once per step.  Scores: 16 lanes per key (8 dims each, G dot
// products, DPP row sums), 4 keys per wavefront per step, into LDS; per-head
// max and exp-sum over the split; P V with lane = 4 dims, two keys per
// wavefront load and the 4 wavefronts on interleaved keys, reduced through
// LDS.  The split's
// unnormalised output, max and sum go to `part`; attn_combine_kernel merges
// the splits of each (b, head) and applies the sigmoid output gate.
constexpr int kDecKeys = 256;
constexpr int kPartStride = kHd + 4;  // floats per (b, head, split) record: o[128], m, l

template <int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(G <= 4 ? 5 : 1))) void attn_decode_split_kernel(AttnArgs a, float *part, int nsplit) {
    __shared__ float sc[G][kDecKeys];
    __shared__ float red[4][G][kHd];
    __shared__ float ml[G][2];
    __shared__ long long prow[kDecKeys / kPage];  // first cache row of each page of the split
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sp = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int L = a.lens[b];
    const int j0 = sp * kDecKeys;
    if (j0 >= L) return;  // whole workgroup
    const int n = min(kDecKeys, L - j0);
    if (tid < kDecKeys / kPage && j0 + tid * kPage < L) prow[tid] = kv_row(a.pages, a.maxp, b, j0 + tid * kPage);
    __syncthreads();
    const int g4 = lane >> 4, gl = lane & 15;
    float4 q[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float *qp = a.q + (static_cast<long long>(b) * a.nh + kvh * G + g) * kHd + 8 * gl;
        q[g][0] = *reinterpret_cast<const float4 *>(qp);
        q[g][1] = *reinterpret_cast<const float4 *>(qp + 4);
    }
    // scores: wave w, step it -> key w*kWK + 4*it + g4 (a wave's keys lie in
    // one page); rows past the split are clamped to its last key, so the
    // loads carry no branches, and their scores are not stored
    constexpr int kWK = kDecKeys / 4;  // keys per wavefront
    static_assert(kPage % kWK == 0, "a wavefront's keys lie in one page");
    const int wkeys = min(kWK, n - wave * kWK);  // keys of this wave (<= 0: none)
    const long long wrow = wkeys > 0 ? prow[wave * kWK / kPage] + wave * kWK % kPage : 0;
    // kB key rows' loads are issued together before their dot products: the
    // conditional score store splits an iteration into several basic blocks,
    // so the compiler would not hoist the next key's loads across it
    constexpr int kB = 4;
    static_assert((kWK / 4) % kB == 0, "whole load batches");
    for (int it0 = 0; it0 < (wkeys > 0 ? kWK / 4 : 0); it0 += kB) {
        float4 k0[kB], k1[kB];
#pragma unroll
        for (int i = 0; i < kB; ++i) {
            const int jj = 4 * (it0 + i) + g4;
            const float *kp = a.kc + ((wrow + min(jj, max(wkeys - 1, 0))) * a.nkv + kvh) * kHd + 8 * gl;
            // the KV cache is read once per step: non-temporal loads
            k0[i] = __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(kp)));
            k1[i] = __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(kp + 4)));
        }
#pragma unroll
        for (int i = 0; i < kB; ++i) {
            const int jj = 4 * (it0 + i) + g4;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d = q[g][0].x * k0[i].x + q[g][0].y * k0[i].y + q[g][0].z * k0[i].z + q[g][0].w * k0[i].w +
                          q[g][1].x * k1[i].x + q[g][1].y * k1[i].y + q[g][1].z * k1[i].z + q[g][1].w * k1[i].w;
                d = row16_sum(d);
                if (gl == 0 && jj < wkeys) sc[g][wave * kWK + jj] = d * a.scale;
            }
        }
    }
    __syncthreads();
    // per-head max and exp-sum over the split (wave w takes heads w, w+4, ...)
    for (int g = wave; g < G; g += 4) {
        float mx = -INFINITY;
        for (int j = lane; j < n; j += 64) mx = fmaxf(mx, sc[g][j]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float sum = 0.f;
        for (int j = lane; j < n; j += 64) {
            const float e = expf(sc[g][j] - mx);
            sc[g][j] = e;
            sum += e;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
        if (lane == 0) {
            ml[g][0] = mx;
            ml[g][1] = sum;
        }
    }
    __syncthreads();
    // P V: wave w, half h (lanes 32h .. 32h+31) take keys 2w + h, +8, ...;
    // lane owns dims 4 (lane % 32) .. +3, so one load instruction reads two
    // whole 512-byte rows; the halves are added at the end
    const int h = lane >> 5, d4 = 4 * (lane & 31);
    float4 acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    const float *vp = a.vc + kvh * kHd + d4;
    const long long vstride = static_cast<long long>(a.nkv) * kHd;
#pragma unroll 8
    for (int j0 = 2 * wave; j0 < n; j0 += 8) {
        const int j = min(j0 + h, n - 1);  // clamped; its weight is zeroed
        const float4 v = __builtin_bit_cast(
            float4, __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(vp + (prow[j / kPage] + j % kPage) * vstride)));
        const bool live = j0 + h < n;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float pj = live ? sc[g][j] : 0.f;
            acc[g].x += pj * v.x;
            acc[g].y += pj * v.y;
            acc[g].z += pj * v.z;
            acc[g].w += pj * v.w;
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        acc[g].x += __shfl_xor(acc[g].x, 32, 64);
        acc[g].y += __shfl_xor(acc[g].y, 32, 64);
        acc[g].z += __shfl_xor(acc[g].z, 32, 64);
        acc[g].w += __shfl_xor(acc[g].w, 32, 64);
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (h == 0) *reinterpret_cast<float4 *>(&red[wave][g][d4]) = acc[g];
    __syncthreads();
    for (int i = tid; i < G * kHd; i += 256) {
        const int g = i / kHd, d = i % kHd;
        const float o = red[0][g][d] + red[1][g][d] + red[2][g][d] + red[3][g][d];
        float *rec = part + ((static_cast<long long>(b) * a.nh + kvh * G + g) * nsplit + sp) * kPartStride;
        rec[d] = o;
        if (d == 0) {
            rec[kHd] = ml[g][0];
            rec[kHd + 1] = ml[g][1];
        }
    }
}

// Merge the splits of (b, head): o = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s,
// times sigmoid(gate) (qwen35.rs:1205-1210).  One 128-thread workgroup per (b, head).
__global__ __launch_bounds__(128) void attn_combine_kernel(AttnArgs a, const float *part, int nsplit) {
    const int b = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
    const int ns = (a.lens[b] + kDecKeys - 1) / kDecKeys;
    const float *rec = part + (static_cast<long long>(b) * a.nh + h) * nsplit * kPartStride;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, rec[s * kPartStride + kHd]);
    float num = 0.f, den = 0.f;
    for (int s = 0; s < ns; ++s) {
        const float w = expf(rec[s * kPartStride + kHd] - M);
        num += w * rec[s * kPartStride + d];
        den += w * rec[s * kPartStride + kHd + 1];
    }
    const long long qo = (static_cast<long long>(b) * a.nh + h) * kHd + d;
    const float g2 = a.gate[qo];
    a.out[qo] = (num / den) * (1.0f / (1.0f + expf(-g2)));
}

// ------------------------------------------------ delta-net prefill inputs --

struct ConvArgs {
    const float *qkv;          // [T][ch]
    const float *ring;         // [N][ch][3] conv state before the batch
    const float *conv_w;       // [ch][4]
    const int32_t *seq, *pos;  // [T]
    const float *beta_raw, *alpha_raw, *dt_bias, *a_log;  // [T][Hv], [Hv]
    uint16_t *qb, *kb, *vb;    // bf16 [T][di], [T][di], [T][Hv*d]
    float *beta, *gate;        // [T][Hv]
    int T, ch, di, Hv;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (128 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(ConvArgs) == 128, "ConvArgs: kernel argument layout");

__device__ __forceinline__ uint16_t to_bf16(float x) { return f32_to_bf16_bits(x); }

// conv_step + SiLU per (token, channel) with the causal window inside the
// token's sequence (inputs before the sequence come from its ring), then
// beta and gate per (token, v-head) (qwen35.rs:1066-1088).
// Grid: x = blocks of 1024 channels (a thread takes 4 adjacent channels:
// 16-byte loads, 8-byte bf16 stores), y = contiguous token ranges.  A
// thread walks its channels along its range with the last three inputs in
// registers (each input read once), taking them from the sequence's ring
// at a sequence start.  The gates of token t are written by the last column
// of workgroups.
__device__ __forceinline__ float silu_f(float y) { return y / (1.0f + expf(-y)); }

__global__ __launch_bounds__(256) void prefill_conv_gate_kernel(ConvArgs a, int per) {
    // tokens go in batches of kB: a batch's loads (inputs and positions) are
    // issued together (the token loop is otherwise one dependent HBM round
    // trip per token)
    constexpr int kB = 16;
    const int ta = static_cast<int>(blockIdx.y) * per, tb = min(ta + per, a.T);
    const int nc4 = a.ch / 4;  // channel quads (the host checks ch % 4 == 0)
    // the last column of workgroups computes the gates (next to the conv
    // workgroups rather than in one of them, which made it the longest)
    if (static_cast<int>(blockIdx.x) == (nc4 + 255) / 256) {
        if (threadIdx.x >= a.Hv) return;
        const int hv = threadIdx.x;
        const float dtb = a.dt_bias[hv], al = a.a_log[hv];
        for (int t0 = ta; t0 < tb; t0 += kB) {
            float br[kB], ar[kB];
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                const long long ig = static_cast<long long>(min(t0 + u, tb - 1)) * a.Hv + hv;
                br[u] = a.beta_raw[ig];
                ar[u] = a.alpha_raw[ig];
            }
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                if (t0 + u >= tb) break;
                const long long ig = static_cast<long long>(t0 + u) * a.Hv + hv;
                a.beta[ig] = 1.0f / (1.0f + expf(-br[u]));
                const float x = ar[u] + dtb;
                a.gate[ig] = al * (x > 20.0f ? x : logf(1.0f + expf(x)));
            }
        }
        return;
    }
    const int c4 = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (c4 >= nc4 || ta >= tb) return;
    const int c = 4 * c4;
    f32x4_t w[4];  // conv weights of channels c .. c + 3
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = *reinterpret_cast<const f32x4_t *>(a.conv_w + 4LL * (c + e));
    const int di = a.di, dv = a.ch - 2 * a.di;
    // the quad lies in one of q, k, v (di % 4 == 0): its output row and column
    uint16_t *dst;
    int dstride, dc;
    if (c < di) dst = a.qb, dstride = di, dc = c;
    else if (c < 2 * di) dst = a.kb, dstride = di, dc = c - di;
    else dst = a.vb, dstride = dv, dc = c - 2 * di;
    // window x[t-3], x[t-2], x[t-1] for the range's first token
    f32x4_t x0, x1, x2;
    auto ring_window = [&](int t) {
        const float *r = a.ring + (static_cast<long long>(a.seq[t]) * a.ch + c) * 3;  // [channel][3]
        const f32x4_t r0 = *reinterpret_cast<const f32x4_t *>(r), r1 = *reinterpret_cast<const f32x4_t *>(r + 4),
                      r2 = *reinterpret_cast<const f32x4_t *>(r + 8);  // 12 floats, channel-major
        const float rr[12] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3], r2[0], r2[1], r2[2], r2[3]};
#pragma unroll
        for (int e = 0; e < 4; ++e) x0[e] = rr[3 * e], x1[e] = rr[3 * e + 1], x2[e] = rr[3 * e + 2];
    };
    {
        // x[ta-3] = ring[p] (p < 3), x[ta-2] = ring[1 + p] (p < 2), x[ta-1] = ring[2] (p < 1)
        const int p = a.pos[ta];
        ring_window(ta);  // x0, x1, x2 = ring[0], ring[1], ring[2]
        const f32x4_t r1 = x1, r2 = x2;
        if (p == 1) x0 = r1, x1 = r2;
        if (p == 2) x0 = r2;
        const float *q = a.qkv + static_cast<long long>(ta) * a.ch + c;
        if (p >= 3) x0 = *reinterpret_cast<const f32x4_t *>(q - 3LL * a.ch);
        if (p >= 2) x1 = *reinterpret_cast<const f32x4_t *>(q - 2LL * a.ch);
        if (p >= 1) x2 = *reinterpret_cast<const f32x4_t *>(q - a.ch);
    }
    for (int t0 = ta; t0 < tb; t0 += kB) {
        f32x4_t xb[kB];
        int pb[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            const int t = min(t0 + u, tb - 1);
            xb[u] = *reinterpret_cast<const f32x4_t *>(a.qkv + static_cast<long long>(t) * a.ch + c);
            pb[u] = a.pos[t];
        }
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            const int t = t0 + u;
            if (t < tb) {
                if (t > ta && pb[u] == 0) ring_window(t);  // a sequence starts: its ring is the window
                const f32x4_t x = xb[u];
                uint32_t o[2];
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    const float y0 = w[e][0] * x0[e] + w[e][1] * x1[e] + w[e][2] * x2[e] + w[e][3] * x[e];
                    const float y1 = w[e + 1][0] * x0[e + 1] + w[e + 1][1] * x1[e + 1] + w[e + 1][2] * x2[e + 1] +
                                     w[e + 1][3] * x[e + 1];
                    o[e / 2] = static_cast<uint32_t>(to_bf16(silu_f(y0))) | (static_cast<uint32_t>(to_bf16(silu_f(y1))) << 16);
                }
                x0 = x1;
                x1 = x2;
                x2 = x;
                *reinterpret_cast<uint2 *>(dst + static_cast<long long>(t) * dstride + dc) = make_uint2(o[0], o[1]);
            }
        }
    }
}

// The conv ring after a sequence: its last three inputs (older ring values
// for sequences shorter than three), one thread per (sequence, channel).
__global__ void ring_update_kernel(const float *qkv, float *ring, const int32_t *cu, int N, int ch) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long long>(N) * ch) return;
    const int s = static_cast<int>(i / ch), c = static_cast<int>(i % ch);
    const int t0 = cu[s], L = cu[s + 1] - t0;
    float *r = ring + i * 3;
    float nr[3];
#pragma unroll
    for (int e = 0; e < 3; ++e) {
        const int j = L - 3 + e;  // input index within the sequence
        nr[e] = j >= 0 ? qkv[(static_cast<long long>(t0) + j) * ch + c] : r[3 + j];
    }
    r[0] = nr[0];
    r[1] = nr[1];
    r[2] = nr[2];
}

// finite_argmax (infer/mod.rs:70-83) of each row in two launches: keys of
// kArgChunk-element chunks (grid chunks x rows), then one
// wavefront per row over its chunk keys.  Keys order values as `>` does and
// break ties toward the lower index, so the split gives the same answer.
constexpr int kArgChunk = 4096;

__global__ __launch_bounds__(256) void argmax_chunk_kernel(const float *y, long long n, unsigned long long *keys) {
    const long long row = blockIdx.y;
    const long long c0 = static_cast<long long>(blockIdx.x) * kArgChunk;
    const float *yr = y + row * n;
    unsigned long long best = 0;
    const long long end = c0 + kArgChunk < n ? c0 + kArgChunk : n;
    for (long long i = c0 + threadIdx.x; i < end; i += 256)
        best = argmax_key_max(best, argmax_key(yr[i], static_cast<unsigned>(i)));
    best = argmax_block_key(best);
    if (threadIdx.x == 0) keys[row * gridDim.x + blockIdx.x] = best;
}

__global__ __launch_bounds__(64) void argmax_final_rows_kernel(const unsigned long long *keys, int nk, int32_t *idx) {
    const long long row = blockIdx.x;
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < nk; i += 64) best = argmax_key_max(best, keys[row * nk + i]);
    best = argmax_block_key(best);
    if (threadIdx.x == 0) idx[row] = argmax_index(best);
}

__global__ void fill_zero_kernel(float *p, long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

// Start of a decode step: the new token of sequence b sits at position
// lens[b], its attention sees lens[b] + 1 keys, and the cache grows by one.
// Pages the host assigned for this step (a sequence entering a new page)
// arrive by value and are written into the page table first.
__global__ void lens_step_kernel(int32_t *lens, int32_t *pos, int32_t *klen, int B, int32_t *pages, PageAssign pa) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < pa.n) pages[pa.slot[b]] = pa.page[b];
    if (b >= B) return;
    const int l = lens[b];
    pos[b] = l;
    klen[b] = l + 1;
    lens[b] = l + 1;
}

unsigned blocks_for(long long n, int per) { return static_cast<unsigned>((n + per - 1) / per); }

}  // namespace

// ------------------------------------------------------- host launchers --

int fill_zero(float *p, size_t n, void *stream) {
    if (!n) return OURO_OK;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks_for(static_cast<long long>(n), 256)), dim3(256), 0,
                       as_stream(stream), p, static_cast<long long>(n));
    return check_launch("fill_zero_kernel");
}

int lens_step(int32_t *lens, int32_t *pos, int32_t *klen, size_t B, int32_t *pages, const PageAssign &pa,
              void *stream) {
    const long long n = static_cast<long long>(B) > pa.n ? static_cast<long long>(B) : pa.n;
    hipLaunchKernelGGL(lens_step_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), lens, pos, klen,
                       static_cast<int>(B), pages, pa);
    return check_launch("lens_step_kernel");
}

int gen_codes(uint32_t seed, uint32_t tensor, size_t rows, size_t cols, uint8_t *dst, void *stream) {
    if (cols % 4 || rows * cols >= (1ull << 32)) return fail(OURO_ERR_SHAPE, "gen_codes: %zu x %zu", rows, cols);
    const long long bytes = static_cast<long long>(rows * cols / 4);
    hipLaunchKernelGGL(gen_codes_kernel, dim3(blocks_for(bytes, 256)), dim3(256), 0, as_stream(stream), seed, tensor,
                       static_cast<long long>(rows), static_cast<int>(cols), dst);
    return check_launch("gen_codes_kernel");
}

int gen_floats(uint32_t seed, uint32_t tensor, size_t n, float lo, float span, float *dst, void *stream) {
    if (n >= (1ull << 32)) return fail(OURO_ERR_SHAPE, "gen_floats: %zu values", n);
    hipLaunchKernelGGL(gen_floats_kernel, dim3(blocks_for(static_cast<long long>(n), 256)), dim3(256), 0,
                       as_stream(stream), seed, tensor, static_cast<long long>(n), lo, span, dst);
    return check_launch("gen_floats_kernel");
}

int embed_rows(const int32_t *tokens, const float *table, float *x, size_t n_tok, size_t n_vocab, size_t n_embd,
               void *stream) {
    hipLaunchKernelGGL(embed_kernel, dim3(blocks_for(static_cast<long long>(n_tok * n_embd), 256)), dim3(256), 0,
                       as_stream(stream), tokens, table, x, static_cast<int>(n_tok), static_cast<int>(n_vocab),
                       static_cast<int>(n_embd));
    return check_launch("embed_kernel");
}

int gather_rows(const float *src, const int32_t *rows_idx, float *dst, size_t n, size_t width, void *stream) {
    hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks_for(static_cast<long long>(n * width), 256)), dim3(256), 0,
                       as_stream(stream), src, rows_idx, dst, static_cast<int>(n), static_cast<int>(width));
    return check_launch("gather_rows_kernel");
}

int attn_prep(const float *qfull, const float *k, const float *v, const float *qn, const float *kn,
              const int32_t *pos, const int32_t *seq, const int32_t *pages, int maxp, float *q_out, float *gate_out,
              float *kc, float *vc, size_t T, int nh, int nkv, int n_rot, float rope_base, float eps,
              void *stream) {
    if (n_rot < 0 || n_rot > kHd || n_rot % 4) return fail(OURO_ERR_SHAPE, "attn_prep: n_rot %d", n_rot);
    if (!T) return OURO_OK;
    AttnPrepArgs a{qfull, k, v, qn, kn, pos, seq, pages, q_out, gate_out, kc, vc,
                   static_cast<int>(T), nh, nkv, n_rot, maxp, rope_base, eps};
    const unsigned gy = T >= 4096 ? 1u : static_cast<unsigned>((nh + nkv + 3) / 4);
    hipLaunchKernelGGL(attn_prep_kernel, dim3(static_cast<unsigned>(T), gy), dim3(256), 0, as_stream(stream), a);
    return check_launch("attn_prep_kernel");
}

int attn_prefill(const float *q, const float *gate, const float *kc, const float *vc, const int32_t *pages, int maxp,
                 const int32_t *cu, const int32_t *tile_seq, const int32_t *tile_p0, size_t n_tiles, float *out,
                 int nh, int nkv, void *stream) {
    if (!n_tiles) return OURO_OK;
    // one opt-in per process for > 64 KiB of dynamic LDS (idempotent)
    static std::atomic<bool> lds_set{false};
    if (!lds_set.load(std::memory_order_acquire)) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(attn_prefill_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kAttnLds);
        if (e != hipSuccess) return fail(OURO_ERR_HIP, "attn_prefill: LDS opt-in: %s", hipGetErrorString(e));
        lds_set.store(true, std::memory_order_release);
    }
    AttnArgs a{q, gate, kc, vc, pages, cu, nullptr, tile_seq, tile_p0, out, nh, nkv, maxp,
               1.0f / sqrtf(static_cast<float>(kHd))};
    hipLaunchKernelGGL(attn_prefill_kernel, dim3(static_cast<unsigned>(n_tiles), nh), dim3(256), kAttnLds,
                       as_stream(stream), a);
    return check_launch("attn_prefill_kernel");
}

size_t attn_decode_ws_bytes(size_t B, int nh, size_t max_ctx) {
    return B * static_cast<size_t>(nh) * ((max_ctx + kDecKeys - 1) / kDecKeys) * kPartStride * sizeof(float);
}

int attn_decode(const float *q, const float *gate, const float *kc, const float *vc, const int32_t *pages, int maxp,
                const int32_t *lens, size_t B, int max_len, float *out, int nh, int nkv, float *part, void *stream) {
    const int G = nh / nkv;
    if (G < 1 || G > 8 || nh % nkv) return fail(OURO_ERR_SHAPE, "attn_decode: %d heads over %d kv heads", nh, nkv);
    if (max_len < 1 || !B) return OURO_OK;
    const int nsplit = (max_len + kDecKeys - 1) / kDecKeys;
    AttnArgs a{q, gate, kc, vc, pages, nullptr, lens, nullptr, nullptr, out, nh, nkv, maxp,
               1.0f / sqrtf(static_cast<float>(kHd))};
    // the split is the fastest grid index: workgroups are dealt to the CUs
    // in launch order, so a long context's splits land on different CUs
    // (with the sequence fastest, every split of one sequence would fall on
    // the same CU and the longest context would set the step time)
    const dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(nkv), static_cast<unsigned>(B));
    hipStream_t s = as_stream(stream);
    switch (G) {
    case 1: hipLaunchKernelGGL(attn_decode_split_kernel<1>, grid, dim3(256), 0, s, a, part, nsplit); break;
    case 2: hipLaunchKernelGGL(attn_decode_split_kernel<2>, grid, dim3(256), 0, s, a, part, nsplit); break;
    case 3: hipLaunchKernelGGL(attn_decode_split_kernel<3>, grid, dim3(256), 0, s, a, part, nsplit); break;
    case 4: hipLaunchKernelGGL(attn_decode_split_kernel<4>, grid, dim3(256), 0, s, a, part, nsplit); break;
    case 5: hipLaunchKernelGGL(attn_decode_split_kernel<5>, grid, dim3(256), 0, s, a, part, nsplit); break;
    case 6: hipLaunchKernelGGL(attn_decode_split_kernel<6>, grid, dim3(256), 0, s, a, part, nsplit); break;
    case 7: hipLaunchKernelGGL(attn_decode_split_kernel<7>, grid, dim3(256), 0, s, a, part, nsplit); break;
    default: hipLaunchKernelGGL(attn_decode_split_kernel<8>, grid, dim3(256), 0, s, a, part, nsplit); break;
    }
    int st = check_launch("attn_decode_split_kernel");
    if (st) return st;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(static_cast<unsigned>(B), static_cast<unsigned>(nh)), dim3(kHd), 0, s,
                       a, part, nsplit);
    return check_launch("attn_combine_kernel");
}

int prefill_conv_gate(const float *qkv, const float *ring, const float *conv_w, const int32_t *seq,
                      const int32_t *pos, const float *beta_raw, const float *alpha_raw, const float *dt_bias,
                      const float *a_log, uint16_t *qb, uint16_t *kb, uint16_t *vb, float *beta, float *gate,
                      size_t T, int ch, int di, int Hv, void *stream) {
    ConvArgs a{qkv, ring, conv_w, seq, pos, beta_raw, alpha_raw, dt_bias, a_log, qb, kb, vb, beta, gate,
               static_cast<int>(T), ch, di, Hv};
    if (!T) return OURO_OK;
    if (Hv > 256) return fail(OURO_ERR_SHAPE, "prefill_conv_gate: %d v-heads (<= 256)", Hv);
    if (ch % 4 || di % 4) return fail(OURO_ERR_SHAPE, "prefill_conv_gate: %d channels, %d per q/k (multiples of 4)", ch, di);
    const int cb = (ch / 4 + 255) / 256;
    // token ranges: enough workgroups to fill the chip, each range long
    // enough that the window is refilled from memory rarely
    const int ranges = static_cast<int>(T < 256 ? T : 256);
    const int per = static_cast<int>((T + ranges - 1) / ranges);
    hipLaunchKernelGGL(prefill_conv_gate_kernel, dim3(static_cast<unsigned>(cb + 1), static_cast<unsigned>((T + per - 1) / per)),
                       dim3(256), 0, as_stream(stream), a, per);
    return check_launch("prefill_conv_gate_kernel");
}

int ring_update(const float *qkv, float *ring, const int32_t *cu, size_t N, int ch, void *stream) {
    hipLaunchKernelGGL(ring_update_kernel, dim3(blocks_for(static_cast<long long>(N) * ch, 256)), dim3(256), 0,
                       as_stream(stream), qkv, ring, cu, static_cast<int>(N), ch);
    return check_launch("ring_update_kernel");
}

size_t argmax_rows_ws_bytes(size_t rows, size_t n) {
    return rows * ((n + kArgChunk - 1) / kArgChunk) * sizeof(unsigned long long);
}

int argmax_rows(const float *y, size_t rows, size_t n, int32_t *idx, unsigned long long *keys, void *stream) {
    if (!rows || !n) return OURO_OK;
    const int nk = static_cast<int>((n + kArgChunk - 1) / kArgChunk);
    hipLaunchKernelGGL(argmax_chunk_kernel, dim3(static_cast<unsigned>(nk), static_cast<unsigned>(rows)), dim3(256), 0,
                       as_stream(stream), y, static_cast<long long>(n), keys);
    int st = check_launch("argmax_chunk_kernel");
    if (st) return st;
    hipLaunchKernelGGL(argmax_final_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, as_stream(stream),
                       keys, nk, idx);
    return check_launch("argmax_final_rows_kernel");
}

}  // namespace ouro
