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

// One wavefront per (token, head of q or k); lane l holds dims 2l, 2l+1.
__global__ __launch_bounds__(256) void attn_prep_kernel(AttnPrepArgs a) {
    const int lane = threadIdx.x & 63;
    const long long item = static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int heads = a.nh + a.nkv;
    if (item >= static_cast<long long>(a.T) * heads) return;  // whole wavefront
    const int t = static_cast<int>(item / heads), hh = static_cast<int>(item % heads);
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
    // rope_partial_neox on the first n_rot dims: pair (i, i + n_rot/2)
    const int half = a.n_rot / 2;
    const int p = a.pos[t];
    const int partner = lane < half / 2 ? lane + half / 2 : lane - half / 2;
    const float px = __shfl(x.x, partner, 64), py = __shfl(x.y, partner, 64);
    if (2 * lane < a.n_rot) {
        float r[2] = {x.x, x.y};
        const float pr[2] = {px, py};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int d = 2 * lane + e;
            const int i = d < half ? d : d - half;
            const float theta = 1.0f / powf(a.rope_base, static_cast<float>(2 * i) / static_cast<float>(a.n_rot));
            const float ang = static_cast<float>(p) * theta;
            const float c = cosf(ang), s = sinf(ang);
            r[e] = d < half ? r[e] * c - pr[e] * s : r[e] * c + pr[e] * s;
        }
        x.x = r[0];
        x.y = r[1];
    }
    if (isq) {
        const long long o = (static_cast<long long>(t) * a.nh + h) * kHd + 2 * lane;
        *reinterpret_cast<float2 *>(a.q_out + o) = x;
        *reinterpret_cast<float2 *>(a.gate_out + o) = *reinterpret_cast<const float2 *>(src + kHd + 2 * lane);
    } else {
        const long long row = kv_row(a.pages, a.maxp, a.seq[t], p);
        const long long o = (row * a.nkv + h) * kHd + 2 * lane;
        *reinterpret_cast<float2 *>(a.kc + o) = x;
        *reinterpret_cast<float2 *>(a.vc + o) =
            *reinterpret_cast<const float2 *>(a.v + (static_cast<long long>(t) * a.nkv + h) * kHd + 2 * lane);
    }
}

// ---------------------------------------------------- attention (prefill) --

constexpr int kQT = 64;        // query rows per tile
constexpr int kKT = 64;        // keys per tile
constexpr int kQP = kHd + 4;   // LDS row pitch (floats) of Q, K, V tiles
constexpr int kPP = kKT + 4;   // LDS row pitch of P

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

// Causal attention over a packed varlen batch on fp32 MFMA
// (v_mfma_f32_16x16x4f32: fp32 products and sums, the reference's f32
// arithmetic up to summation order).  One workgroup per (query tile of 64
// tokens of one sequence, q head); wavefront w owns query rows 16w..16w+15
// and keeps their Q in registers as A operands.  Per key tile of 64 (one KV
// page): S = Q K^T as 4 MFMA tiles of 16 keys (k = 128 dims, the dims of
// k-step s and lane group g being 32g + s), online softmax per row with DPP
// row reductions, P to the wavefront's LDS rows, then O += P V as 8 MFMA
// tiles of 16 dims (k = 64 keys, key 16g + s at step s) with V staged
// transposed.  The sigmoid output gate is applied at the end.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false)));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
    return v;
}

constexpr int kVTP = kKT + 4;  // LDS row pitch of V^T (floats)
// P reuses the K tile's space once every wavefront has its scores: 68 KiB,
// two workgroups per CU
constexpr int kAttnLds = (kKT * kQP + kHd * kVTP) * 4;
static_assert(kQT * kPP <= kKT * kQP, "P fits in the K tile");

__device__ __forceinline__ f32x4_t mfma_f32(float a, float b, const f32x4_t &c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__global__ __launch_bounds__(256) void attn_prefill_kernel(AttnArgs a) {
    extern __shared__ float lds[];
    float *Ks = lds, *Vt = Ks + kKT * kQP;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int s = a.tile_seq[blockIdx.x], p0 = a.tile_p0[blockIdx.x];
    const int h = blockIdx.y;
    const int kvh = h / (a.nh / a.nkv);
    const int t0 = a.cu[s], L = a.cu[s + 1] - t0;
    float *Pw = Ks + 16 * wave * kPP;  // this wavefront's 16 rows of P (over the K tile)

    // Q row 16w + lr, dims 32g .. 32g + 31 as the A operand of k-steps 0..31
    float qa[32];
    {
        const int qp = min(p0 + 16 * wave + lr, L - 1);  // rows past the end: any valid row, never stored
        const float *qr = a.q + ((static_cast<long long>(t0) + qp) * a.nh + h) * kHd + 32 * lg;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = *reinterpret_cast<const float4 *>(qr + 4 * i);
            qa[4 * i] = v.x, qa[4 * i + 1] = v.y, qa[4 * i + 2] = v.z, qa[4 * i + 3] = v.w;
        }
    }
    f32x4_t o[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        m[e] = -INFINITY;
        l[e] = 0.f;
    }
    const int last = min(p0 + kQT, L) - 1;  // last query position in the tile
    // K and V of the next key tile are loaded into registers while the
    // current one is used (a key tile is one KV page; rows past L read the
    // page's unused rows and are zeroed)
    constexpr int kPer = kKT * (kHd / 4) / 256;  // float4 of K (and of V) per thread
    float4 kpre[kPer], vpre[kPer];
    auto load_kv = [&](int k0) {
        const long long row0 = kv_row(a.pages, a.maxp, s, k0);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = tid + 256 * j, r = i / (kHd / 4), c4 = i % (kHd / 4);
            const long long off = ((row0 + r) * a.nkv + kvh) * kHd + 4 * c4;
            kpre[j] = *reinterpret_cast<const float4 *>(a.kc + off);
            vpre[j] = *reinterpret_cast<const float4 *>(a.vc + off);
        }
    };
    load_kv(0);
    for (int k0 = 0; k0 <= last; k0 += kKT) {
        __syncthreads();  // the previous tile's K and V are consumed
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = tid + 256 * j, r = i / (kHd / 4), c4 = i % (kHd / 4);
            const bool live = k0 + r < L;
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 kv = live ? kpre[j] : z, vv = live ? vpre[j] : z;
            *reinterpret_cast<float4 *>(Ks + r * kQP + 4 * c4) = kv;
            Vt[(4 * c4) * kVTP + r] = vv.x;
            Vt[(4 * c4 + 1) * kVTP + r] = vv.y;
            Vt[(4 * c4 + 2) * kVTP + r] = vv.z;
            Vt[(4 * c4 + 3) * kVTP + r] = vv.w;
        }
        __syncthreads();
        if (k0 + kKT <= last) load_kv(k0 + kKT);
        // S: tile t holds S[16w + 4g + e][k0 + 16t + lr]
        f32x4_t sc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            const float *kr = Ks + (16 * t + lr) * kQP + 32 * lg;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 kv = *reinterpret_cast<const float4 *>(kr + 4 * i);
                sc[t] = mfma_f32(qa[4 * i], kv.x, sc[t]);
                sc[t] = mfma_f32(qa[4 * i + 1], kv.y, sc[t]);
                sc[t] = mfma_f32(qa[4 * i + 2], kv.z, sc[t]);
                sc[t] = mfma_f32(qa[4 * i + 3], kv.w, sc[t]);
            }
        }
        __syncthreads();  // every wavefront's scores are done: P may overwrite the K tile
        float corr[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int qp = p0 + 16 * wave + 4 * lg + e;
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int kp = k0 + 16 * t + lr;
                sc[t][e] = (kp <= qp && kp < L) ? sc[t][e] * a.scale : -INFINITY;
                mx = fmaxf(mx, sc[t][e]);
            }
            mx = row16_max(mx);
            const float mn = fmaxf(m[e], mx);
            // rows with no visible key yet keep m = -inf; use 0 to avoid inf - inf
            const float mref = mn == -INFINITY ? 0.f : mn;
            corr[e] = expf(m[e] - mref);
            float ps = 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float pv = expf(sc[t][e] - mref);
                Pw[(4 * lg + e) * kPP + 16 * t + lr] = pv;
                ps += pv;
            }
            l[e] = l[e] * corr[e] + row16_sum(ps);
            m[e] = mn;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[t][e] *= corr[e];
        __builtin_amdgcn_wave_barrier();  // P rows written by this wavefront only
        // O += P V: A = P[16w + lr][16g + s], B = V[16g + s][16t + lr]
        float pa[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = *reinterpret_cast<const float4 *>(Pw + lr * kPP + 16 * lg + 4 * i);
            pa[4 * i] = v.x, pa[4 * i + 1] = v.y, pa[4 * i + 2] = v.z, pa[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float *vr = Vt + (16 * t + lr) * kVTP + 16 * lg;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 vv = *reinterpret_cast<const float4 *>(vr + 4 * i);
                o[t] = mfma_f32(pa[4 * i], vv.x, o[t]);
                o[t] = mfma_f32(pa[4 * i + 1], vv.y, o[t]);
                o[t] = mfma_f32(pa[4 * i + 2], vv.z, o[t]);
                o[t] = mfma_f32(pa[4 * i + 3], vv.w, o[t]);
            }
        }
        __builtin_amdgcn_wave_barrier();  // P reads done before the next tile's writes
    }
    // o / l, times sigmoid(gate) (qwen35.rs:1208-1210); lane holds rows 4g + e, dims 16t + lr
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int qp = p0 + 16 * wave + 4 * lg + e;
        if (qp >= L) continue;
        const long long base = ((static_cast<long long>(t0) + qp) * a.nh + h) * kHd + lr;
        const float il = 1.0f / l[e];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float g = a.gate[base + 16 * t];
            a.out[base + 16 * t] = (o[t][e] * il) * (1.0f / (1.0f + expf(-g)));
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
__global__ __launch_bounds__(256) void attn_decode_split_kernel(AttnArgs a, float *part, int nsplit) {
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
    constexpr int kB = 8;
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
// Grid: x = channel blocks of 256, y = contiguous token ranges.  A thread
// walks its channel along its range with the last three inputs in registers
// (each input read once), taking them from the sequence's ring at a
// sequence start.  The gates of token t are written by channel block 0.
__global__ __launch_bounds__(256) void prefill_conv_gate_kernel(ConvArgs a, int per) {
    // tokens go in batches of kB: a batch's loads are issued together (the
    // token loop is otherwise one dependent HBM round trip per token)
    constexpr int kB = 16;
    const int c = static_cast<int>(blockIdx.x) * 256 + threadIdx.x;
    const int ta = static_cast<int>(blockIdx.y) * per, tb = min(ta + per, a.T);
    // the last column of workgroups computes the gates (next to the conv
    // workgroups rather than in one of them, which made it the longest)
    if (static_cast<int>(blockIdx.x) == (a.ch + 255) / 256) {
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
    if (c >= a.ch || ta >= tb) return;
    const float4 w = *reinterpret_cast<const float4 *>(a.conv_w + 4LL * c);
    const int di = a.di, dv = a.ch - 2 * a.di;
    // window x[t-3], x[t-2], x[t-1] for the range's first token
    float x0, x1, x2;
    {
        const int p = a.pos[ta];
        const float *r = a.ring + (static_cast<long long>(a.seq[ta]) * a.ch + c) * 3;
        x0 = p >= 3 ? a.qkv[(static_cast<long long>(ta) - 3) * a.ch + c] : r[p];
        x1 = p >= 2 ? a.qkv[(static_cast<long long>(ta) - 2) * a.ch + c] : r[1 + p];
        x2 = p >= 1 ? a.qkv[(static_cast<long long>(ta) - 1) * a.ch + c] : r[2];
    }
    for (int t0 = ta; t0 < tb; t0 += kB) {
        float xb[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) xb[u] = a.qkv[static_cast<long long>(min(t0 + u, tb - 1)) * a.ch + c];
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            const int t = t0 + u;
            if (t >= tb) break;
            if (t > ta && a.pos[t] == 0) {  // a sequence starts: its ring is the window
                const float *r = a.ring + (static_cast<long long>(a.seq[t]) * a.ch + c) * 3;
                x0 = r[0];
                x1 = r[1];
                x2 = r[2];
            }
            const float x = xb[u];
            const float y = w.x * x0 + w.y * x1 + w.z * x2 + w.w * x;
            x0 = x1;
            x1 = x2;
            x2 = x;
            const uint16_t sy = to_bf16(y / (1.0f + expf(-y)));
            if (c < di)
                a.qb[static_cast<long long>(t) * di + c] = sy;
            else if (c < 2 * di)
                a.kb[static_cast<long long>(t) * di + c - di] = sy;
            else
                a.vb[static_cast<long long>(t) * dv + c - 2 * di] = sy;
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
    AttnPrepArgs a{qfull, k, v, qn, kn, pos, seq, pages, q_out, gate_out, kc, vc,
                   static_cast<int>(T), nh, nkv, n_rot, maxp, rope_base, eps};
    const long long items = static_cast<long long>(T) * (nh + nkv);
    hipLaunchKernelGGL(attn_prep_kernel, dim3(blocks_for(items, 4)), dim3(256), 0, as_stream(stream), a);
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
    const int cb = (ch + 255) / 256;
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
