// gdn_decode.hip - gated delta-net recurrent decode step on the GPU.
//
// Follows delta_head_dim (qwen35.rs:27-57) per (sequence, v-head) with the
// per-head preprocessing of run_delta (qwen35.rs:1096-1112):
//   decay = exp(gate); sk = decay * S^T k; dv = beta * (v - sk);
//   S' = decay * S + k dv^T; out = S'^T q.
// With S(i, j) at i + j*d, output column j touches only column j of S, so
// the state is split by columns: a 64-lane wavefront owns CPW columns, lanes
// 0-31 walking one column of each pair and lanes 32-63 the other, four k
// values per lane.  Each wavefront issues all of its state loads up front
// (non-temporal: the state is touched once per step), reduces S^T k across
// its 32-lane halves (permlane16 swaps and DPP, no LDS), broadcasts dv,
// updates the columns in registers, writes them back and reduces S'^T q.  The state
// makes exactly one HBM round trip.
#include "common.hpp"

namespace ouro {
namespace {

constexpr int kD = 128;          // d_state of the qwen35 family (qwen35.rs:8)

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct DecodeArgs {
    float *state;
    const void *q, *k, *v;
    const float *gate, *beta;  // NULL: use gate_s / beta_s for every head
    float gate_s, beta_s;
    float *out;
    long long qk_bs, v_bs;  // elements between consecutive sequences of q/k and of v
    int B, Hk, Hv;
    unsigned flags;
    float eps;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (104 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(DecodeArgs) == 104, "DecodeArgs: kernel argument layout");

// conv_step (qwen35.rs:64-70) of one channel, then SiLU (ops.rs:34-36), in
// the reference's operation order.
__device__ __forceinline__ float conv_silu(const float4 &w, float r0, float r1, float r2, float x) {
#pragma clang fp contract(off)
    const float y = w.x * r0 + w.y * r1 + w.z * r2 + w.w * x;
    return y / (1.0f + expf(-y));
}


template <typename T>
__device__ __forceinline__ float4 ld4(const T *p);
template <>
__device__ __forceinline__ float4 ld4<float>(const float *p) {
    return *reinterpret_cast<const float4 *>(p);
}
template <>
__device__ __forceinline__ float4 ld4<uint16_t>(const uint16_t *p) {
    const uint2 u = *reinterpret_cast<const uint2 *>(p);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                       __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
}
template <typename T>
__device__ __forceinline__ float ld1(const T *p);
template <>
__device__ __forceinline__ float ld1<float>(const float *p) { return *p; }
template <>
__device__ __forceinline__ float ld1<uint16_t>(const uint16_t *p) { return bf16_bits_to_f32(*p); }

// Cross-lane float sums without LDS.  dpp(v, ctrl) moves v across lanes
// of a 16-lane row: 0x128 row_ror:8 (lane ^ 8), 0x141 row_half_mirror
// (lane ^ 7 within 8), 0x4E quad_perm [2,3,0,1] (lane ^ 2), 0xB1 quad_perm
// [1,0,3,2] (lane ^ 1); the four steps make every lane of a row hold the
// row's sum (the lane sets {l, l^8}, {.., ^7}, {.., ^2}, {.., ^1} cover the
// 16 lanes once).
#define OURO_DPP(v, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false))
__device__ __forceinline__ float sum_row16(float v) {
    v += OURO_DPP(v, 0x128);
    v += OURO_DPP(v, 0x141);
    v += OURO_DPP(v, 0x4E);
    v += OURO_DPP(v, 0xB1);
    return v;
}
// v_permlane16_swap(a, b) exchanges the odd 16-lane rows of a with the even
// rows of b; adding the two results sums rows 0+1 and 2+3.
__device__ __forceinline__ float sum_rows_pair(float a, float b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float sum_half(float v) {  // over the 32 lanes of a half, every lane
    return sum_row16(sum_rows_pair(v, v));
}

__device__ __forceinline__ float dot4(const float4 &a, const float4 &b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// One wavefront's update of state columns col0 .. col0+3 of a head (S):
// lanes 0-31 hold rows i0 .. i0+3 of columns col0 + 2p, lanes 32-63 of
// col0 + 2p + 1 (p = 0, 1), loaded by the caller into s.  k and q are
// normalised; vcol(j) is v of column j.  Writes the columns back and
// returns o of column myj (set here) in every lane of its 8-lane group.
constexpr int kCPW = 4;   // state columns per wavefront
constexpr int kPairs = kCPW / 2;
constexpr int kSpan = 32 / kPairs;  // lanes of a half that end up holding one pair

__device__ __forceinline__ void load_cols(const float *S, int col0, int lane, float4 (&s)[kPairs]) {
    const int half = lane >> 5, i0 = 4 * (lane & 31);
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
        const f32x4 t = __builtin_nontemporal_load(
            reinterpret_cast<const f32x4 *>(S + (col0 + 2 * p + half) * kD + i0));
        s[p] = make_float4(t[0], t[1], t[2], t[3]);
    }
}

template <typename VF>
__device__ __forceinline__ float update_cols(float *S, int col0, int lane, const float4 (&s)[kPairs], const float4 &k,
                                             const float4 &q, float decay, float beta, VF vcol, int &myj) {
    const int half = lane >> 5, i0 = 4 * (lane & 31);
    // sk for the column pairs: over each 32-lane half, row r of the half
    // (16 lanes) ends up holding pair r.
    float part[kPairs];
#pragma unroll
    for (int p = 0; p < kPairs; ++p) part[p] = dot4(s[p], k);
    const float skj = sum_row16(sum_rows_pair(part[0], part[1])) * decay;
    // This lane now holds column pair (lane & 31) / kSpan of its half.
    const int myp = (lane & 31) / kSpan;
    myj = col0 + 2 * myp + half;
    const float vj = vcol(myj);
    const float dj = beta * (vj - skj);
    // dv of pair p in half hh sits in every lane of row 2*hh + p (named
    // scalars: an array indexed by the half would be placed in memory).
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dj), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dj), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dj), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dj), 48));
    const float dv0 = half ? r2 : r0, dv1 = half ? r3 : r1;

    float o[kPairs];
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
        const float dp = p == 0 ? dv0 : dv1;
        float4 t;
        t.x = s[p].x * decay + k.x * dp;
        t.y = s[p].y * decay + k.y * dp;
        t.z = s[p].z * decay + k.z * dp;
        t.w = s[p].w * decay + k.w * dp;
        const f32x4 tv = {t.x, t.y, t.z, t.w};
        __builtin_nontemporal_store(tv, reinterpret_cast<f32x4 *>(S + (col0 + 2 * p + half) * kD + i0));
        o[p] = dot4(t, q);
    }
    return sum_row16(sum_rows_pair(o[0], o[1]));
}

// l2_norm of k and q (1 / (sqrt(sum) + eps)) and the 1/sqrt(d) scale of q,
// per the flags, over the 32 lanes of each half (rows i0 .. i0+3 per lane).
__device__ __forceinline__ void norm_qk(float4 &k, float4 &q, unsigned flags, float eps) {
    if (flags & OURO_GDN_L2NORM_QK) {
        const float ik = 1.0f / (sqrtf(sum_half(dot4(k, k))) + eps);
        const float iq = 1.0f / (sqrtf(sum_half(dot4(q, q))) + eps);
        k = make_float4(k.x * ik, k.y * ik, k.z * ik, k.w * ik);
        q = make_float4(q.x * iq, q.y * iq, q.z * iq, q.w * iq);
    }
    if (flags & OURO_GDN_SCALE_Q) {
        const float sc = 1.0f / sqrtf(static_cast<float>(kD));
        q = make_float4(q.x * sc, q.y * sc, q.z * sc, q.w * sc);
    }
}

// kCPW state columns per wavefront, WPB wavefronts per block.
template <typename TQK, typename TV, int WPB>
__global__ __launch_bounds__(64 * WPB) void gdn_decode_kernel(DecodeArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i0 = 4 * (lane & 31);
    const int bh = blockIdx.x;  // b * Hv + h
    const int b = bh / a.Hv, h = bh % a.Hv;
    const int kh = (a.flags & OURO_GDN_KHEAD_DIV) ? h / (a.Hv / a.Hk) : h % a.Hk;
    const int col0 = (blockIdx.y * WPB + wave) * kCPW;

    float *S = a.state + static_cast<long long>(bh) * kD * kD;
    // State columns first: they are the bytes that matter.
    float4 s[kPairs];
    load_cols(S, col0, lane, s);

    const long long qk_off = b * a.qk_bs + static_cast<long long>(kh) * kD + i0;
    float4 k = ld4(static_cast<const TQK *>(a.k) + qk_off);
    float4 q = ld4(static_cast<const TQK *>(a.q) + qk_off);
    const float gate = a.gate ? a.gate[bh] : a.gate_s;
    const float beta = a.beta ? a.beta[bh] : a.beta_s;
    norm_qk(k, q, a.flags, a.eps);
    const float decay = expf(gate);
    const TV *v = static_cast<const TV *>(a.v) + b * a.v_bs + static_cast<long long>(h) * kD;
    int myj;
    const float oj = update_cols(S, col0, lane, s, k, q, decay, beta, [&](int j) { return ld1(v + j); }, myj);
    if ((lane & (kSpan - 1)) == 0) a.out[static_cast<long long>(bh) * kD + myj] = oj;
}

// Any other head dimension d <= 256 (delta_head_dim is the runtime-dim
// variant, qwen35.rs:26-27): one 256-thread workgroup per (sequence, head),
// each wavefront walking columns w, w + 4, ..; lane l holds rows
// i = l + 64m (m < M = ceil(d / 64)) of a column, so every column access is
// coalesced, and S^T k and S'^T q are wavefront reductions.
constexpr int kAnyWaves = 4;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += xor_shfl(v, off);
    return v;
}

template <typename TQK, typename TV, int M>
__global__ __launch_bounds__(64 * kAnyWaves) void gdn_decode_any_kernel(DecodeArgs a, int d) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int bh = blockIdx.x;
    const int b = bh / a.Hv, h = bh % a.Hv;
    const int kh = (a.flags & OURO_GDN_KHEAD_DIV) ? h / (a.Hv / a.Hk) : h % a.Hk;
    const long long qk_off = b * a.qk_bs + static_cast<long long>(kh) * d;
    float k[M], q[M];
    float kk = 0.f, qq = 0.f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int i = lane + 64 * m;
        k[m] = i < d ? ld1(static_cast<const TQK *>(a.k) + qk_off + i) : 0.f;
        q[m] = i < d ? ld1(static_cast<const TQK *>(a.q) + qk_off + i) : 0.f;
        kk += k[m] * k[m];
        qq += q[m] * q[m];
    }
    if (a.flags & OURO_GDN_L2NORM_QK) {  // l2_norm: 1 / (sqrt(sum) + eps)
        const float ik = 1.0f / (sqrtf(wave_sum(kk)) + a.eps);
        const float iq = 1.0f / (sqrtf(wave_sum(qq)) + a.eps);
#pragma unroll
        for (int m = 0; m < M; ++m) k[m] = k[m] * ik, q[m] = q[m] * iq;
    }
    if (a.flags & OURO_GDN_SCALE_Q) {
        const float sc = 1.0f / sqrtf(static_cast<float>(d));
#pragma unroll
        for (int m = 0; m < M; ++m) q[m] = q[m] * sc;
    }
    const float gate = a.gate ? a.gate[bh] : a.gate_s;
    const float beta = a.beta ? a.beta[bh] : a.beta_s;
    const float decay = expf(gate);
    float *S = a.state + static_cast<long long>(bh) * d * d;
    const TV *v = static_cast<const TV *>(a.v) + b * a.v_bs + static_cast<long long>(h) * d;
    for (int j = wave; j < d; j += kAnyWaves) {
        float s[M];
        float part = 0.f;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const int i = lane + 64 * m;
            s[m] = i < d ? S[static_cast<long long>(j) * d + i] : 0.f;
            part += s[m] * k[m];
        }
        const float sk = wave_sum(part) * decay;
        const float dv = beta * (ld1(v + j) - sk);
        float o = 0.f;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const int i = lane + 64 * m;
            const float t = s[m] * decay + k[m] * dv;
            if (i < d) S[static_cast<long long>(j) * d + i] = t;
            o += t * q[m];
        }
        o = wave_sum(o);
        if (lane == 0) a.out[static_cast<long long>(bh) * d + j] = o;
    }
}

template <typename TQK, typename TV>
int launch_any(const DecodeArgs &a, int d, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(a.B * a.Hv)), block(64 * kAnyWaves);
    switch ((d + 63) / 64) {
    case 1: hipLaunchKernelGGL((gdn_decode_any_kernel<TQK, TV, 1>), grid, block, 0, s, a, d); break;
    case 2: hipLaunchKernelGGL((gdn_decode_any_kernel<TQK, TV, 2>), grid, block, 0, s, a, d); break;
    case 3: hipLaunchKernelGGL((gdn_decode_any_kernel<TQK, TV, 3>), grid, block, 0, s, a, d); break;
    default: hipLaunchKernelGGL((gdn_decode_any_kernel<TQK, TV, 4>), grid, block, 0, s, a, d); break;
    }
    return check_launch("gdn_decode_any_kernel");
}

// Measured on B=32, Hv=32 with 8 rotating 64 MiB state sets: 4 columns per
// wavefront in 8-wavefront blocks streams the state at ~91% of the in-place
// read-modify-write rate of a plain copy-style kernel on the same bytes.
constexpr int kWPB = 8;

template <typename TQK, typename TV>
int launch(const DecodeArgs &a, int d, hipStream_t s) {
    if (d != kD) return launch_any<TQK, TV>(a, d, s);
    dim3 grid(static_cast<unsigned>(a.B * a.Hv), kD / (kCPW * kWPB));
    hipLaunchKernelGGL((gdn_decode_kernel<TQK, TV, kWPB>), grid, dim3(64 * kWPB), 0, s, a);
    return check_launch("gdn_decode_kernel");
}

// ---- the whole delta-net layer block between the projections -------------
// run_delta (qwen35.rs:1048-1151) for one decode token per sequence, in one
// launch: one workgroup per (sequence b, k-head kh) with the g = Hv / Hk
// v-heads that read it, so every conv channel it reads belongs to it alone.
//   1. conv_step + SiLU (qwen35.rs:64-70, 1080-1088) of the k-head's q and k
//      channels and of each v-head's v channels from the ring (read only),
//      and beta, decay per v-head (qwen35.rs:1066-1070, 1241-1243), in LDS;
//   2. the normed recurrence of every v-head (update_cols, as the decode
//      kernel), outputs o in LDS;
//   3. gated_norm_rms per v-head (qwen35.rs:82-92) written at its V-grouped
//      position when asked (qwen35.rs:1122-1138);
//   4. the ring shift of every channel read in 1.
struct LayerArgs {
    const float *qkv, *z, *beta_raw, *alpha_raw, *dt_bias, *a_log, *conv_w, *norm_w;
    float *ring, *state, *out;
    int Hk, Hv, ch;
    unsigned flags;  // OURO_GDN_KHEAD_DIV, OURO_GDN_V_GROUPED
    float eps;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (112 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(LayerArgs) == 112, "LayerArgs: kernel argument layout");
constexpr int kLayerWaves = 16;

// The conv channel of item t of the workgroup's (2 + g) * d: q, k, then v
// of each v-head.
__device__ __forceinline__ int layer_channel(const LayerArgs &a, int kh, int g, int t) {
    const int blk = t / kD, i = t % kD;
    if (blk == 0) return kh * kD + i;
    if (blk == 1) return (a.Hk + kh) * kD + i;
    const int j = blk - 2;
    const int h = (a.flags & OURO_GDN_KHEAD_DIV) ? kh * g + j : kh + a.Hk * j;
    return (2 * a.Hk + h) * kD + i;
}

__global__ __launch_bounds__(64 * kLayerWaves) void gdn_layer_kernel(LayerArgs a) {
    extern __shared__ float lsm[];  // q[d] k[d] v[g][d] o[g][d] beta[g] decay[g]
    const int g = a.Hv / a.Hk;
    const int b = blockIdx.x / a.Hk, kh = blockIdx.x % a.Hk;
    const bool div = (a.flags & OURO_GDN_KHEAD_DIV) != 0;
    float *os = lsm + (2 + g) * kD, *bs = os + g * kD, *ds = bs + g;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int nthr = 64 * kLayerWaves;
    const long long row = static_cast<long long>(b) * a.ch;

    for (int t = tid; t < (2 + g) * kD; t += nthr) {
        const long long c = row + layer_channel(a, kh, g, t);
        const float *r = a.ring + c * 3;
        lsm[t] = conv_silu(reinterpret_cast<const float4 *>(a.conv_w)[c - row], r[0], r[1], r[2], a.qkv[c]);
    }
    if (tid < g) {
#pragma clang fp contract(off)
        const int h = div ? kh * g + tid : kh + a.Hk * tid;
        const long long bh = static_cast<long long>(b) * a.Hv + h;
        bs[tid] = 1.0f / (1.0f + expf(-a.beta_raw[bh]));
        const float x = a.alpha_raw[bh] + a.dt_bias[h];
        ds[tid] = expf(a.a_log[h] * (x > 20.0f ? x : logf(1.0f + expf(x))));
    }
    __syncthreads();

    const int i0 = 4 * (lane & 31);
    float4 q = *reinterpret_cast<const float4 *>(lsm + i0);
    float4 k = *reinterpret_cast<const float4 *>(lsm + kD + i0);
    norm_qk(k, q, OURO_GDN_L2NORM_QK | OURO_GDN_SCALE_Q, a.eps);
    for (int gi = wave; gi < g * (kD / kCPW); gi += kLayerWaves) {  // column groups of the g heads
        const int j = gi / (kD / kCPW), col0 = gi % (kD / kCPW) * kCPW;
        const int h = div ? kh * g + j : kh + a.Hk * j;
        float *S = a.state + (static_cast<long long>(b) * a.Hv + h) * kD * kD;
        float4 s[kPairs];
        load_cols(S, col0, lane, s);
        const float *vs = lsm + (2 + j) * kD;
        int myj;
        const float oj = update_cols(S, col0, lane, s, k, q, ds[j], bs[j], [&](int c) { return vs[c]; }, myj);
        if ((lane & (kSpan - 1)) == 0) os[j * kD + myj] = oj;
    }
    __syncthreads();

    for (int j = wave; j < g; j += kLayerWaves) {
#pragma clang fp contract(off)
        const int h = div ? kh * g + j : kh + a.Hk * j;
        const long long bh = static_cast<long long>(b) * a.Hv + h;
        const float2 x = *reinterpret_cast<const float2 *>(os + j * kD + 2 * lane);
        float ss = x.x * x.x + x.y * x.y;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss += xor_shfl(ss, off);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(kD) + a.eps);
        const float2 zz = *reinterpret_cast<const float2 *>(a.z + bh * kD + 2 * lane);
        const float2 w = *reinterpret_cast<const float2 *>(a.norm_w + 2 * lane);
        const float g0 = zz.x / (1.0f + expf(-zz.x)), g1 = zz.y / (1.0f + expf(-zz.y));
        const int dst = (a.flags & OURO_GDN_V_GROUPED) ? (h % a.Hk) * g + h / a.Hk : h;
        *reinterpret_cast<float2 *>(a.out + (static_cast<long long>(b) * a.Hv + dst) * kD + 2 * lane) =
            make_float2(x.x * inv * w.x * g0, x.y * inv * w.y * g1);
    }
    for (int t = tid; t < (2 + g) * kD; t += nthr) {  // the window moves by one, the new input enters last
        const long long c = row + layer_channel(a, kh, g, t);
        float *r = a.ring + c * 3;
        const float r1 = r[1], r2 = r[2];
        r[0] = r1;
        r[1] = r2;
        r[2] = a.qkv[c];
    }
}

}  // namespace

size_t gdn_layer_lds_bytes(size_t Hk, size_t Hv) { return ((2 + 2 * (Hv / Hk)) * kD + 2 * (Hv / Hk)) * 4; }

// The layer block in one launch (d = 128, f32; shapes and alignment checked
// by the caller).
int gdn_layer_fused(const float *qkv, const float *z, const float *beta_raw, const float *alpha_raw,
                    const float *dt_bias, const float *a_log, const float *conv_w, const float *norm_w, float *ring,
                    float *state, float *out, size_t B, size_t Hk, size_t Hv, unsigned flags, float eps,
                    void *stream) {
    const LayerArgs a{qkv, z, beta_raw, alpha_raw, dt_bias, a_log, conv_w, norm_w, ring, state, out,
                      static_cast<int>(Hk), static_cast<int>(Hv), static_cast<int>((2 * Hk + Hv) * kD), flags, eps};
    const size_t lds = gdn_layer_lds_bytes(Hk, Hv);
    if (lds > 64 * 1024) return fail(OURO_ERR_SHAPE, "gdn layer: %zu v-heads per k-head is too many", Hv / Hk);
    hipLaunchKernelGGL(gdn_layer_kernel, dim3(static_cast<unsigned>(B * Hk)), dim3(64 * kLayerWaves),
                       static_cast<unsigned>(lds), as_stream(stream), a);
    return check_launch("gdn_layer_kernel");
}

int gdn_decode(float *state, const void *q, const void *k, int qk_dtype, const void *v, int v_dtype,
               const float *gate, const float *beta, float gate_s, float beta_s, float *out,
               size_t B, size_t Hk, size_t Hv, size_t d, unsigned flags, float eps, void *stream,
               size_t qk_bs, size_t v_bs) {
    if (!state || !q || !k || !v || !out) return fail(OURO_ERR_INVALID_ARG, "gdn decode: NULL argument");
    if (!d || d > 256) return fail(OURO_ERR_SHAPE, "gdn decode: d = %zu, supported 1..256", d);
    if (!B || !Hk || !Hv || Hv % Hk) return fail(OURO_ERR_SHAPE, "gdn decode: bad heads B=%zu Hk=%zu Hv=%zu", B, Hk, Hv);
    if (B * Hv > 0x7fffffffULL) return fail(OURO_ERR_SHAPE, "gdn decode: too many heads");
    if (flags & ~(OURO_GDN_L2NORM_QK | OURO_GDN_SCALE_Q | OURO_GDN_KHEAD_DIV))
        return fail(OURO_ERR_INVALID_ARG, "gdn decode: bad flags 0x%x", flags);
    // d = 128 reads q, k and the state in 16-byte pieces; other d element-wise
    const bool wide = d == static_cast<size_t>(kD);
    if (reinterpret_cast<uintptr_t>(state) % (wide ? 16 : 4))
        return fail(OURO_ERR_ALIGN, "gdn decode: state needs %d-byte alignment", wide ? 16 : 4);
    const size_t qa = wide ? (qk_dtype == OURO_DT_F32 ? 16 : 8) : (qk_dtype == OURO_DT_F32 ? 4 : 2);
    if (reinterpret_cast<uintptr_t>(q) % qa || reinterpret_cast<uintptr_t>(k) % qa)
        return fail(OURO_ERR_ALIGN, "gdn decode: q/k need %zu-byte alignment", qa);
    if ((qk_bs * (qk_dtype == OURO_DT_F32 ? 4 : 2)) % qa)
        return fail(OURO_ERR_ALIGN, "gdn decode: q/k sequence stride breaks %zu-byte alignment", qa);
    DecodeArgs a{};
    a.state = state;
    a.q = q;
    a.k = k;
    a.v = v;
    a.gate = gate;
    a.beta = beta;
    a.gate_s = gate_s;
    a.beta_s = beta_s;
    a.out = out;
    a.qk_bs = static_cast<long long>(qk_bs ? qk_bs : Hk * d);
    a.v_bs = static_cast<long long>(v_bs ? v_bs : Hv * d);
    a.B = static_cast<int>(B);
    a.Hk = static_cast<int>(Hk);
    a.Hv = static_cast<int>(Hv);
    a.flags = flags;
    a.eps = eps;
    hipStream_t s = as_stream(stream);
    const bool qf = qk_dtype == OURO_DT_F32, vf = v_dtype == OURO_DT_F32;
    if ((qk_dtype != OURO_DT_F32 && qk_dtype != OURO_DT_BF16) || (v_dtype != OURO_DT_F32 && v_dtype != OURO_DT_BF16))
        return fail(OURO_ERR_INVALID_ARG, "gdn decode: bad dtype");
    const int dd = static_cast<int>(d);
    if (qf && vf) return launch<float, float>(a, dd, s);
    if (qf) return launch<float, uint16_t>(a, dd, s);
    if (vf) return launch<uint16_t, float>(a, dd, s);
    return launch<uint16_t, uint16_t>(a, dd, s);
}

}  // namespace ouro

using namespace ouro;

extern "C" {

int ouro_gdn_decode(float *state, const void *q, const void *k, int qk_dtype, const void *v, int v_dtype,
                    const float *gate, const float *beta, float *out, size_t B, size_t Hk, size_t Hv,
                    size_t d, unsigned flags, float eps, void *stream) {
    OURO_REQUIRE_INIT();
    if (!gate || !beta) return fail(OURO_ERR_INVALID_ARG, "ouro_gdn_decode: gate/beta NULL");
    return gdn_decode(state, q, k, qk_dtype, v, v_dtype, gate, beta, 0.f, 0.f, out, B, Hk, Hv, d,
                      flags, eps, stream, 0, 0);
}

int ouro_delta_head_dim(float *state, size_t sdim, const float *q, const float *k, const float *v,
                        float gate, float beta, float *out, void *stream) {
    OURO_REQUIRE_INIT();
    return gdn_decode(state, q, k, OURO_DT_F32, v, OURO_DT_F32, nullptr, nullptr, gate, beta, out, 1,
                      1, 1, sdim, 0u, 0.f, stream, 0, 0);
}

}  // extern "C"
