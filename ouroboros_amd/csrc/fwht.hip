// fwht.hip - blockwise Walsh-Hadamard rotation of activation rows
// (hadamard::rotate_fwd / rotate_inv, hadamard.rs:41-66).
//
// One 256-thread workgroup owns one row, staged in LDS.  The butterfly
// stages of wht_inplace (hadamard.rs:15-31) run in the reference's order
// h = 1, 2, 4, ..., block/2, four stages per pass: pass 0 in registers over
// 16 contiguous elements per thread, each later pass over the 16 elements
// that differ only in index bits 4p..4p+3.  Every stage is the same set of
// independent (a+b, a-b) pairs as in the reference, so the fp32 result is
// bit-identical.  Optional fused epilogue: per-row int8 absmax quantisation
// of the stored output (bitnet.cpp's quantize_row_i8_s, the activation
// quantiser of the ternary GEMV).
#include "common.hpp"

#pragma clang fp contract(off)

namespace ouro {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxN = 32768;  // row length limit of the LDS-resident design

__device__ __forceinline__ int pad_idx(int i) { return i + (i >> 4); }

// 16 contiguous elements <-> registers with 16-byte global accesses.
__device__ __forceinline__ void ld16(const float *p, float (&v)[16]) {
    const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 t = q[i];
        v[4 * i] = t.x, v[4 * i + 1] = t.y, v[4 * i + 2] = t.z, v[4 * i + 3] = t.w;
    }
}
__device__ __forceinline__ void ld16(const uint16_t *p, float (&v)[16]) {
    const uint4 *q = reinterpret_cast<const uint4 *>(p);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint4 t = q[i];
        const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[8 * i + 2 * e] = __uint_as_float(w[e] << 16);
            v[8 * i + 2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
        }
    }
}
__device__ __forceinline__ void st16(float *p, const float (&v)[16]) {
    float4 *q = reinterpret_cast<float4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}
__device__ __forceinline__ void st16(uint16_t *p, const float (&v)[16]) {
    uint4 *q = reinterpret_cast<uint4 *>(p);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = static_cast<uint32_t>(f32_to_bf16_bits(v[8 * i + 2 * e])) |
                   (static_cast<uint32_t>(f32_to_bf16_bits(v[8 * i + 2 * e + 1])) << 16);
        q[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Value as it will be stored in the output dtype (bf16 rounds).
template <typename T>
__device__ __forceinline__ float as_stored(float v);
template <>
__device__ __forceinline__ float as_stored<float>(float v) { return v; }
template <>
__device__ __forceinline__ float as_stored<uint16_t>(float v) {
    return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// In-register stages h = 1..min(8, block/2) over 16 contiguous values.
template <int LOGB>
__device__ __forceinline__ void wht16(float (&v)[16]) {
#pragma unroll
    for (int s = 0; s < (LOGB < 4 ? LOGB : 4); ++s) {
        const int h = 1 << s;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if ((i & h) == 0) {
                const float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
        }
    }
}

struct FwhtArgs {
    const void *x;
    void *y;
    const float *signs;
    int8_t *xq;
    float *act_scale;
    long long rows;
    int n;
    float scale;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (56 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(FwhtArgs) == 56, "FwhtArgs: kernel argument layout");

// Pass P (P >= 1) of a block of 2^LOGB: stages 2^(4P) .. over the <= 16
// elements of one set, which differ only in index bits 4P .. 4P+NB-1.  The
// padded LDS index of element e is e + e/16, so the set's elements sit at a
// constant stride from its base and every access is an immediate offset.
template <int LOGB, int P>
__device__ __forceinline__ void wht_pass(float *lds, int n, int tid) {
    constexpr int LO = 4 * P;
    constexpr int NB = (LOGB - LO) < 4 ? (LOGB - LO) : 4;
    constexpr int SPAN = 1 << NB;
    constexpr int STRIDE = (1 << LO) + (1 << (LO - 4));  // padded distance of index bit LO
    const int sets = n >> NB;
    for (int s = tid; s < sets; s += kThreads) {
        const int low = s & ((1 << LO) - 1);
        const int high = s >> LO;
        const int base = (high << (LO + NB)) + low;
        float *p = lds + pad_idx(base);
        float v[16];
#pragma unroll
        for (int j = 0; j < SPAN; ++j) v[j] = p[j * STRIDE];
#pragma unroll
        for (int st_ = 0; st_ < NB; ++st_) {
            const int h = 1 << st_;
#pragma unroll
            for (int j = 0; j < SPAN; ++j) {
                if ((j & h) == 0) {
                    const float u = v[j], w = v[j + h];
                    v[j] = u + w;
                    v[j + h] = u - w;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < SPAN; ++j) p[j * STRIDE] = v[j];
    }
}

// The last pass of a plain rotation (no quantisation) straight to the
// output: the same stages as wht_pass<LOGB, P>, then each value scaled (and,
// inverse, signed) exactly as the epilogue does and stored at its element
// index.  For a fixed j the lanes of a wavefront hold consecutive elements,
// so every store instruction is contiguous; this saves the epilogue's LDS
// round trip and its barrier.
template <typename TO, bool INV, int LOGB, int P>
__device__ __forceinline__ void wht_pass_store(const float *lds, int n, int tid, const FwhtArgs &a, long long row) {
    constexpr int LO = 4 * P;
    constexpr int NB = (LOGB - LO) < 4 ? (LOGB - LO) : 4;
    constexpr int SPAN = 1 << NB;
    constexpr int STRIDE = (1 << LO) + (1 << (LO - 4));
    TO *y = static_cast<TO *>(a.y) + row * n;
    const int sets = n >> NB;
    for (int s = tid; s < sets; s += kThreads) {
        const int low = s & ((1 << LO) - 1);
        const int high = s >> LO;
        const int base = (high << (LO + NB)) + low;
        const float *p = lds + pad_idx(base);
        float v[16];
#pragma unroll
        for (int j = 0; j < SPAN; ++j) v[j] = p[j * STRIDE];
#pragma unroll
        for (int st_ = 0; st_ < NB; ++st_) {
            const int h = 1 << st_;
#pragma unroll
            for (int j = 0; j < SPAN; ++j) {
                if ((j & h) == 0) {
                    const float u = v[j], w = v[j + h];
                    v[j] = u + w;
                    v[j + h] = u - w;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < SPAN; ++j) {
            const int e = base + (j << LO);
            const float t = (INV && a.signs) ? v[j] * (a.signs[e] * a.scale) : v[j] * a.scale;
            if constexpr (sizeof(TO) == 2) y[e] = f32_to_bf16_bits(t);
            else y[e] = t;
        }
    }
}

template <typename TI, typename TO, bool INV, bool QUANT, bool STORE, int LOGB>
__global__ __launch_bounds__(kThreads) void fwht_row_kernel(FwhtArgs a) {
    extern __shared__ float lds[];
    __shared__ float red[kThreads / 64];
    const long long row = blockIdx.x;
    const int n = a.n;
    const int tid = threadIdx.x;
    const TI *x = static_cast<const TI *>(a.x) + row * n;
    const int chunks = n / 16;

    // Pass 0: load 16 contiguous values, apply forward signs, stages 1..8.
    for (int c = tid; c < chunks; c += kThreads) {
        float v[16];
        ld16(x + 16LL * c, v);
        if (!INV && a.signs) {
            float sg[16];
            ld16(a.signs + 16 * c, sg);
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = v[i] * sg[i];
        }
        wht16<LOGB>(v);
        float *p = lds + 17 * c;
#pragma unroll
        for (int i = 0; i < 16; ++i) p[i] = v[i];
    }

    // Passes 1..3: stages 16, 32, ... in the reference's order, 4 per pass;
    // a plain rotation stores its last pass straight to the output.
    constexpr int kLast = (LOGB - 1) / 4;  // index of the last pass
    constexpr bool kDirect = !QUANT && STORE && LOGB > 4;
    if constexpr (LOGB > 4) {
        __syncthreads();
        if constexpr (kDirect && kLast == 1) {
            wht_pass_store<TO, INV, LOGB, 1>(lds, n, tid, a, row);
            return;
        } else {
            wht_pass<LOGB, 1>(lds, n, tid);
        }
    }
    if constexpr (LOGB > 8) {
        __syncthreads();
        if constexpr (kDirect && kLast == 2) {
            wht_pass_store<TO, INV, LOGB, 2>(lds, n, tid, a, row);
            return;
        } else {
            wht_pass<LOGB, 2>(lds, n, tid);
        }
    }
    if constexpr (LOGB > 12) {
        __syncthreads();
        if constexpr (kDirect && kLast == 3) {
            wht_pass_store<TO, INV, LOGB, 3>(lds, n, tid, a, row);
            return;
        } else {
            wht_pass<LOGB, 3>(lds, n, tid);
        }
    }
    __syncthreads();

    // Epilogue: scale (and inverse signs), store, track |max| of stored values.
    TO *y = STORE ? static_cast<TO *>(a.y) + row * n : nullptr;
    float amax = 0.f;
    for (int c = tid; c < chunks; c += kThreads) {
        float v[16], sg[16];
        if (INV && a.signs) ld16(a.signs + 16 * c, sg);
        float *p = lds + 17 * c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float t = p[i];
            if (INV && a.signs)
                t = t * (sg[i] * a.scale);
            else
                t = t * a.scale;
            v[i] = as_stored<TO>(t);
        }
        if (STORE) st16(y + 16LL * c, v);
        if (QUANT) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                amax = fmaxf(amax, fabsf(v[i]));
                p[i] = v[i];
            }
        }
    }
    if (!QUANT) return;

    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, xor_shfl(amax, off));
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int8_t *q = a.xq + row * n;
    const float s = i8s_scale(amax);
    for (int c = tid; c < chunks; c += kThreads) {
        const float *p = lds + 17 * c;
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i)
            w[i >> 2] |= (static_cast<uint32_t>(i8s_quant(p[i], s)) & 0xffu) << (8 * (i & 3));
        *reinterpret_cast<uint4 *>(q + 16 * c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    if (tid == 0) a.act_scale[row] = s;
}

// ------------------------------------------------------------------------
// Fused row kernels: a prologue that produces the row to be rotated, then
// the same butterfly passes and int8 absmax epilogue as fwht_row_kernel.
//   RQ_COPY    v = a
//   RQ_NORM    s = a (+ b) (optionally stored), v = s * inv * w with
//              inv = 1 / sqrt(mean(s^2) + eps) (rmsnorm, ops.rs:12-17);
//              Q2 also quantises the unrotated v (no rotation) into xq2
//   RQ_SWIGLU  v = silu(a) * b (run_ffn, qwen35.rs:802)
//   RQ_GNORM   per 128-wide head of a: v = a * inv_h * w * silu(b)
//              (gated_norm_rms, qwen35.rs:82-92), heads optionally placed in
//              the V-grouped order (qwen35.rs:1122-1138)
// then v * signs -> WHT blocks -> * 1/sqrt(block) -> int8 absmax.  The int8
// rows go out row-major, or (tiles > 0) in the B-fragment order of the
// few-column ternary GEMM: 16-byte chunk k/16 of row r at
// (((k/256)*4 + (k%256)/64) * tiles + r/16) * 1024 + (16*((k%64)/16) + r%16) * 16.
enum { RQ_COPY = 0, RQ_NORM = 1, RQ_SWIGLU = 2, RQ_GNORM = 3 };

struct RowRqArgs {
    const float *a, *b, *w;
    float *sum_out;
    const float *signs;
    int8_t *xq, *xq2;
    float *ds, *ds2;
    int n, tiles, Hk, Hv;
    unsigned flags;
    float eps, scale;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (104 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(RowRqArgs) == 104, "RowRqArgs: kernel argument layout");

__device__ __forceinline__ long long rq_offset(long long row, int c16, int n, int tiles) {
    if (!tiles) return row * n + 16LL * c16;
    const int kb = c16 >> 4, s = (c16 >> 2) & 3, g = c16 & 3;
    return ((static_cast<long long>(kb * 4 + s) * tiles + (row >> 4)) * 64 + 16 * g + (row & 15)) * 16;
}

__device__ __forceinline__ void quant16_store(const float *p, float s, int8_t *dst) {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i)
        w[i >> 2] |= (static_cast<uint32_t>(i8s_quant(p[i], s)) & 0xffu) << (8 * (i & 3));
    *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
}

template <int LOGB, int PRO, bool Q2>
__global__ __launch_bounds__(kThreads) void row_rq_kernel(RowRqArgs a) {
    extern __shared__ float lds[];
    __shared__ float red[8];
    const long long row = blockIdx.x;
    const int n = a.n, tid = threadIdx.x, chunks = n / 16;
    float *hl = lds + 17 * chunks + 16;  // Q2: the unrotated row, same padded layout
    const float *ar = a.a + row * n;
    float inv = 0.f;
    // RQ_NORM with one chunk per thread: the norm weights and signs of the
    // thread's chunk are loaded with the row, not after the sum of squares
    const bool pre = PRO == RQ_NORM && chunks <= kThreads;
    float wpre[16], spre[16];
    if constexpr (PRO == RQ_NORM) {
        if (pre && tid < chunks) {
            ld16(a.w + 16 * tid, wpre);
            if (a.signs) ld16(a.signs + 16 * tid, spre);
        }
        const float *br = a.b ? a.b + row * n : nullptr;
        float ss = 0.f;
        for (int c = tid; c < chunks; c += kThreads) {
            float v[16];
            ld16(ar + 16 * c, v);
            if (br) {
                float u[16];
                ld16(br + 16 * c, u);
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = v[i] + u[i];
            }
            if (a.sum_out) st16(a.sum_out + row * n + 16 * c, v);
            float *p = lds + 17 * c;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                ss += v[i] * v[i];
                p[i] = v[i];
            }
        }
        for (int off = 32; off >= 1; off >>= 1) ss += xor_shfl(ss, off);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        ss = red[0] + red[1] + red[2] + red[3];
        inv = 1.0f / sqrtf(ss / static_cast<float>(n) + a.eps);
    }
    float amax2 = 0.f;
    for (int c = tid; c < chunks; c += kThreads) {
        float v[16];
        int dc = c;
        if constexpr (PRO == RQ_NORM) {
            const float *p = lds + 17 * c;
            float wv[16];
            if (pre) {
#pragma unroll
                for (int i = 0; i < 16; ++i) wv[i] = wpre[i];
            } else {
                ld16(a.w + 16 * c, wv);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = p[i] * inv * wv[i];
            if constexpr (Q2) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    hl[17 * c + i] = v[i];
                    amax2 = fmaxf(amax2, fabsf(v[i]));
                }
            }
        } else if constexpr (PRO == RQ_SWIGLU) {
            float u[16];
            ld16(ar + 16 * c, v);
            ld16(a.b + row * n + 16 * c, u);
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = v[i] / (1.0f + expf(-v[i])) * u[i];
        } else if constexpr (PRO == RQ_GNORM) {
            // the 8 chunks of a head sit on 8 consecutive lanes (n = Hv * 128)
            ld16(ar + 16 * c, v);
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) ss += v[i] * v[i];
            ss += xor_shfl(ss, 1);
            ss += xor_shfl(ss, 2);
            ss += xor_shfl(ss, 4);
            const float invh = 1.0f / sqrtf(ss / 128.0f + a.eps);
            float z[16], wv[16];
            ld16(a.b + row * n + 16 * c, z);
            ld16(a.w + 16 * (c & 7), wv);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float g = z[i] / (1.0f + expf(-z[i]));
                v[i] = v[i] * invh * wv[i] * g;
            }
            if (a.flags & OURO_GDN_V_GROUPED) {
                const int h = c >> 3;
                dc = ((h % a.Hk) * (a.Hv / a.Hk) + h / a.Hk) * 8 + (c & 7);
            }
        } else {
            ld16(ar + 16 * c, v);
        }
        if (a.signs) {
            float sg[16];
            if (pre) {
#pragma unroll
                for (int i = 0; i < 16; ++i) sg[i] = spre[i];
            } else {
                ld16(a.signs + 16 * dc, sg);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = v[i] * sg[i];
        }
        wht16<LOGB>(v);
        float *p = lds + 17 * dc;
#pragma unroll
        for (int i = 0; i < 16; ++i) p[i] = v[i];
    }
    if constexpr (LOGB > 4) {
        __syncthreads();
        wht_pass<LOGB, 1>(lds, n, tid);
    }
    if constexpr (LOGB > 8) {
        __syncthreads();
        wht_pass<LOGB, 2>(lds, n, tid);
    }
    if constexpr (LOGB > 12) {
        __syncthreads();
        wht_pass<LOGB, 3>(lds, n, tid);
    }
    __syncthreads();
    float amax = 0.f;
    for (int c = tid; c < chunks; c += kThreads) {
        float *p = lds + 17 * c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float t = p[i] * a.scale;
            p[i] = t;
            amax = fmaxf(amax, fabsf(t));
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        amax = fmaxf(amax, xor_shfl(amax, off));
        if constexpr (Q2) amax2 = fmaxf(amax2, xor_shfl(amax2, off));
    }
    if ((tid & 63) == 0) {
        red[4 + (tid >> 6)] = amax;
        if constexpr (Q2) red[tid >> 6] = amax2;
    }
    __syncthreads();
    amax = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
    {
        const float s = i8s_scale(amax);
        for (int c = tid; c < chunks; c += kThreads) quant16_store(lds + 17 * c, s, a.xq + rq_offset(row, c, n, a.tiles));
        if (tid == 0) a.ds[row] = s;
    }
    if constexpr (Q2) {
        amax2 = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float s = i8s_scale(amax2);
        for (int c = tid; c < chunks; c += kThreads) quant16_store(hl + 17 * c, s, a.xq2 + rq_offset(row, c, n, a.tiles));
        if (tid == 0) a.ds2[row] = s;
    }
}

template <int PRO, bool Q2>
void (*pick_rq(int logb))(RowRqArgs) {
    switch (logb) {
    case 8: return row_rq_kernel<8, PRO, Q2>;
    case 9: return row_rq_kernel<9, PRO, Q2>;
    case 10: return row_rq_kernel<10, PRO, Q2>;
    case 11: return row_rq_kernel<11, PRO, Q2>;
    case 12: return row_rq_kernel<12, PRO, Q2>;
    case 13: return row_rq_kernel<13, PRO, Q2>;
    default: return nullptr;
    }
}

template <typename TI, typename TO, bool INV, bool QUANT, bool STORE>
void (*pick_logb(int logb))(FwhtArgs) {
    switch (logb) {
    case 1: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 1>;
    case 2: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 2>;
    case 3: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 3>;
    case 4: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 4>;
    case 5: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 5>;
    case 6: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 6>;
    case 7: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 7>;
    case 8: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 8>;
    case 9: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 9>;
    case 10: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 10>;
    case 11: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 11>;
    case 12: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 12>;
    case 13: return fwht_row_kernel<TI, TO, INV, QUANT, STORE, 13>;
    default: return nullptr;
    }
}

template <typename TI, typename TO, bool INV>
int launch_t(const FwhtArgs &a, int logb, bool quant, bool store, hipStream_t s) {
    const size_t lds = sizeof(float) * static_cast<size_t>(a.n + a.n / 16 + 1);
    void (*kern)(FwhtArgs) = quant ? (store ? pick_logb<TI, TO, INV, true, true>(logb)
                                            : pick_logb<TI, TO, INV, true, false>(logb))
                                   : pick_logb<TI, TO, INV, false, true>(logb);
    if (!kern) return fail(OURO_ERR_SHAPE, "ouro_fwht_rows: no kernel for log2(block) = %d", logb);
    if (lds > 64 * 1024) {
        // Rows longer than ~15K elements need the opt-in for >64 KiB of LDS.
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(lds));
        if (e != hipSuccess)
            return fail(OURO_ERR_SHAPE, "ouro_fwht_rows: %zu B of LDS for len %d refused: %s", lds,
                        a.n, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(a.rows)), dim3(kThreads), lds, s, a);
    return check_launch("fwht_row_kernel");
}

template <typename TI, typename TO>
int launch_io(const FwhtArgs &a, int logb, bool inv, bool quant, bool store, hipStream_t s) {
    return inv ? launch_t<TI, TO, true>(a, logb, quant, store, s)
               : launch_t<TI, TO, false>(a, logb, quant, store, s);
}

}  // namespace

int fwht_rows(const void *x, int x_dtype, void *y, int y_dtype, size_t rows, size_t n,
              size_t block, const float *signs, unsigned flags, int8_t *xq, float *act_scale,
              void *stream) {
    if (!x) return fail(OURO_ERR_INVALID_ARG, "ouro_fwht_rows: x is NULL");
    const bool quant = xq || act_scale;
    if (quant && !(xq && act_scale))
        return fail(OURO_ERR_INVALID_ARG, "ouro_fwht_rows: xq and act_scale go together");
    if (!y && !quant) return fail(OURO_ERR_INVALID_ARG, "ouro_fwht_rows: nothing to store");
    if (flags & ~OURO_FWHT_INVERSE) return fail(OURO_ERR_INVALID_ARG, "ouro_fwht_rows: bad flags");
    if ((x_dtype != OURO_DT_F32 && x_dtype != OURO_DT_BF16) ||
        (y_dtype != OURO_DT_F32 && y_dtype != OURO_DT_BF16))
        return fail(OURO_ERR_INVALID_ARG, "ouro_fwht_rows: bad dtype");
    // check_args (hadamard.rs:33-37): block a power of two dividing n.
    if (block < 2 || (block & (block - 1)) || block > 8192)
        return fail(OURO_ERR_SHAPE, "ouro_fwht_rows: block %zu not a power of two in [2, 8192]", block);
    if (!n || n % block) return fail(OURO_ERR_SHAPE, "ouro_fwht_rows: len %zu not multiple of block %zu", n, block);
    if (n % 16 || n > static_cast<size_t>(kMaxN))
        return fail(OURO_ERR_SHAPE, "ouro_fwht_rows: len %zu must be a multiple of 16 and <= %d", n, kMaxN);
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(signs)) % 16)
        return fail(OURO_ERR_ALIGN, "ouro_fwht_rows: x, y and signs need 16-byte alignment");
    if (!rows) return OURO_OK;
    if (rows > 0x7fffffffULL) return fail(OURO_ERR_SHAPE, "ouro_fwht_rows: too many rows");
    FwhtArgs a{};
    a.x = x;
    a.y = y;
    a.signs = signs;
    a.xq = xq;
    a.act_scale = act_scale;
    a.rows = static_cast<long long>(rows);
    a.n = static_cast<int>(n);
    int logb = 0;
    while ((size_t(1) << logb) < block) ++logb;
    a.scale = 1.0f / sqrtf(static_cast<float>(block));  // hadamard.rs:43
    const bool inv = (flags & OURO_FWHT_INVERSE) != 0;
    const bool store = y != nullptr;
    hipStream_t s = as_stream(stream);
    const bool fi = x_dtype == OURO_DT_F32, fo = y_dtype == OURO_DT_F32;
    if (fi && fo) return launch_io<float, float>(a, logb, inv, quant, store, s);
    if (fi && !fo) return launch_io<float, uint16_t>(a, logb, inv, quant, store, s);
    if (!fi && fo) return launch_io<uint16_t, float>(a, logb, inv, quant, store, s);
    return launch_io<uint16_t, uint16_t>(a, logb, inv, quant, store, s);
}

// Fused prologue + rotation + int8 quantisation of rows x n (n a multiple
// of block, block a power of two in 256..8192).  pro: RQ_COPY, RQ_NORM
// (a + b optional, sum_out optional, w[n]; xq2/ds2 optional: the unrotated
// row quantised too), RQ_SWIGLU (gate a, up b), RQ_GNORM (o a, z b, w[128],
// n = Hv * 128, flags OURO_GDN_V_GROUPED).  tiles > 0 writes the int8 rows
// in the few-column GEMM's fragment order for 16 * tiles >= rows columns.
int row_rotate_quant(int pro, const float *a, const float *b, const float *w, float *sum_out, size_t rows,
                     size_t n, size_t block, const float *signs, int8_t *xq, float *ds, int8_t *xq2, float *ds2,
                     int tiles, int Hk, int Hv, unsigned flags, float eps, void *stream) {
    if (!a || !xq || !ds) return fail(OURO_ERR_INVALID_ARG, "row_rotate_quant: NULL argument");
    if (block < 256 || (block & (block - 1)) || block > 8192 || n % block || n > 12288)
        return fail(OURO_ERR_SHAPE, "row_rotate_quant: len %zu, block %zu", n, block);
    if (pro == RQ_GNORM && (n != static_cast<size_t>(Hv) * 128 || Hk < 1 || Hv % Hk))
        return fail(OURO_ERR_SHAPE, "row_rotate_quant: gated norm over %d heads of 128 (len %zu)", Hv, n);
    if (tiles && static_cast<size_t>(tiles) * 16 < rows)
        return fail(OURO_ERR_SHAPE, "row_rotate_quant: %d fragment tiles for %zu rows", tiles, rows);
    if (!rows) return OURO_OK;
    RowRqArgs r{a, b, w, sum_out, signs, xq, xq2, ds, ds2, static_cast<int>(n), tiles, Hk, Hv, flags, eps,
                1.0f / sqrtf(static_cast<float>(block))};
    int logb = 0;
    while ((size_t(1) << logb) < block) ++logb;
    const bool q2 = pro == RQ_NORM && xq2 && ds2;
    void (*kern)(RowRqArgs) = nullptr;
    switch (pro) {
    case RQ_COPY: kern = pick_rq<RQ_COPY, false>(logb); break;
    case RQ_NORM: kern = q2 ? pick_rq<RQ_NORM, true>(logb) : pick_rq<RQ_NORM, false>(logb); break;
    case RQ_SWIGLU: kern = pick_rq<RQ_SWIGLU, false>(logb); break;
    case RQ_GNORM: kern = pick_rq<RQ_GNORM, false>(logb); break;
    default: return fail(OURO_ERR_INVALID_ARG, "row_rotate_quant: prologue %d", pro);
    }
    if (!kern) return fail(OURO_ERR_SHAPE, "row_rotate_quant: block %zu", block);
    const size_t lds = sizeof(float) * ((q2 ? 2 : 1) * (n + n / 16) + 16);
    if (lds > 64 * 1024) return fail(OURO_ERR_SHAPE, "row_rotate_quant: len %zu needs %zu B of LDS", n, lds);
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(rows)), dim3(kThreads), lds, as_stream(stream), r);
    return check_launch("row_rq_kernel");
}

}  // namespace ouro

using namespace ouro;

extern "C" {

int ouro_fwht_rows(const void *x, int x_dtype, void *y, int y_dtype, size_t rows, size_t n,
                   size_t block, const float *signs, unsigned flags, int8_t *xq, float *act_scale,
                   void *stream) {
    OURO_REQUIRE_INIT();
    return fwht_rows(x, x_dtype, y, y_dtype, rows, n, block, signs, flags, xq, act_scale, stream);
}

int ouro_rotate_fwd(float *x, const float *signs, size_t n, size_t block, void *stream) {
    OURO_REQUIRE_INIT();
    if (!signs) return fail(OURO_ERR_INVALID_ARG, "ouro_rotate_fwd: signs is NULL");
    return fwht_rows(x, OURO_DT_F32, x, OURO_DT_F32, 1, n, block, signs, 0, nullptr, nullptr, stream);
}

int ouro_rotate_inv(float *x, const float *signs, size_t n, size_t block, void *stream) {
    OURO_REQUIRE_INIT();
    if (!signs) return fail(OURO_ERR_INVALID_ARG, "ouro_rotate_inv: signs is NULL");
    return fwht_rows(x, OURO_DT_F32, x, OURO_DT_F32, 1, n, block, signs, OURO_FWHT_INVERSE,
                     nullptr, nullptr, stream);
}

}  // extern "C"
