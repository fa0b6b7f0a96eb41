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
// of the stored output (the activation quantiser of the ternary GEMV).
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
    float *dscale;
    long long rows;
    int n;
    float scale;
};

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

    // Passes 1..3: stages 16, 32, ... in the reference's order, 4 per pass.
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
    if (amax == 0.f) {
        for (int c = tid; c < chunks; c += kThreads)
            *reinterpret_cast<uint4 *>(q + 16 * c) = make_uint4(0, 0, 0, 0);
        if (tid == 0) a.dscale[row] = 0.f;
        return;
    }
    const float s = 127.0f / amax;
    for (int c = tid; c < chunks; c += kThreads) {
        const float *p = lds + 17 * c;
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float t = rintf(p[i] * s);
            t = fminf(fmaxf(t, -127.f), 127.f);
            w[i >> 2] |= (static_cast<uint32_t>(static_cast<int>(t)) & 0xffu) << (8 * (i & 3));
        }
        *reinterpret_cast<uint4 *>(q + 16 * c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    if (tid == 0) a.dscale[row] = amax / 127.0f;
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
              size_t block, const float *signs, unsigned flags, int8_t *xq, float *dscale,
              void *stream) {
    if (!x) return fail(OURO_ERR_INVALID_ARG, "ouro_fwht_rows: x is NULL");
    const bool quant = xq || dscale;
    if (quant && !(xq && dscale))
        return fail(OURO_ERR_INVALID_ARG, "ouro_fwht_rows: xq and dscale go together");
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
    a.dscale = dscale;
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

}  // namespace ouro

using namespace ouro;

extern "C" {

int ouro_fwht_rows(const void *x, int x_dtype, void *y, int y_dtype, size_t rows, size_t n,
                   size_t block, const float *signs, unsigned flags, int8_t *xq, float *dscale,
                   void *stream) {
    OURO_REQUIRE_INIT();
    return fwht_rows(x, x_dtype, y, y_dtype, rows, n, block, signs, flags, xq, dscale, stream);
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
