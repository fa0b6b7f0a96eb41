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

template <typename T>
__device__ __forceinline__ float ld(const T *p, long long i);
template <>
__device__ __forceinline__ float ld<float>(const float *p, long long i) { return p[i]; }
template <>
__device__ __forceinline__ float ld<uint16_t>(const uint16_t *p, long long i) {
    return bf16_bits_to_f32(p[i]);
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

template <typename T>
__device__ __forceinline__ void st(T *p, long long i, float v);
template <>
__device__ __forceinline__ void st<float>(float *p, long long i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void st<uint16_t>(uint16_t *p, long long i, float v) {
    p[i] = f32_to_bf16_bits(v);
}

// In-register stages h = 1..min(8, block/2) over 16 contiguous values.
__device__ __forceinline__ void wht16(float (&v)[16], int logb) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (s >= logb) break;
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
    int n, logb;
    float scale;
};

template <typename TI, typename TO, bool INV, bool QUANT, bool STORE>
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
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = ld(x, 16LL * c + i);
        if (!INV && a.signs) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = v[i] * a.signs[16 * c + i];
        }
        wht16(v, a.logb);
#pragma unroll
        for (int i = 0; i < 16; ++i) lds[pad_idx(16 * c + i)] = v[i];
    }

    // Passes 1..: stages 16, 32, ... in order, 4 per pass.
    for (int p = 1; 4 * p < a.logb; ++p) {
        const int nb = min(4, a.logb - 4 * p);
        const int span = 1 << nb;
        const int sets = n >> nb;
        const int lo_bits = 4 * p;
        __syncthreads();
        for (int s = tid; s < sets; s += kThreads) {
            const int low = s & ((1 << lo_bits) - 1);
            const int high = s >> lo_bits;
            const int base = (high << (lo_bits + nb)) + low;
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j < span) v[j] = lds[pad_idx(base + (j << lo_bits))];
#pragma unroll
            for (int st_ = 0; st_ < 4; ++st_) {
                if (st_ >= nb) break;
                const int h = 1 << st_;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    if ((j & h) == 0 && j + h < span) {
                        const float u = v[j], w = v[j + h];
                        v[j] = u + w;
                        v[j + h] = u - w;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j < span) lds[pad_idx(base + (j << lo_bits))] = v[j];
        }
    }
    __syncthreads();

    // Epilogue: scale (and inverse signs), store, track |max| of stored values.
    TO *y = STORE ? static_cast<TO *>(a.y) + row * n : nullptr;
    float amax = 0.f;
    for (int c = tid; c < chunks; c += kThreads) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float t = lds[pad_idx(16 * c + i)];
            if (INV && a.signs)
                t = t * (a.signs[16 * c + i] * a.scale);
            else
                t = t * a.scale;
            v[i] = as_stored<TO>(t);
        }
        if (STORE) {
#pragma unroll
            for (int i = 0; i < 16; ++i) st(y, 16LL * c + i, v[i]);
        }
        if (QUANT) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                amax = fmaxf(amax, fabsf(v[i]));
                lds[pad_idx(16 * c + i)] = v[i];
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
        for (int i = tid; i < n; i += kThreads) q[i] = 0;
        if (tid == 0) a.dscale[row] = 0.f;
        return;
    }
    const float s = 127.0f / amax;
    for (int c = tid; c < chunks; c += kThreads) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float t = rintf(lds[pad_idx(16 * c + i)] * s);
            t = fminf(fmaxf(t, -127.f), 127.f);
            q[16 * c + i] = static_cast<int8_t>(t);
        }
    }
    if (tid == 0) a.dscale[row] = amax / 127.0f;
}

template <typename TI, typename TO, bool INV>
int launch_t(const FwhtArgs &a, bool quant, bool store, hipStream_t s) {
    const size_t lds = sizeof(float) * static_cast<size_t>(a.n + a.n / 16 + 1);
    void (*kern)(FwhtArgs) = quant ? (store ? fwht_row_kernel<TI, TO, INV, true, true>
                                            : fwht_row_kernel<TI, TO, INV, true, false>)
                                   : fwht_row_kernel<TI, TO, INV, false, true>;
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
int launch_io(const FwhtArgs &a, bool inv, bool quant, bool store, hipStream_t s) {
    return inv ? launch_t<TI, TO, true>(a, quant, store, s) : launch_t<TI, TO, false>(a, quant, store, s);
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
    a.logb = logb;
    a.scale = 1.0f / sqrtf(static_cast<float>(block));  // hadamard.rs:43
    const bool inv = (flags & OURO_FWHT_INVERSE) != 0;
    const bool store = y != nullptr;
    hipStream_t s = as_stream(stream);
    const bool fi = x_dtype == OURO_DT_F32, fo = y_dtype == OURO_DT_F32;
    if (fi && fo) return launch_io<float, float>(a, inv, quant, store, s);
    if (fi && !fo) return launch_io<float, uint16_t>(a, inv, quant, store, s);
    if (!fi && fo) return launch_io<uint16_t, float>(a, inv, quant, store, s);
    return launch_io<uint16_t, uint16_t>(a, inv, quant, store, s);
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
