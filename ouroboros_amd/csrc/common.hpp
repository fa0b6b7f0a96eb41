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

// Per-device workspace owned by the library (grown on demand, freed by
// ouro_shutdown).  Returns nullptr and sets the error on failure.
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

}  // namespace ouro
