// tl1_lut.hip - TL1 (PTQ1_0) matvec by table lookup, for resident weights.
//
// A PTQ1_0 group (dequant.rs:140-171) is 28 bytes: qs[0..16] carry the
// elements n*16 + m, qs[16..24] the elements 80 + n*8 + m, qh[0..2] the
// elements 120 + n*2 + h (5, 5 and 4 trits per byte, digit of byte v at
// stage n = ((v * 3^n mod 256) * 3) >> 8, trit = digit - 1), then an f16
// scale d.  matvec_tl1 (ops.rs:294-363) computes y[r] = sum over groups of
// sum over elements (trit * d) * x.
//
// Here every payload byte is one lookup: for a block of 4 groups the
// workgroup builds, in LDS, the partial dot of each of the 256 byte values
// of each of the 26 byte positions with its 4 or 5 x values
// (T[g][b][v] = sum_n trit_n(v) x[...]); a row then costs 26 lookups and
// adds per group and one multiply by d.  Weights are repacked on upload so
// that the 112 bytes of a row's group block sit in 7 x 16 B lane-interleaved
// chunks ([block][row tile of 64][chunk][lane]): every load instruction
// reads 1 KiB contiguously.  Each group block writes a partial sum per row;
// a second kernel adds the blocks (and can take the finite_argmax of the
// result on the way, for a greedy sample).
#include "common.hpp"

#include <algorithm>

namespace ouro {
namespace {

constexpr int kGB = 4;                 // groups per block
constexpr int kChunks = kGB * 28 / 16; // 7 x 16 B per row per block
constexpr int kThreads = 1024;
constexpr int kAhead = 1;             // tiles of weights in flight per wave (deeper is slower)
constexpr int kTable = kGB * 26 * 256; // floats
constexpr int LUT_LDS = kTable * 4 + kGB * 128 * 4;

__device__ __forceinline__ int tl1_trit(uint32_t v, uint32_t pow3) {
    const uint32_t q = (v * pow3) & 0xffu;  // u8 wrapping_mul
    return static_cast<int>((q * 3u) >> 8) - 1;
}

// Raw row-major payload [rows][groups][28] -> [block][tile][chunk][lane] x 16 B,
// zero-padded (a padded group has d = 0).  One thread per (row, block, 16 B chunk).
__global__ void tl1_repack_kernel(const uint8_t *raw, uint4 *dst, int out_len, int groups, int nb, int ntiles) {
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    const long long total = static_cast<long long>(nb) * ntiles * 64 * kChunks;
    if (i >= total) return;
    const int lane = static_cast<int>(i % 64);
    const int c = static_cast<int>((i / 64) % kChunks);
    const long long bt = i / (64 * kChunks);
    const int tile = static_cast<int>(bt % ntiles), b = static_cast<int>(bt / ntiles);
    const int row = tile * 64 + lane;
    uint32_t w[4] = {0, 0, 0, 0};
    if (row < out_len) {
        const long long rb = static_cast<long long>(groups) * 28;
        for (int k = 0; k < 16; ++k) {
            const int off = c * 16 + k;          // byte within the block's 112
            const int g = b * kGB + off / 28;   // group
            if (g < groups) {
                const uint32_t v = raw[row * rb + static_cast<long long>(g) * 28 + off % 28];
                w[k / 4] |= v << (8 * (k % 4));
            }
        }
    }
    dst[i] = make_uint4(w[0], w[1], w[2], w[3]);
}

// One group block per blockIdx.y; waves walk row tiles.  RAW = 0 reads the
// repacked layout; RAW = 16, 8 or 4 reads the reference's row-major payload
// itself (matvec_q on device bytes), the 112 bytes of a lane's row block as
// RAW-byte loads (the widest the row pitch groups * 28 keeps aligned).
template <int RAW>
__global__ __launch_bounds__(kThreads) void tl1_lut_kernel(const uint4 *w, const float *x, float *partial,
                                                           int out_len, int groups, int ntiles) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float *T = lds;               // [g][b][256]
    float *xs = lds + kTable;     // [g * 128]
    const int b = blockIdx.y;
    const int gcnt = min(kGB, groups - b * kGB);
    const int tid = threadIdx.x;
    for (int i = tid; i < gcnt * 128; i += kThreads) xs[i] = x[b * kGB * 128 + i];
    __syncthreads();
    // thread (g = tid / 256, v = tid % 256) decodes byte value v once and
    // fills T[g][bb][v] for the 26 byte positions (x reads are broadcasts)
    static_assert(kThreads == kGB * 256, "one thread per (group, byte value)");
    {
        const int v = tid & 255, g = tid >> 8;
        if (g < gcnt) {
            float tr[5];
            uint32_t p3 = 1;
#pragma unroll
            for (int n = 0; n < 5; ++n, p3 *= 3) tr[n] = static_cast<float>(tl1_trit(static_cast<uint32_t>(v), p3));
            const float *xg = xs + g * 128;
            float *Tg = T + g * 26 * 256 + v;
#pragma unroll
            for (int bb = 0; bb < 26; ++bb) {
                const int base = bb < 16 ? bb : bb < 24 ? 80 + (bb - 16) : 120 + (bb - 24);
                const int stride = bb < 16 ? 16 : bb < 24 ? 8 : 2;
                float s = 0.f;
#pragma unroll
                for (int n = 0; n < (bb < 24 ? 5 : 4); ++n) s += tr[n] * xg[base + n * stride];
                Tg[bb * 256] = s;
            }
        }
    }
    __syncthreads();

    const int lane = tid & 63;
    const int wglobal = blockIdx.x * (kThreads / 64) + (tid >> 6);
    const int wstride = gridDim.x * (kThreads / 64);
    const uint4 *wb = w + static_cast<long long>(b) * ntiles * kChunks * 64;
    float *pb = partial + static_cast<long long>(b) * out_len;
    // a wave keeps the 112-byte rows of its next kAhead tiles in flight
    // while it looks up the current one
    uint4 nx[kAhead][kChunks];
    auto load_tile = [&](uint4 (&dst)[kChunks], int tile) {
        if constexpr (RAW == 0) {
            const uint4 *src = wb + static_cast<long long>(tile) * kChunks * 64 + lane;
#pragma unroll
            for (int c = 0; c < kChunks; ++c) dst[c] = src[c * 64];
        } else {
            // row-major: this lane's row, bytes b*112 .. b*112 + 28*gcnt - 1
            // (rows past the end read the last row and are never stored)
            const int row = min(tile * 64 + lane, out_len - 1);
            const uint8_t *src = reinterpret_cast<const uint8_t *>(w) + static_cast<long long>(row) * groups * 28 +
                                 static_cast<long long>(b) * kGB * 28;
            uint32_t u[kChunks * 4];
            constexpr int kW = RAW / 4;  // words per load
#pragma unroll
            for (int i = 0; i < kChunks * 4; i += kW) {
                if (i * 4 < gcnt * 28) {
                    if constexpr (kW == 4) {
                        const uint4 t = *reinterpret_cast<const uint4 *>(src + 4 * i);
                        u[i] = t.x, u[i + 1] = t.y, u[i + 2] = t.z, u[i + 3] = t.w;
                    } else if constexpr (kW == 2) {
                        const uint2 t = *reinterpret_cast<const uint2 *>(src + 4 * i);
                        u[i] = t.x, u[i + 1] = t.y;
                    } else {
                        u[i] = *reinterpret_cast<const uint32_t *>(src + 4 * i);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < kW; ++j) u[i + j] = 0u;
                }
            }
#pragma unroll
            for (int c = 0; c < kChunks; ++c) dst[c] = make_uint4(u[4 * c], u[4 * c + 1], u[4 * c + 2], u[4 * c + 3]);
        }
    };
#pragma unroll
    for (int a = 0; a < kAhead; ++a)
        if (wglobal + a * wstride < ntiles) load_tile(nx[a], wglobal + a * wstride);
    for (int tile0 = wglobal; tile0 < ntiles; tile0 += kAhead * wstride) {
#pragma unroll
        for (int a = 0; a < kAhead; ++a) {
            const int tile = tile0 + a * wstride;  // wave-uniform
            if (tile >= ntiles) break;
            uint32_t u[kChunks * 4];
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                u[4 * c] = nx[a][c].x, u[4 * c + 1] = nx[a][c].y, u[4 * c + 2] = nx[a][c].z,
                u[4 * c + 3] = nx[a][c].w;
            }
            if (tile + kAhead * wstride < ntiles) load_tile(nx[a], tile + kAhead * wstride);
            float acc = 0.f;
#pragma unroll
            for (int g = 0; g < kGB; ++g) {
                if (g < gcnt) {
                    const float *Tg = T + g * 26 * 256;
                    float gs = 0.f;
#pragma unroll
                    for (int bb = 0; bb < 26; ++bb) {
                        const int by = g * 28 + bb;  // byte within the row's 112
                        const uint32_t v = (u[by >> 2] >> (8 * (by & 3))) & 0xffu;
                        gs += Tg[bb * 256 + v];
                    }
                    const uint32_t dw = u[(g * 28 + 24) >> 2] >> 16;  // bytes 26, 27 of the group
                    const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(dw)));
                    acc += d * gs;
                }
            }
            const int row = tile * 64 + lane;
            if (row < out_len) pb[row] = acc;
        }
    }
}

// The same lookups on the reference's row-major payload when a row's group
// blocks are 16-byte aligned (groups % 4 == 0): each wave stages a tile of
// 64 rows x 112 bytes through its own LDS region so the loads stay
// coalesced -- load k of the tile has lane 7j + c read 16-byte chunk c of
// row 9k + j (63 lanes, nine 112-byte row segments per instruction), which
// lands at byte 16 * (63k + lane) of the staging; then lane r reads row r's
// 112 bytes back (both access patterns are bank-conflict free) and looks
// them up exactly as above.  The next tile's loads are in flight during the
// lookups.  Eight waves: the table and 8 x 7 KiB of staging fill the 160 KiB
// of LDS, so x is read from global memory (L1/L2 broadcasts) in the build.
// (Measured alternatives, on 248320x5120: one row per lane read straight
// from global memory, 113 us; 16 waves staging 32-row tiles with a row's
// groups split over lanes l and l ^ 32, 144 us; this one 100 us; the
// repacked layout of a resident weight, 61 us.)
typedef unsigned v4u __attribute__((ext_vector_type(4)));
constexpr int kRawThreads = 512;
constexpr int kRawStage = 64 * kGB * 28;                              // bytes per wave
constexpr int RAW_LDS = kTable * 4 + (kRawThreads / 64) * kRawStage;  // 163840

// Orders a wave's LDS accesses across lanes: LDS executes one wave's
// instructions in issue order, so only the compiler must not move them
// across this point (a memory fence here would also wait for the global
// loads of the next tile that are meant to stay in flight).
__device__ __forceinline__ void wave_sync() { __builtin_amdgcn_wave_barrier(); }

__global__ __launch_bounds__(kRawThreads) void tl1_lut_raw_kernel(const uint8_t *w, const float *x, float *partial,
                                                                  int out_len, int groups, int ntiles) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float *T = lds;  // [g][b][256]
    const int tid = threadIdx.x;
    const int b = blockIdx.y;  // groups % 4 == 0: every block has kGB groups
    uint8_t *stage = reinterpret_cast<uint8_t *>(lds + kTable) + (tid >> 6) * kRawStage;
    for (int p = tid; p < kGB * 256; p += kRawThreads) {  // (group, byte value) pairs
        const int v = p & 255, g = p >> 8;
        float tr[5];
        uint32_t p3 = 1;
#pragma unroll
        for (int n = 0; n < 5; ++n, p3 *= 3) tr[n] = static_cast<float>(tl1_trit(static_cast<uint32_t>(v), p3));
        const float *xg = x + (b * kGB + g) * 128;
        float *Tg = T + g * 26 * 256 + v;
#pragma unroll
        for (int bb = 0; bb < 26; ++bb) {
            const int base = bb < 16 ? bb : bb < 24 ? 80 + (bb - 16) : 120 + (bb - 24);
            const int stride = bb < 16 ? 16 : bb < 24 ? 8 : 2;
            float s = 0.f;
#pragma unroll
            for (int n = 0; n < (bb < 24 ? 5 : 4); ++n) s += tr[n] * xg[base + n * stride];
            Tg[bb * 256] = s;
        }
    }
    __syncthreads();

    const int lane = tid & 63;
    const int j = lane / 7, cc = lane - 7 * j;  // loading: row 9k + j of the tile, 16-byte chunk cc
    const int wglobal = blockIdx.x * (kRawThreads / 64) + (tid >> 6);
    const int wstride = gridDim.x * (kRawThreads / 64);
    const long long rowb = static_cast<long long>(groups) * 28;
    const uint8_t *wb = w + static_cast<long long>(b) * kGB * 28 + 16 * cc;
    float *pb = partial + static_cast<long long>(b) * out_len;
    v4u ld[8];  // native vectors: an array of uint4 structs would live in scratch memory
    auto load_tile = [&](int tile) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int row = min(tile * 64 + 9 * k + j, out_len - 1);  // rows past the end: never stored
            ld[k] = *reinterpret_cast<const v4u *>(wb + row * rowb);
        }
    };
    if (wglobal < ntiles) load_tile(wglobal);
    for (int tile = wglobal; tile < ntiles; tile += wstride) {  // wave-uniform
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (lane < 63 && 9 * k + j < 64) *reinterpret_cast<v4u *>(stage + 16 * (63 * k + lane)) = ld[k];
        wave_sync();
        if (tile + wstride < ntiles) load_tile(tile + wstride);
        uint32_t u[kChunks * 4];
#pragma unroll
        for (int q = 0; q < kChunks; ++q) {
            const v4u t = *reinterpret_cast<const v4u *>(stage + 112 * lane + 16 * q);
            u[4 * q] = t[0], u[4 * q + 1] = t[1], u[4 * q + 2] = t[2], u[4 * q + 3] = t[3];
        }
        wave_sync();  // the staging is free for the next tile
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < kGB; ++g) {
            const float *Tg = T + g * 26 * 256;
            float gs = 0.f;
#pragma unroll
            for (int bb = 0; bb < 26; ++bb) {
                const int by = g * 28 + bb;
                const uint32_t v = (u[by >> 2] >> (8 * (by & 3))) & 0xffu;
                gs += Tg[bb * 256 + v];
            }
            const uint32_t dw = u[(g * 28 + 24) >> 2] >> 16;  // bytes 26, 27 of the group
            const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(dw)));
            acc += d * gs;
        }
        const int row = tile * 64 + lane;
        if (row < out_len) pb[row] = acc;
    }
}

// y[r] = sum over blocks of partial[b][r], blocks in order; with ARGMAX the
// finite_argmax of y is reduced on the way (few workgroups: one atomic each).
template <bool ARGMAX>
__global__ __launch_bounds__(256) void tl1_sum_kernel(const float *partial, float *y, int out_len, int nb,
                                                      unsigned long long *keys) {
    unsigned long long k = 0;
    for (int r = blockIdx.x * 256 + threadIdx.x; r < out_len; r += gridDim.x * 256) {
        float s = 0.f;
        for (int b = 0; b < nb; ++b) s += partial[static_cast<long long>(b) * out_len + r];
        y[r] = s;
        if (ARGMAX) k = argmax_key_max(k, argmax_key(s, static_cast<unsigned>(r)));
    }
    if (ARGMAX) {
        k = argmax_block_key(k);
        if (threadIdx.x == 0) keys[blockIdx.x] = k;
    }
}

}  // namespace

size_t tl1_lut_bytes(size_t out_len, size_t in_len) {
    const size_t groups = in_len / 128, nb = (groups + kGB - 1) / kGB, ntiles = (out_len + 63) / 64;
    return nb * ntiles * 64 * kChunks * 16;
}

size_t tl1_lut_partial_floats(size_t out_len, size_t in_len) {
    const size_t groups = in_len / 128, nb = (groups + kGB - 1) / kGB;
    return nb * out_len;
}

int tl1_repack(const uint8_t *raw, size_t out_len, size_t in_len, void *dst, void *stream) {
    const size_t groups = in_len / 128, nb = (groups + kGB - 1) / kGB, ntiles = (out_len + 63) / 64;
    const size_t total = nb * ntiles * 64 * kChunks;
    hipLaunchKernelGGL(tl1_repack_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                       as_stream(stream), raw, static_cast<uint4 *>(dst), static_cast<int>(out_len),
                       static_cast<int>(groups), static_cast<int>(nb), static_cast<int>(ntiles));
    return check_launch("tl1_repack_kernel");
}

// raw: 0 for the repacked layout, else the payload is the reference's
// row-major bytes (4-byte aligned).
int tl1_lut_matvec(const void *packed, size_t out_len, size_t in_len, const float *x, float *y, float *partial,
                   void *amax_scratch, int32_t *idx, void *stream, int raw) {
    const int groups = static_cast<int>(in_len / 128), nb = (groups + kGB - 1) / kGB;
    // the widest load the row pitch (groups * 28 bytes) and the base keep aligned
    const uintptr_t base = reinterpret_cast<uintptr_t>(packed);
    const int width = !raw ? 0 : (groups % 4 == 0 && base % 16 == 0) ? 16 : (groups % 2 == 0 && base % 8 == 0) ? 8 : 4;
    void (*kern)(const uint4 *, const float *, float *, int, int, int) =
        width == 0 ? tl1_lut_kernel<0> : width == 8 ? tl1_lut_kernel<8> : tl1_lut_kernel<4>;
    const bool staged = width == 16;  // coalesced loads through LDS staging
    static bool attr[4] = {false, false, false, false};
    const int ai = width == 0 ? 0 : width == 16 ? 1 : width == 8 ? 2 : 3;
    const int lds_bytes = staged ? RAW_LDS : LUT_LDS;
    if (!attr[ai]) {
        const void *f = staged ? reinterpret_cast<const void *>(tl1_lut_raw_kernel) : reinterpret_cast<const void *>(kern);
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes) != hipSuccess)
            return fail(OURO_ERR_HIP, "tl1 lut: %d B of LDS refused", lds_bytes);
        attr[ai] = true;
    }
    const int ntiles = static_cast<int>((out_len + 63) / 64);
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    // at most one workgroup per CU in all (LDS holds one): a grid larger than
    // the CU count would run a second round on a few CUs
    const int wpb = (staged ? kRawThreads : kThreads) / 64;
    int gx = cus / nb;
    gx = std::max(1, std::min(gx, (ntiles + wpb - 1) / wpb));
    hipStream_t s = as_stream(stream);
    if (staged)
        hipLaunchKernelGGL(tl1_lut_raw_kernel, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(nb)),
                           dim3(kRawThreads), RAW_LDS, s, static_cast<const uint8_t *>(packed), x, partial,
                           static_cast<int>(out_len), groups, ntiles);
    else
        hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(nb)), dim3(kThreads), LUT_LDS,
                           s, static_cast<const uint4 *>(packed), x, partial, static_cast<int>(out_len), groups,
                           ntiles);
    int st = check_launch("tl1_lut_kernel");
    if (st) return st;
    if (!idx) {
        hipLaunchKernelGGL(tl1_sum_kernel<false>, dim3(static_cast<unsigned>((out_len + 255) / 256)), dim3(256), 0, s,
                           partial, y, static_cast<int>(out_len), nb, nullptr);
        return check_launch("tl1_sum_kernel");
    }
    auto *keys = static_cast<unsigned long long *>(amax_scratch);
    const int blocks = static_cast<int>(std::min<size_t>((out_len + 255) / 256, kArgmaxBlocks));
    hipLaunchKernelGGL(tl1_sum_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, partial, y,
                       static_cast<int>(out_len), nb, keys);
    st = check_launch("tl1_sum_kernel");
    if (st) return st;
    return argmax_final(keys, blocks, idx, stream);
}

}  // namespace ouro
