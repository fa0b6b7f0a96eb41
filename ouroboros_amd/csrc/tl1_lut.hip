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
#include <atomic>

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

// Table slot of byte value v: v ^ (v >> 6), a bijection on 0..255.  A table
// row is 256 floats, so values that agree in their low six bits share an
// LDS bank; payloads whose rows are correlated (the lm_head probe payload of
// ops.rs:694-717 has bytes (i ^ i >> 13) * 0x9E, even and equal mod 32 down
// a column) put most lanes of a lookup on a few banks.  Folding the top two
// bits into the bottom two spreads such values over four banks; on random
// bytes it changes nothing.
__device__ __forceinline__ uint32_t tl1_slot(uint32_t v) { return v ^ (v >> 6); }
// The same on the bytes of a word that carry trits (mask 0x03 per trit byte;
// the group's f16 scale bytes keep their value).
__device__ __forceinline__ uint32_t tl1_slot4(uint32_t w, uint32_t mask) { return w ^ ((w >> 6) & mask); }
// Trit-byte mask of word i of a row's 28-byte group (word 6 holds trit
// bytes 24, 25 and the scale bytes 26, 27).
__host__ __device__ constexpr uint32_t tl1_word_mask(int i) { return i % 7 == 6 ? 0x00000303u : 0x03030303u; }

// Raw row-major payload [rows][groups][28] -> [block][tile][chunk][lane] x 16 B,
// trit bytes replaced by their table slots, zero-padded (a padded group has
// d = 0).  One thread per (row, block, 16 B chunk).
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
                uint32_t v = raw[row * rb + static_cast<long long>(g) * 28 + off % 28];
                if (off % 28 < 26) v = tl1_slot(v);  // trit bytes; 26, 27 are the scale
                w[k / 4] |= v << (8 * (k % 4));
            }
        }
    }
    dst[i] = make_uint4(w[0], w[1], w[2], w[3]);
}

// One group block per blockIdx.y; waves walk row tiles of the repacked layout.
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
            float *Tg = T + g * 26 * 256 + tl1_slot(static_cast<uint32_t>(v));
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
        const uint4 *src = wb + static_cast<long long>(tile) * kChunks * 64 + lane;
#pragma unroll
        for (int c = 0; c < kChunks; ++c) dst[c] = src[c * 64];
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

// The same lookups on the reference's row-major payload (matvec_q on device
// bytes, 4-byte aligned).  Lane 4j + g of a wave owns group g of the block
// for row 16k + j of a 64-row tile: it reads the group's 28 bytes as one
// 16-byte and one 12-byte load (dword-aligned; the 16 rows of a load are
// 16 contiguous 112-byte segments), looks up its 26 trit bytes, scales by
// the group's own f16 d, and the four lanes of a row add their products
// with two DPP quad swaps.  No byte leaves the lane that loaded it, so the
// weights need no LDS staging and every lookup instruction has 64 live
// lanes.  Each group's table starts 16 banks after the previous one, so the
// four groups of a lookup spread over the banks.  The next tile's loads are
// in flight during the lookups.
// A block's 112-byte segments share 128-byte lines with the neighbouring
// blocks' segments, so the workgroups of all blocks of one set of tiles are
// placed on one XCD (workgroup i runs on XCD i mod 8) and read those lines
// through one L2: reading the 248320x5120 payload in this pattern alone
// takes 45 us that way and 76 us with the blocks spread over XCDs.
// (Measured alternatives, on 248320x5120: one row per lane, its 112 bytes
// read straight from global memory, 113 us; whole rows staged through LDS
// per wave, 92-96 us; this kernel with the blocks on different XCDs, 92 us;
// the repacked layout of a resident weight, 55-62 us.)
typedef unsigned v4a __attribute__((ext_vector_type(4), aligned(4)));
typedef unsigned v3a __attribute__((ext_vector_type(3), aligned(4)));
constexpr int kRawThreads = 1024;
constexpr int kGStride = 26 * 256 + 16;  // floats per group table
constexpr int RAW_LDS = kGB * kGStride * 4;
constexpr int kXcds = 8;  // MI355X: workgroup i of a launch runs on XCD i mod 8

template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// 1D grid of kXcds * per_xcd * nb workgroups: workgroup i is block
// (i / kXcds) % nb of tile set (i % kXcds) * per_xcd + i / (kXcds * nb).
__global__ __launch_bounds__(kRawThreads) void tl1_lut_raw_kernel(const uint8_t *w, const float *x, float *partial,
                                                                  int out_len, int groups, int ntiles, int nb,
                                                                  int per_xcd) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x;
    const int slot = blockIdx.x / kXcds;
    const int b = slot % nb;
    const int set = (blockIdx.x % kXcds) * per_xcd + slot / nb;
    const int gcnt = min(kGB, groups - b * kGB);
    static_assert(kRawThreads == kGB * 256, "one thread per (group, byte value)");
    {
        const int v = tid & 255, g = tid >> 8;
        if (g < gcnt) {
            float tr[5];
            uint32_t p3 = 1;
#pragma unroll
            for (int n = 0; n < 5; ++n, p3 *= 3) tr[n] = static_cast<float>(tl1_trit(static_cast<uint32_t>(v), p3));
            const float *xg = x + (b * kGB + g) * 128;
            float *Tg = lds + g * kGStride + tl1_slot(static_cast<uint32_t>(v));
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
    const int j = lane >> 2, g = lane & 3;
    const bool live = g < gcnt;  // lanes past a short last block load group 0 and add nothing
    const int wglobal = set * (kRawThreads / 64) + (tid >> 6);
    const int wstride = kXcds * per_xcd * (kRawThreads / 64);
    const long long rowb = static_cast<long long>(groups) * 28;
    const uint8_t *wb = w + static_cast<long long>(b * kGB + (live ? g : 0)) * 28;
    const float *Tg = lds + g * kGStride;
    float *pb = partial + static_cast<long long>(b) * out_len;
    v4a ld4[4];
    v3a ld3[4];
    auto load_tile = [&](int tile) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int row = min(tile * 64 + 16 * k + j, out_len - 1);  // rows past the end: never stored
            const uint8_t *p = wb + row * rowb;
            // ordinary loads: the lines this block shares with its neighbours
            // must stay in L2 for them (non-temporal loads: 65 -> 117 us)
            ld4[k] = *reinterpret_cast<const v4a *>(p);
            ld3[k] = *reinterpret_cast<const v3a *>(p + 16);
        }
    };
    if (wglobal < ntiles) load_tile(wglobal);
    for (int tile = wglobal; tile < ntiles; tile += wstride) {  // wave-uniform
        uint32_t u[4][7];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            u[k][0] = ld4[k][0], u[k][1] = ld4[k][1], u[k][2] = ld4[k][2], u[k][3] = ld4[k][3];
            u[k][4] = ld3[k][0], u[k][5] = ld3[k][1], u[k][6] = ld3[k][2];
        }
        if (tile + wstride < ntiles) load_tile(tile + wstride);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int i = 0; i < 7; ++i) u[k][i] = tl1_slot4(u[k][i], tl1_word_mask(i));
            float gs = 0.f;
#pragma unroll
            for (int bb = 0; bb < 26; ++bb) {
                const uint32_t v = (u[k][bb >> 2] >> (8 * (bb & 3))) & 0xffu;
                gs += Tg[bb * 256 + v];
            }
            const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u[k][6] >> 16)));
            float part = live ? d * gs : 0.f;
            part += quad_perm<0xB1>(part);  // lanes [1,0,3,2] of each quad
            part += quad_perm<0x4E>(part);  // lanes [2,3,0,1]
            const int row = tile * 64 + 16 * k + j;
            if (g == 0 && row < out_len) pb[row] = part;
        }
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

// ---------------------------------------------------------------------------
// TQ1_0 (dequant.rs:49-105, ggml's block_tq1_0) by the same table lookups,
// on the raw row-major payload (matvec_q on device bytes).  A 256-element
// block is 54 bytes: qs[0..32] hold elements m + 32n, qs[32..48] elements
// 160 + m + 16n (n = 0..4), qh[0..4] elements 240 + m + 4n (n = 0..3), then
// the f16 d; a byte's digits decode as TL1's.  A workgroup takes a pair of
// blocks (two tables of 52 positions x 256 values, 104 KiB; the second
// starts 16 banks after the first).  Lane 2j + g owns block g of the pair for
// row 32k + j of a 64-row tile: it reads the block as 14 dwords (an odd
// block starts 2 bytes past a dword, so it reads from 2 bytes earlier and
// realigns with one funnel shift per word), looks up its 52 trit bytes,
// scales by its own d, and the pair of lanes adds with one DPP swap.  Needs
// an even block count per row (so every pair is whole and every row starts
// on a dword) and a 4-byte-aligned payload.  Workgroups of one tile set sit
// on one XCD, as for TL1.
constexpr int kTqPos = 52;
constexpr int kTqGStride = kTqPos * 256 + 16;  // floats per block table
constexpr int TQ_LDS = 2 * kTqGStride * 4;
typedef unsigned v2a __attribute__((ext_vector_type(2), aligned(4)));

__global__ __launch_bounds__(kRawThreads) void tq1_lut_raw_kernel(const uint8_t *w, const float *x, float *partial,
                                                                  int out_len, int blocks, int ntiles, int npairs,
                                                                  int per_xcd) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x;
    const int slot = blockIdx.x / kXcds;
    const int pr = slot % npairs;  // block pair
    const int set = (blockIdx.x % kXcds) * per_xcd + slot / npairs;
    static_assert(kRawThreads == 4 * 256, "one thread per (block, byte value, half of the positions)");
    {
        const int v = tid & 255, g = (tid >> 8) & 1, half = tid >> 9;  // g and half are wave-uniform
        float tr[5];
        uint32_t p3 = 1;
#pragma unroll
        for (int n = 0; n < 5; ++n, p3 *= 3) tr[n] = static_cast<float>(tl1_trit(static_cast<uint32_t>(v), p3));
        const float *xg = x + (2 * pr + g) * 256;
        float *Tg = lds + g * kTqGStride + tl1_slot(static_cast<uint32_t>(v));
#pragma unroll
        for (int bb = 0; bb < kTqPos; ++bb) {
            if ((bb >= kTqPos / 2) != (half == 1)) continue;
            const int base = bb < 32 ? bb : bb < 48 ? 160 + (bb - 32) : 240 + (bb - 48);
            const int stride = bb < 32 ? 32 : bb < 48 ? 16 : 4;
            float s = 0.f;
#pragma unroll
            for (int n = 0; n < (bb < 48 ? 5 : 4); ++n) s += tr[n] * xg[base + n * stride];
            Tg[bb * 256] = s;
        }
    }
    __syncthreads();

    const int lane = tid & 63;
    const int j = lane >> 1, g = lane & 1;
    const int wglobal = set * (kRawThreads / 64) + (tid >> 6);
    const int wstride = kXcds * per_xcd * (kRawThreads / 64);
    const long long rowb = static_cast<long long>(blocks) * 54;
    const uint8_t *wb = w + static_cast<long long>(2 * pr + g) * 54 - 2 * g;  // dword-aligned
    const float *Tg = lds + g * kTqGStride;
    float *pb = partial + static_cast<long long>(pr) * out_len;
    v4a l0[2], l1[2], l2[2];
    v2a l3[2];
    auto load_tile = [&](int tile) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int row = min(tile * 64 + 32 * k + j, out_len - 1);  // rows past the end: never stored
            const uint8_t *p = wb + row * rowb;
            l0[k] = *reinterpret_cast<const v4a *>(p);  // ordinary loads, as for TL1
            l1[k] = *reinterpret_cast<const v4a *>(p + 16);
            l2[k] = *reinterpret_cast<const v4a *>(p + 32);
            l3[k] = *reinterpret_cast<const v2a *>(p + 48);
        }
    };
    if (wglobal < ntiles) load_tile(wglobal);
    for (int tile = wglobal; tile < ntiles; tile += wstride) {  // wave-uniform
        uint32_t wd[2][14];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
#pragma unroll
            for (int i = 0; i < 4; ++i) wd[k][i] = l0[k][i], wd[k][4 + i] = l1[k][i], wd[k][8 + i] = l2[k][i];
            wd[k][12] = l3[k][0], wd[k][13] = l3[k][1];
        }
        if (tile + wstride < ntiles) load_tile(tile + wstride);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            uint32_t u[13];
#pragma unroll
            for (int i = 0; i < 13; ++i) {
                const uint32_t t = g ? __builtin_amdgcn_alignbit(wd[k][i + 1], wd[k][i], 16) : wd[k][i];
                u[i] = tl1_slot4(t, 0x03030303u);
            }
            const uint32_t dbits = g ? (wd[k][13] >> 16) : (wd[k][13] & 0xffffu);
            float gs = 0.f;
#pragma unroll
            for (int bb = 0; bb < kTqPos; ++bb) {
                const uint32_t v = (u[bb >> 2] >> (8 * (bb & 3))) & 0xffu;
                gs += Tg[bb * 256 + v];
            }
            const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(dbits)));
            float part = d * gs;
            part += quad_perm<0xB1>(part);  // lanes [1,0,3,2]: the other block of the pair
            const int row = tile * 64 + 32 * k + j;
            if (g == 0 && row < out_len) pb[row] = part;
        }
    }
}

// y = the sum of the nb block partials; with idx, also its finite_argmax.
static int tl1_sum(const float *partial, float *y, size_t out_len, int nb, void *amax_scratch, int32_t *idx,
                   void *stream) {
    hipStream_t s = as_stream(stream);
    if (!idx) {
        hipLaunchKernelGGL(tl1_sum_kernel<false>, dim3(static_cast<unsigned>((out_len + 255) / 256)), dim3(256), 0, s,
                           partial, y, static_cast<int>(out_len), nb, nullptr);
        return check_launch("tl1_sum_kernel");
    }
    auto *keys = static_cast<unsigned long long *>(amax_scratch);
    const int blocks = static_cast<int>(std::min<size_t>((out_len + 255) / 256, kArgmaxBlocks));
    hipLaunchKernelGGL(tl1_sum_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, partial, y,
                       static_cast<int>(out_len), nb, keys);
    const int st = check_launch("tl1_sum_kernel");
    if (st) return st;
    return argmax_final(keys, blocks, idx, stream);
}

// raw: 0 for the repacked layout, else the payload is the reference's
// row-major bytes (4-byte aligned).
int tl1_lut_matvec(const void *packed, size_t out_len, size_t in_len, const float *x, float *y, float *partial,
                   void *amax_scratch, int32_t *idx, void *stream, int raw) {
    const int groups = static_cast<int>(in_len / 128), nb = (groups + kGB - 1) / kGB;
    // LDS opt-in once per process and kernel (idempotent)
    static std::atomic<bool> attr[2] = {{false}, {false}};
    const int lds_bytes = raw ? RAW_LDS : LUT_LDS;
    if (!attr[raw ? 1 : 0].load(std::memory_order_acquire)) {
        const void *f = raw ? reinterpret_cast<const void *>(tl1_lut_raw_kernel)
                            : reinterpret_cast<const void *>(tl1_lut_kernel);
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes) != hipSuccess)
            return fail(OURO_ERR_HIP, "tl1 lut: %d B of LDS refused", lds_bytes);
        attr[raw ? 1 : 0].store(true, std::memory_order_release);
    }
    const int ntiles = static_cast<int>((out_len + 63) / 64);
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    // at most one workgroup per CU in all (LDS holds one): a grid larger than
    // the CU count would run a second round on a few CUs
    hipStream_t s = as_stream(stream);
    if (raw) {
        const int per_xcd = std::max(1, std::min(cus / kXcds / nb, (ntiles + 16 * kXcds - 1) / (16 * kXcds)));
        hipLaunchKernelGGL(tl1_lut_raw_kernel, dim3(static_cast<unsigned>(kXcds * per_xcd * nb)), dim3(kRawThreads),
                           RAW_LDS, s, static_cast<const uint8_t *>(packed), x, partial, static_cast<int>(out_len),
                           groups, ntiles, nb, per_xcd);
        const int st = check_launch("tl1_lut_raw_kernel");
        if (st) return st;
        return tl1_sum(partial, y, out_len, nb, amax_scratch, idx, stream);
    }
    const int wpb = kThreads / 64;
    int gx = cus / nb;
    gx = std::max(1, std::min(gx, (ntiles + wpb - 1) / wpb));
        hipLaunchKernelGGL(tl1_lut_kernel, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(nb)), dim3(kThreads),
                           LUT_LDS, s, static_cast<const uint4 *>(packed), x, partial, static_cast<int>(out_len),
                           groups, ntiles);
    const int st = check_launch("tl1_lut_kernel");
    if (st) return st;
    return tl1_sum(partial, y, out_len, nb, amax_scratch, idx, stream);
}

size_t tq1_lut_partial_floats(size_t out_len, size_t in_len) { return (in_len / 512) * out_len; }

// The lookup path takes TQ1_0 rows of an even block count on a 4-byte-aligned payload.
bool tq1_lut_fits(const void *payload, size_t in_len) {
    return in_len % 512 == 0 && in_len <= 65536 && reinterpret_cast<uintptr_t>(payload) % 4 == 0;
}

int tq1_lut_matvec(const void *payload, size_t out_len, size_t in_len, const float *x, float *y, float *partial,
                   void *amax_scratch, int32_t *idx, void *stream) {
    const int blocks = static_cast<int>(in_len / 256), npairs = blocks / 2;
    static std::atomic<bool> attr{false};  // LDS opt-in once per process (idempotent)
    if (!attr.load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(tq1_lut_raw_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, TQ_LDS) != hipSuccess)
            return fail(OURO_ERR_HIP, "tq1 lut: %d B of LDS refused", TQ_LDS);
        attr.store(true, std::memory_order_release);
    }
    const int ntiles = static_cast<int>((out_len + 63) / 64);
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int per_xcd = std::max(1, std::min(cus / kXcds / npairs, (ntiles + 16 * kXcds - 1) / (16 * kXcds)));
    hipLaunchKernelGGL(tq1_lut_raw_kernel, dim3(static_cast<unsigned>(kXcds * per_xcd * npairs)), dim3(kRawThreads),
                       TQ_LDS, as_stream(stream), static_cast<const uint8_t *>(payload), x, partial,
                       static_cast<int>(out_len), blocks, ntiles, npairs, per_xcd);
    const int st = check_launch("tq1_lut_raw_kernel");
    if (st) return st;
    return tl1_sum(partial, y, out_len, npairs, amax_scratch, idx, stream);
}

}  // namespace ouro
