// i2_gemv.hip - int8 per-token-absmax activations x 2-bit ternary weights.
//
// The weight stream is the whole cost of a decode GEMV (ops.rs:288-293 says
// the same of the reference's fused decode+dot), so the kernel is built
// around HBM: the device-tiled I2 layout (ouro_hip.h) makes every 16-byte
// load of a 64-lane wavefront one contiguous 1 KiB segment, each lane keeps
// its activation slice in registers for all rows it visits, and 2-bit codes
// are expanded to int8 in registers and consumed by v_dot4_i32_i8.
//
// Activations are bitnet.cpp's I8_S rows (quantize_row_i8_s) and the
// epilogue is its I2_S mul_mat one, y = (acc / s) * w_scale.  Integer
// accumulation is exact in any order and the epilogue is two separately
// rounded operations, so results are bit-identical to the oracle.
#include "common.hpp"

#include <type_traits>

#pragma clang fp contract(off)

namespace ouro {
namespace {

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Tiles are 8 rows.  A lane's share of a tile (8 * G bytes) is stored, and
// read, in units of 16 bytes when G is even and of 8 bytes when G is odd.
constexpr int kTileRows = 8;
__host__ __device__ constexpr int unit_bytes(int G) { return G % 2 ? 8 : 16; }

// The G groups a lane owns in each row are split into chunks of 4 groups,
// then one of 2 (if G % 4 >= 2), then one of 1 (if G is odd).  Chunk c of
// size s starting at lane-local group o covers, for lane l, the k-groups
// 64*o + s*l + (g - o), so the activations of one chunk are a contiguous
// 64*s*4-byte segment read by one coalesced load of s*4 bytes per lane.
__host__ __device__ constexpr int chunk_start(int G, int g) {
    return g < G / 4 * 4 ? g / 4 * 4 : (g < G / 4 * 4 + (G % 4 >= 2 ? 2 : 0) ? G / 4 * 4 : G - 1);
}
__host__ __device__ constexpr int chunk_size(int G, int g) {
    return g < G / 4 * 4 ? 4 : (g < G / 4 * 4 + (G % 4 >= 2 ? 2 : 0) ? 2 : 1);
}
// k-group (canonical byte column) of lane-local group g of lane l.
__host__ __device__ constexpr int kgroup(int G, int l, int g) {
    return 64 * chunk_start(G, g) + chunk_size(G, g) * l + (g - chunk_start(G, g));
}

// ------------------------------------------------------------ tiling --

// One thread per 32-bit word of the tiled layout.  The source is canonical
// codes, or (src_i2s) the codes of a bitnet.cpp I2_S tensor.
__global__ void i2_tile_kernel(const uint8_t *__restrict__ canon, uint32_t *__restrict__ tiled,
                               int out_len, int G, long long total_words, int src_i2s) {
    long long id = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= total_words) return;
    constexpr int R = kTileRows;
    const int wu = unit_bytes(G) / 4;           // words per unit
    const long long tile_words = 16LL * R * G;  // 64 lanes * R*G bytes / 4
    const long long t = id / tile_words;
    const int w = static_cast<int>(id % tile_words);
    const int lane = (w % (64 * wu)) / wu;
    const int d = wu * (w / (64 * wu)) + (w % wu);
    const long long row_bytes = 64LL * G;
    uint32_t word = 0;
#pragma unroll
    for (int f = 0; f < 4; ++f) {
        const int gi = 4 * d + f;
        const int r = gi / G, g = gi % G;
        const long long row = t * R + r;
        uint32_t byte = 0x55;  // padding rows: code 1 (w = 0) everywhere
        if (row < out_len)
            byte = src_i2s ? i2s_canon_byte(canon, row, 256 * G, kgroup(G, lane, g))
                           : canon[row * row_bytes + kgroup(G, lane, g)];
#pragma unroll
        for (int b = 0; b < 4; ++b) word |= ((byte >> (2 * b)) & 3u) << (8 * b + 2 * f);
    }
    tiled[id] = word;
}

__global__ void copy_scale_kernel(const float *src, float *dst) { *dst = *src; }

// ------------------------------------------------------- act quant --

template <typename T>
__device__ __forceinline__ float load_act(const T *p, long long i);
template <>
__device__ __forceinline__ float load_act<float>(const float *p, long long i) { return p[i]; }
template <>
__device__ __forceinline__ float load_act<uint16_t>(const uint16_t *p, long long i) {
    return bf16_bits_to_f32(p[i]);
}

__device__ __forceinline__ float block_max_256(float v, float *red) {
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, xor_shfl(v, off));
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < static_cast<int>(blockDim.x / kWave); ++i) m = fmaxf(m, red[i]);
    __syncthreads();
    return m;
}

// One 256-thread block per row: quantize_row_i8_s (bitnet.cpp), s = 127 /
// max(max|x|, 1e-5), q = clamp(round(x * s), -128, 127).
template <typename T>
__global__ __launch_bounds__(256) void act_quant_kernel(const T *__restrict__ x, long long n,
                                                        int8_t *__restrict__ xq,
                                                        float *__restrict__ act_scale) {
    __shared__ float red[4];
    const long long row = blockIdx.x;
    const T *xr = x + row * n;
    float amax = 0.f;
    for (long long i = threadIdx.x; i < n; i += blockDim.x) amax = fmaxf(amax, fabsf(load_act(xr, i)));
    amax = block_max_256(amax, red);
    int8_t *qr = xq + row * n;
    const float s = i8s_scale(amax);
    for (long long i = threadIdx.x; i < n; i += blockDim.x)
        qr[i] = static_cast<int8_t>(i8s_quant(load_act(xr, i), s));
    if (threadIdx.x == 0) act_scale[row] = s;
}

// ------------------------------------------------------------- GEMV --

struct GemvArgs {
    const uint8_t *w;       // tiled codes of matrix 0
    long long w_stride;     // bytes between matrices
    const float *w_scale;   // per matrix, stride 1
    const int8_t *xq;       // [ncols][in_len] of matrix 0
    long long x_stride;     // elements between matrices
    const float *act_scale;    // [ncols] of matrix 0, per matrix stride ncols
    float *y;               // [ncols][out_len] of matrix 0
    long long y_stride;     // elements between matrices
    int32_t *acc;           // optional, same layout as y (matrix 0 only)
    int out_len, in_len, ncols, tiles;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (88 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(GemvArgs) == 88, "GemvArgs: kernel argument layout");

// Row totals of a tile: each lane holds R partial sums (one per row of the
// tile); row r's total is the sum over the span = 64 / R lanes of group r.
// The first log2(R) lane stages halve the value count (lanes whose stage bit
// is set keep the upper half), the rest add within the span.  Offsets 32 and
// 16 use v_permlane32_swap / v_permlane16_swap (upper 32 lanes of the first
// operand <-> lower 32 of the second; odd 16-lane rows of the first <-> even
// rows of the second), offset 8 a DPP row rotation by 8 (lane L ^ 8), the
// fourth halving (R = 16) a DPP half-row mirror and the in-span tail a DPP
// shift-right scan, so no stage goes through LDS.  On
// return lane L with L % span == span - 1 holds the total of row L / span.
template <int R>
__device__ __forceinline__ int row_totals(int (&v)[R], int lane) {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8 || R == 16, "R is a power of two <= 16");
    constexpr int span = kWave / R;
    // offset 32
    if constexpr (R > 1) {
#pragma unroll
        for (int i = 0; i < R / 2; ++i) {
            const auto p = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v[i]),
                                                            static_cast<unsigned>(v[i + R / 2]), false, false);
            v[i] = static_cast<int>(p[0] + p[1]);
        }
    } else {
        const auto p = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v[0]), static_cast<unsigned>(v[0]),
                                                        false, false);
        v[0] = static_cast<int>(p[0] + p[1]);
    }
    // offset 16
    if constexpr (R > 2) {
#pragma unroll
        for (int i = 0; i < R / 4; ++i) {
            const auto p = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v[i]),
                                                            static_cast<unsigned>(v[i + R / 4]), false, false);
            v[i] = static_cast<int>(p[0] + p[1]);
        }
    } else {
        const auto p = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v[0]), static_cast<unsigned>(v[0]),
                                                        false, false);
        v[0] = static_cast<int>(p[0] + p[1]);
    }
    // offset 8 (row_ror:8 = dpp_ctrl 0x128)
    if constexpr (R > 4) {
        const bool upper = (lane & 8) != 0;
#pragma unroll
        for (int i = 0; i < R / 8; ++i) {
            const int keep = upper ? v[i + R / 8] : v[i];
            const int send = upper ? v[i] : v[i + R / 8];
            v[i] = keep + __builtin_amdgcn_update_dpp(0, send, 0x128, 0xf, 0xf, false);
        }
    }
    // Last halving stage of R = 16: row_half_mirror (0x141) pairs lane L
    // with L ^ 7, whose bit 2 is the opposite one; the partial sums then
    // cover {l, l ^ 7}, and the tail below over each aligned group of four
    // lanes adds up all eight lanes of the half-row.
    if constexpr (R > 8) {
        const bool upper = (lane & 4) != 0;
        const int keep = upper ? v[1] : v[0];
        const int send = upper ? v[0] : v[1];
        v[0] = keep + __builtin_amdgcn_update_dpp(0, send, 0x141, 0xf, 0xf, false);
    }
    // In-span tail: after shift-right steps 1, 2, .., lane L holds the sum
    // of lanes L - s + 1 .. L of its 16-lane row (row_shr:k = 0x110 + k).
    constexpr int tail = span < 16 ? span : 16;
    if constexpr (tail > 1) v[0] += __builtin_amdgcn_update_dpp(0, v[0], 0x111, 0xf, 0xf, false);
    if constexpr (tail > 2) v[0] += __builtin_amdgcn_update_dpp(0, v[0], 0x112, 0xf, 0xf, false);
    if constexpr (tail > 4) v[0] += __builtin_amdgcn_update_dpp(0, v[0], 0x114, 0xf, 0xf, false);
    if constexpr (tail > 8) v[0] += __builtin_amdgcn_update_dpp(0, v[0], 0x118, 0xf, 0xf, false);
    return v[0];
}

// G: 4-weight groups per lane per row; R rows per tile; NC activation
// columns per pass; TPW tiles per wavefront, taken in order with DEPTH of
// them in flight (the load of tile t + DEPTH is issued as soon as tile t
// has been consumed); WPB wavefronts per block.  SPLIT selects how the four
// 2-bit fields of a code byte reach v_dot4_i32_i8:
//   SPLIT = 1: each field shifted down and masked (7 operations per word),
//              one accumulator per row;
//   SPLIT = 2: fields 0 and 2 at scale 1 (w & 0x03.., (w >> 4) & 0x03..),
//              fields 1 and 3 at scale 4 (w & 0x0c.., (w >> 4) & 0x0c..),
//              5 operations per word and two accumulators per row,
//              recombined exactly as s1 + (s4 >> 2) (s4 is a multiple of 4).
template <int G, int NC, int TPW, int DEPTH, int WPB, int SPLIT>
__global__ __launch_bounds__(kWave *WPB) void i2_gemv_kernel(GemvArgs a) {
    constexpr int R = kTileRows;
    constexpr int U = unit_bytes(G);  // bytes per load
    constexpr int WU = U / 4;         // words per load
    constexpr int CHUNK = R * G;      // bytes per lane per tile
    constexpr int NV = CHUNK / U;     // loads per lane per tile
    using unit_t = typename std::conditional<U == 16, u32x4, u32x2>::type;
    static_assert(CHUNK % U == 0, "tile chunk must be whole loads");
    static_assert(DEPTH >= 1 && DEPTH <= TPW, "1 <= DEPTH <= TPW");
    static_assert(SPLIT == 1 || SPLIT == 2, "SPLIT is 1 or 2");

    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int mat = blockIdx.z;
    const int c0 = blockIdx.y * NC;
    const int tile0 = (blockIdx.x * WPB + wave) * TPW;
    if (tile0 >= a.tiles) return;  // whole wavefront leaves together

    const uint8_t *w = a.w + mat * a.w_stride;
    const int8_t *xq = a.xq + mat * a.x_stride;
    const float *act_scale = a.act_scale + static_cast<long long>(mat) * a.ncols;
    float *y = a.y + mat * a.y_stride;
    const float wscale = a.w_scale[mat];

    // Tiles past the end are loaded from tile0 (in bounds) and never used.
    // The weights are read once: non-temporal loads (on the 1.14 GB stream of
    // 256 matrices 6.26 -> 6.98 TB/s).
    unit_t buf[DEPTH][NV];
    auto load_tile = [&](int t, unit_t(&dst)[NV]) {
        const int tile = tile0 + t;
        const unit_t *tp = reinterpret_cast<const unit_t *>(
            w + static_cast<long long>(tile < a.tiles ? tile : tile0) * (R * 64 * G));
#pragma unroll
        for (int j = 0; j < NV; ++j) dst[j] = __builtin_nontemporal_load(&tp[j * kWave + lane]);
    };
#pragma unroll
    for (int t = 0; t < DEPTH; ++t) load_tile(t, buf[t]);

    // Activation groups of this lane (kgroup order): one 16-, 8- or 4-byte
    // load per chunk.
    uint32_t xw[NC][G];
    int sx[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        sx[c] = 0;
        const bool live = c0 + c < a.ncols;
        const uint32_t *xr = reinterpret_cast<const uint32_t *>(xq + static_cast<long long>(c0 + c) * a.in_len);
        constexpr int N4 = G / 4 * 4;  // groups in chunks of 4
#pragma unroll
        for (int g = 0; g < N4; g += 4) {
            const u32x4 v = live ? *reinterpret_cast<const u32x4 *>(xr + kgroup(G, lane, g)) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 4; ++i) xw[c][g + i] = v[i];
        }
        if constexpr (G % 4 >= 2) {
            const u32x2 v = live ? *reinterpret_cast<const u32x2 *>(xr + kgroup(G, lane, N4)) : u32x2{0u, 0u};
            xw[c][N4] = v[0];
            xw[c][N4 + 1] = v[1];
        }
        if constexpr (G % 2) xw[c][G - 1] = live ? xr[kgroup(G, lane, G - 1)] : 0u;
#pragma unroll
        for (int g = 0; g < G; ++g)
            sx[c] = __builtin_amdgcn_sdot4(static_cast<int>(xw[c][g]), 0x01010101, sx[c], false);
    }

#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int tile = tile0 + t;
        if (tile >= a.tiles) break;  // uniform across the wavefront
        unit_t(&cur)[NV] = buf[t % DEPTH];
        int s1[NC][R], s4[NC][R];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                s1[c][r] = -sx[c];  // codes are w + 1
                s4[c][r] = 0;
            }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
#pragma unroll
            for (int q = 0; q < WU; ++q) {
                const int d = WU * j + q;
                const uint32_t word = cur[j][q];
                const uint32_t hi = word >> 4;
                int fields[4];
                if constexpr (SPLIT == 2) {
                    fields[0] = static_cast<int>(word & 0x03030303u);
                    fields[1] = static_cast<int>(word & 0x0c0c0c0cu);
                    fields[2] = static_cast<int>(hi & 0x03030303u);
                    fields[3] = static_cast<int>(hi & 0x0c0c0c0cu);
                } else {
#pragma unroll
                    for (int f = 0; f < 4; ++f) fields[f] = static_cast<int>((word >> (2 * f)) & 0x03030303u);
                }
#pragma unroll
                for (int f = 0; f < 4; ++f) {
                    const int gi = 4 * d + f;
                    const int r = gi / G, g = gi % G;
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        const int xv = static_cast<int>(xw[c][g]);
                        if (SPLIT == 2 && (f & 1))
                            s4[c][r] = __builtin_amdgcn_sdot4(fields[f], xv, s4[c][r], false);
                        else
                            s1[c][r] = __builtin_amdgcn_sdot4(fields[f], xv, s1[c][r], false);
                    }
                }
            }
        }
        if (t + DEPTH < TPW) load_tile(t + DEPTH, cur);  // the slot is free again
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            int acc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = SPLIT == 2 ? s1[c][r] + (s4[c][r] >> 2) : s1[c][r];
            const int total = row_totals<R>(acc, lane);
            constexpr int span = kWave / R;
            const int row = tile * R + lane / span;
            if (lane % span == span - 1 && row < a.out_len && c0 + c < a.ncols) {
                const long long o = static_cast<long long>(c0 + c) * a.out_len + row;
                const float v = i8s_out(total, act_scale[c0 + c], wscale);
                y[o] = v;
                if (a.acc) a.acc[o] = total;
            }
        }
    }
}

using GemvFn = void (*)(GemvArgs);

struct GemvPick {
    GemvFn fn;
    int nc, tpw, wpb;
};

constexpr int kGemvWpb = 4;
// Enough wavefronts to keep every CU's load pipes busy (256 CUs x 8).
constexpr long long kGemvWaves = 2048;

// One activation column.  Measured on streams of 6912x2560, 2560x6912,
// 4096x4096, 8192x8192 and 248320x5120 matrices: one 8-row tile per
// wavefront in 4-wavefront blocks is the fastest shape, or within 2 % of
// it, for every in_len >= 2048, and clearly the fastest once the stream is
// larger than the last-level cache.  For in_len <= 1024 a tile is at most
// 8 KiB per wavefront and two tiles (both in flight) pay for the fixed
// per-tile cost, when that still leaves kGemvWaves wavefronts.
// Several columns: NC = 4 or 2 with the single-accumulator unpack, NC = 4
// only while 4 * G words of activations fit in 40 registers, NC = 2 while
// 2 * G fit in 64.
template <int G>
GemvPick pick_g(int ncols, long long total_tiles) {
    if constexpr (4 * G <= 40)
        if (ncols >= 4) return {i2_gemv_kernel<G, 4, 1, 1, kGemvWpb, 1>, 4, 1, kGemvWpb};
    if constexpr (2 * G <= 64)
        if (ncols >= 2) return {i2_gemv_kernel<G, 2, 1, 1, kGemvWpb, 1>, 2, 1, kGemvWpb};
    if constexpr (G <= 4)
        if (total_tiles >= 2 * kGemvWaves) return {i2_gemv_kernel<G, 1, 2, 2, kGemvWpb, 2>, 1, 2, kGemvWpb};
    return {i2_gemv_kernel<G, 1, 1, 1, kGemvWpb, 2>, 1, 1, kGemvWpb};
}

GemvPick pick_gemv(int G, int ncols, long long total_tiles) {
    switch (G) {
    case 1: return pick_g<1>(ncols, total_tiles);
    case 2: return pick_g<2>(ncols, total_tiles);
    case 4: return pick_g<4>(ncols, total_tiles);
    case 8: return pick_g<8>(ncols, total_tiles);
    case 10: return pick_g<10>(ncols, total_tiles);
    case 12: return pick_g<12>(ncols, total_tiles);
    case 16: return pick_g<16>(ncols, total_tiles);
    case 20: return pick_g<20>(ncols, total_tiles);
    case 24: return pick_g<24>(ncols, total_tiles);
    case 27: return pick_g<27>(ncols, total_tiles);
    case 32: return pick_g<32>(ncols, total_tiles);
    default: return {nullptr, 0, 0, 0};
    }
}

// ------------------------------------------------------- raw I2_S GEMV --
//
// y = W x straight from a bitnet.cpp I2_S tensor (ouro_matvec_q with
// OURO_KIND_I2_S).  Row r is in_len/4 bytes at r*in_len/4 (in_len % 256 == 0,
// so no 128-block straddles two rows), i.e. in_len/64 chunks of 16 bytes;
// chunk c is half h = c%2 of block c/2, and field f (bits 6-2f) of its word
// w (bytes 4w..4w+3) holds the codes of weights
// k = 128*(c/2) + 32*f + 16*h + 4*w + i (byte i of the word), so every
// field of a word meets four consecutive activations.  Lane l owns chunks
// c = l + 64*s (s < NS) of every row: its activations (one 16-byte load per
// field and chunk) stay in registers while the wavefront reads its 8 rows,
// each row one contiguous in_len/4-byte span.  Lanes past the last chunk read a
// clamped chunk against zero activations.
struct I2sArgs {
    const uint8_t *w;
    const float *w_scale;
    const int8_t *xq;        // [ncols][in_len]
    const float *act_scale;  // [ncols]
    float *y;                // [ncols][out_len]
    int32_t *acc;            // optional, same layout as y
    int out_len, in_len;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (56 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(I2sArgs) == 56, "I2sArgs: kernel argument layout");

constexpr int kI2sWaves = 4;

template <int NS>
__global__ __launch_bounds__(kWave *kI2sWaves) void i2s_gemv_kernel(I2sArgs a) {
    constexpr int R = kTileRows;  // rows per wavefront, reduced as in the tiled GEMV
    const int lane = threadIdx.x % kWave;
    const int row0 = (blockIdx.x * kI2sWaves + static_cast<int>(threadIdx.x / kWave)) * R;
    if (row0 >= a.out_len) return;  // whole wavefront leaves together
    const int col = blockIdx.y;
    const int chunks = a.in_len / 64;
    const int8_t *xr = a.xq + static_cast<long long>(col) * a.in_len;
    u32x4 xv[NS][4];
    int sx = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int c = lane + 64 * s;
        const int cc = c < chunks ? c : chunks - 1;
        const int k0 = 128 * (cc >> 1) + 16 * (cc & 1);
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(xr + k0 + 32 * f);
            xv[s][f] = c < chunks ? v : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                sx = __builtin_amdgcn_sdot4(static_cast<int>(xv[s][f][q]), 0x01010101, sx, false);
        }
    }
    const long long rb = a.in_len / 4;
    int s1[R], s4[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        s1[r] = -sx;  // codes are w + 1
        s4[r] = 0;
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int c = lane + 64 * s;
        const int cc = c < chunks ? c : chunks - 1;
        u32x4 wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + r < a.out_len ? row0 + r : a.out_len - 1;
            wv[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(a.w + row * rb + 16 * cc));
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t word = wv[r][q], hi = word >> 4;
                // fields 0 and 2 masked at scale 4, fields 1 and 3 at scale 1
                s4[r] = __builtin_amdgcn_sdot4(static_cast<int>(hi & 0x0c0c0c0cu), static_cast<int>(xv[s][0][q]), s4[r], false);
                s1[r] = __builtin_amdgcn_sdot4(static_cast<int>(hi & 0x03030303u), static_cast<int>(xv[s][1][q]), s1[r], false);
                s4[r] = __builtin_amdgcn_sdot4(static_cast<int>(word & 0x0c0c0c0cu), static_cast<int>(xv[s][2][q]), s4[r], false);
                s1[r] = __builtin_amdgcn_sdot4(static_cast<int>(word & 0x03030303u), static_cast<int>(xv[s][3][q]), s1[r], false);
            }
    }
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = s1[r] + (s4[r] >> 2);  // s4 is a multiple of 4
    const int total = row_totals<R>(acc, lane);
    constexpr int span = kWave / R;
    const int row = row0 + lane / span;
    if (lane % span == span - 1 && row < a.out_len) {
        const long long o = static_cast<long long>(col) * a.out_len + row;
        a.y[o] = i8s_out(total, a.act_scale[col], *a.w_scale);
        if (a.acc) a.acc[o] = total;
    }
}

int launch_gemv(const GemvArgs &base, int count, void *stream) {
    const int G = base.in_len / 256;
    const int tiles = base.tiles;
    const long long total_tiles = static_cast<long long>(tiles) * count;
    const GemvPick p = pick_gemv(G, base.ncols, total_tiles);
    if (!p.fn) return fail(OURO_ERR_SHAPE, "i2 gemv: in_len %d (G=%d) has no kernel instance", base.in_len, G);
    const int nc = p.nc;
    const int per_block = p.wpb * p.tpw;
    dim3 grid((tiles + per_block - 1) / per_block, (base.ncols + nc - 1) / nc, count);
    if (grid.y > 65535 || grid.z > 65535) return fail(OURO_ERR_SHAPE, "i2 gemv: grid too large");
    hipLaunchKernelGGL(p.fn, grid, dim3(kWave * p.wpb), 0, as_stream(stream), base);
    return check_launch("i2_gemv_kernel");
}

int check_i2_shape(size_t out_len, size_t in_len) {
    if (!out_len || !in_len) return fail(OURO_ERR_SHAPE, "i2: empty shape");
    if (in_len % 256) return fail(OURO_ERR_SHAPE, "i2: in_len %zu is not a multiple of 256", in_len);
    if (out_len > (1u << 30) || in_len > (1u << 20)) return fail(OURO_ERR_SHAPE, "i2: shape too large");
    return OURO_OK;
}

}  // namespace

// Internal entry shared with the matvec_q surface and resident weights.
int i2_gemm(const uint8_t *w_tiled, size_t out_len, size_t in_len, const float *w_scale,
            const int8_t *xq, const float *act_scale, size_t ncols, float *y, int32_t *acc,
            void *stream) {
    int st = check_i2_shape(out_len, in_len);
    if (st) return st;
    if (!w_tiled || !w_scale || !xq || !act_scale || !y || !ncols)
        return fail(OURO_ERR_INVALID_ARG, "ouro_gemm_i2: NULL argument or ncols == 0");
    if (reinterpret_cast<uintptr_t>(w_tiled) % 16 || reinterpret_cast<uintptr_t>(xq) % 16)
        return fail(OURO_ERR_ALIGN, "ouro_gemm_i2: weights and xq need 16-byte alignment");
    constexpr int R = kTileRows;
    GemvArgs a{};
    a.w = w_tiled;
    a.w_stride = 0;
    a.w_scale = w_scale;
    a.xq = xq;
    a.x_stride = 0;
    a.act_scale = act_scale;
    a.y = y;
    a.y_stride = 0;
    a.acc = acc;
    a.out_len = static_cast<int>(out_len);
    a.in_len = static_cast<int>(in_len);
    a.ncols = static_cast<int>(ncols);
    a.tiles = static_cast<int>((out_len + R - 1) / R);
    return launch_gemv(a, 1, stream);
}

int act_quant(const void *x, int x_dtype, size_t rows, size_t n, int8_t *xq, float *act_scale,
              void *stream) {
    if (!x || !xq || !act_scale) return fail(OURO_ERR_INVALID_ARG, "ouro_act_quant_i8: NULL argument");
    if (!rows || !n) return fail(OURO_ERR_SHAPE, "ouro_act_quant_i8: empty shape");
    if (rows > 0x7fffffff) return fail(OURO_ERR_SHAPE, "ouro_act_quant_i8: too many rows");
    dim3 grid(static_cast<unsigned>(rows)), block(256);
    if (x_dtype == OURO_DT_F32)
        hipLaunchKernelGGL(act_quant_kernel<float>, grid, block, 0, as_stream(stream),
                           static_cast<const float *>(x), static_cast<long long>(n), xq, act_scale);
    else if (x_dtype == OURO_DT_BF16)
        hipLaunchKernelGGL(act_quant_kernel<uint16_t>, grid, block, 0, as_stream(stream),
                           static_cast<const uint16_t *>(x), static_cast<long long>(n), xq, act_scale);
    else
        return fail(OURO_ERR_INVALID_ARG, "ouro_act_quant_i8: bad dtype %d", x_dtype);
    return check_launch("act_quant_kernel");
}

size_t i2_tiled_bytes(size_t out_len, size_t in_len) {
    if (!in_len || in_len % 256) return 0;
    const size_t R = kTileRows;
    const size_t tiles = (out_len + R - 1) / R;
    return tiles * R * (in_len / 4);
}

// Tiles canonical codes (src_i2s = 0) or the codes of an I2_S tensor.
int i2_tile(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *tiled,
            const float *w_scale, void *stream, int src_i2s) {
    int st = check_i2_shape(out_len, in_len);
    if (st) return st;
    if (!canonical || !tiled) return fail(OURO_ERR_INVALID_ARG, "ouro_i2_tile: NULL argument");
    if (reinterpret_cast<uintptr_t>(tiled) % 16) return fail(OURO_ERR_ALIGN, "ouro_i2_tile: tiled needs 16-byte alignment");
    const int G = static_cast<int>(in_len / 256);
    const size_t bytes = i2_tiled_bytes(out_len, in_len);
    const long long words = static_cast<long long>(bytes / 4);
    const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
    hipLaunchKernelGGL(i2_tile_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), canonical,
                       reinterpret_cast<uint32_t *>(tiled), static_cast<int>(out_len), G, words, src_i2s);
    st = check_launch("i2_tile_kernel");
    if (st) return st;
    if (w_scale) {
        hipLaunchKernelGGL(copy_scale_kernel, dim3(1), dim3(1), 0, as_stream(stream), w_scale,
                           reinterpret_cast<float *>(tiled + bytes));
        st = check_launch("copy_scale_kernel");
    }
    return st;
}

// y = W x on a raw I2_S tensor (codes, then the fp32 scale at byte
// out_len*in_len/4) for ncols int8 rows xq with their act_scale.
int i2s_gemm(const uint8_t *i2s, size_t out_len, size_t in_len, const int8_t *xq, const float *act_scale,
             size_t ncols, float *y, int32_t *acc, void *stream) {
    int st = check_i2_shape(out_len, in_len);
    if (st) return st;
    if (!i2s || !xq || !act_scale || !y || !ncols)
        return fail(OURO_ERR_INVALID_ARG, "i2_s gemv: NULL argument or ncols == 0");
    if (reinterpret_cast<uintptr_t>(i2s) % 16 || reinterpret_cast<uintptr_t>(xq) % 16)
        return fail(OURO_ERR_ALIGN, "i2_s gemv: payload and xq need 16-byte alignment");
    if (ncols > 65535) return fail(OURO_ERR_SHAPE, "i2_s gemv: more than 65535 columns");
    const int ns = static_cast<int>((in_len / 64 + 63) / 64);
    I2sArgs a{i2s, reinterpret_cast<const float *>(i2s + out_len * in_len / 4), xq, act_scale, y, acc,
              static_cast<int>(out_len), static_cast<int>(in_len)};
    void (*fn)(I2sArgs) = nullptr;
    switch (ns) {
    case 1: fn = i2s_gemv_kernel<1>; break;
    case 2: fn = i2s_gemv_kernel<2>; break;
    case 3: fn = i2s_gemv_kernel<3>; break;
    case 4: fn = i2s_gemv_kernel<4>; break;
    case 5: fn = i2s_gemv_kernel<5>; break;
    case 6: fn = i2s_gemv_kernel<6>; break;
    case 7: fn = i2s_gemv_kernel<7>; break;
    case 8: fn = i2s_gemv_kernel<8>; break;
    default: return fail(OURO_ERR_SHAPE, "i2_s gemv: in_len %zu > 32768", in_len);
    }
    const size_t rows_per_block = static_cast<size_t>(kTileRows) * kI2sWaves;
    dim3 grid(static_cast<unsigned>((out_len + rows_per_block - 1) / rows_per_block), static_cast<unsigned>(ncols));
    hipLaunchKernelGGL(fn, grid, dim3(kWave * kI2sWaves), 0, as_stream(stream), a);
    return check_launch("i2s_gemv_kernel");
}

}  // namespace ouro

using namespace ouro;

extern "C" {

size_t ouro_i2_tiled_bytes(size_t out_len, size_t in_len) { return i2_tiled_bytes(out_len, in_len); }

int ouro_i2_tile(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *tiled,
                 const float *w_scale_or_null, void *stream) {
    OURO_REQUIRE_INIT();
    return i2_tile(canonical, out_len, in_len, tiled, w_scale_or_null, stream, 0);
}

int ouro_i2s_tile(const uint8_t *i2s, size_t out_len, size_t in_len, uint8_t *tiled, void *stream) {
    OURO_REQUIRE_INIT();
    if (!i2s) return fail(OURO_ERR_INVALID_ARG, "ouro_i2s_tile: NULL argument");
    return i2_tile(i2s, out_len, in_len, tiled, reinterpret_cast<const float *>(i2s + out_len * in_len / 4), stream, 1);
}

int ouro_act_quant_i8(const void *x, int x_dtype, size_t rows, size_t n, int8_t *xq,
                      float *act_scale, void *stream) {
    OURO_REQUIRE_INIT();
    return act_quant(x, x_dtype, rows, n, xq, act_scale, stream);
}

int ouro_gemm_i2(const uint8_t *w_tiled, size_t out_len, size_t in_len, const float *w_scale,
                 const int8_t *xq, const float *act_scale, size_t ncols, float *y,
                 int32_t *acc_or_null, void *stream) {
    OURO_REQUIRE_INIT();
    return i2_gemm(w_tiled, out_len, in_len, w_scale, xq, act_scale, ncols, y, acc_or_null, stream);
}

int ouro_gemv_i2_grouped(const uint8_t *w_tiled, size_t w_stride, const float *w_scale,
                         const int8_t *xq, size_t x_stride, const float *act_scale, float *y,
                         size_t y_stride, size_t out_len, size_t in_len, size_t count,
                         void *stream) {
    OURO_REQUIRE_INIT();
    int st = check_i2_shape(out_len, in_len);
    if (st) return st;
    if (!w_tiled || !w_scale || !xq || !act_scale || !y || !count)
        return fail(OURO_ERR_INVALID_ARG, "ouro_gemv_i2_grouped: NULL argument or count == 0");
    if (count > 65535) return fail(OURO_ERR_SHAPE, "ouro_gemv_i2_grouped: count > 65535");
    if (w_stride < i2_tiled_bytes(out_len, in_len) || w_stride % 16 || x_stride < in_len ||
        x_stride % 16 || y_stride < out_len)
        return fail(OURO_ERR_SHAPE, "ouro_gemv_i2_grouped: strides overlap or misaligned");
    if (reinterpret_cast<uintptr_t>(w_tiled) % 16 || reinterpret_cast<uintptr_t>(xq) % 16)
        return fail(OURO_ERR_ALIGN, "ouro_gemv_i2_grouped: weights and xq need 16-byte alignment");
    constexpr int R = kTileRows;
    GemvArgs a{};
    a.w = w_tiled;
    a.w_stride = static_cast<long long>(w_stride);
    a.w_scale = w_scale;
    a.xq = xq;
    a.x_stride = static_cast<long long>(x_stride);
    a.act_scale = act_scale;
    a.y = y;
    a.y_stride = static_cast<long long>(y_stride);
    a.acc = nullptr;
    a.out_len = static_cast<int>(out_len);
    a.in_len = static_cast<int>(in_len);
    a.ncols = 1;
    a.tiles = static_cast<int>((out_len + R - 1) / R);
    return launch_gemv(a, static_cast<int>(count), stream);
}

}  // extern "C"
