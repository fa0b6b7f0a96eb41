// i2_gemm.hip - ternary x int8 GEMM for many activation columns on int8 MFMA.
//
// matmul_q (ops.rs:156-230) amortises one decode of the weights over K input
// columns; at K in the tens to thousands (batched verify, prefill
// projections) the product is compute-bound, so it runs on
// v_mfma_i32_16x16x64_i8 with the 2-bit weights expanded to int8 MFMA A
// fragments in registers and the int8 activations staged through LDS as B
// fragments.  Accumulation is exact int32 and the fp32 epilogue is the same
// two separately rounded products as the GEMV, so every output is
// bit-identical to the oracle for any K.
//
// MFMA layout of the codes (ouro_i2_tile_mfma): 1 KiB units, one per
// (row tile of 16 rows, k block of 256); unit (rt, kb) at byte
// (rt * in_len/256 + kb) * 1024.  Lane l's 16 bytes of a unit are its A
// fragments for the block's four 64-deep MFMA steps: 32-bit word s holds
// row 16*rt + l%16, k = 256*kb + 64*s + 16*(l/16) + 4*j + i at bits
// 8*i + 2*j as the 2-bit two's complement of v = 1 - code = -w (so every
// 2-bit code, including the never-produced 3, is representable).  One
// shift and one mask, (word << (6 - 2j)) & 0xC0C0C0C0, turn field j of all
// four bytes into the int8 values 64*v for k = 4j + i; the MFMA sum is
// -64 * sum(w*x), and acc = -(D >> 6) exactly.
#include "common.hpp"

#include <cstddef>

#pragma clang fp contract(off)

namespace ouro {
namespace {

constexpr int kWave = 64;
constexpr int kGemmWaves = 4;
constexpr int kXPitch = 272;  // LDS bytes per activation row of a 256-k block
constexpr int kSkinnyCols = 64;  // column counts up to this use the split-k kernel
constexpr int kSkinnyWaves = 16; // its wavefronts per workgroup (one per k block; half for > 32 columns)
constexpr int kSkinnyGroup = 4;  // products per grouped launch
constexpr long long kSkinnyTallTiles = 4096;  // row tiles from which a workgroup takes 4 of them

typedef int v4i __attribute__((ext_vector_type(4)));
// Register arrays of 16-byte pieces use the native vector type: arrays of
// HIP's uint4 struct are kept in scratch memory by the compiler.
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// One thread per 32-bit word of the MFMA layout.  The source is canonical
// codes, or (src_i2s) the codes of a bitnet.cpp I2_S tensor.
__global__ void i2_tile_mfma_kernel(const uint8_t *__restrict__ canon, uint32_t *__restrict__ dst,
                                    int out_len, int in_len, long long total_words, int src_i2s) {
    const long long id = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= total_words) return;
    const int nkb = in_len / 256;
    const long long unit = id / 256;
    const int rem = static_cast<int>(id % 256);
    const int l = rem / 4, s = rem % 4;
    const long long rt = unit / nkb;
    const int kb = static_cast<int>(unit % nkb);
    const long long row = rt * 16 + (l % 16);
    const int kbase = 256 * kb + 64 * s + 16 * (l / 16);
    uint32_t word = 0;
    if (row < out_len) {
        const uint8_t *cr = canon + row * (in_len / 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kg = (kbase + 4 * j) / 4;  // the four k of field j share a canonical byte
            const uint32_t byte = src_i2s ? i2s_canon_byte(canon, row, in_len, kg) : cr[kg];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t code = (byte >> (2 * i)) & 3u;
                word |= ((1u - code) & 3u) << (8 * i + 2 * j);
            }
        }
    }
    dst[id] = word;
}

__global__ void copy_scale_mfma_kernel(const float *src, float *dst) { *dst = *src; }

struct GemmArgs {
    const uint4 *w;        // MFMA-layout units
    const float *w_scale;  // device scalar
    const int8_t *xq;      // [N][K] int8
    const float *act_scale;   // [N]
    float *y;              // [N][M]
    int32_t *acc;          // optional, same layout as y
    int M, K, N, nkb, nrb;
    int x_tiled;           // xq in the few-column fragment order (ceil(N/16) column tiles)
    int swiglu;            // rows are (up, gate) pairs: y[N][M/2] = silu(gate) * up (no acc)
    GemmEpilogue epi;      // element-wise step on every stored output (not with acc or swiglu)
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (120 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(GemmArgs) == 120, "GemmArgs: kernel argument layout");

// The SwiGLU of an interleaved (up, gate) row pair, in the row kernel's
// arithmetic (silu(gate) * up, run_ffn qwen35.rs:802).
__device__ __forceinline__ float swiglu_pair(float up, float gate) { return gate / (1.0f + expf(-gate)) * up; }

// Up to four products with the same k and column count in one launch of the
// 16x16 kernel: workgroups bstart[p] .. bstart[p+1]-1 belong to product p.
constexpr int kMfmaGroup = 4;
static_assert(kMfmaGroup >= kSkinnyGroup, "a few-column group fits one 16x16 launch");
struct MfmaGroup {
    GemmArgs p[kMfmaGroup];
    int bstart[kMfmaGroup + 1];
    int np;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (504 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(MfmaGroup) == 504, "MfmaGroup: kernel argument layout");

// Block: 4 wavefronts stacked along rows; wavefront w owns row tiles
// (4*rb + w)*WR .. +WR-1 and the block's WC column tiles of 16 columns.
// Per 256-deep k block: the block copies its WC*16 activation rows into
// one of two LDS buffers (prefetched a block ahead in registers), every
// wavefront loads its WR 1 KiB weight units (also a block ahead), and runs
// 4 steps x WR x WC MFMAs.  XT: the activations are in the few-column
// fragment order, whose 1 KiB pieces (k block, step, column tile) are the
// MFMA B operands lane by lane; they are copied to LDS as they are and read
// back at lane * 16.  A launch may hold several products (MfmaGroup).
// KS > 1: KS groups of 4 wavefronts split the k blocks (each group its own
// LDS buffers), so the latency chain is nkb / KS blocks long; the groups'
// int32 tiles are added in LDS at the end (exact) and group 0 stores.
template <int WR, int WC, bool XT, int KS>
__global__ __launch_bounds__(kWave *kGemmWaves *KS) void i2_gemm_mfma_kernel(MfmaGroup grp) {
    __shared__ __attribute__((aligned(16))) uint8_t xs[KS][2][WC * 16 * kXPitch];
    static_assert(WC * 4 * 1024 <= WC * 16 * kXPitch, "fragment-ordered tile fits the LDS buffer");
    static_assert((KS - 1) * kGemmWaves * WR * WC * 4 * kWave * 4 <= KS * 2 * WC * 16 * kXPitch,
                  "the k groups' partial tiles fit the LDS buffers");
    const int tid0 = threadIdx.x, lane = tid0 & 63, kg = tid0 / (kWave * kGemmWaves);
    const int tid = tid0 % (kWave * kGemmWaves), wave = tid >> 6;  // within the k group
    int pi = 0;
    while (pi + 1 < grp.np && static_cast<int>(blockIdx.x) >= grp.bstart[pi + 1]) ++pi;
    const GemmArgs &a = grp.p[pi];
    const int local = static_cast<int>(blockIdx.x) - grp.bstart[pi];
    const int rb = local % a.nrb, cb = local / a.nrb;
    const int n0 = cb * WC * 16;
    const int rt0 = (rb * kGemmWaves + wave) * WR;
    const int nrt = (a.M + 15) / 16;
    const int tiles = (a.N + 15) / 16;

    v4u xr[WC];
    auto load_x = [&](int kb) {
#pragma unroll
        for (int i = 0; i < WC; ++i) {
            const int c = tid + kWave * kGemmWaves * i;
            if (XT) {
                // piece c: step c / (64 WC), column tile c / 64 % WC, lane c % 64
                const int ct = min(n0 / 16 + (c / 64) % WC, tiles - 1);  // clamped: never stored
                xr[i] = *reinterpret_cast<const v4u *>(
                    a.xq + ((static_cast<long long>(kb) * 4 + c / (64 * WC)) * tiles + ct) * 1024 + (c % 64) * 16);
            } else {
                const int n = min(n0 + c / 16, a.N - 1);  // clamped: columns past N are never stored
                xr[i] = *reinterpret_cast<const v4u *>(a.xq + static_cast<long long>(n) * a.K + 256 * kb +
                                                       16 * (c % 16));
            }
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < WC; ++i) {
            const int c = tid + kWave * kGemmWaves * i;
            const int off = XT ? 16 * c : (c / 16) * kXPitch + 16 * (c % 16);
            *reinterpret_cast<v4u *>(&xs[kg][buf][off]) = xr[i];
        }
    };
    v4u wr[WR];
    auto load_w = [&](int kb) {
#pragma unroll
        for (int r = 0; r < WR; ++r) {
            const int rt = min(rt0 + r, nrt - 1);  // clamped: rows past M are never stored
            wr[r] = reinterpret_cast<const v4u *>(a.w)[(static_cast<long long>(rt) * a.nkb + kb) * kWave + lane];
        }
    };

    // every column's activation scale, for the epilogue, ahead of the k loop:
    // its stores would keep the compiler from moving a later load above them
    float as[WC];
#pragma unroll
    for (int c = 0; c < WC; ++c) as[c] = a.act_scale[min(n0 + 16 * c + (lane & 15), a.N - 1)];

    v4i acc[WR][WC];
#pragma unroll
    for (int r = 0; r < WR; ++r)
#pragma unroll
        for (int c = 0; c < WC; ++c) acc[r][c] = v4i{0, 0, 0, 0};

    // k blocks kb0 .. kb1-1 of this group; every group runs `per` steps (the
    // same barriers), a group past its range loads a valid block and skips
    // the products
    const int per = (a.nkb + KS - 1) / KS;
    const int kb0 = min(kg * per, a.nkb), kb1 = min(kb0 + per, a.nkb);
    const auto kbc = [&](int it) { return min(kb0 + it, a.nkb - 1); };
    load_x(kbc(0));
    load_w(kbc(0));
    store_x(0);
    __syncthreads();
    for (int it = 0; it < per; ++it) {
        v4u wc[WR];
#pragma unroll
        for (int r = 0; r < WR; ++r) wc[r] = wr[r];
        const bool more = it + 1 < per;
        if (more) {
            load_x(kbc(it + 1));
            load_w(kbc(it + 1));
        }
        const uint8_t *xb = XT ? xs[kg][it & 1] + 16 * lane : xs[kg][it & 1] + (lane & 15) * kXPitch + 16 * (lane >> 4);
        if (kb0 + it < kb1) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v4i A[WR];
#pragma unroll
            for (int r = 0; r < WR; ++r) {
                const uint32_t wd = s == 0 ? wc[r][0] : s == 1 ? wc[r][1] : s == 2 ? wc[r][2] : wc[r][3];
                A[r] = v4i{static_cast<int>((wd << 6) & 0xC0C0C0C0u), static_cast<int>((wd << 4) & 0xC0C0C0C0u),
                           static_cast<int>((wd << 2) & 0xC0C0C0C0u), static_cast<int>(wd & 0xC0C0C0C0u)};
            }
#pragma unroll
            for (int c = 0; c < WC; ++c) {
                const v4i B = *reinterpret_cast<const v4i *>(XT ? xb + (s * WC + c) * 1024 : xb + c * 16 * kXPitch + 64 * s);
#pragma unroll
                for (int r = 0; r < WR; ++r)
                    acc[r][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[r], B, acc[r][c], 0, 0, 0);
            }
        }
        }
        if (more) store_x((it + 1) & 1);
        __syncthreads();
    }
    if constexpr (KS > 1) {  // every LDS read of the loop is behind its last barrier
        int *red = reinterpret_cast<int *>(&xs[0][0][0]);
        constexpr int kAcc = WR * WC * 4;
        if (kg > 0) {
#pragma unroll
            for (int r = 0; r < WR; ++r)
#pragma unroll
                for (int c = 0; c < WC; ++c)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        red[(((kg - 1) * kGemmWaves + wave) * kAcc + (r * WC + c) * 4 + e) * kWave + lane] = acc[r][c][e];
        }
        __syncthreads();
        if (kg > 0) return;  // no barrier follows
#pragma unroll
        for (int g = 1; g < KS; ++g)
#pragma unroll
            for (int r = 0; r < WR; ++r)
#pragma unroll
                for (int c = 0; c < WC; ++c)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[r][c][e] += red[(((g - 1) * kGemmWaves + wave) * kAcc + (r * WC + c) * 4 + e) * kWave + lane];
    }

    // D lane l: rows 4*(l/16) + e of the row tile, column l % 16.  With the
    // row count a multiple of 4 and 16-byte aligned outputs and operands, a
    // lane's four rows are stored (and the epilogue's operands moved) as one
    // 16-byte piece.
    const float wscale = *a.w_scale;
    const bool vec = (a.M & 3) == 0 &&
                     ((reinterpret_cast<uintptr_t>(a.y) | reinterpret_cast<uintptr_t>(a.acc) |
                       reinterpret_cast<uintptr_t>(a.epi.b) | reinterpret_cast<uintptr_t>(a.epi.ring) |
                       reinterpret_cast<uintptr_t>(a.epi.w)) & 15) == 0;
#pragma unroll
    for (int c = 0; c < WC; ++c) {
        const int n = n0 + 16 * c + (lane & 15);
        if (n >= a.N) continue;
        const I8sInv ds = i8s_inv(as[c]);  // (acc / s) without a division per output
#pragma unroll
        for (int r = 0; r < WR; ++r) {
            const int row = (rt0 + r) * 16 + 4 * (lane >> 4);
            if (vec && row + 3 < a.M) {
                int t[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) t[e] = -(acc[r][c][e] >> 6);
                const float4 v = make_float4(i8s_out_inv(t[0], ds, wscale), i8s_out_inv(t[1], ds, wscale),
                                             i8s_out_inv(t[2], ds, wscale), i8s_out_inv(t[3], ds, wscale));
                if (a.swiglu) {  // outputs row/2 and row/2 + 1: an 8-byte piece
                    *reinterpret_cast<float2 *>(a.y + static_cast<long long>(n) * (a.M / 2) + row / 2) =
                        make_float2(swiglu_pair(v.x, v.y), swiglu_pair(v.z, v.w));
                    continue;
                }
                const long long o = static_cast<long long>(n) * a.M + row;
                *reinterpret_cast<float4 *>(a.y + o) = gemm_epilogue4(a.epi, v, n, row, a.M);
                if (a.acc) *reinterpret_cast<int4 *>(a.acc + o) = make_int4(t[0], t[1], t[2], t[3]);
                continue;
            }
            if (a.swiglu) {  // rows row .. row+3 = (up, gate) of outputs row/2, row/2 + 1
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    if (row + e + 1 >= a.M) break;
                    const float up = i8s_out_inv(-(acc[r][c][e] >> 6), ds, wscale);
                    const float gt = i8s_out_inv(-(acc[r][c][e + 1] >> 6), ds, wscale);
                    a.y[static_cast<long long>(n) * (a.M / 2) + (row + e) / 2] = swiglu_pair(up, gt);
                }
                continue;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (row + e >= a.M) break;
                const int total = -(acc[r][c][e] >> 6);
                const long long o = static_cast<long long>(n) * a.M + row + e;
                a.y[o] = gemm_epilogue(a.epi, i8s_out_inv(total, ds, wscale), n, row + e, a.M);
                if (a.acc) a.acc[o] = total;
            }
        }
    }
}

// Large products (prefill projections, thousands of columns) on
// v_mfma_i32_32x32x32_i8, which sustains ~1.4x the rate of the 16x16x64
// form on MI355X.  Workgroup tile 256 rows x 128 columns: four wavefronts
// stacked along the rows, each with a 64 x 128 register tile (2 x 4 MFMA
// tiles of 32 x 32), so each decoded weight fragment feeds 4 MFMAs (the
// 2-bit decode is the VALU work that competes with the MFMA issue) and each
// 16-byte activation fragment from LDS feeds 2.
//
// The weights stay in the 16-row unit layout: the 32x32x32 A operand of
// lane l is row l % 32 and 16 k values chosen per lane, so lane l reads
// lane slot (l % 16) + 16 (2p + l / 32) of unit 2 RT + (l % 32) / 16 for
// p = 0, 1; word s of that slot is MFMA step (s, p) over k = 64 s + 32 p +
// 16 (l / 32) + 0..15, and the B operand reads the same 16 activation bytes
// of column l % 32.  D lane l register e: column l % 32, row
// 8 (e / 4) + 4 (l / 32) + e % 4.
//
// The activation tile of a 256-deep k block (32 KiB) is double-buffered in
// LDS and filled a k block ahead by direct global-to-LDS loads
// (global_load_lds_dwordx4: lane i of a wavefront's load lands at the
// wavefront's LDS base + 16 i, from an address the lane chooses), so the
// tile takes no registers and no LDS write instructions; column n's 256
// bytes are one LDS row, its 16-byte chunk u at slot u ^ (n % 16), so the
// B-fragment reads (32 columns, one chunk) hit distinct banks.  The
// weights are prefetched a k block ahead in registers.  Indices are
// clamped, not guarded, so the loads are unconditional and the waits count
// them exactly.  Workgroups are handed out XCD by XCD
// (blockIdx % 8 is the XCD): each XCD takes a contiguous run of tiles, row
// blocks fastest, so the 128 activation columns a run shares stay in that
// XCD's L2.
typedef int v16i __attribute__((ext_vector_type(16)));
constexpr int kBigTM = 2, kBigTN = 4;  // 32 x 32 MFMA tiles per wavefront
constexpr int kBigCols = kBigTN * 32;  // columns per workgroup (rows: 4 kBigTM 32)
constexpr int kBigMinBlocks = 192;  // fewer tiles than this: the 16x16 kernel (faster there)

typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

__global__ __launch_bounds__(kWave *kGemmWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void i2_gemm_big_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t xs[2][kBigCols * 256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nblk = static_cast<int>(gridDim.x), xcd = static_cast<int>(blockIdx.x) % 8;
    const int q8 = nblk / 8, r8 = nblk % 8;
    const int t = xcd * q8 + min(xcd, r8) + static_cast<int>(blockIdx.x) / 8;
    const int rb = t % a.nrb, cb = t / a.nrb;
    const int n0 = cb * kBigCols;
    const int RT0 = (rb * kGemmWaves + wave) * kBigTM;  // the wavefront's first 32-row tile
    const int nrt = (a.M + 15) / 16;
    const int half = (lane & 31) >> 4, g = lane >> 5;

    constexpr int XV = kBigCols * 16 / (kWave * kGemmWaves);  // 16-byte pieces per thread per k block
    v4u wr[kBigTM][2];
    // load i of wavefront `wave` fills LDS bytes 1024 (XV wave + i) .. +1023 of
    // buffer buf: slot 16 lane of that KiB is column n = 4 (XV wave + i) +
    // lane / 16, chunk (lane % 16) ^ (n % 16)
    auto load_x = [&](int kb, int buf) {
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int piece = XV * wave + i;
            const int nl = 4 * piece + (lane >> 4);
            const int u = (lane & 15) ^ (nl & 15);
            const int n = min(n0 + nl, a.N - 1);  // clamped: columns past N are never stored
            __builtin_amdgcn_global_load_lds(
                (global_void *)(a.xq + static_cast<long long>(n) * a.K + 256 * kb + 16 * u),
                (lds_void *)(&xs[buf][1024 * piece]), 16, 0, 0);
        }
    };
    auto load_w = [&](int kb) {
#pragma unroll
        for (int r = 0; r < kBigTM; ++r) {
            const int rt = min(2 * (RT0 + r) + half, nrt - 1);  // clamped: rows past M are never stored
#pragma unroll
            for (int p = 0; p < 2; ++p)
                wr[r][p] = reinterpret_cast<const v4u *>(
                    a.w)[(static_cast<long long>(rt) * a.nkb + kb) * kWave + (lane & 15) + 16 * (2 * p + g)];
        }
    };

    v16i acc[kBigTM][kBigTN];
#pragma unroll
    for (int r = 0; r < kBigTM; ++r)
#pragma unroll
        for (int c = 0; c < kBigTN; ++c)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[r][c][e] = 0;

    // every column's activation scale, for the epilogue, ahead of the k loop:
    // its stores would keep the compiler from moving a later load above them
    float as[kBigTN];
#pragma unroll
    for (int c = 0; c < kBigTN; ++c) as[c] = a.act_scale[min(n0 + c * 32 + (lane & 31), a.N - 1)];
    load_x(0, 0);
    load_w(0);
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0): this wavefront's LDS fills have landed
    __syncthreads();
    const int ncol = lane & 31;  // the B fragment's column within its 32-column tile (same low bits for every tile)
    for (int kb = 0; kb < a.nkb; ++kb) {
        v4u wc[kBigTM][2];
#pragma unroll
        for (int r = 0; r < kBigTM; ++r) wc[r][0] = wr[r][0], wc[r][1] = wr[r][1];
        const bool more = kb + 1 < a.nkb;
        if (more) {  // the other buffer: its last reads were before the previous barrier
            load_x(kb + 1, (kb + 1) & 1);
            load_w(kb + 1);
        }
        const uint8_t *xb = xs[kb & 1] + ncol * 256;
#pragma unroll
        for (int sp = 0; sp < 8; ++sp) {
            const int s = sp / 2, p = sp % 2;  // MFMA step (s, p): k = 64 s + 32 p + 16 g
            v4i A[kBigTM];
#pragma unroll
            for (int r = 0; r < kBigTM; ++r) {
                const uint32_t wd = wc[r][p][s];
                A[r] = v4i{static_cast<int>((wd << 6) & 0xC0C0C0C0u), static_cast<int>((wd << 4) & 0xC0C0C0C0u),
                           static_cast<int>((wd << 2) & 0xC0C0C0C0u), static_cast<int>(wd & 0xC0C0C0C0u)};
            }
            const int slot = 16 * ((2 * sp + g) ^ (ncol & 15));  // chunk 2 sp + g of column 32 c + ncol
#pragma unroll
            for (int c = 0; c < kBigTN; ++c) {
                const v4i B = *reinterpret_cast<const v4i *>(xb + c * 32 * 256 + slot);
#pragma unroll
                for (int r = 0; r < kBigTM; ++r)
                    acc[r][c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[r], B, acc[r][c], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0): the next block's LDS fills (and weights) have landed
        __syncthreads();
    }

    // registers 4q .. 4q+3 of a tile are 4 consecutive rows of one column,
    // contiguous in y: a full quad goes out as one 16-byte store
    const float wscale = *a.w_scale;
    const bool quad = (a.M % 4) == 0 && !a.acc && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 &&
                      (a.epi.op != EPI_RESID || (reinterpret_cast<uintptr_t>(a.epi.b) & 15) == 0);
    if (quad && a.swiglu && a.M % 8 == 0) {
        // SwiGLU: the wavefront's 64 rows are 32 (up, gate) pairs, so its
        // outputs are 32 rows of each column: one pass through LDS (output
        // chunk 4 r + q of column n, at chunk (4 r + q) ^ (n % 8)) and 8
        // lanes to a 128-byte line on the way out, as above.
        float *tw = reinterpret_cast<float *>(&xs[0][0]) + wave * (kBigCols * 32);
#pragma unroll
        for (int r = 0; r < kBigTM; ++r)
#pragma unroll
            for (int c = 0; c < kBigTN; ++c) {
                const int nl = c * 32 + (lane & 31);
                const I8sInv ds = i8s_inv(as[c]);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float2 v;  // outputs 16 r + 4 q + 2 g + {0, 1} of the wavefront
                    v.x = swiglu_pair(i8s_out_inv(-(acc[r][c][4 * q] >> 6), ds, wscale),
                                      i8s_out_inv(-(acc[r][c][4 * q + 1] >> 6), ds, wscale));
                    v.y = swiglu_pair(i8s_out_inv(-(acc[r][c][4 * q + 2] >> 6), ds, wscale),
                                      i8s_out_inv(-(acc[r][c][4 * q + 3] >> 6), ds, wscale));
                    *reinterpret_cast<float2 *>(tw + nl * 32 + 4 * ((4 * r + q) ^ (nl & 7)) + 2 * g) = v;
                }
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int col = lane >> 3, j = lane & 7, mh = a.M / 2;
        const int o0 = RT0 * 16;  // the wavefront's first output row
#pragma unroll
        for (int i = 0; i < kBigCols / 8; ++i) {
            const int nl = 8 * i + col, n = n0 + nl, orow = o0 + 4 * j;
            const float4 v = *reinterpret_cast<const float4 *>(tw + nl * 32 + 4 * (j ^ (nl & 7)));
            if (n < a.N && orow < mh)  // mh % 4 == 0: a chunk of 4 outputs is all in or all out
                *reinterpret_cast<float4 *>(a.y + static_cast<long long>(n) * mh + orow) = v;
        }
        return;
    }
    if (quad && !a.swiglu && (a.epi.op == EPI_NONE || a.epi.op == EPI_RESID)) {
        // Through LDS, one 32-row tile at a time: the wavefront writes its
        // 32 x 128 outputs column by column into its own 16 KiB of the
        // (now idle) activation buffers, 16-byte chunk j of column n at
        // chunk j ^ (n % 8), then reads them back so that 8 lanes hold one
        // column's 32 rows and each store instruction writes 8 whole
        // 128-byte lines (the register layout gives 32 partial lines).
        float *tw = reinterpret_cast<float *>(&xs[0][0]) + wave * (kBigCols * 32);
        const int col = lane >> 3, j = lane & 7;  // read back: column 8 i + col, rows 4 j .. 4 j + 3
#pragma unroll
        for (int r = 0; r < kBigTM; ++r) {
            const int r0 = (RT0 + r) * 32;
#pragma unroll
            for (int c = 0; c < kBigTN; ++c) {
                const int nl = c * 32 + (lane & 31);  // the lane's column in the tile
                const I8sInv ds = i8s_inv(as[c]);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float4 v;
                    v.x = i8s_out_inv(-(acc[r][c][4 * q] >> 6), ds, wscale);
                    v.y = i8s_out_inv(-(acc[r][c][4 * q + 1] >> 6), ds, wscale);
                    v.z = i8s_out_inv(-(acc[r][c][4 * q + 2] >> 6), ds, wscale);
                    v.w = i8s_out_inv(-(acc[r][c][4 * q + 3] >> 6), ds, wscale);
                    *reinterpret_cast<float4 *>(tw + nl * 32 + 4 * ((2 * q + g) ^ (nl & 7))) = v;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int i = 0; i < kBigCols / 8; ++i) {
                const int nl = 8 * i + col, n = n0 + nl, row = r0 + 4 * j;
                float4 v = *reinterpret_cast<const float4 *>(tw + nl * 32 + 4 * (j ^ (nl & 7)));
                if (n < a.N && row + 3 < a.M) {
                    const long long o = static_cast<long long>(n) * a.M + row;
                    if (a.epi.op == EPI_RESID) {
                        const float4 res = *reinterpret_cast<const float4 *>(a.epi.b + o);
                        v.x = res.x + v.x;
                        v.y = res.y + v.y;
                        v.z = res.z + v.z;
                        v.w = res.w + v.w;
                    }
                    *reinterpret_cast<float4 *>(a.y + o) = v;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();  // the reads are done before the next tile's writes
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        return;
    }
#pragma unroll
    for (int c = 0; c < kBigTN; ++c) {
        const int n = n0 + c * 32 + (lane & 31);
        if (n >= a.N) continue;
        const I8sInv ds = i8s_inv(as[c]);  // (acc / s) without a division per output
#pragma unroll
        for (int r = 0; r < kBigTM; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = (RT0 + r) * 32 + 8 * q + 4 * g;
                const long long o = static_cast<long long>(n) * a.M + row;
                if (a.swiglu) {  // rows row .. row+3 = (up, gate) of outputs row/2, row/2 + 1
#pragma unroll
                    for (int e = 0; e < 4; e += 2) {
                        if (row + e + 1 >= a.M) break;
                        const float up = i8s_out_inv(-(acc[r][c][4 * q + e] >> 6), ds, wscale);
                        const float gt = i8s_out_inv(-(acc[r][c][4 * q + e + 1] >> 6), ds, wscale);
                        a.y[static_cast<long long>(n) * (a.M / 2) + (row + e) / 2] = swiglu_pair(up, gt);
                    }
                    continue;
                }
                if (quad && row + 3 < a.M) {
                    float4 v;
                    float4 res = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (a.epi.op == EPI_RESID) res = *reinterpret_cast<const float4 *>(a.epi.b + o);
                    v.x = i8s_out_inv(-(acc[r][c][4 * q] >> 6), ds, wscale);
                    v.y = i8s_out_inv(-(acc[r][c][4 * q + 1] >> 6), ds, wscale);
                    v.z = i8s_out_inv(-(acc[r][c][4 * q + 2] >> 6), ds, wscale);
                    v.w = i8s_out_inv(-(acc[r][c][4 * q + 3] >> 6), ds, wscale);
                    if (a.epi.op == EPI_RESID) {
                        v.x = res.x + v.x;
                        v.y = res.y + v.y;
                        v.z = res.z + v.z;
                        v.w = res.w + v.w;
                    }
                    *reinterpret_cast<float4 *>(a.y + o) = v;
                    continue;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (row + e >= a.M) break;
                    const int total = -(acc[r][c][4 * q + e] >> 6);
                    a.y[o + e] = gemm_epilogue(a.epi, i8s_out_inv(total, ds, wscale), n, row + e, a.M);
                    if (a.acc) a.acc[o + e] = total;
                }
            }
    }
}

// Few columns (N <= 64, e.g. one decode step of a batch of sequences): the
// product is a weight stream, so every weight unit must be read once and
// the k loop must not be a latency chain.  Workgroup = 2 (or 4) row tiles
// x all N columns, with one wavefront per k block (up to 16; beyond that
// each wavefront takes every 16th block), so all of a workgroup's loads are
// in flight at once.  Wavefronts read their activation fragments straight
// from global memory (L2-resident: 16*WC rows of in_len bytes) and add their
// int32 tiles into one LDS tile with integer atomics (exact, order-free).
constexpr int skinny_waves(int wc) { return wc <= 2 ? kSkinnyWaves : kSkinnyWaves / 2; }

// Up to kSkinnyGroup products with the same k and column count share one
// launch (the projections of one activation): workgroups
// bstart[p] .. bstart[p+1]-1 belong to product p.
struct SkinnyProblem {
    const uint4 *w;
    const float *w_scale;
    const int8_t *xq;
    const float *act_scale;
    float *y;
    int32_t *acc;
    int M;
    GemmEpilogue epi;
    int swiglu;
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (104 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(SkinnyProblem) == 104, "SkinnyProblem: kernel argument layout");
struct SkinnyGroup {
    SkinnyProblem p[kSkinnyGroup];
    int bstart[kSkinnyGroup + 1];
    int np, K, N, nkb, x_tiled;
    int tiles;  // column tiles of the whole launch, ceil(N / 16)
    int ncg;    // column groups of WC tiles; workgroup x = row block * ncg + column group
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (464 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(SkinnyGroup) == 464, "SkinnyGroup: kernel argument layout");
static_assert(offsetof(SkinnyGroup, bstart) == 416 && offsetof(SkinnyGroup, np) == 436 &&
                  offsetof(SkinnyGroup, ncg) == 460, "SkinnyGroup: kernel argument layout");

template <int WC, int WR>
__global__ __launch_bounds__(kWave *skinny_waves(WC)) void i2_gemm_skinny_kernel(SkinnyGroup g) {
    constexpr int TR = 16 * WR, TC = 16 * WC + 1;
    __shared__ int tile[TR * TC];
    __shared__ float sas[16 * WC];  // the columns' activation scales, read before the k loop
    // Workgroups numbered XCD by XCD (workgroup i runs on XCD i % 8), so the
    // ncg column groups of a row block, which read the same weight units,
    // are served by one L2: numbered round-robin, each group's XCD fetched
    // the units from HBM again (2560x6912 at 64 columns: 19.3 MB of L2
    // misses for 4.4 MB of weights).
    const int nblk = static_cast<int>(gridDim.x), xcd = static_cast<int>(blockIdx.x) % 8;
    const int q8 = nblk / 8, r8 = nblk % 8;
    const int wg = xcd * q8 + min(xcd, r8) + static_cast<int>(blockIdx.x) / 8;
    const int bx = wg / g.ncg, cg = wg % g.ncg;
    int pi = 0;
    while (pi + 1 < g.np && bx >= g.bstart[pi + 1]) ++pi;
    const SkinnyProblem &pb = g.p[pi];
    struct {
        const uint4 *w;
        const float *w_scale;
        const int8_t *xq;
        const float *act_scale;
        float *y;
        int32_t *acc;
        int M, K, N, nkb, x_tiled;
    } a{pb.w, pb.w_scale, pb.xq, pb.act_scale, pb.y, pb.acc, pb.M, g.K, g.N, g.nkb, g.x_tiled};
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int ct0 = cg * WC;  // first column tile of this workgroup
    const int rt0 = (bx - g.bstart[pi]) * WR;
    const int nrt = (a.M + 15) / 16;
    for (int i = tid; i < TR * TC; i += blockDim.x) tile[i] = 0;
    // (the epilogue's loads would otherwise wait behind its own stores)
    if (tid < 16 * WC) sas[tid] = a.act_scale[min(16 * ct0 + tid, a.N - 1)];
    v4i acc[WR][WC];
#pragma unroll
    for (int r = 0; r < WR; ++r)
#pragma unroll
        for (int c = 0; c < WC; ++c) acc[r][c] = v4i{0, 0, 0, 0};
    // Rows past M and columns past N are clamped to the last valid ones
    // (unconditional loads, no branches between them); their sums land in
    // tile rows / columns that the epilogue never stores.
    // Row-major x: lane l of column tile c reads row 16c + l%16 (clamped),
    // bytes 16*(l/16) of each 64-deep step.  Fragment-ordered x: one
    // contiguous 1 KiB per (k block, step, column tile), 16 bytes per lane.
    const int8_t *xr[WC];
#pragma unroll
    for (int c = 0; c < WC; ++c)
        xr[c] = a.x_tiled ? a.xq + (static_cast<long long>(ct0 + c) * kWave + lane) * 16
                          : a.xq + static_cast<long long>(min(16 * (ct0 + c) + (lane & 15), a.N - 1)) * a.K +
                                16 * (lane >> 4);
    const long long xkb = a.x_tiled ? 4LL * g.tiles * 1024 : 256, xs = a.x_tiled ? g.tiles * 1024 : 64;
    const uint4 *wp[WR];
#pragma unroll
    for (int r = 0; r < WR; ++r) wp[r] = a.w + static_cast<long long>(min(rt0 + r, nrt - 1)) * a.nkb * kWave + lane;
    const int nl = lane & 15;
    for (int kb = wave; kb < a.nkb; kb += nw) {
        uint4 wr[WR];
#pragma unroll
        for (int r = 0; r < WR; ++r) wr[r] = wp[r][kb * kWave];
        v4i B[WC][4];
#pragma unroll
        for (int c = 0; c < WC; ++c)
#pragma unroll
            for (int s = 0; s < 4; ++s) B[c][s] = *reinterpret_cast<const v4i *>(xr[c] + xkb * kb + xs * s);
        __builtin_amdgcn_sched_barrier(0);  // every load of the k block is issued before the first wait
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v4i A[WR];
#pragma unroll
            for (int r = 0; r < WR; ++r) {
                const uint32_t wd = s == 0 ? wr[r].x : s == 1 ? wr[r].y : s == 2 ? wr[r].z : wr[r].w;
                A[r] = v4i{static_cast<int>((wd << 6) & 0xC0C0C0C0u), static_cast<int>((wd << 4) & 0xC0C0C0C0u),
                           static_cast<int>((wd << 2) & 0xC0C0C0C0u), static_cast<int>(wd & 0xC0C0C0C0u)};
            }
#pragma unroll
            for (int c = 0; c < WC; ++c)
#pragma unroll
                for (int r = 0; r < WR; ++r)
                    acc[r][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[r], B[c][s], acc[r][c], 0, 0, 0);
        }
    }
    __syncthreads();  // tile zeroed
    // D lane l: rows 4*(l/16) + e of the row tile, column l % 16.
    if (wave < a.nkb) {
#pragma unroll
        for (int r = 0; r < WR; ++r)
#pragma unroll
            for (int c = 0; c < WC; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    atomicAdd(&tile[(16 * r + 4 * (lane >> 4) + e) * TC + 16 * c + nl], acc[r][c][e]);
    }
    __syncthreads();
    const float wscale = *a.w_scale;
    if (pb.swiglu) {  // tile rows 2p, 2p+1 = (up, gate) of output row (rt0 * 16 + 2p) / 2
        for (int i = tid; i < TR * 8 * WC; i += blockDim.x) {
            const int nt = i / (TR / 2), rr = 2 * (i % (TR / 2)), row = rt0 * 16 + rr, n = 16 * ct0 + nt;
            if (n >= a.N || row + 1 >= a.M) continue;
            const float ds = sas[nt];
            const float up = i8s_out(-(tile[rr * TC + nt] >> 6), ds, wscale);
            const float gt = i8s_out(-(tile[(rr + 1) * TC + nt] >> 6), ds, wscale);
            a.y[static_cast<long long>(n) * (a.M / 2) + row / 2] = swiglu_pair(up, gt);
        }
        return;
    }
    for (int i = tid; i < TR * 16 * WC; i += blockDim.x) {
        const int nt = i / TR, rr = i % TR, row = rt0 * 16 + rr, n = 16 * ct0 + nt;
        if (n >= a.N || row >= a.M) continue;
        const int total = -(tile[rr * TC + nt] >> 6);
        const long long o = static_cast<long long>(n) * a.M + row;
        a.y[o] = gemm_epilogue(pb.epi, i8s_out(total, sas[nt], wscale), n, row, a.M);
        if (a.acc) a.acc[o] = total;
    }
}

using GemmFn = void (*)(MfmaGroup);
using SkinnyFn = void (*)(SkinnyGroup);

struct GemmPick {
    GemmFn fn;
    int wr, wc, ks;
};

// Row tiles per wavefront WR and column tiles per block WC, from sweeps on
// MI355X (6912x2560, 2560x6912 and 2560x2560 at 4 .. 8192 columns): the
// largest wavefront tile (2x4: 32 rows x 64 columns, 8 MFMAs per pair of
// fragment loads) while it still gives >= 1024 workgroups, then 2x2 while
// >= 512, else 1x1 (16x16 per wavefront, the most workgroups, which is what
// few columns need).  Few-column launches of 17 .. 64 columns (the decode
// step's tall projections) take 1x2 with the k blocks split over two groups
// of four wavefronts: half the activation traffic of 1x1 and half its chain
// (12352x2560 and 13824x2560 at 64 columns, weights streamed from HBM:
// 10.4 -> 9.1 and 9.7 -> 8.7 us).  nrt = row tiles of all products of the
// launch.
template <bool XT>
GemmPick pick_gemm_xt(long long nrt, int N) {
    const auto blocks = [&](int wr, int wc) {
        const long long nrb = (nrt + kGemmWaves * wr - 1) / (kGemmWaves * wr);
        return nrb * ((N + 16 * wc - 1) / (16 * wc));
    };
    if (blocks(2, 4) >= 1024) return {i2_gemm_mfma_kernel<2, 4, XT, 1>, 2, 4, 1};
    if (blocks(2, 2) >= 512) return {i2_gemm_mfma_kernel<2, 2, XT, 1>, 2, 2, 1};
    if (N > 16 && N <= kSkinnyCols) return {i2_gemm_mfma_kernel<1, 2, XT, 2>, 1, 2, 2};
    return {i2_gemm_mfma_kernel<1, 1, XT, 1>, 1, 1, 1};
}

// One launch of the 16x16 kernel over np products (shared k, column count
// and activation layout); shapes are checked by the callers.
int launch_mfma_group(const GemmArgs *args, int np, void *stream) {
    long long nrt = 0;
    for (int i = 0; i < np; ++i) nrt += (args[i].M + 15) / 16;
    const int N = args[0].N;
    const GemmPick p = args[0].x_tiled ? pick_gemm_xt<true>(nrt, N) : pick_gemm_xt<false>(nrt, N);
    const long long ncb = (N + 16LL * p.wc - 1) / (16LL * p.wc);
    MfmaGroup g{};
    g.np = np;
    long long grid = 0;
    for (int i = 0; i < np; ++i) {
        g.p[i] = args[i];
        g.p[i].nrb = ((args[i].M + 15) / 16 + kGemmWaves * p.wr - 1) / (kGemmWaves * p.wr);
        g.bstart[i] = static_cast<int>(grid);
        grid += static_cast<long long>(g.p[i].nrb) * ncb;
        if (grid > 0x7fffffffLL) return fail(OURO_ERR_SHAPE, "ouro_gemm_i2_mfma: grid too large");
    }
    g.bstart[np] = static_cast<int>(grid);
    hipLaunchKernelGGL(p.fn, dim3(static_cast<unsigned>(grid)), dim3(kWave * kGemmWaves * p.ks), 0, as_stream(stream), g);
    return check_launch("i2_gemm_mfma_kernel");
}

// Few columns: the split-k kernel below unless the launch is tall (its
// activation re-reads grow with the rows) and has more than 32 columns (16
// on the tallest weights); the 16x16 kernel then streams the activations
// once per 64 rows.  Short products (2560 rows, some with 6912-deep k) keep
// the split-k kernel, which spreads k over the waves (sweeps on MI355X at
// 8 .. 64 columns, 2560 .. 248320 rows, singly and in the hybrid stack).
constexpr long long kFewColsMfmaTiles = 640;
bool few_cols_on_mfma(int N, long long row_tiles) {
    return (N > 32 && row_tiles >= kFewColsMfmaTiles) || (N > 16 && row_tiles >= kSkinnyTallTiles);
}

// Few-column launches: column tiles WC = ceil(N / 16) <= 4; row tiles per
// workgroup WR = 2, or 4 for very tall products, where re-reading the
// activations once per workgroup (from L2) costs more than the weights.
template <int WR>
SkinnyFn pick_skinny_wr(int N) {
    switch ((N + 15) / 16) {
    case 1: return i2_gemm_skinny_kernel<1, WR>;
    case 2: return i2_gemm_skinny_kernel<2, WR>;
    case 3: return i2_gemm_skinny_kernel<3, WR>;
    default: return i2_gemm_skinny_kernel<4, WR>;
    }
}
SkinnyFn pick_skinny(int N, int wr) { return wr == 4 ? pick_skinny_wr<4>(N) : pick_skinny_wr<2>(N); }

int check_mfma_shape(size_t out_len, size_t in_len) {
    if (!out_len || !in_len) return fail(OURO_ERR_SHAPE, "i2 mfma: empty shape");
    if (in_len % 256) return fail(OURO_ERR_SHAPE, "i2 mfma: in_len %zu is not a multiple of 256", in_len);
    if (out_len > (1u << 30) || in_len > (1u << 18)) return fail(OURO_ERR_SHAPE, "i2 mfma: shape too large");
    return OURO_OK;
}

}  // namespace

size_t i2_mfma_bytes(size_t out_len, size_t in_len) {
    if (!in_len || in_len % 256) return 0;
    return (out_len + 15) / 16 * (in_len / 256) * 1024;
}

int i2_tile_mfma(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *dst,
                 const float *w_scale, void *stream, int src_i2s) {
    int st = check_mfma_shape(out_len, in_len);
    if (st) return st;
    if (!canonical || !dst) return fail(OURO_ERR_INVALID_ARG, "ouro_i2_tile_mfma: NULL argument");
    if (reinterpret_cast<uintptr_t>(dst) % 16) return fail(OURO_ERR_ALIGN, "ouro_i2_tile_mfma: dst needs 16-byte alignment");
    const size_t bytes = i2_mfma_bytes(out_len, in_len);
    const long long words = static_cast<long long>(bytes / 4);
    hipLaunchKernelGGL(i2_tile_mfma_kernel, dim3(static_cast<unsigned>((words + 255) / 256)), dim3(256), 0,
                       as_stream(stream), canonical, reinterpret_cast<uint32_t *>(dst), static_cast<int>(out_len),
                       static_cast<int>(in_len), words, src_i2s);
    st = check_launch("i2_tile_mfma_kernel");
    if (st || !w_scale) return st;
    hipLaunchKernelGGL(copy_scale_mfma_kernel, dim3(1), dim3(1), 0, as_stream(stream), w_scale,
                       reinterpret_cast<float *>(dst + bytes));
    return check_launch("copy_scale_mfma_kernel");
}

// Up to 4 few-column products of the same activations (k = in_len, ncols
// <= 64 columns, each with its own weights, activations, scales and
// output) in one launch.
int i2_gemm_skinny_group(const GemmProblem *probs, int np, size_t in_len, size_t ncols, int x_tiled, void *stream) {
    if (np < 1 || np > kSkinnyGroup) return fail(OURO_ERR_INVALID_ARG, "i2 gemm group: %d products", np);
    if (!ncols || ncols > static_cast<size_t>(kSkinnyCols))
        return fail(OURO_ERR_SHAPE, "i2 gemm group: %zu columns (1..%d)", ncols, kSkinnyCols);
    SkinnyGroup g{};
    g.np = np;
    g.K = static_cast<int>(in_len);
    g.N = static_cast<int>(ncols);
    g.nkb = g.K / 256;
    g.x_tiled = x_tiled;
    long long blocks = 0;
    for (int i = 0; i < np; ++i) {
        const GemmProblem &p = probs[i];
        int st = check_mfma_shape(p.out_len, in_len);
        if (st) return st;
        if (!p.w || !p.w_scale || !p.xq || !p.act_scale || !p.y)
            return fail(OURO_ERR_INVALID_ARG, "i2 gemm group: NULL argument in product %d", i);
        if (reinterpret_cast<uintptr_t>(p.w) % 16 || reinterpret_cast<uintptr_t>(p.xq) % 16)
            return fail(OURO_ERR_ALIGN, "ouro_gemm_i2_mfma: weights and xq need 16-byte alignment");
        if ((p.epi.op != EPI_NONE || p.swiglu) && p.acc)
            return fail(OURO_ERR_INVALID_ARG, "i2 gemm group: an epilogue with int32 output in product %d", i);
        if (p.swiglu && (p.epi.op != EPI_NONE || p.out_len % 2))
            return fail(OURO_ERR_SHAPE, "i2 gemm group: SwiGLU pairs need an even row count and no other epilogue");
        g.p[i] = SkinnyProblem{reinterpret_cast<const uint4 *>(p.w), p.w_scale, p.xq, p.act_scale, p.y, p.acc,
                               static_cast<int>(p.out_len), p.epi, p.swiglu};
    }
    long long row_tiles = 0;
    for (int i = 0; i < np; ++i) row_tiles += (static_cast<long long>(probs[i].out_len) + 15) / 16;
    if (few_cols_on_mfma(g.N, row_tiles)) {
        GemmArgs args[kMfmaGroup];
        for (int i = 0; i < np; ++i)
            args[i] = GemmArgs{reinterpret_cast<const uint4 *>(probs[i].w), probs[i].w_scale, probs[i].xq,
                               probs[i].act_scale, probs[i].y, probs[i].acc, static_cast<int>(probs[i].out_len),
                               g.K, g.N, g.nkb, 0, x_tiled, probs[i].swiglu, probs[i].epi};
        return launch_mfma_group(args, np, stream);
    }
    const int wr = row_tiles >= kSkinnyTallTiles ? 4 : 2;
    for (int i = 0; i < np; ++i) {
        g.bstart[i] = static_cast<int>(blocks);
        blocks += ((static_cast<long long>(probs[i].out_len) + 15) / 16 + wr - 1) / wr;
    }
    g.bstart[np] = static_cast<int>(blocks);
    if (blocks > 0x7fffffffLL) return fail(OURO_ERR_SHAPE, "i2 gemm group: grid too large");
    // Few row blocks: split the column tiles into groups so the launch still
    // fills the chip; a row block's column groups are adjacent workgroups,
    // so the weights they share are read from HBM once and then from L2.
    g.tiles = (g.N + 15) / 16;
    int ncg = 1;
    if (g.tiles == 4 && blocks < 96) ncg = 4;
    else if (g.tiles % 2 == 0 && blocks < 192) ncg = 2;
    g.ncg = ncg;
    const int wc = g.tiles / ncg;
    const int maxw = skinny_waves(wc);
    const int waves = g.nkb < maxw ? g.nkb : maxw;
    if (blocks * ncg > 0x7fffffffLL) return fail(OURO_ERR_SHAPE, "i2 gemm group: grid too large");
    hipLaunchKernelGGL(pick_skinny(16 * wc, wr), dim3(static_cast<unsigned>(blocks * ncg)), dim3(kWave * waves), 0,
                       as_stream(stream), g);
    return check_launch("i2_gemm_skinny_kernel");
}

int i2_gemm_mfma(const uint8_t *w_mfma, size_t out_len, size_t in_len, const float *w_scale, const int8_t *xq,
                 const float *act_scale, size_t ncols, float *y, int32_t *acc, void *stream, int x_tiled, int swiglu,
                 const GemmEpilogue *epi) {
    int st = check_mfma_shape(out_len, in_len);
    if (st) return st;
    if (!w_mfma || !w_scale || !xq || !act_scale || !y || !ncols)
        return fail(OURO_ERR_INVALID_ARG, "ouro_gemm_i2_mfma: NULL argument or ncols == 0");
    if (ncols > (1u << 24)) return fail(OURO_ERR_SHAPE, "ouro_gemm_i2_mfma: ncols %zu too large", ncols);
    if (reinterpret_cast<uintptr_t>(w_mfma) % 16 || reinterpret_cast<uintptr_t>(xq) % 16)
        return fail(OURO_ERR_ALIGN, "ouro_gemm_i2_mfma: weights and xq need 16-byte alignment");
    GemmArgs a{};
    a.w = reinterpret_cast<const uint4 *>(w_mfma);
    a.w_scale = w_scale;
    a.xq = xq;
    a.act_scale = act_scale;
    a.y = y;
    a.acc = acc;
    a.M = static_cast<int>(out_len);
    a.K = static_cast<int>(in_len);
    a.N = static_cast<int>(ncols);
    a.nkb = a.K / 256;
    a.x_tiled = x_tiled;
    a.swiglu = swiglu;
    if (epi) a.epi = *epi;
    if (epi && (acc || swiglu || (epi->op != EPI_NONE && epi->op != EPI_RESID && ncols > static_cast<size_t>(kSkinnyCols))))
        return fail(OURO_ERR_INVALID_ARG, "i2 gemm: epilogue not supported with this output");
    if (swiglu && (x_tiled || acc || out_len % 2 || ncols <= static_cast<size_t>(kSkinnyCols)))
        return fail(OURO_ERR_SHAPE, "i2 gemm: the SwiGLU epilogue takes > %d row-major columns, an even row count "
                    "and no int32 output", kSkinnyCols);
    if (x_tiled && ncols > static_cast<size_t>(kSkinnyCols))
        return fail(OURO_ERR_SHAPE, "i2 gemm: fragment-ordered x is for <= %d columns", kSkinnyCols);
    if (ncols <= static_cast<size_t>(kSkinnyCols)) {
        const GemmProblem one{w_mfma, out_len, w_scale, xq, act_scale, y, acc, epi ? *epi : GemmEpilogue{}, 0};
        return i2_gemm_skinny_group(&one, 1, in_len, ncols, x_tiled, stream);
    }
    const int nrt = (a.M + 15) / 16;
    {
        const long long nrb = (nrt + 8LL * kBigTM - 1) / (8LL * kBigTM);  // 16-row tiles per workgroup: 8 kBigTM
        const long long big = nrb * ((a.N + kBigCols - 1) / kBigCols);
        if (big >= kBigMinBlocks) {
            if (big > 0x7fffffffLL) return fail(OURO_ERR_SHAPE, "ouro_gemm_i2_mfma: grid too large");
            a.nrb = static_cast<int>(nrb);
            hipLaunchKernelGGL(i2_gemm_big_kernel, dim3(static_cast<unsigned>(big)), dim3(kWave * kGemmWaves), 0,
                               as_stream(stream), a);
            return check_launch("i2_gemm_big_kernel");
        }
    }
    return launch_mfma_group(&a, 1, stream);
}

}  // namespace ouro

extern "C" {

size_t ouro_i2_mfma_bytes(size_t out_len, size_t in_len) { return ouro::i2_mfma_bytes(out_len, in_len); }

int ouro_i2_tile_mfma(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *dst,
                      const float *w_scale_or_null, void *stream) {
    OURO_REQUIRE_INIT();
    return ouro::i2_tile_mfma(canonical, out_len, in_len, dst, w_scale_or_null, stream, 0);
}

int ouro_i2s_tile_mfma(const uint8_t *i2s, size_t out_len, size_t in_len, uint8_t *dst, void *stream) {
    OURO_REQUIRE_INIT();
    if (!i2s) return ouro::fail(OURO_ERR_INVALID_ARG, "ouro_i2s_tile_mfma: NULL argument");
    return ouro::i2_tile_mfma(i2s, out_len, in_len, dst, reinterpret_cast<const float *>(i2s + out_len * in_len / 4),
                              stream, 1);
}

int ouro_gemm_i2_mfma(const uint8_t *w_mfma, size_t out_len, size_t in_len, const float *w_scale,
                      const int8_t *xq, const float *act_scale, size_t ncols, float *y, int32_t *acc_or_null,
                      void *stream) {
    OURO_REQUIRE_INIT();
    return ouro::i2_gemm_mfma(w_mfma, out_len, in_len, w_scale, xq, act_scale, ncols, y, acc_or_null, stream, 0, 0, nullptr);
}

}  // extern "C"
