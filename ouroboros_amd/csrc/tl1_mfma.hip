// tl1_mfma.hip - TL1 (PTQ1_0) matmul for K columns in one pass over the
// weights: matmul_tl1 (ops.rs:156-286) amortises one decode of each weight
// byte over K columns; here the trits are int8 MFMA operands and x is exact
// fixed point, so the K columns cost one weight stream.
//
// Weights.  A resident TL1 handle for several columns also keeps its trits
// in the int8 MFMA unit layout of the ternary GEMM (1 KiB per 16-row tile and
// 256-deep k block; lane l's word s holds row 16 rt + l%16, k = 256 kb +
// 64 s + 16 (l/16) + 4 j + i at bits 8 i + 2 j as the 2-bit two's complement
// of -trit; k padded to a multiple of 256 with zero trits), and the f16 scale
// d of every (row, group of 128) in an array [rows][groups].
//
// Activations.  Column c of x, group g (128 elements): with E the binary
// exponent of the group's largest |x| (|x| < 2^E), x_int = rint(x 2^(22-E)),
// |x_int| <= 2^22, split into balanced base-256 digits x_int = 65536 p0 +
// 256 p1 + p2 (each int8, |p0| <= 65).  The three digit planes of column c
// are the rows 4c + p of the MFMA A operand (row 4c + 3 is zero), laid out
// in its fragment order (one 1 KiB piece per k block, step and tile of 16
// rows: lane l holds A row l%16, k = 64 s + 16 (l/16) .. +16).  Elements
// below 2^(E-23) of a group lose their low bits (error <= 2^-23 of the
// group's largest |x|).
//
// Product.  The weights are the B operand, so D row 4c + p, column r is row
// r's sum against plane p of column c, and lane l = 16 q + r of the D
// fragment holds the three planes of column 4 t + q (tile t) for its own
// weight row r.  Per group, two 16x16x64 int8 MFMA steps give exact int32
// plane sums, which the lane combines exactly into T = sum_k trit x_int
// (65536 S0 + 256 S1 + S2, scaled back from the encoding), and adds
// d(r, g) 2^(E-22) T to an fp32 accumulator per (row, column).
#include "common.hpp"

#include <algorithm>
#include <cstddef>

namespace ouro {

namespace {

constexpr int kWave = 64;
constexpr int kWaves = 4;  // wavefronts per workgroup, stacked along the rows
constexpr int kRowsPerCol = 4;  // A rows of an x column: its three digit planes and a zero row
typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int tl1_trit_at(const uint8_t *grp, int e) {
    // element e of a 28-byte PTQ1_0 group (dequant.rs:146-171)
    int byte, n;
    if (e < 80) byte = e & 15, n = e >> 4;
    else if (e < 120) byte = 16 + ((e - 80) & 7), n = (e - 80) >> 3;
    else byte = 24 + ((e - 120) & 1), n = (e - 120) >> 1;
    uint32_t p3 = 1;
    for (int i = 0; i < n; ++i) p3 *= 3;
    const uint32_t q = (static_cast<uint32_t>(grp[byte]) * p3) & 0xffu;
    return static_cast<int>((q * 3u) >> 8) - 1;
}

__device__ __forceinline__ int tq1_trit_at(const uint8_t *blk, int e) {
    // element e of a 54-byte TQ1_0 block (dequant.rs:50-80): qs bytes 0..31
    // carry elements 32 n + m, bytes 32..47 elements 160 + 16 n + m, qh
    // bytes 48..51 elements 240 + 4 n + m, n the base-3 digit
    int byte, n;
    if (e < 160) byte = e & 31, n = e >> 5;
    else if (e < 240) byte = 32 + ((e - 160) & 15), n = (e - 160) >> 4;
    else byte = 48 + ((e - 240) & 3), n = (e - 240) >> 2;
    uint32_t p3 = 1;
    for (int i = 0; i < n; ++i) p3 *= 3;
    const uint32_t q = (static_cast<uint32_t>(blk[byte]) * p3) & 0xffu;
    return static_cast<int>((q * 3u) >> 8) - 1;
}

// One thread per 32-bit word of the unit layout (rows past M and k past K
// hold zero trits).  TQ: the source is TQ1_0 (54-byte blocks of 256), else
// TL1 (28-byte groups of 128).
template <bool TQ>
__global__ void tl1_tile_mfma_kernel(const uint8_t *__restrict__ raw, uint32_t *__restrict__ dst, int M, int K,
                                     int nkb, long long total_words) {
    const long long id = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= total_words) return;
    const long long unit = id / 256;
    const int rem = static_cast<int>(id % 256);
    const int l = rem / 4, s = rem % 4;
    const long long rt = unit / nkb;
    const int kb = static_cast<int>(unit % nkb);
    const long long row = rt * 16 + (l % 16);
    const int kbase = 256 * kb + 64 * s + 16 * (l / 16);
    const long long rowb = TQ ? static_cast<long long>(K / 256) * 54 : static_cast<long long>(K / 128) * 28;
    uint32_t word = 0;
    if (row < M) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = kbase + 4 * j + i;
                if (k < K) {
                    const int t = TQ ? tq1_trit_at(raw + row * rowb + static_cast<long long>(k / 256) * 54, k % 256)
                                     : tl1_trit_at(raw + row * rowb + static_cast<long long>(k / 128) * 28, k % 128);
                    word |= (static_cast<uint32_t>(-t) & 3u) << (8 * i + 2 * j);
                }
            }
    }
    dst[id] = word;
}

// d of every (row, group of 128) as f16 bits; groups past K / 128 are 0.
// TQ: both 128-groups of a TQ1_0 block take the block's d (bytes 52, 53).
template <bool TQ>
__global__ void tl1_scales_kernel(const uint8_t *__restrict__ raw, uint16_t *__restrict__ d, int M, int K, int G) {
    const long long id = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= static_cast<long long>(M) * G) return;
    const long long row = id / G;
    const int g = static_cast<int>(id % G);
    uint16_t v = 0;
    if (g < K / 128) {
        const uint8_t *p = TQ ? raw + row * (static_cast<long long>(K / 256) * 54) + static_cast<long long>(g / 2) * 54 + 52
                              : raw + row * (static_cast<long long>(K / 128) * 28) + static_cast<long long>(g) * 28 + 26;
        v = static_cast<uint16_t>(p[0] | (p[1] << 8));
    }
    d[id] = v;
}

struct XprepArgs {
    const float *x;  // [ncols][K]
    int8_t *xb;      // A fragments: [nkb][4 steps][tiles][64 lanes][16 bytes]
    float *wt;       // [G][4 tiles] 2^(E-22) of each column
    int32_t *sx;     // [G][4 tiles] each column's sum of x_int over the group
    int K, G, tiles, ncols;
};
static_assert(sizeof(XprepArgs) == 48, "XprepArgs: kernel argument layout");

// One workgroup of 128 threads per (group g, virtual column c); columns past
// ncols (up to the last tile's end) and k past K write zero digits.
__global__ __launch_bounds__(128) void tl1_xprep_kernel(XprepArgs a) {
    __shared__ float red[2];
    __shared__ int xsum[2];
    const int g = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
    const int k = g * 128 + t;
    const float x = (c < a.ncols && k < a.K) ? a.x[static_cast<long long>(c) * a.K + k] : 0.f;
    float m = fabsf(x);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, xor_shfl(m, off));
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    m = fmaxf(red[0], red[1]);
    int E = 0;
    (void)frexpf(m, &E);  // m = f 2^E, f in [0.5, 1): |x| < 2^E (E = 0 for m = 0)
    const int xi = static_cast<int>(rintf(ldexpf(x, 22 - E)));  // exact scaling, one rounding
    const int p2 = ((xi + 128) & 255) - 128;
    const int r1 = (xi - p2) >> 8;  // exact: xi - p2 is a multiple of 256
    const int p1 = ((r1 + 128) & 255) - 128;
    const int p0 = (r1 - p1) >> 8;
    const int dig[kRowsPerCol] = {p0, p1, p2, 0};
    const int kb = k >> 8, s = (k & 255) >> 6, quarter = (k & 63) >> 4, byte = k & 15;
    int v = xi;  // the group's sum of x_int (|sum| <= 2^29)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += xor_shfl(v, off);
    if ((t & 63) == 0) xsum[t >> 6] = v;
    __syncthreads();
#pragma unroll
    for (int p = 0; p < kRowsPerCol; ++p) {
        const int j = kRowsPerCol * c + p;
        const int ct = j >> 4, lane = (j & 15) + 16 * quarter;
        a.xb[((static_cast<long long>(kb) * 4 + s) * a.tiles + ct) * 1024 + lane * 16 + byte] = static_cast<int8_t>(dig[p]);
    }
    if (t == 0) {
        a.wt[static_cast<long long>(g) * 4 * a.tiles + c] = (c < a.ncols) ? ldexpf(1.0f, E - 22) : 0.f;
        a.sx[static_cast<long long>(g) * 4 * a.tiles + c] = xsum[0] + xsum[1];
    }
}

struct Tl1MmArgs {
    const v4u *w;        // unit layout [nrt][nkb][64] x 16 B (RAW: unused)
    const uint16_t *d;   // [M][G] f16 (RAW: unused)
    const uint8_t *raw;  // RAW: the reference's row-major groups of 28 bytes
    const int8_t *xb;    // A fragments
    const float *wt;     // [G][4 tiles]
    const int32_t *sx;   // [G][4 tiles] sums of x_int (RAW)
    float *y;            // [ncols][M]
    int M, nkb, G, tiles, ncols, nrb, graw;  // graw: groups of a raw row (K / 128)
};
static_assert(sizeof(Tl1MmArgs) == 88, "Tl1MmArgs: kernel argument layout");

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned v4a __attribute__((ext_vector_type(4), aligned(4)));
typedef unsigned v3a __attribute__((ext_vector_type(3), aligned(4)));

// Base-3 digits (0..2) of the four bytes of S, byte b taking digit n_b
// (dequant.rs:134-138: ((v * 3^n mod 256) * 3) >> 8), with the multipliers
// packed per 16-bit half: me = 3^n0 | 3^n2 << 16 for bytes 0 and 2, mo the
// same for bytes 1 and 3.  One byte per 16-bit lane keeps every product
// within 16 bits.
__device__ __forceinline__ uint32_t digits4(uint32_t S, uint32_t me, uint32_t mo) {
    const u16x2 e = __builtin_bit_cast(u16x2, S & 0x00ff00ffu);
    const u16x2 o = __builtin_bit_cast(u16x2, (S >> 8) & 0x00ff00ffu);
    const u16x2 k3 = {3, 3};
    const u16x2 ff = {0xff, 0xff};
    const u16x2 qe = ((e * __builtin_bit_cast(u16x2, me)) & ff) * k3;
    const u16x2 qo = ((o * __builtin_bit_cast(u16x2, mo)) & ff) * k3;
    const uint32_t de = __builtin_bit_cast(uint32_t, static_cast<u16x2>(qe >> 8));
    const uint32_t dd = __builtin_bit_cast(uint32_t, static_cast<u16x2>(qo >> 8));
    return de | (dd << 8);
}

// Workgroup: 4 wavefronts along the rows, wavefront w owns row tiles
// (4 rb + w) WR .. +WR-1 and all WC column tiles.  Per 256-deep k block the
// workgroup stages the block's 4 WC A pieces of x in LDS (double-buffered,
// prefetched a block ahead in registers) and each wavefront loads its WR
// weight units and their scales a block ahead.  Indices are clamped, so
// every load is unconditional.
//
// RAW: the weights are the reference's row-major payload.  Lane l loads the
// 28 bytes of group g of row 16 rt + l%16 (one 16- and one 12-byte load) and
// makes its B fragment of each step from them: the base-3 digit (0..2) of
// every element, elements 16 (l/16) .. +15 of the step's half group in the
// payload's order (qs bytes 0..15 carry elements 16 n + m, bytes 16..23
// elements 80 + 8 n + m, bytes 24, 25 elements 120 + 2 n + h).  The MFMA
// then sums digit * x; the trit sum is that minus the group's sum of x_int
// (exact integers), and the group scale d comes from bytes 26, 27 of the
// lane's own row.
template <int WR, int WC, bool RAW, bool STG = false>
__global__ __launch_bounds__(kWave *kWaves) void tl1_mfma_kernel(Tl1MmArgs a) {
    constexpr int kPiece = 1024;
    __shared__ __attribute__((aligned(16))) int8_t xs[2][4 * WC * kPiece];
    // STG (RAW, one row tile a wavefront, groups a row a multiple of 4, the
    // payload 16-byte aligned): each wavefront copies its 16 rows' 112
    // contiguous bytes of two k blocks (four groups) into its own LDS rows
    // with contiguous 16-byte loads, instead of each lane loading its row's
    // groups (a 16-lane quarter of a load then reads 16 rows).  Rows lie 144
    // bytes apart, so a dword read of the 16 rows hits each bank at most twice
    // (128 bytes apart they all fell in one bank: twice as slow).
    __shared__ __attribute__((aligned(16))) uint8_t wst[STG ? kWaves : 1][STG ? 16 * 144 : 16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rt0 = (static_cast<int>(blockIdx.x) * kWaves + wave) * WR;
    const int nrt = (a.M + 15) / 16;
    const int q = lane >> 4;

    // RAW: per-lane digit multipliers of the odd steps' four B dwords (the
    // even steps take digit q of qs bytes 0..15: 3^q in both halves)
    uint32_t m_even = 0, me1[4] = {0, 0, 0, 0}, mo1[4] = {0, 0, 0, 0};
    if constexpr (RAW) {
        const uint32_t p3q = q == 0 ? 1u : q == 1 ? 3u : q == 2 ? 9u : 27u;
        m_even = p3q | (p3q << 16);
        const uint32_t lo = q == 0 ? 81u : q == 1 ? 1u : q == 2 ? 9u : 81u;   // dwords 0, 1
        const uint32_t hi = q == 0 ? 81u : q == 1 ? 3u : q == 2 ? 27u : 0u;   // dwords 2, 3 (q = 3: below)
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            const uint32_t m = dw < 2 ? lo : hi;
            me1[dw] = mo1[dw] = m | (m << 16);
        }
        if (q == 3) {  // bytes (24, 25, 24, 25): digits (0, 0, 1, 1), then (2, 2, 3, 3)
            me1[2] = mo1[2] = 1u | (3u << 16);
            me1[3] = mo1[3] = 9u | (27u << 16);
        }
    }

    v4u xr[WC];
    auto load_x = [&](int kb) {
#pragma unroll
        for (int i = 0; i < WC; ++i) {
            const int c = tid + kWave * kWaves * i;  // chunk c: piece c / 64 (step-major), lane c % 64
            const int pq = c / 64, s = pq / WC, ct = pq % WC;
            xr[i] = *reinterpret_cast<const v4u *>(a.xb + ((static_cast<long long>(kb) * 4 + s) * a.tiles + ct) * kPiece +
                                                   (c % 64) * 16);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < WC; ++i) *reinterpret_cast<v4u *>(&xs[buf][16 * (tid + kWave * kWaves * i)]) = xr[i];
    };
    // unit layout: the lane's word of each step and the f16 scales of its row
    // for the block's two groups; RAW: the 7 dwords of its row's groups
    v4u wr[WR];
    uint32_t dr[WR];
    uint32_t rr[WR][2][7];
    auto load_w = [&](int kb) {
#pragma unroll
        for (int r = 0; r < WR; ++r) {
            const int rt = min(rt0 + r, nrt - 1);
            const long long row = min(rt * 16 + (lane & 15), a.M - 1);
            if constexpr (RAW) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int g = min(2 * kb + h, a.graw - 1);  // the padding group loads a real one, d = 0 below
                    const uint8_t *p = a.raw + row * (static_cast<long long>(a.graw) * 28) + static_cast<long long>(g) * 28;
                    const v4a u4 = *reinterpret_cast<const v4a *>(p);
                    const v3a u3 = *reinterpret_cast<const v3a *>(p + 16);
                    rr[r][h][0] = u4.x, rr[r][h][1] = u4.y, rr[r][h][2] = u4.z, rr[r][h][3] = u4.w;
                    rr[r][h][4] = u3.x, rr[r][h][5] = u3.y, rr[r][h][6] = u3.z;
                }
            } else {
                wr[r] = a.w[(static_cast<long long>(rt) * a.nkb + kb) * kWave + lane];
                dr[r] = *reinterpret_cast<const uint32_t *>(a.d + row * a.G + 2 * kb);
            }
        }
    };

    float yacc[WR][WC];
#pragma unroll
    for (int r = 0; r < WR; ++r)
#pragma unroll
        for (int c = 0; c < WC; ++c) yacc[r][c] = 0.f;

    v4u sg[2];
    const int rowt = min(rt0, nrt - 1) * 16;
    auto issue_seg = [&](int pair) {
        const int pc = min(pair, a.nkb / 2 - 1);  // past the last pair: loaded again, never staged
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int id = min(64 * i + lane, 111);
            const long long row = min(rowt + id / 7, a.M - 1);
            sg[i] = *reinterpret_cast<const v4u *>(a.raw + row * (static_cast<long long>(a.graw) * 28) + 112LL * pc +
                                                   16 * (id % 7));
        }
    };
    auto stage_seg = [&]() {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int id = 64 * i + lane;
            if (id < 112) *reinterpret_cast<v4u *>(&wst[wave][144 * (id / 7) + 16 * (id % 7)]) = sg[i];
        }
    };

    load_x(0);
    if constexpr (STG) issue_seg(0);
    else load_w(0);
    store_x(0);
    __syncthreads();
    for (int kb = 0; kb < a.nkb; ++kb) {
        v4u wc[WR];
        uint32_t dc[WR];
        uint32_t rc[WR][2][7];
        if constexpr (STG) {
            if ((kb & 1) == 0) {  // uniform
                stage_seg();
                issue_seg(kb / 2 + 1);
            }
            const uint8_t *gp = &wst[wave][144 * (lane & 15) + 56 * (kb & 1)];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 7; ++i) rc[0][h][i] = *reinterpret_cast<const uint32_t *>(gp + 28 * h + 4 * i);
        }
#pragma unroll
        for (int r = 0; r < WR; ++r) {
            if constexpr (STG) {
            } else if constexpr (RAW) {
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int i = 0; i < 7; ++i) rc[r][h][i] = rr[r][h][i];
            } else {
                wc[r] = wr[r];
                dc[r] = dr[r];
            }
        }
        const bool more = kb + 1 < a.nkb;
        if (more) {
            load_x(kb + 1);
            if constexpr (!STG) load_w(kb + 1);
        }
        const int8_t *xbuf = xs[kb & 1] + 16 * lane;
#pragma unroll
        for (int half = 0; half < 2; ++half) {  // the block's two groups
            const int g = 2 * kb + half;
            v4i acc[WR][WC];
#pragma unroll
            for (int r = 0; r < WR; ++r)
#pragma unroll
                for (int c = 0; c < WC; ++c) acc[r][c] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const int s = 2 * half + s2;
                v4i Bw[WR];
#pragma unroll
                for (int r = 0; r < WR; ++r) {
                    if constexpr (RAW) {
                        const uint32_t *w7 = rc[r][half];
                        uint32_t d4[4];
                        if (s2 == 0) {
#pragma unroll
                            for (int dw = 0; dw < 4; ++dw) d4[dw] = digits4(w7[dw], m_even, m_even);
                        } else {
                            const uint32_t qh = (w7[6] & 0xffffu) * 0x00010001u;  // bytes 24, 25, 24, 25
                            const uint32_t src[4] = {q == 0 ? w7[0] : w7[4], q == 0 ? w7[1] : w7[5],
                                                     q == 0 ? w7[2] : q == 3 ? qh : w7[4],
                                                     q == 0 ? w7[3] : q == 3 ? qh : w7[5]};
#pragma unroll
                            for (int dw = 0; dw < 4; ++dw) d4[dw] = digits4(src[dw], me1[dw], mo1[dw]);
                        }
                        Bw[r] = v4i{static_cast<int>(d4[0]), static_cast<int>(d4[1]), static_cast<int>(d4[2]),
                                    static_cast<int>(d4[3])};
                    } else {
                        const uint32_t wd = s == 0 ? wc[r][0] : s == 1 ? wc[r][1] : s == 2 ? wc[r][2] : wc[r][3];
                        Bw[r] = v4i{static_cast<int>((wd << 6) & 0xC0C0C0C0u), static_cast<int>((wd << 4) & 0xC0C0C0C0u),
                                    static_cast<int>((wd << 2) & 0xC0C0C0C0u), static_cast<int>(wd & 0xC0C0C0C0u)};
                    }
                }
#pragma unroll
                for (int c = 0; c < WC; ++c) {
                    const v4i Ax = *reinterpret_cast<const v4i *>(xbuf + (s * WC + c) * kPiece);
#pragma unroll
                    for (int r = 0; r < WR; ++r)
                        acc[r][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Ax, Bw[r], acc[r][c], 0, 0, 0);
                }
            }
            // the group's term: d(row) 2^(E-22) T, T = sum_k trit x_int from the
            // three plane sums (D rows 4 q + p of the lane)
#pragma unroll
            for (int r = 0; r < WR; ++r) {
                float dv;
                if constexpr (RAW) {
                    dv = g < a.graw
                        ? static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(rc[r][half][6] >> 16)))
                        : 0.f;
                } else {
                    dv = static_cast<float>(
                        __builtin_bit_cast(_Float16, static_cast<uint16_t>(half ? dc[r] >> 16 : dc[r] & 0xffffu)));
                }
#pragma unroll
                for (int c = 0; c < WC; ++c) {
                    const long long wi = static_cast<long long>(g) * 4 * a.tiles + 4 * c + q;
                    int T;
                    if constexpr (RAW)  // digit = trit + 1: the digit sum less the group's sum of x_int
                        T = (acc[r][c][0] << 16) + (acc[r][c][1] << 8) + acc[r][c][2] - a.sx[wi];
                    else  // the codes are -64 trit: every plane sum is a multiple of 64
                        T = -((acc[r][c][0] << 10) + (acc[r][c][1] << 2) + (acc[r][c][2] >> 6));
                    yacc[r][c] = __builtin_fmaf(static_cast<float>(T), dv * a.wt[wi], yacc[r][c]);
                }
            }
        }
        if (more) store_x((kb + 1) & 1);
        __syncthreads();
    }
    // lane 16 q + r holds row 16 rt + r of columns 4 c + q
#pragma unroll
    for (int r = 0; r < WR; ++r) {
        const int rt = rt0 + r, row = rt * 16 + (lane & 15);
#pragma unroll
        for (int c = 0; c < WC; ++c) {
            const int col = 4 * c + q;
            if (rt < nrt && row < a.M && col < a.ncols) a.y[static_cast<long long>(col) * a.M + row] = yacc[r][c];
        }
    }
}

}  // namespace

// Columns one launch handles: 4 A rows each, up to 4 tiles of 16.
constexpr int kTl1MmCols = 16;

size_t tl1_mfma_code_bytes(size_t M, size_t K) { return (M + 15) / 16 * ((K + 255) / 256) * 1024; }
size_t tl1_mfma_scale_bytes(size_t M, size_t K) { return M * ((K + 255) / 256 * 2) * sizeof(uint16_t); }
// A fragments and column weights for up to ncols columns (one launch's share).
size_t tl1_xprep_bytes(size_t K, size_t ncols) {
    const size_t nc = std::min(ncols, static_cast<size_t>(kTl1MmCols));
    const size_t tiles = (kRowsPerCol * nc + 15) / 16;
    const size_t nkb = (K + 255) / 256;
    return nkb * 4 * tiles * 1024 + nkb * 2 * 4 * tiles * (sizeof(float) + sizeof(int32_t));
}

namespace {
template <bool TQ>
int tile_mfma(const uint8_t *raw, size_t M, size_t K, uint8_t *codes, uint16_t *scales, void *stream) {
    if (!raw || !codes || !scales || !M || !K || K % (TQ ? 256 : 128) || M > 0x7fffffffULL || K > 0x7fffffffULL)
        return fail(OURO_ERR_SHAPE, "%s mfma tiling: bad shape %zu x %zu", TQ ? "tq1_0" : "tl1", M, K);
    const int nkb = static_cast<int>((K + 255) / 256), G = 2 * nkb;
    const long long words = static_cast<long long>(tl1_mfma_code_bytes(M, K) / 4);
    const hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(tl1_tile_mfma_kernel<TQ>, dim3(static_cast<unsigned>((words + 255) / 256)), dim3(256), 0, s,
                       raw, reinterpret_cast<uint32_t *>(codes), static_cast<int>(M), static_cast<int>(K), nkb, words);
    int st = check_launch("tl1_tile_mfma_kernel");
    if (st) return st;
    const long long n = static_cast<long long>(M) * G;
    hipLaunchKernelGGL(tl1_scales_kernel<TQ>, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, raw,
                       scales, static_cast<int>(M), static_cast<int>(K), G);
    return check_launch("tl1_scales_kernel");
}
}  // namespace

// Raw TL1 payload (device, row-major groups) -> unit layout + scales.
int tl1_tile_mfma(const uint8_t *raw, size_t M, size_t K, uint8_t *codes, uint16_t *scales, void *stream) {
    return tile_mfma<false>(raw, M, K, codes, scales, stream);
}

// Raw TQ1_0 payload (device, row-major 54-byte blocks) -> the same unit
// layout + scales (each block's d for both of its 128-groups).
int tq1_tile_mfma(const uint8_t *raw, size_t M, size_t K, uint8_t *codes, uint16_t *scales, void *stream) {
    return tile_mfma<true>(raw, M, K, codes, scales, stream);
}

namespace {
// y[c][M] = W x_c for ncols columns of x [ncols][K]; W in the unit layout
// (codes, scales) or, raw != nullptr, the reference's payload.
int tl1_mfma_run(const uint8_t *codes, const uint16_t *scales, const uint8_t *raw, size_t M, size_t K, const float *x,
                 size_t ncols, float *y, void *scratch, void *stream) {
    if ((!raw && (!codes || !scales)) || !x || !y || !scratch) return fail(OURO_ERR_INVALID_ARG, "tl1 matmul: NULL argument");
    if (!M || !K || K % 128 || !ncols || M > 0x7fffffffULL || K > 0x7fffffffULL)
        return fail(OURO_ERR_SHAPE, "tl1 matmul: bad shape");
    if ((reinterpret_cast<uintptr_t>(codes) | reinterpret_cast<uintptr_t>(scratch)) % 16 ||
        (reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(raw)) % 4)
        return fail(OURO_ERR_ALIGN, "tl1 matmul: alignment");
    const hipStream_t s = as_stream(stream);
    const int nkb = static_cast<int>((K + 255) / 256);
    for (size_t c0 = 0; c0 < ncols; c0 += kTl1MmCols) {
        const int nc = static_cast<int>(std::min(ncols - c0, static_cast<size_t>(kTl1MmCols)));
        const int tiles = (kRowsPerCol * nc + 15) / 16;
        int8_t *xb = static_cast<int8_t *>(scratch);
        float *wt = reinterpret_cast<float *>(xb + static_cast<size_t>(nkb) * 4 * tiles * 1024);
        int32_t *sx = reinterpret_cast<int32_t *>(wt + static_cast<size_t>(nkb) * 2 * 4 * tiles);
        XprepArgs xa{x + c0 * K, xb, wt, sx, static_cast<int>(K), 2 * nkb, tiles, nc};
        const int vcols = 4 * tiles;  // virtual columns cover every A row
        hipLaunchKernelGGL(tl1_xprep_kernel, dim3(2 * nkb, vcols), dim3(128), 0, s, xa);
        int st = check_launch("tl1_xprep_kernel");
        if (st) return st;
        Tl1MmArgs a{reinterpret_cast<const v4u *>(codes), scales, raw, xb, wt, sx, y + c0 * M, static_cast<int>(M), nkb,
                    2 * nkb, tiles, nc, 0, static_cast<int>(K / 128)};
        const int nrt = static_cast<int>((M + 15) / 16);
        // the raw payload's digit decode fills the registers: one row tile a
        // wavefront there (184 against 219 us at 8 columns of 248320x5120),
        // two on the unit layout (102 against 116 us)
        const int wr = raw ? 1 : 2;
        a.nrb = (nrt + kWaves * wr - 1) / (kWaves * wr);
        const dim3 grid(a.nrb), block(kWave * kWaves);
        if (raw && a.graw % 4 == 0 && reinterpret_cast<uintptr_t>(raw) % 16 == 0) {
            if (tiles == 1) hipLaunchKernelGGL((tl1_mfma_kernel<1, 1, true, true>), grid, block, 0, s, a);
            else if (tiles == 2) hipLaunchKernelGGL((tl1_mfma_kernel<1, 2, true, true>), grid, block, 0, s, a);
            else if (tiles == 3) hipLaunchKernelGGL((tl1_mfma_kernel<1, 3, true, true>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((tl1_mfma_kernel<1, 4, true, true>), grid, block, 0, s, a);
        } else if (raw) {
            if (tiles == 1) hipLaunchKernelGGL((tl1_mfma_kernel<1, 1, true>), grid, block, 0, s, a);
            else if (tiles == 2) hipLaunchKernelGGL((tl1_mfma_kernel<1, 2, true>), grid, block, 0, s, a);
            else if (tiles == 3) hipLaunchKernelGGL((tl1_mfma_kernel<1, 3, true>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((tl1_mfma_kernel<1, 4, true>), grid, block, 0, s, a);
        } else {
            if (tiles == 1) hipLaunchKernelGGL((tl1_mfma_kernel<2, 1, false>), grid, block, 0, s, a);
            else if (tiles == 2) hipLaunchKernelGGL((tl1_mfma_kernel<2, 2, false>), grid, block, 0, s, a);
            else if (tiles == 3) hipLaunchKernelGGL((tl1_mfma_kernel<2, 3, false>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((tl1_mfma_kernel<2, 4, false>), grid, block, 0, s, a);
        }
        st = check_launch("tl1_mfma_kernel");
        if (st) return st;
    }
    return OURO_OK;
}
}  // namespace

// W in the unit layout (a resident handle).  scratch: tl1_xprep_bytes(K,
// ncols) bytes, 16-byte aligned.
int tl1_mfma_matmul(const uint8_t *codes, const uint16_t *scales, size_t M, size_t K, const float *x, size_t ncols,
                    float *y, void *scratch, void *stream) {
    return tl1_mfma_run(codes, scales, nullptr, M, K, x, ncols, y, scratch, stream);
}

// W the reference's row-major payload on the device (4-byte aligned).
int tl1_mfma_matmul_raw(const uint8_t *raw, size_t M, size_t K, const float *x, size_t ncols, float *y, void *scratch,
                        void *stream) {
    return tl1_mfma_run(nullptr, nullptr, raw, M, K, x, ncols, y, scratch, stream);
}

}  // namespace ouro
