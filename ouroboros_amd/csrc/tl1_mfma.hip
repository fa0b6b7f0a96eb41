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
// 256 p1 + p2 (each int8).  The three digit planes of every column are the
// columns 3c + p of the MFMA B operand, laid out in its fragment order (one
// 1 KiB piece per k block, step and tile of 16 B columns: lane l holds B
// column l%16, k = 64 s + 16 (l/16) .. +16).  Elements below 2^(E-23) of a
// group lose their low bits (error <= 2^-23 of the group's largest |x|).
//
// Product.  Per group, two 16x16x64 int8 MFMA steps give the exact int32 sum
// A = -64 sum_k trit x_int_p for every (row, plane column); the group's term
// d(row, g) * w(g, column) * A, w = -2^(E - 28 + 8 (2 - p)) (the digit weight,
// the exponent and the -64 of the A encoding), is added to an fp32
// accumulator per (row, plane column); the three planes of a column are added
// at the end.
#include "common.hpp"

#include <algorithm>
#include <cstddef>

namespace ouro {

namespace {

constexpr int kWave = 64;
constexpr int kWaves = 4;  // wavefronts per workgroup, stacked along the rows
constexpr int kPlanes = 3;
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

// One thread per 32-bit word of the unit layout (rows past M and k past K
// hold zero trits).
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
    const long long rowb = static_cast<long long>(K / 128) * 28;
    uint32_t word = 0;
    if (row < M) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = kbase + 4 * j + i;
                if (k < K) {
                    const int t = tl1_trit_at(raw + row * rowb + static_cast<long long>(k / 128) * 28, k % 128);
                    word |= (static_cast<uint32_t>(-t) & 3u) << (8 * i + 2 * j);
                }
            }
    }
    dst[id] = word;
}

// d of every (row, group) as f16 bits; groups past K / 128 are 0.
__global__ void tl1_scales_kernel(const uint8_t *__restrict__ raw, uint16_t *__restrict__ d, int M, int K, int G) {
    const long long id = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= static_cast<long long>(M) * G) return;
    const long long row = id / G;
    const int g = static_cast<int>(id % G);
    uint16_t v = 0;
    if (g < K / 128) {
        const uint8_t *p = raw + row * (static_cast<long long>(K / 128) * 28) + static_cast<long long>(g) * 28;
        v = static_cast<uint16_t>(p[26] | (p[27] << 8));
    }
    d[id] = v;
}

struct XprepArgs {
    const float *x;  // [ncols][K]
    int8_t *xb;      // B fragments: [nkb][4 steps][tiles][64 lanes][16 bytes]
    float *wt;       // [G][16 tiles] plane weights
    int K, G, tiles, ncols;
};
static_assert(sizeof(XprepArgs) == 40, "XprepArgs: kernel argument layout");

// One workgroup of 128 threads per (group g, virtual column c); columns past
// ncols (up to the last tile's end) and k past K write zero digits.
__global__ __launch_bounds__(128) void tl1_xprep_kernel(XprepArgs a) {
    __shared__ float red[2];
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
    const int dig[kPlanes] = {p0, p1, p2};
    const int kb = k >> 8, s = (k & 255) >> 6, quarter = (k & 63) >> 4, byte = k & 15;
#pragma unroll
    for (int p = 0; p < kPlanes; ++p) {
        const int j = kPlanes * c + p;
        if (j >= 16 * a.tiles) continue;
        const int ct = j >> 4, lane = (j & 15) + 16 * quarter;
        a.xb[((static_cast<long long>(kb) * 4 + s) * a.tiles + ct) * 1024 + lane * 16 + byte] = static_cast<int8_t>(dig[p]);
        if (t == 0) a.wt[static_cast<long long>(g) * 16 * a.tiles + j] = (c < a.ncols) ? -ldexpf(1.0f, E - 28 + 8 * (2 - p)) : 0.f;
    }
}

struct Tl1MmArgs {
    const v4u *w;        // unit layout [nrt][nkb][64] x 16 B
    const uint16_t *d;   // [M][G] f16
    const int8_t *xb;    // B fragments
    const float *wt;     // [G][16 tiles]
    float *y;            // [ncols][M]
    int M, nkb, G, tiles, ncols, nrb;
};
static_assert(sizeof(Tl1MmArgs) == 64, "Tl1MmArgs: kernel argument layout");

// Workgroup: 4 wavefronts along the rows, wavefront w owns row tiles
// (4 rb + w) WR .. +WR-1 and all WC column tiles.  Per 256-deep k block the
// workgroup stages the block's 4 WC B pieces in LDS (double-buffered,
// prefetched a block ahead in registers) and each wavefront loads its WR
// weight units and their scales a block ahead.  Indices are clamped, so
// every load is unconditional.
template <int WR, int WC>
__global__ __launch_bounds__(kWave *kWaves) void tl1_mfma_kernel(Tl1MmArgs a) {
    constexpr int kPiece = 1024;
    __shared__ __attribute__((aligned(16))) int8_t xs[2][4 * WC * kPiece];
    __shared__ float comb[kWaves][16][16 * WC + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rt0 = (static_cast<int>(blockIdx.x) * kWaves + wave) * WR;
    const int nrt = (a.M + 15) / 16;

    v4u xr[WC];
    auto load_x = [&](int kb) {
#pragma unroll
        for (int i = 0; i < WC; ++i) {
            const int c = tid + kWave * kWaves * i;  // chunk c: piece c / 64 (step-major), lane c % 64
            const int q = c / 64, s = q / WC, ct = q % WC;
            xr[i] = *reinterpret_cast<const v4u *>(a.xb + ((static_cast<long long>(kb) * 4 + s) * a.tiles + ct) * kPiece +
                                                   (c % 64) * 16);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < WC; ++i) *reinterpret_cast<v4u *>(&xs[buf][16 * (tid + kWave * kWaves * i)]) = xr[i];
    };
    v4u wr[WR];
    uint32_t dr[WR][4];  // f16 scales of the lane's 4 rows, groups 2 kb (low half) and 2 kb + 1 (high half)
    auto load_w = [&](int kb) {
#pragma unroll
        for (int r = 0; r < WR; ++r) {
            const int rt = min(rt0 + r, nrt - 1);
            wr[r] = a.w[(static_cast<long long>(rt) * a.nkb + kb) * kWave + lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = min(rt * 16 + 4 * (lane >> 4) + e, a.M - 1);
                dr[r][e] = *reinterpret_cast<const uint32_t *>(a.d + static_cast<long long>(row) * a.G + 2 * kb);
            }
        }
    };

    float yacc[WR][WC][4];
#pragma unroll
    for (int r = 0; r < WR; ++r)
#pragma unroll
        for (int c = 0; c < WC; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) yacc[r][c][e] = 0.f;

    load_x(0);
    load_w(0);
    store_x(0);
    __syncthreads();
    for (int kb = 0; kb < a.nkb; ++kb) {
        v4u wc[WR];
        uint32_t dc[WR][4];
#pragma unroll
        for (int r = 0; r < WR; ++r) {
            wc[r] = wr[r];
#pragma unroll
            for (int e = 0; e < 4; ++e) dc[r][e] = dr[r][e];
        }
        const bool more = kb + 1 < a.nkb;
        if (more) {
            load_x(kb + 1);
            load_w(kb + 1);
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
                v4i A[WR];
#pragma unroll
                for (int r = 0; r < WR; ++r) {
                    const uint32_t wd = s == 0 ? wc[r][0] : s == 1 ? wc[r][1] : s == 2 ? wc[r][2] : wc[r][3];
                    A[r] = v4i{static_cast<int>((wd << 6) & 0xC0C0C0C0u), static_cast<int>((wd << 4) & 0xC0C0C0C0u),
                               static_cast<int>((wd << 2) & 0xC0C0C0C0u), static_cast<int>(wd & 0xC0C0C0C0u)};
                }
#pragma unroll
                for (int c = 0; c < WC; ++c) {
                    const v4i B = *reinterpret_cast<const v4i *>(xbuf + (s * WC + c) * kPiece);
#pragma unroll
                    for (int r = 0; r < WR; ++r)
                        acc[r][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[r], B, acc[r][c], 0, 0, 0);
                }
            }
            // the group's term: d(row) * w(g, column) * acc
#pragma unroll
            for (int c = 0; c < WC; ++c) {
                const float wv = a.wt[static_cast<long long>(g) * 16 * a.tiles + 16 * c + (lane & 15)];
#pragma unroll
                for (int r = 0; r < WR; ++r)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint16_t db = static_cast<uint16_t>(half ? dc[r][e] >> 16 : dc[r][e] & 0xffffu);
                        const float dv = static_cast<float>(__builtin_bit_cast(_Float16, db));
                        yacc[r][c][e] = __builtin_fmaf(static_cast<float>(acc[r][c][e]), dv * wv, yacc[r][c][e]);
                    }
            }
        }
        if (more) store_x((kb + 1) & 1);
        __syncthreads();
    }
    // the planes of a column lie in three B columns: add them through LDS,
    // one row tile at a time (each wavefront its own region)
#pragma unroll
    for (int r = 0; r < WR; ++r) {
        const int rt = rt0 + r;
#pragma unroll
        for (int c = 0; c < WC; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) comb[wave][4 * (lane >> 4) + e][16 * c + (lane & 15)] = yacc[r][c][e];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int idx = lane; idx < 16 * a.ncols; idx += kWave) {
            const int rr = idx & 15, col = idx >> 4;
            const float v = comb[wave][rr][kPlanes * col] + comb[wave][rr][kPlanes * col + 1] +
                            comb[wave][rr][kPlanes * col + 2];
            const int row = rt * 16 + rr;
            if (rt < nrt && row < a.M) a.y[static_cast<long long>(col) * a.M + row] = v;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

}  // namespace

// Columns one launch handles: 3 B columns each, up to 3 tiles of 16.
constexpr int kTl1MmCols = 16;

size_t tl1_mfma_code_bytes(size_t M, size_t K) { return (M + 15) / 16 * ((K + 255) / 256) * 1024; }
size_t tl1_mfma_scale_bytes(size_t M, size_t K) { return M * ((K + 255) / 256 * 2) * sizeof(uint16_t); }
// B fragments and plane weights for up to ncols columns (one launch's share).
size_t tl1_xprep_bytes(size_t K, size_t ncols) {
    const size_t nc = std::min(ncols, static_cast<size_t>(kTl1MmCols));
    const size_t tiles = (kPlanes * nc + 15) / 16;
    const size_t nkb = (K + 255) / 256;
    return nkb * 4 * tiles * 1024 + nkb * 2 * 16 * tiles * sizeof(float);
}

// Raw TL1 payload (device, row-major groups) -> unit layout + scales.
int tl1_tile_mfma(const uint8_t *raw, size_t M, size_t K, uint8_t *codes, uint16_t *scales, void *stream) {
    if (!raw || !codes || !scales || !M || !K || K % 128 || M > 0x7fffffffULL || K > 0x7fffffffULL)
        return fail(OURO_ERR_SHAPE, "tl1 mfma tiling: bad shape %zu x %zu", M, K);
    const int nkb = static_cast<int>((K + 255) / 256), G = 2 * nkb;
    const long long words = static_cast<long long>(tl1_mfma_code_bytes(M, K) / 4);
    const hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(tl1_tile_mfma_kernel, dim3(static_cast<unsigned>((words + 255) / 256)), dim3(256), 0, s, raw,
                       reinterpret_cast<uint32_t *>(codes), static_cast<int>(M), static_cast<int>(K), nkb, words);
    int st = check_launch("tl1_tile_mfma_kernel");
    if (st) return st;
    const long long n = static_cast<long long>(M) * G;
    hipLaunchKernelGGL(tl1_scales_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, raw, scales,
                       static_cast<int>(M), static_cast<int>(K), G);
    return check_launch("tl1_scales_kernel");
}

// y[c][M] = W x_c for ncols columns of x [ncols][K], W in the unit layout.
// scratch: tl1_xprep_bytes(K, ncols) bytes, 16-byte aligned.
int tl1_mfma_matmul(const uint8_t *codes, const uint16_t *scales, size_t M, size_t K, const float *x, size_t ncols,
                    float *y, void *scratch, void *stream) {
    if (!codes || !scales || !x || !y || !scratch) return fail(OURO_ERR_INVALID_ARG, "tl1 matmul: NULL argument");
    if (!M || !K || K % 128 || !ncols || M > 0x7fffffffULL || K > 0x7fffffffULL)
        return fail(OURO_ERR_SHAPE, "tl1 matmul: bad shape");
    if ((reinterpret_cast<uintptr_t>(codes) | reinterpret_cast<uintptr_t>(scratch)) % 16 ||
        reinterpret_cast<uintptr_t>(scales) % 4)
        return fail(OURO_ERR_ALIGN, "tl1 matmul: alignment");
    const hipStream_t s = as_stream(stream);
    const int nkb = static_cast<int>((K + 255) / 256);
    for (size_t c0 = 0; c0 < ncols; c0 += kTl1MmCols) {
        const int nc = static_cast<int>(std::min(ncols - c0, static_cast<size_t>(kTl1MmCols)));
        const int tiles = (kPlanes * nc + 15) / 16;
        int8_t *xb = static_cast<int8_t *>(scratch);
        float *wt = reinterpret_cast<float *>(xb + static_cast<size_t>(nkb) * 4 * tiles * 1024);
        XprepArgs xa{x + c0 * K, xb, wt, static_cast<int>(K), 2 * nkb, tiles, nc};
        const int vcols = (16 * tiles + kPlanes - 1) / kPlanes;  // virtual columns cover every B column
        hipLaunchKernelGGL(tl1_xprep_kernel, dim3(2 * nkb, vcols), dim3(128), 0, s, xa);
        int st = check_launch("tl1_xprep_kernel");
        if (st) return st;
        Tl1MmArgs a{reinterpret_cast<const v4u *>(codes), scales, xb, wt, y + c0 * M, static_cast<int>(M), nkb,
                    2 * nkb, tiles, nc, 0};
        const int nrt = static_cast<int>((M + 15) / 16);
        constexpr int WR = 2;
        a.nrb = (nrt + kWaves * WR - 1) / (kWaves * WR);
        if (tiles == 1) hipLaunchKernelGGL((tl1_mfma_kernel<WR, 1>), dim3(a.nrb), dim3(kWave * kWaves), 0, s, a);
        else if (tiles == 2) hipLaunchKernelGGL((tl1_mfma_kernel<WR, 2>), dim3(a.nrb), dim3(kWave * kWaves), 0, s, a);
        else hipLaunchKernelGGL((tl1_mfma_kernel<WR, 3>), dim3(a.nrb), dim3(kWave * kWaves), 0, s, a);
        st = check_launch("tl1_mfma_kernel");
        if (st) return st;
    }
    return OURO_OK;
}

}  // namespace ouro
