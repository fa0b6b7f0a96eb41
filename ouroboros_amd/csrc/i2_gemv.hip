// i2_gemv.hip - int8 per-token-absmax activations x 2-bit ternary weights.
//
// The weight stream is the whole cost of a decode GEMV (ops.rs:288-293 says
// the same of the reference's fused decode+dot), so the kernel is built
// around HBM: the device-tiled I2 layout (ouro_hip.h) makes every 16-byte
// load of a 64-lane wavefront one contiguous 1 KiB segment, each lane keeps
// its activation slice in registers for all rows it visits, and 2-bit codes
// are expanded to int8 in registers and consumed by v_dot4_i32_i8.
//
// Integer accumulation is exact in any order; the fp32 epilogue is two
// separately rounded products, so results are bit-identical to the oracle.
#include "common.hpp"

#pragma clang fp contract(off)

namespace ouro {
namespace {

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int gcd_i(int a, int b) { return b == 0 ? a : gcd_i(b, a % b); }
__host__ __device__ constexpr int rows_per_tile(int G) { return 16 / gcd_i(G, 16); }

// ------------------------------------------------------------ tiling --

// One thread per 32-bit word of the tiled layout.
__global__ void i2_tile_kernel(const uint8_t *__restrict__ canon, uint32_t *__restrict__ tiled,
                               int out_len, int G, int R, long long total_words) {
    long long id = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= total_words) return;
    const long long tile_words = 16LL * R * G;  // 64 lanes * R*G bytes / 4
    const long long t = id / tile_words;
    const int w = static_cast<int>(id % tile_words);
    const int lane = (w % 256) / 4;
    const int d = 4 * (w / 256) + (w % 4);
    const long long row_bytes = 64LL * G;
    uint32_t word = 0;
#pragma unroll
    for (int f = 0; f < 4; ++f) {
        const int gi = 4 * d + f;
        const int r = gi / G, g = gi % G;
        const long long row = t * R + r;
        uint32_t byte = 0x55;  // padding rows: code 1 (w = 0) everywhere
        if (row < out_len) byte = canon[row * row_bytes + static_cast<long long>(G) * lane + g];
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

// One 256-thread block per row.
template <typename T>
__global__ __launch_bounds__(256) void act_quant_kernel(const T *__restrict__ x, long long n,
                                                        int8_t *__restrict__ xq,
                                                        float *__restrict__ dscale) {
    __shared__ float red[4];
    const long long row = blockIdx.x;
    const T *xr = x + row * n;
    float amax = 0.f;
    for (long long i = threadIdx.x; i < n; i += blockDim.x) amax = fmaxf(amax, fabsf(load_act(xr, i)));
    amax = block_max_256(amax, red);
    int8_t *qr = xq + row * n;
    if (amax == 0.f) {
        for (long long i = threadIdx.x; i < n; i += blockDim.x) qr[i] = 0;
        if (threadIdx.x == 0) dscale[row] = 0.f;
        return;
    }
    const float s = 127.0f / amax;
    for (long long i = threadIdx.x; i < n; i += blockDim.x) {
        float t = rintf(load_act(xr, i) * s);
        t = fminf(fmaxf(t, -127.f), 127.f);
        qr[i] = static_cast<int8_t>(t);
    }
    if (threadIdx.x == 0) dscale[row] = amax / 127.0f;
}

// ------------------------------------------------------------- GEMV --

struct GemvArgs {
    const uint8_t *w;       // tiled codes of matrix 0
    long long w_stride;     // bytes between matrices
    const float *w_scale;   // per matrix, stride 1
    const int8_t *xq;       // [ncols][in_len] of matrix 0
    long long x_stride;     // elements between matrices
    const float *dscale;    // [ncols] of matrix 0, per matrix stride ncols
    float *y;               // [ncols][out_len] of matrix 0
    long long y_stride;     // elements between matrices
    int32_t *acc;           // optional, same layout as y (matrix 0 only)
    int out_len, in_len, ncols, tiles;
};

// G: 4-weight groups per lane per row; R rows per tile; NC activation
// columns per pass; TPW tiles per wavefront; WPB wavefronts per block.
template <int G, int NC, int TPW, int WPB>
__global__ __launch_bounds__(kWave *WPB) void i2_gemv_kernel(GemvArgs a) {
    constexpr int R = rows_per_tile(G);
    constexpr int CHUNK = R * G;      // bytes per lane per tile
    constexpr int NV = CHUNK / 16;    // 16-byte loads per lane per tile
    static_assert(CHUNK % 16 == 0, "tile chunk must be whole 16-byte loads");

    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int mat = blockIdx.z;
    const int c0 = blockIdx.y * NC;
    const int tile0 = (blockIdx.x * WPB + wave) * TPW;
    if (tile0 >= a.tiles) return;  // whole wavefront leaves together

    const uint8_t *w = a.w + mat * a.w_stride;
    const int8_t *xq = a.xq + mat * a.x_stride;
    const float *dscale = a.dscale + static_cast<long long>(mat) * a.ncols;
    float *y = a.y + mat * a.y_stride;
    const float wscale = a.w_scale[mat];

    // Activation slice of this lane: k in [4*G*lane, 4*G*(lane+1)).
    uint32_t xw[NC][G];
    int sx[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        sx[c] = 0;
        const bool live = c0 + c < a.ncols;
        const uint32_t *xp = reinterpret_cast<const uint32_t *>(
            xq + static_cast<long long>(c0 + c) * a.in_len + 4 * G * lane);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            xw[c][g] = live ? xp[g] : 0u;
            sx[c] = __builtin_amdgcn_sdot4(static_cast<int>(xw[c][g]), 0x01010101, sx[c], false);
        }
    }

    // Issue every load of this wavefront's tiles before any arithmetic.
    u32x4 buf[TPW][NV];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int tile = tile0 + t;
        const u32x4 *tp = reinterpret_cast<const u32x4 *>(
            w + static_cast<long long>(tile < a.tiles ? tile : tile0) * (R * 64 * G));
#pragma unroll
        for (int j = 0; j < NV; ++j) buf[t][j] = tp[j * kWave + lane];
    }

#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int tile = tile0 + t;
        if (tile >= a.tiles) break;  // uniform across the wavefront
        int acc[NC][R];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[c][r] = -sx[c];  // codes are w + 1
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t words[4] = {buf[t][j].x, buf[t][j].y, buf[t][j].z, buf[t][j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int d = 4 * j + q;
#pragma unroll
                for (int f = 0; f < 4; ++f) {
                    const int gi = 4 * d + f;
                    const int r = gi / G, g = gi % G;
                    const int codes = static_cast<int>((words[q] >> (2 * f)) & 0x03030303u);
#pragma unroll
                    for (int c = 0; c < NC; ++c)
                        acc[c][r] = __builtin_amdgcn_sdot4(codes, static_cast<int>(xw[c][g]),
                                                           acc[c][r], false);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int total = reduce_scatter<R, kWave>(acc[c], lane);
            constexpr int span = kWave / R;
            const int row = tile * R + lane / span;
            if (lane % span == 0 && row < a.out_len && c0 + c < a.ncols) {
                const long long o = static_cast<long long>(c0 + c) * a.out_len + row;
                const float v = (static_cast<float>(total) * dscale[c0 + c]) * wscale;
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

// Tiles per wavefront are capped so that the in-flight tile buffers stay
// within about 32 VGPRs (NV 16-byte loads per tile).
template <int G>
GemvPick pick_g(int ncols, int want_tpw) {
    constexpr int NV = rows_per_tile(G) * G / 16;
    if (ncols >= 4) return {i2_gemv_kernel<G, 4, 1, 4>, 4, 1, 4};
    if (ncols >= 2) return {i2_gemv_kernel<G, 2, 1, 4>, 2, 1, 4};
    // Measured on the 64 x 6912x2560 stream: 2 tiles per wavefront in
    // 8-wavefront blocks for large grouped launches, 1 tile per wavefront
    // when a single matrix has to spread over the whole chip.
    if (want_tpw >= 2 && 2 * NV <= 32) return {i2_gemv_kernel<G, 1, 2, 8>, 1, 2, 8};
    return {i2_gemv_kernel<G, 1, 1, 4>, 1, 1, 4};
}

GemvPick pick_gemv(int G, int ncols, int tpw) {
    switch (G) {
    case 1: return pick_g<1>(ncols, tpw);
    case 2: return pick_g<2>(ncols, tpw);
    case 4: return pick_g<4>(ncols, tpw);
    case 8: return pick_g<8>(ncols, tpw);
    case 10: return pick_g<10>(ncols, tpw);
    case 12: return pick_g<12>(ncols, tpw);
    case 16: return pick_g<16>(ncols, tpw);
    case 20: return pick_g<20>(ncols, tpw);
    case 24: return pick_g<24>(ncols, tpw);
    case 27: return pick_g<27>(ncols, tpw);
    case 32: return pick_g<32>(ncols, tpw);
    default: return {nullptr, 0, 0};
    }
}

int launch_gemv(const GemvArgs &base, int count, void *stream) {
    const int G = base.in_len / 256;
    const int tiles = base.tiles;
    // Tiles per wavefront: enough in flight for a large grouped launch,
    // one per wavefront when a single matrix has to fill the chip alone.
    const long long total_tiles = static_cast<long long>(tiles) * count;
    const int want = total_tiles >= 8192 ? 2 : 1;
    const GemvPick p = pick_gemv(G, base.ncols, want);
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
            const int8_t *xq, const float *dscale, size_t ncols, float *y, int32_t *acc,
            void *stream) {
    int st = check_i2_shape(out_len, in_len);
    if (st) return st;
    if (!w_tiled || !w_scale || !xq || !dscale || !y || !ncols)
        return fail(OURO_ERR_INVALID_ARG, "ouro_gemm_i2: NULL argument or ncols == 0");
    if (reinterpret_cast<uintptr_t>(w_tiled) % 16 || reinterpret_cast<uintptr_t>(xq) % 4)
        return fail(OURO_ERR_ALIGN, "ouro_gemm_i2: weights need 16-byte, xq 4-byte alignment");
    const int G = static_cast<int>(in_len / 256);
    const int R = rows_per_tile(G);
    GemvArgs a{};
    a.w = w_tiled;
    a.w_stride = 0;
    a.w_scale = w_scale;
    a.xq = xq;
    a.x_stride = 0;
    a.dscale = dscale;
    a.y = y;
    a.y_stride = 0;
    a.acc = acc;
    a.out_len = static_cast<int>(out_len);
    a.in_len = static_cast<int>(in_len);
    a.ncols = static_cast<int>(ncols);
    a.tiles = static_cast<int>((out_len + R - 1) / R);
    return launch_gemv(a, 1, stream);
}

int act_quant(const void *x, int x_dtype, size_t rows, size_t n, int8_t *xq, float *dscale,
              void *stream) {
    if (!x || !xq || !dscale) return fail(OURO_ERR_INVALID_ARG, "ouro_act_quant_i8: NULL argument");
    if (!rows || !n) return fail(OURO_ERR_SHAPE, "ouro_act_quant_i8: empty shape");
    if (rows > 0x7fffffff) return fail(OURO_ERR_SHAPE, "ouro_act_quant_i8: too many rows");
    dim3 grid(static_cast<unsigned>(rows)), block(256);
    if (x_dtype == OURO_DT_F32)
        hipLaunchKernelGGL(act_quant_kernel<float>, grid, block, 0, as_stream(stream),
                           static_cast<const float *>(x), static_cast<long long>(n), xq, dscale);
    else if (x_dtype == OURO_DT_BF16)
        hipLaunchKernelGGL(act_quant_kernel<uint16_t>, grid, block, 0, as_stream(stream),
                           static_cast<const uint16_t *>(x), static_cast<long long>(n), xq, dscale);
    else
        return fail(OURO_ERR_INVALID_ARG, "ouro_act_quant_i8: bad dtype %d", x_dtype);
    return check_launch("act_quant_kernel");
}

size_t i2_tiled_bytes(size_t out_len, size_t in_len) {
    if (!in_len || in_len % 256) return 0;
    const size_t G = in_len / 256;
    const size_t R = static_cast<size_t>(rows_per_tile(static_cast<int>(G)));
    const size_t tiles = (out_len + R - 1) / R;
    return tiles * R * (in_len / 4);
}

int i2_tile(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *tiled,
            const float *w_scale, void *stream) {
    int st = check_i2_shape(out_len, in_len);
    if (st) return st;
    if (!canonical || !tiled) return fail(OURO_ERR_INVALID_ARG, "ouro_i2_tile: NULL argument");
    if (reinterpret_cast<uintptr_t>(tiled) % 16) return fail(OURO_ERR_ALIGN, "ouro_i2_tile: tiled needs 16-byte alignment");
    const int G = static_cast<int>(in_len / 256);
    const int R = rows_per_tile(G);
    const size_t bytes = i2_tiled_bytes(out_len, in_len);
    const long long words = static_cast<long long>(bytes / 4);
    const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
    hipLaunchKernelGGL(i2_tile_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), canonical,
                       reinterpret_cast<uint32_t *>(tiled), static_cast<int>(out_len), G, R, words);
    st = check_launch("i2_tile_kernel");
    if (st) return st;
    if (w_scale) {
        hipLaunchKernelGGL(copy_scale_kernel, dim3(1), dim3(1), 0, as_stream(stream), w_scale,
                           reinterpret_cast<float *>(tiled + bytes));
        st = check_launch("copy_scale_kernel");
    }
    return st;
}

}  // namespace ouro

using namespace ouro;

extern "C" {

size_t ouro_i2_tiled_bytes(size_t out_len, size_t in_len) { return i2_tiled_bytes(out_len, in_len); }

int ouro_i2_tile(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *tiled,
                 const float *w_scale_or_null, void *stream) {
    OURO_REQUIRE_INIT();
    return i2_tile(canonical, out_len, in_len, tiled, w_scale_or_null, stream);
}

int ouro_act_quant_i8(const void *x, int x_dtype, size_t rows, size_t n, int8_t *xq,
                      float *dscale, void *stream) {
    OURO_REQUIRE_INIT();
    return act_quant(x, x_dtype, rows, n, xq, dscale, stream);
}

int ouro_gemm_i2(const uint8_t *w_tiled, size_t out_len, size_t in_len, const float *w_scale,
                 const int8_t *xq, const float *dscale, size_t ncols, float *y,
                 int32_t *acc_or_null, void *stream) {
    OURO_REQUIRE_INIT();
    return i2_gemm(w_tiled, out_len, in_len, w_scale, xq, dscale, ncols, y, acc_or_null, stream);
}

int ouro_gemv_i2_grouped(const uint8_t *w_tiled, size_t w_stride, const float *w_scale,
                         const int8_t *xq, size_t x_stride, const float *dscale, float *y,
                         size_t y_stride, size_t out_len, size_t in_len, size_t count,
                         void *stream) {
    OURO_REQUIRE_INIT();
    int st = check_i2_shape(out_len, in_len);
    if (st) return st;
    if (!w_tiled || !w_scale || !xq || !dscale || !y || !count)
        return fail(OURO_ERR_INVALID_ARG, "ouro_gemv_i2_grouped: NULL argument or count == 0");
    if (count > 65535) return fail(OURO_ERR_SHAPE, "ouro_gemv_i2_grouped: count > 65535");
    if (w_stride < i2_tiled_bytes(out_len, in_len) || w_stride % 16 || x_stride < in_len ||
        x_stride % 4 || y_stride < out_len)
        return fail(OURO_ERR_SHAPE, "ouro_gemv_i2_grouped: strides overlap or misaligned");
    if (reinterpret_cast<uintptr_t>(w_tiled) % 16 || reinterpret_cast<uintptr_t>(xq) % 4)
        return fail(OURO_ERR_ALIGN, "ouro_gemv_i2_grouped: weights need 16-byte, xq 4-byte alignment");
    const int G = static_cast<int>(in_len / 256);
    const int R = rows_per_tile(G);
    GemvArgs a{};
    a.w = w_tiled;
    a.w_stride = static_cast<long long>(w_stride);
    a.w_scale = w_scale;
    a.xq = xq;
    a.x_stride = static_cast<long long>(x_stride);
    a.dscale = dscale;
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
