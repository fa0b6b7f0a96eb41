// matvec_q.hip - the reference kernel-call surface matvec_q / matmul_q
// (ops.rs:76-84, 219-230) on device payloads of every ternary and dense kind.
//
// TL1 (PTQ1_0) and TQ1_0 are decoded in registers exactly as the reference
// does (digit of byte b at stage n: q = b * 3^n mod 256, digit = (q*3) >> 8,
// trit = digit - 1; dequant.rs:55-59, 134-138), one packed byte per lane
// task, and multiplied straight into fp32 accumulators: trits never touch
// memory (ops.rs:288-293).  One wavefront per output row; a task is one
// payload byte with its 4 or 5 trits, so consecutive lanes read consecutive
// payload bytes.  matmul_q decodes each byte once for up to 8 columns; a
// 4-byte-aligned TL1 payload of several columns goes to the int8 MFMA pass of
// tl1_mfma.hip instead (one pass over the payload for all columns).
#include "common.hpp"

#include <mutex>

namespace ouro {

int i2_gemm(const uint8_t *w_tiled, size_t out_len, size_t in_len, const float *w_scale,
            const int8_t *xq, const float *act_scale, size_t ncols, float *y, int32_t *acc,
            void *stream);
int act_quant(const void *x, int x_dtype, size_t rows, size_t n, int8_t *xq, float *act_scale,
              void *stream);
size_t i2_tiled_bytes(size_t out_len, size_t in_len);
int i2s_gemm(const uint8_t *i2s, size_t out_len, size_t in_len, const int8_t *xq, const float *act_scale,
             size_t ncols, float *y, int32_t *acc, void *stream);
size_t tl1_lut_partial_floats(size_t out_len, size_t in_len);
int tl1_lut_matvec(const void *packed, size_t out_len, size_t in_len, const float *x, float *y, float *partial,
                   void *amax_scratch, int32_t *idx, void *stream, int raw);
bool is_kquant(int kind);
size_t tl1_xprep_bytes(size_t K, size_t ncols);
int tl1_mfma_matmul_raw(const uint8_t *raw, size_t M, size_t K, const float *x, size_t ncols, float *y, void *scratch,
                        void *stream);
int kq_matmul(const void *payload, int kind, size_t out_len, size_t in_len, const float *x, size_t k, float *y,
              void *stream);
size_t tq1_lut_partial_floats(size_t out_len, size_t in_len);
bool tq1_lut_fits(const void *payload, size_t in_len);
int tq1_lut_matvec(const void *payload, size_t out_len, size_t in_len, const float *x, float *y, float *partial,
                   void *amax_scratch, int32_t *idx, void *stream);

// TL1 and TQ1_0 matvecs with at least this many rows run the table-lookup
// kernels on the raw payload: the table build and the partial-sum launch
// cost ~14 us, which the direct kernels undercut below ~8192 rows (measured
// at in_len 2560 and 5120).
constexpr size_t kLutRows = 8192;

namespace {

constexpr int kWaves = 4;

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

__device__ __forceinline__ int trit(uint32_t byte, uint32_t pow3) {
    const uint32_t q = (byte * pow3) & 0xffu;  // u8 wrapping_mul
    return static_cast<int>((q * 3u) >> 8) - 1;
}

struct MvArgs {
    const uint8_t *w;
    const float *x;  // [k][in_len]
    float *y;        // column-major [k][out_len]
    int out_len, in_len, k;
};

template <int NC>
__device__ __forceinline__ void wave_store(float (&acc)[NC], const MvArgs &a, int row, int c0, int lane) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        float v = acc[c];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += xor_shfl(v, off);
        if (lane == 0 && c0 + c < a.k) a.y[static_cast<long long>(c0 + c) * a.out_len + row] = v;
    }
}

// PTQ1_0 group (dequant.rs:140-171): qs[0..16] hold elements n*16 + m,
// qs[16..24] elements 80 + n*8 + m, qh[0..2] elements 120 + n*2 + h.
template <int NC>
__global__ __launch_bounds__(64 * kWaves) void tl1_kernel(MvArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int c0 = blockIdx.y * NC;
    if (row >= a.out_len) return;
    const int gpr = a.in_len / 128;
    const uint8_t *rw = a.w + static_cast<long long>(row) * gpr * 28;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.f;
    const int tasks = gpr * 26;
    for (int t = lane; t < tasks; t += 64) {
        const int g = t / 26, b = t % 26;
        const uint8_t *gp = rw + g * 28;
        const uint32_t byte = gp[b];
        const float d = f16_bits_to_f32(gp[26] | (static_cast<uint32_t>(gp[27]) << 8));
        const int xg = g * 128;
        int base, stride, cnt;
        if (b < 16) {
            base = xg + b, stride = 16, cnt = 5;
        } else if (b < 24) {
            base = xg + 80 + (b - 16), stride = 8, cnt = 5;
        } else {
            base = xg + 120 + (b - 24), stride = 2, cnt = 4;
        }
        uint32_t pow3 = 1;
#pragma unroll
        for (int n = 0; n < 5; ++n) {
            if (n < cnt) {
                const float w = static_cast<float>(trit(byte, pow3)) * d;
                const int xi = base + n * stride;
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    if (c0 + c < a.k) acc[c] += w * a.x[static_cast<long long>(c0 + c) * a.in_len + xi];
            }
            pow3 *= 3;
        }
    }
    wave_store<NC>(acc, a, row, c0, lane);
}

// TQ1_0 block (dequant.rs:49-80): qs[0..32] hold elements n*32 + m,
// qs[32..48] elements 160 + n*16 + m, qh[0..4] elements 240 + n*4 + m;
// f16 scale at bytes 52..53.
template <int NC>
__global__ __launch_bounds__(64 * kWaves) void tq1_kernel(MvArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int c0 = blockIdx.y * NC;
    if (row >= a.out_len) return;
    const int bpr = a.in_len / 256;
    const uint8_t *rw = a.w + static_cast<long long>(row) * bpr * 54;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.f;
    const int tasks = bpr * 52;
    for (int t = lane; t < tasks; t += 64) {
        const int blk = t / 52, b = t % 52;
        const uint8_t *bp = rw + blk * 54;
        const uint32_t byte = bp[b];
        const float d = f16_bits_to_f32(bp[52] | (static_cast<uint32_t>(bp[53]) << 8));
        const int xb = blk * 256;
        int base, stride, cnt;
        if (b < 32) {
            base = xb + b, stride = 32, cnt = 5;
        } else if (b < 48) {
            base = xb + 160 + (b - 32), stride = 16, cnt = 5;
        } else {
            base = xb + 240 + (b - 48), stride = 4, cnt = 4;
        }
        uint32_t pow3 = 1;
#pragma unroll
        for (int n = 0; n < 5; ++n) {
            if (n < cnt) {
                const float w = static_cast<float>(trit(byte, pow3)) * d;
                const int xi = base + n * stride;
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    if (c0 + c < a.k) acc[c] += w * a.x[static_cast<long long>(c0 + c) * a.in_len + xi];
            }
            pow3 *= 3;
        }
    }
    wave_store<NC>(acc, a, row, c0, lane);
}

template <int KIND>
__device__ __forceinline__ float dense_w(const uint8_t *w, long long i);
template <>
__device__ __forceinline__ float dense_w<OURO_KIND_F32>(const uint8_t *w, long long i) {
    return reinterpret_cast<const float *>(w)[i];
}
template <>
__device__ __forceinline__ float dense_w<OURO_KIND_F16>(const uint8_t *w, long long i) {
    return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(w)[i]);
}
template <>
__device__ __forceinline__ float dense_w<OURO_KIND_BF16>(const uint8_t *w, long long i) {
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(w)[i]);
}

template <int KIND, int NC>
__global__ __launch_bounds__(64 * kWaves) void dense_kernel(MvArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int c0 = blockIdx.y * NC;
    if (row >= a.out_len) return;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.f;
    const long long rb = static_cast<long long>(row) * a.in_len;
    for (int i = lane; i < a.in_len; i += 64) {
        const float w = dense_w<KIND>(a.w, rb + i);
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (c0 + c < a.k) acc[c] += w * a.x[static_cast<long long>(c0 + c) * a.in_len + i];
    }
    wave_store<NC>(acc, a, row, c0, lane);
}

int launch_mv(int kind, const MvArgs &a, hipStream_t s) {
    const int nc = a.k >= 8 ? 8 : (a.k >= 4 ? 4 : (a.k >= 2 ? 2 : 1));
    dim3 grid((a.out_len + kWaves - 1) / kWaves, (a.k + nc - 1) / nc), block(64 * kWaves);
    if (grid.y > 65535) return fail(OURO_ERR_SHAPE, "matmul_q: too many columns");
#define OURO_MV_LAUNCH(KERNEL)                                                        \
    do {                                                                              \
        if (nc == 8) hipLaunchKernelGGL(KERNEL<8>, grid, block, 0, s, a);             \
        else if (nc == 4) hipLaunchKernelGGL(KERNEL<4>, grid, block, 0, s, a);        \
        else if (nc == 2) hipLaunchKernelGGL(KERNEL<2>, grid, block, 0, s, a);        \
        else hipLaunchKernelGGL(KERNEL<1>, grid, block, 0, s, a);                     \
    } while (0)
    switch (kind) {
    case OURO_KIND_TL1: OURO_MV_LAUNCH(tl1_kernel); break;
    case OURO_KIND_TQ1_0: OURO_MV_LAUNCH(tq1_kernel); break;
    case OURO_KIND_F32:
        if (nc == 8) hipLaunchKernelGGL((dense_kernel<OURO_KIND_F32, 8>), grid, block, 0, s, a);
        else if (nc == 4) hipLaunchKernelGGL((dense_kernel<OURO_KIND_F32, 4>), grid, block, 0, s, a);
        else if (nc == 2) hipLaunchKernelGGL((dense_kernel<OURO_KIND_F32, 2>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((dense_kernel<OURO_KIND_F32, 1>), grid, block, 0, s, a);
        break;
    case OURO_KIND_F16:
        if (nc == 8) hipLaunchKernelGGL((dense_kernel<OURO_KIND_F16, 8>), grid, block, 0, s, a);
        else if (nc == 4) hipLaunchKernelGGL((dense_kernel<OURO_KIND_F16, 4>), grid, block, 0, s, a);
        else if (nc == 2) hipLaunchKernelGGL((dense_kernel<OURO_KIND_F16, 2>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((dense_kernel<OURO_KIND_F16, 1>), grid, block, 0, s, a);
        break;
    case OURO_KIND_BF16:
        if (nc == 8) hipLaunchKernelGGL((dense_kernel<OURO_KIND_BF16, 8>), grid, block, 0, s, a);
        else if (nc == 4) hipLaunchKernelGGL((dense_kernel<OURO_KIND_BF16, 4>), grid, block, 0, s, a);
        else if (nc == 2) hipLaunchKernelGGL((dense_kernel<OURO_KIND_BF16, 2>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((dense_kernel<OURO_KIND_BF16, 1>), grid, block, 0, s, a);
        break;
    default:
        return fail(OURO_ERR_KIND, "matvec_q: kind %d not supported", kind);
    }
#undef OURO_MV_LAUNCH
    return check_launch("matvec_q kernel");
}

}  // namespace

// Shape rules of the reference decoders: TL1 rows are whole 128-groups
// (ops.rs:296), TQ1_0 rows whole 256-blocks (QuantKind::row_bytes,
// dequant.rs:376-387).
// use_workspace = false keeps every path off the library workspace (the
// 2-bit kinds then need xq_scratch / act_scale_scratch; a TL1 or TQ1_0
// lookup GEMV runs only if lut_partial holds its partial sums, else the
// direct kernel does).
int matmul_q(const void *payload, int kind, size_t out_len, size_t in_len, const float *x, size_t k,
             float *y, int8_t *xq_scratch, float *act_scale_scratch, void *stream, bool use_workspace,
             float *lut_partial, size_t lut_partial_bytes) {
    // partial sums of a lookup GEMV: the library workspace, or the caller's
    // buffer if it is large enough (nullptr: run the direct kernel)
    auto partials = [&](size_t floats, bool &failed) -> float * {
        failed = false;
        if (use_workspace) {
            float *p = static_cast<float *>(workspace(floats * 4, stream));
            failed = !p;
            return p;
        }
        return lut_partial && floats * 4 <= lut_partial_bytes ? lut_partial : nullptr;
    };
    if (!payload || !x || !y) return fail(OURO_ERR_INVALID_ARG, "matvec_q: NULL argument");
    if (!out_len || !in_len || !k) return fail(OURO_ERR_SHAPE, "matvec_q: empty shape");
    if (out_len > 0x7fffffffULL || in_len > 0x7fffffffULL || k > 0x7fffffffULL)
        return fail(OURO_ERR_SHAPE, "matvec_q: shape too large");
    if (is_kquant(kind)) return kq_matmul(payload, kind, out_len, in_len, x, k, y, stream);
    switch (kind) {
    case OURO_KIND_TL1:
        if (in_len % 128) return fail(OURO_ERR_SHAPE, "matvec_q TL1: in_len %zu not a multiple of 128", in_len);
        // one column of a large matrix: the lookup kernel straight on the
        // reference bytes (per-block partial sums in the library workspace or
        // the caller's buffer)
        if (k == 1 && out_len >= kLutRows && reinterpret_cast<uintptr_t>(payload) % 4 == 0 && in_len <= 65536) {
            bool failed = false;
            float *partial = partials(tl1_lut_partial_floats(out_len, in_len), failed);
            if (failed) return OURO_ERR_HIP;
            if (partial) return tl1_lut_matvec(payload, out_len, in_len, x, y, partial, nullptr, nullptr, stream, 1);
        }
        // several columns: one pass over the payload for all of them (int8 MFMA
        // on the decoded digits, x as exact digit planes in the workspace)
        if (k >= 2 && use_workspace && reinterpret_cast<uintptr_t>(payload) % 4 == 0 &&
            reinterpret_cast<uintptr_t>(x) % 4 == 0) {
            void *ws = workspace(tl1_xprep_bytes(in_len, k), stream);
            if (!ws) return OURO_ERR_HIP;
            return tl1_mfma_matmul_raw(static_cast<const uint8_t *>(payload), out_len, in_len, x, k, y, ws, stream);
        }
        break;
    case OURO_KIND_TQ1_0:
        if (in_len % 256) return fail(OURO_ERR_SHAPE, "matvec_q TQ1_0: in_len %zu not a multiple of 256", in_len);
        // one column of a large matrix: the lookup kernel on the reference bytes
        if (k == 1 && out_len >= kLutRows && tq1_lut_fits(payload, in_len)) {
            bool failed = false;
            float *partial = partials(tq1_lut_partial_floats(out_len, in_len), failed);
            if (failed) return OURO_ERR_HIP;
            if (partial) return tq1_lut_matvec(payload, out_len, in_len, x, y, partial, nullptr, nullptr, stream);
        }
        break;
    case OURO_KIND_F32:
        if (reinterpret_cast<uintptr_t>(payload) % 4) return fail(OURO_ERR_ALIGN, "matvec_q F32: payload alignment");
        break;
    case OURO_KIND_F16:
    case OURO_KIND_BF16:
        if (reinterpret_cast<uintptr_t>(payload) % 2) return fail(OURO_ERR_ALIGN, "matvec_q F16: payload alignment");
        break;
    case OURO_KIND_I2:
    case OURO_KIND_I2_S: {
        const size_t tb = i2_tiled_bytes(out_len, in_len);
        if (!tb) return fail(OURO_ERR_SHAPE, "matvec_q I2: in_len %zu not a multiple of 256", in_len);
        int8_t *xq = xq_scratch;
        float *ds = act_scale_scratch;
        if (!xq) {
            if (!use_workspace) return fail(OURO_ERR_INVALID_ARG, "matvec_q: no activation scratch");
            const size_t xb = (k * in_len + 255) & ~size_t(255);
            uint8_t *ws = static_cast<uint8_t *>(workspace(xb + k * sizeof(float), stream));
            if (!ws) return OURO_ERR_HIP;
            xq = reinterpret_cast<int8_t *>(ws);
            ds = reinterpret_cast<float *>(ws + xb);
        }
        int st = act_quant(x, OURO_DT_F32, k, in_len, xq, ds, stream);
        if (st) return st;
        const uint8_t *w = static_cast<const uint8_t *>(payload);
        if (kind == OURO_KIND_I2_S) return i2s_gemm(w, out_len, in_len, xq, ds, k, y, nullptr, stream);
        return i2_gemm(w, out_len, in_len, reinterpret_cast<const float *>(w + tb), xq, ds, k, y,
                       nullptr, stream);
    }
    default:
        return fail(OURO_ERR_KIND, "matvec_q: kind %d not supported", kind);
    }
    MvArgs a{static_cast<const uint8_t *>(payload), x, y, static_cast<int>(out_len),
             static_cast<int>(in_len), static_cast<int>(k)};
    return launch_mv(kind, a, as_stream(stream));
}

// ---- the allocation-free variant of matvec_q ----
//
// Callers that cannot allocate (code under HIP graph capture, tight serving
// loops) get ouro_matvec_q_noalloc: its 2-bit kinds quantise x into this
// file-scope device array, and its TL1 / TQ1_0 lookup GEMVs keep their
// per-block partial sums there, instead of the library workspace.  Each
// device holds its own copy until the process ends; its address on a device
// comes from hipGetSymbolAddress (the array's name is not a device address
// in host code).  All calls on one device share it, so calls that overlap
// on one device race.  Nothing in it needs to start at zero: each call
// writes the in_len int8 values and the scale, or every partial sum, before
// the next kernel reads them.
constexpr size_t kNoAllocMaxIn = 32768;          // the raw I2_S kernel's limit
constexpr size_t kNoAllocLut = size_t(16) << 20;  // lookup partial sums (the 248320x5120 lm_head needs 9.9 MB)
constexpr size_t kNoAllocScratch = kNoAllocLut;  // 2-bit kinds: int8 row at 0, act_scale at kNoAllocMaxIn
static_assert(kNoAllocMaxIn + 256 <= kNoAllocScratch, "noalloc scratch layout");
static __device__ __align__(256) uint8_t scratch[kNoAllocScratch];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up once per device).
int scratch_ptr(void **out) {
    const int dev = current_device();
    if (dev < 0 || dev >= kMaxDevices) return fail(OURO_ERR_NO_DEVICE, "matvec_q_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(OURO_ERR_HIP, "matvec_q_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return OURO_OK;
}
}  // namespace

}  // namespace ouro

using namespace ouro;

extern "C" {

int ouro_matvec_q_noalloc(const void *payload, int kind, size_t out_len, size_t in_len, const float *x,
                          float *y, void *stream) {
    OURO_REQUIRE_INIT();
    if (kind == OURO_KIND_TL1 || kind == OURO_KIND_TQ1_0) {
        // the lookup GEMV's partial sums in the static array when they fit;
        // larger shapes (and fewer than 8192 rows) run the direct kernel,
        // which needs no scratch
        void *p = nullptr;
        const int st = scratch_ptr(&p);
        if (st) return st;
        return matmul_q(payload, kind, out_len, in_len, x, 1, y, nullptr, nullptr, stream, false,
                        static_cast<float *>(p), kNoAllocLut);
    }
    if (kind != OURO_KIND_I2 && kind != OURO_KIND_I2_S)  // no scratch, and no workspace
        return matmul_q(payload, kind, out_len, in_len, x, 1, y, nullptr, nullptr, stream, false, nullptr, 0);
    if (in_len > kNoAllocMaxIn)
        return fail(OURO_ERR_SHAPE, "ouro_matvec_q_noalloc: in_len %zu exceeds the %zu-element static scratch",
                    in_len, kNoAllocMaxIn);
    void *p = nullptr;
    const int st = scratch_ptr(&p);
    if (st) return st;
    int8_t *xq = static_cast<int8_t *>(p);
    float *s = reinterpret_cast<float *>(static_cast<uint8_t *>(p) + kNoAllocMaxIn);
    return matmul_q(payload, kind, out_len, in_len, x, 1, y, xq, s, stream, false, nullptr, 0);
}

int ouro_matvec_q(const void *payload, int kind, size_t out_len, size_t in_len, const float *x,
                  float *y, void *stream) {
    OURO_REQUIRE_INIT();
    return matmul_q(payload, kind, out_len, in_len, x, 1, y, nullptr, nullptr, stream, true, nullptr, 0);
}

int ouro_matmul_q(const void *payload, int kind, size_t out_len, size_t in_len, const float *x,
                  size_t k, float *y, void *stream) {
    OURO_REQUIRE_INIT();
    return matmul_q(payload, kind, out_len, in_len, x, k, y, nullptr, nullptr, stream, true, nullptr, 0);
}

}  // extern "C"
