// kquant.hip - matvec_q / matmul_q on the block-quantised kinds Q8_0, Q3_K,
// Q4_K, Q5_K and Q6_K: the reference's matvec_qblock (ops.rs:101-128, the
// row decoded by dequant_{q8,q3k,q4k,q5k,q6k}_row, dequant.rs:218-310,
// 390-560, then dot with x) fused into one pass over the payload as it lies
// in device memory (ggml's block layouts, unchanged).
//
// Work unit.  Every block splits into tasks of 32 elements whose codes sit in
// one 16-byte piece of the block (plus, for Q3_K, Q5_K and Q6_K, a 16-byte
// piece of high bits) and whose x values are two runs of 16: elements
// A + i and A + G + i, i < 16.  A 256-element block has 8 tasks, a Q8_0 block
// one.  Per task the codes are summed against x as integers-in-float
// (S = sum q x, an fma chain) and scaled once per run: the contribution is
// cA S_A - mA X_A + cB S_B - mB X_B with X the run's sum of x (the min, or the
// code offset -32 / -4 of Q6_K / Q3_K, taken out of the sum).  That keeps the
// per-element work at a mask, a byte-to-float conversion and an fma.
//
// Mapping.  A thread owns one task position of a row (k-stationary): its 32 x
// values and their run sums stay in registers while the workgroup walks row
// tiles, so x is read once per workgroup.  A workgroup is `slots` side-by-side
// copies of one row's task set (slots * tasks_per_row threads, rounded up to a
// whole wavefront, at most 256 unless one row needs more), each copy walking
// R consecutive rows per tile; the next tile's loads are issued before the
// current tile is summed; the per-thread sums of a tile meet in LDS and one
// wavefront per output row adds them.  Blocks of Q8_0, Q3_K
// and Q6_K (34, 110, 210 bytes) are only 2-byte aligned: their 16-byte pieces
// are read as the aligned dwords that cover them and shifted into place with
// v_alignbyte.  Scale bytes are read as bytes.
#include "common.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace ouro {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));

constexpr int kMaxThreads = 1024;

// 16 bytes at any address: the 4-byte-aligned dwords that cover them, shifted
// into place.  Every dword read holds at least one of the 16 bytes, so the
// read stays inside the pages the bytes are on.
__device__ __forceinline__ u32x4 load16_any(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const u32x4 lo = *reinterpret_cast<const u32x4_a4 *>(a & ~uintptr_t(3));
    const uint32_t e = *reinterpret_cast<const uint32_t *>((a + 15) & ~uintptr_t(3));
    const uint32_t s = static_cast<uint32_t>(a & 3);
    u32x4 r;
    r.x = __builtin_amdgcn_alignbyte(lo.y, lo.x, s);
    r.y = __builtin_amdgcn_alignbyte(lo.z, lo.y, s);
    r.z = __builtin_amdgcn_alignbyte(lo.w, lo.z, s);
    r.w = __builtin_amdgcn_alignbyte(e, lo.w, s);
    return r;
}

template <bool AL16>
__device__ __forceinline__ u32x4 load16(const uint8_t *p) {
    if constexpr (AL16) return *reinterpret_cast<const u32x4 *>(p);
    else return load16_any(p);
}

__device__ __forceinline__ float f16f(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t w) {
    return __builtin_amdgcn_ubfe(v, off, w);
}

// Byte b of a 16-byte piece as a float (unsigned).
__device__ __forceinline__ float ub(uint32_t w, int b) { return static_cast<float>((w >> (8 * b)) & 0xffu); }

// sum over the 16 bytes of v (each an unsigned code) times x[0..15]
__device__ __forceinline__ float dot16u(const u32x4 &v, const float (&x)[16]) {
    float s = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t w = v[d];
#pragma unroll
        for (int b = 0; b < 4; ++b) s = __builtin_fmaf(ub(w, b), x[4 * d + b], s);
    }
    return s;
}

// the same with signed bytes (Q8_0); the builtin returns the sign-extended
// field as an unsigned int, so it is read back as int32 before conversion
__device__ __forceinline__ float dot16s(const u32x4 &v, const float (&x)[16]) {
    float s = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t w = v[d];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int32_t q = static_cast<int32_t>(__builtin_amdgcn_sbfe(w, 8 * b, 8));
            s = __builtin_fmaf(static_cast<float>(q), x[4 * d + b], s);
        }
    }
    return s;
}

__device__ __forceinline__ u32x4 vmap(const u32x4 &a, uint32_t mask, uint32_t sh) {
    return u32x4{(a.x >> sh) & mask, (a.y >> sh) & mask, (a.z >> sh) & mask, (a.w >> sh) & mask};
}

// ---- per kind: block geometry, a task's x runs, its raw loads, its sum ----

template <int KIND> struct Fmt;

// Q8_0 (dequant.rs:225-231): d f16, then 32 int8 codes; one task per block.
template <> struct Fmt<OURO_KIND_Q8_0> {
    static constexpr int BB = 34, EPB = 32, TPB = 1, G = 16;
    __device__ static int A(int) { return 0; }
    struct Raw { u32x4 a, b; uint32_t d0, d1; };
    template <bool AL16> __device__ static Raw load(const uint8_t *bp, int) {
        Raw r;
        r.a = load16_any(bp + 2);
        r.b = load16_any(bp + 18);
        r.d0 = bp[0];
        r.d1 = bp[1];
        return r;
    }
    __device__ static float dot(const Raw &r, int, const float (&xa)[16], const float (&xb)[16], float, float) {
        const float d = f16f(r.d0 | (r.d1 << 8));
        return d * (dot16s(r.a, xa) + dot16s(r.b, xb));
    }
};

// Q4_K / Q5_K scales (scale_min_k4, dequant.rs:245-254) of sub-block k from
// the 12 scale bytes held in words h1 (bytes 0..3), h2 (4..7), h3 (8..11):
// for k < 4 the low six bits of byte k (scale) and k + 4 (min); for k >= 4
// the low / high nibble of byte k + 4 below the top two bits of byte k - 4 /
// k.  Branch-free (k differs between the lanes of a wavefront): v_bfe with
// width 0 yields 0.
__device__ __forceinline__ void scale_min_k4(int k, uint32_t h1, uint32_t h2, uint32_t h3, uint32_t &s, uint32_t &m) {
    const bool hi = k >= 4;
    const uint32_t o = 8 * (k & 3);
    const uint32_t wa = hi ? 4 : 6, wb = hi ? 2 : 0;
    s = bfe(hi ? h3 : h1, o, wa) | (bfe(h1, o + 6, wb) << 4);
    m = bfe(hi ? h3 : h2, o + (hi ? 4 : 0), wa) | (bfe(h2, o + 6, wb) << 4);
}

// Q4_K (dequant.rs:257-282): d, dmin f16, scales[12], qs[128].  Task u:
// pair j = u / 2, half h = u % 2; qs bytes 32j + 16h + i give element
// 64j + 16h + i (low nibble, sub-block 2j) and 64j + 32 + 16h + i (high
// nibble, sub-block 2j + 1).
template <> struct Fmt<OURO_KIND_Q4K> {
    static constexpr int BB = 144, EPB = 256, TPB = 8, G = 32;
    __device__ static int A(int u) { return 64 * (u >> 1) + 16 * (u & 1); }
    struct Raw { u32x4 h, q; };
    template <bool AL16> __device__ static Raw load(const uint8_t *bp, int u) {
        return Raw{load16<AL16>(bp), load16<AL16>(bp + 16 + 16 * u)};
    }
    __device__ static float dot(const Raw &r, int u, const float (&xa)[16], const float (&xb)[16], float XA, float XB) {
#pragma clang fp contract(off)
        const int j = u >> 1;
        uint32_t s1, m1, s2, m2;
        scale_min_k4(2 * j, r.h.y, r.h.z, r.h.w, s1, m1);
        scale_min_k4(2 * j + 1, r.h.y, r.h.z, r.h.w, s2, m2);
        const float d = f16f(r.h.x & 0xffffu), dmin = f16f(r.h.x >> 16);
        const float SA = dot16u(vmap(r.q, 0x0f0f0f0fu, 0), xa);
        const float SB = dot16u(vmap(r.q, 0x0f0f0f0fu, 4), xb);
        return (d * static_cast<float>(s1)) * SA - (dmin * static_cast<float>(m1)) * XA +
               ((d * static_cast<float>(s2)) * SB - (dmin * static_cast<float>(m2)) * XB);
    }
};

// Q5_K (dequant.rs:454-481): d, dmin, scales[12], qh[32], qs[128].  As Q4_K,
// with bit 2j (low nibble) / 2j + 1 (high nibble) of qh[16h + i] adding 16.
template <> struct Fmt<OURO_KIND_Q5K> {
    static constexpr int BB = 176, EPB = 256, TPB = 8, G = 32;
    __device__ static int A(int u) { return 64 * (u >> 1) + 16 * (u & 1); }
    struct Raw { u32x4 h, qh, q; };
    template <bool AL16> __device__ static Raw load(const uint8_t *bp, int u) {
        return Raw{load16<AL16>(bp), load16<AL16>(bp + 16 + 16 * (u & 1)), load16<AL16>(bp + 48 + 16 * u)};
    }
    __device__ static float dot(const Raw &r, int u, const float (&xa)[16], const float (&xb)[16], float XA, float XB) {
#pragma clang fp contract(off)
        const int j = u >> 1;
        uint32_t s1, m1, s2, m2;
        scale_min_k4(2 * j, r.h.y, r.h.z, r.h.w, s1, m1);
        scale_min_k4(2 * j + 1, r.h.y, r.h.z, r.h.w, s2, m2);
        const float d = f16f(r.h.x & 0xffffu), dmin = f16f(r.h.x >> 16);
        const u32x4 lo = vmap(r.q, 0x0f0f0f0fu, 0) | (vmap(r.qh, 0x01010101u, 2 * j) << 4);
        const u32x4 hi = vmap(r.q, 0x0f0f0f0fu, 4) | (vmap(r.qh, 0x01010101u, 2 * j + 1) << 4);
        const float SA = dot16u(lo, xa);
        const float SB = dot16u(hi, xb);
        return (d * static_cast<float>(s1)) * SA - (dmin * static_cast<float>(m1)) * XA +
               ((d * static_cast<float>(s2)) * SB - (dmin * static_cast<float>(m2)) * XB);
    }
};

// Q6_K (dequant.rs:484-510): ql[128], qh[64], scales int8[16], d.  Task u:
// half n = u / 4, l0 = 16 ((u / 2) % 2), s = u % 2: ql bytes 64n + 32s + l0 + i
// with bits 2s (low nibble) / 4 + 2s (high nibble) of qh[32n + l0 + i] give
// element 128n + 32s + l0 + i (scale 8n + l0/16 + 2s) and that + 64 (scale + 4),
// code - 32.
template <> struct Fmt<OURO_KIND_Q6K> {
    static constexpr int BB = 210, EPB = 256, TPB = 8, G = 64;
    __device__ static int A(int u) { return 128 * (u >> 2) + 32 * (u & 1) + 16 * ((u >> 1) & 1); }
    struct Raw { u32x4 ql, qh; uint32_t sa, sb, d0, d1; };
    template <bool AL16> __device__ static Raw load(const uint8_t *bp, int u) {
        const int n = u >> 2, s = u & 1, l0 = 16 * ((u >> 1) & 1);
        Raw r;
        r.ql = load16_any(bp + 64 * n + 32 * s + l0);
        r.qh = load16_any(bp + 128 + 32 * n + l0);
        const uint8_t *sc = bp + 192 + 8 * n + (l0 >> 4) + 2 * s;
        r.sa = sc[0];
        r.sb = sc[4];
        r.d0 = bp[208];
        r.d1 = bp[209];
        return r;
    }
    __device__ static float dot(const Raw &r, int u, const float (&xa)[16], const float (&xb)[16], float XA, float XB) {
#pragma clang fp contract(off)
        const int s = u & 1;
        const float d = f16f(r.d0 | (r.d1 << 8));
        const u32x4 lo = vmap(r.ql, 0x0f0f0f0fu, 0) | (vmap(r.qh, 0x03030303u, 2 * s) << 4);
        const u32x4 hi = vmap(r.ql, 0x0f0f0f0fu, 4) | (vmap(r.qh, 0x03030303u, 4 + 2 * s) << 4);
        const float SA = dot16u(lo, xa) - 32.f * XA;
        const float SB = dot16u(hi, xb) - 32.f * XB;
        const float ca = d * static_cast<float>(static_cast<int8_t>(r.sa));
        const float cb = d * static_cast<float>(static_cast<int8_t>(r.sb));
        return ca * SA + cb * SB;
    }
};

// Q3_K (dequant.rs:398-451): hmask[32], qs[64], scales[12], d.  Task u: half
// n = u / 4, l0 = 16 ((u / 2) % 2), pair t = u % 2 (j = 2t, 2t + 1): bits 2j of
// qs[32n + l0 + i] with bit 4n + j of hmask[l0 + i] give element
// 128n + 32j + l0 + i, code (bits | hbit << 2) - 4, scale 8n + 2j + l0/16 (its
// low four bits nibble k / 8 of scale byte k % 8, its high two bits field
// k / 4 of byte 8 + k % 4), value d (scale - 32) code.
template <> struct Fmt<OURO_KIND_Q3K> {
    static constexpr int BB = 110, EPB = 256, TPB = 8, G = 32;
    __device__ static int A(int u) { return 128 * (u >> 2) + 64 * (u & 1) + 16 * ((u >> 1) & 1); }
    struct Raw { u32x4 q, hm; uint32_t la, ha, lb, hb, d0, d1; };
    template <bool AL16> __device__ static Raw load(const uint8_t *bp, int u) {
        const int n = u >> 2, t = u & 1, l0 = 16 * ((u >> 1) & 1);
        const int ka = 8 * n + 4 * t + (l0 >> 4), kb = ka + 2;
        Raw r;
        r.q = load16_any(bp + 32 + 32 * n + l0);
        r.hm = load16_any(bp + l0);
        const uint8_t *sc = bp + 96;
        r.la = sc[ka & 7];
        r.ha = sc[8 + (ka & 3)];
        r.lb = sc[kb & 7];
        r.hb = sc[8 + (kb & 3)];
        r.d0 = bp[108];
        r.d1 = bp[109];
        return r;
    }
    __device__ static float dot(const Raw &r, int u, const float (&xa)[16], const float (&xb)[16], float XA, float XB) {
#pragma clang fp contract(off)
        const int n = u >> 2, t = u & 1, l0 = 16 * ((u >> 1) & 1);
        const int ka = 8 * n + 4 * t + (l0 >> 4), kb = ka + 2;
        const int j0 = 2 * t;
        const float d = f16f(r.d0 | (r.d1 << 8));
        const uint32_t sa = bfe(r.la, 4 * (ka >> 3), 4) | (bfe(r.ha, 2 * (ka >> 2), 2) << 4);
        const uint32_t sb = bfe(r.lb, 4 * (kb >> 3), 4) | (bfe(r.hb, 2 * (kb >> 2), 2) << 4);
        const u32x4 ca = vmap(r.q, 0x03030303u, 2 * j0) | (vmap(r.hm, 0x01010101u, 4 * n + j0) << 2);
        const u32x4 cb = vmap(r.q, 0x03030303u, 2 * j0 + 2) | (vmap(r.hm, 0x01010101u, 4 * n + j0 + 1) << 2);
        const float SA = dot16u(ca, xa) - 4.f * XA;
        const float SB = dot16u(cb, xb) - 4.f * XB;
        const float fa = d * (static_cast<float>(sa) - 32.f);
        const float fb = d * (static_cast<float>(sb) - 32.f);
        return fa * SA + fb * SB;
    }
};

struct KqArgs {
    const uint8_t *w;
    const float *x;  // [k][in_len]
    float *y;        // [k][out_len] (column-major, as matmul_q returns it)
    long long row_bytes;
    int out_len, in_len;
    int tpr;    // tasks per row
    int slots;  // row task sets side by side in a workgroup
    int tiles;  // ceil(out_len / (slots * R))
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (56 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(KqArgs) == 56, "KqArgs: kernel argument layout");

template <int KIND>
__device__ __forceinline__ void load_x(const float *xc, int blk, int u, float (&xa)[16], float (&xb)[16], float &XA,
                                       float &XB) {
    using F = Fmt<KIND>;
    const float *p = xc + static_cast<long long>(blk) * F::EPB + F::A(u);
    XA = 0.f;
    XB = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        xa[i] = p[i];
        xb[i] = p[F::G + i];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        XA += xa[i];
        XB += xb[i];
    }
}

// The per-thread sums of one tile (R rows of each slot) into LDS, then one
// wavefront per output row adds its task set's sums.
template <int R>
__device__ __forceinline__ void tile_reduce(const KqArgs &a, float *red, const float (&v)[R], int tile, int col) {
    const int t = threadIdx.x, nt = blockDim.x;
    const int rows_per_tile = a.slots * R;
    const int wave = t >> 6, lane = t & 63, nwaves = nt >> 6;
#pragma unroll
    for (int r = 0; r < R; ++r) red[r * nt + t] = v[r];
    __syncthreads();
    for (int o = wave; o < rows_per_tile; o += nwaves) {
        const int s = o / R, r = o - s * R;
        const float *src = red + r * nt + s * a.tpr;
        float acc = 0.f;
        for (int i = lane; i < a.tpr; i += 64) acc += src[i];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc += xor_shfl(acc, off);
        const int row = tile * rows_per_tile + o;
        if (lane == 0 && row < a.out_len) a.y[static_cast<long long>(col) * a.out_len + row] = acc;
    }
    __syncthreads();
}

// One workgroup walks tiles blockIdx.x, + gridDim.x, ...; the loads of the
// next tile are issued before the current one is summed (two register sets).
// Lanes past the last slot (padding to a whole wavefront) run a clamped copy
// of a real task whose sums are never read, so no load sits behind a branch.
template <int KIND, int R, bool AL16, int MAXT>
__global__ __launch_bounds__(MAXT) void kq_gemv_kernel(KqArgs a) {
    using F = Fmt<KIND>;
    extern __shared__ float red[];  // [R][blockDim.x]
    const int t = threadIdx.x;
    const int slot = min(t / a.tpr, a.slots - 1);
    const int task = min(t - slot * a.tpr, a.tpr - 1);
    const int blk = task / F::TPB, u = task % F::TPB;
    const int col = blockIdx.y;
    float xa[16], xb[16], XA, XB;
    load_x<KIND>(a.x + static_cast<long long>(col) * a.in_len, blk, u, xa, xb, XA, XB);
    const int rows_per_tile = a.slots * R;
    const uint8_t *wb = a.w + static_cast<long long>(blk) * F::BB;
    auto issue = [&](typename F::Raw(&raw)[R], int tile) {
        const int row0 = min(tile, a.tiles - 1) * rows_per_tile + slot * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, a.out_len - 1);  // clamped rows are computed and dropped
            raw[r] = F::template load<AL16>(wb + row * a.row_bytes, u);
        }
    };
    auto sum = [&](const typename F::Raw(&raw)[R], int tile) {
        float v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = F::dot(raw[r], u, xa, xb, XA, XB);
        tile_reduce<R>(a, red, v, tile, col);
    };
    typename F::Raw ra[R], rb[R];
    const int g = gridDim.x;
    int tile = blockIdx.x;
    if (tile >= a.tiles) return;
    issue(ra, tile);
    for (;;) {
        issue(rb, tile + g);
        sum(ra, tile);
        tile += g;
        if (tile >= a.tiles) break;
        issue(ra, tile + g);
        sum(rb, tile);
        tile += g;
        if (tile >= a.tiles) break;
    }
}

// Rows longer than one workgroup's task set (more than 1024 tasks): one
// wavefront per row, x read per task.
template <int KIND>
__global__ __launch_bounds__(256) void kq_row_kernel(KqArgs a) {
    using F = Fmt<KIND>;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int col = blockIdx.y;
    if (row >= a.out_len) return;
    const float *xc = a.x + static_cast<long long>(col) * a.in_len;
    float acc = 0.f;
    for (int task = lane; task < a.tpr; task += 64) {
        const int blk = task / F::TPB, u = task % F::TPB;
        float xa[16], xb[16], XA, XB;
        load_x<KIND>(xc, blk, u, xa, xb, XA, XB);
        const typename F::Raw raw =
            F::template load<false>(a.w + row * a.row_bytes + static_cast<long long>(blk) * F::BB, u);
        acc += F::dot(raw, u, xa, xb, XA, XB);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += xor_shfl(acc, off);
    if (lane == 0) a.y[static_cast<long long>(col) * a.out_len + row] = acc;
}

// Rows per slot per tile (two tiles' loads in flight): measured best on
// 248320x5120 and 6912x2560, with workgroups of at most 256 threads (larger
// ones, 320-512 threads, were 10-40 % slower at the same rows per tile).
template <int KIND> constexpr int kRows = KIND == OURO_KIND_Q3K ? 1 : (KIND == OURO_KIND_Q5K || KIND == OURO_KIND_Q6K) ? 2 : 4;
constexpr int kSlotCap = 256;

int cu_count() {
    static std::once_flag once;
    static int n = 256;
    std::call_once(once, [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
    });
    return n;
}

template <int KIND>
int launch_kind(KqArgs a, int k, bool al16, hipStream_t s) {
    using F = Fmt<KIND>;
    a.tpr = a.in_len / F::EPB * F::TPB;
    if (a.tpr > kMaxThreads) {
        dim3 grid((a.out_len + 3) / 4, k);
        hipLaunchKernelGGL(kq_row_kernel<KIND>, grid, dim3(256), 0, s, a);
        return check_launch("kq_row_kernel");
    }
    // slots: up to 256 threads, the most rows side by side with the fewest
    // idle lanes; a longer row is one task set of up to 1024 threads
    int best = 1;
    if (a.tpr <= kSlotCap) {
        double best_util = 0.0;
        for (int sl = 1; sl * a.tpr <= kSlotCap; ++sl) {
            const int nt = (sl * a.tpr + 63) / 64 * 64;
            if (nt > kSlotCap) break;
            const double util = static_cast<double>(sl * a.tpr) / nt;
            if (util > best_util + 1e-9) best_util = util, best = sl;
        }
    }
    a.slots = best;
    const int nt = (best * a.tpr + 63) / 64 * 64;
    const hipStream_t ss = s;
    auto go = [&](auto rows_c, auto maxt_c) {
        constexpr int R = decltype(rows_c)::value, MAXT = decltype(maxt_c)::value;
        a.tiles = (a.out_len + best * R - 1) / (best * R);
        const int grid_x = std::min(a.tiles, cu_count() * std::max(1, 2048 / nt));
        const size_t lds = static_cast<size_t>(R) * nt * sizeof(float);
        dim3 grid(grid_x, k);
        if (al16) hipLaunchKernelGGL((kq_gemv_kernel<KIND, R, true, MAXT>), grid, dim3(nt), lds, ss, a);
        else hipLaunchKernelGGL((kq_gemv_kernel<KIND, R, false, MAXT>), grid, dim3(nt), lds, ss, a);
    };
    if (nt <= 512) go(std::integral_constant<int, kRows<KIND>>{}, std::integral_constant<int, 512>{});
    else go(std::integral_constant<int, 1>{}, std::integral_constant<int, kMaxThreads>{});
    return check_launch("kq_gemv_kernel");
}

}  // namespace

bool is_kquant(int kind) {
    return kind == OURO_KIND_Q8_0 || kind == OURO_KIND_Q3K || kind == OURO_KIND_Q4K || kind == OURO_KIND_Q5K ||
           kind == OURO_KIND_Q6K;
}

// matvec_qblock for k columns of x (row-major [k][in_len]) into y[k][out_len].
int kq_matmul(const void *payload, int kind, size_t out_len, size_t in_len, const float *x, size_t k, float *y,
              void *stream) {
    const size_t epb = kind == OURO_KIND_Q8_0 ? 32 : 256;
    if (in_len % epb)
        return fail(OURO_ERR_SHAPE, "matvec_q kind %d: in_len %zu not a multiple of %zu", kind, in_len, epb);
    if (reinterpret_cast<uintptr_t>(x) % 4) return fail(OURO_ERR_ALIGN, "matvec_q: x not 4-byte aligned");
    if (k > 65535) return fail(OURO_ERR_SHAPE, "matmul_q: too many columns");
    size_t bb = 0;
    switch (kind) {
    case OURO_KIND_Q8_0: bb = 34; break;
    case OURO_KIND_Q3K: bb = 110; break;
    case OURO_KIND_Q4K: bb = 144; break;
    case OURO_KIND_Q5K: bb = 176; break;
    case OURO_KIND_Q6K: bb = 210; break;
    default: return fail(OURO_ERR_KIND, "matvec_q: kind %d is not block-quantised", kind);
    }
    KqArgs a{};
    a.w = static_cast<const uint8_t *>(payload);
    a.x = x;
    a.y = y;
    a.row_bytes = static_cast<long long>(in_len / epb * bb);
    a.out_len = static_cast<int>(out_len);
    a.in_len = static_cast<int>(in_len);
    // the 144- and 176-byte blocks keep 16-byte alignment when the payload has it
    const bool al16 = reinterpret_cast<uintptr_t>(payload) % 16 == 0;
    const hipStream_t s = as_stream(stream);
    const int kk = static_cast<int>(k);
    switch (kind) {
    case OURO_KIND_Q8_0: return launch_kind<OURO_KIND_Q8_0>(a, kk, false, s);
    case OURO_KIND_Q3K: return launch_kind<OURO_KIND_Q3K>(a, kk, false, s);
    case OURO_KIND_Q4K: return launch_kind<OURO_KIND_Q4K>(a, kk, al16, s);
    case OURO_KIND_Q5K: return launch_kind<OURO_KIND_Q5K>(a, kk, al16, s);
    default: return launch_kind<OURO_KIND_Q6K>(a, kk, false, s);
    }
}

}  // namespace ouro
