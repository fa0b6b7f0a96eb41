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
// one.  Per task the codes are summed against x (S = sum q x) and scaled once
// per run: the contribution is cA S_A - mA X_A + cB S_B - mB X_B with X the
// run's sum of x (the min, or the code offset -32 / -4 of Q6_K / Q3_K, taken
// out of the sum).
//
// Integer sums.  Each run of x is held as exact fixed point: with E the binary
// exponent of the run's largest |x| (|x| < 2^E), x_int = rint(x 2^(22-E)) =
// 65536 p0 + 256 p1 + p2 in balanced int8 digits (elements below 2^(E-23) of
// the run's largest lose their low bits).  The codes, unpacked to one byte
// each, are dotted with the three digit planes by v_dot4_i32_i8 (4 products
// a lane operation, exact int32 sums), and S = 2^(E-22) (65536 S0 + 256 S1 +
// S2) in float.  x is converted once per thread (it stays in registers for
// the whole launch), so the per-element work is a share of a mask and three
// quarter-width dot steps.
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
//
// Q3_K rows of up to 64 blocks, Q4_K / Q5_K payloads on a 16-byte boundary,
// dword-aligned Q6_K rows of an even number of blocks (up to 42) and Q8_0
// rows of a multiple of 8 blocks on a 16-byte boundary, in matrices of 2048
// rows or more, go to kq3_mfma_kernel / kq45_mfma_kernel / kq6_mfma_kernel /
// kq8_mfma_kernel instead: the same digit planes, but the products on the
// int8 matrix cores, in 64-row tiles or 16-row tiles shared by a
// workgroup's wavefronts (kq_tiling).
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
// Ordinary loads: the lines a block shares with its neighbours, and the
// dword a piece shares with the next piece, are read again from L2.
__device__ __forceinline__ u32x4 load16_any(const uint8_t *p) {
    // pointer arithmetic (not integer masks) keeps the global address space
    const uint32_t s = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3);
    const uint8_t *base = p - s;
    const u32x4 lo = *reinterpret_cast<const u32x4_a4 *>(base);
    const uint32_t e = *reinterpret_cast<const uint32_t *>(base + ((s + 15) & ~3u));
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

// The same at a known phase s = (bp + off) & 3: when every row is a whole
// number of dwords, a lane's phase is the same on every row, so it is worked
// out once and each load costs one address add per row.
__device__ __forceinline__ u32x4 load16_at(const uint8_t *bp, int off, uint32_t s) {
    const uint8_t *base = bp + (off - static_cast<int>(s));
    const u32x4 lo = *reinterpret_cast<const u32x4_a4 *>(base);
    const uint32_t e = *reinterpret_cast<const uint32_t *>(base + ((s + 15) & ~3u));
    u32x4 r;
    r.x = __builtin_amdgcn_alignbyte(lo.y, lo.x, s);
    r.y = __builtin_amdgcn_alignbyte(lo.z, lo.y, s);
    r.z = __builtin_amdgcn_alignbyte(lo.w, lo.z, s);
    r.w = __builtin_amdgcn_alignbyte(e, lo.w, s);
    return r;
}

// Piece j of a block, at offset off: aligned (AL16), at the lane's fixed
// phase sh[j] (PH), or at any address.
template <bool AL16, bool PH>
__device__ __forceinline__ u32x4 piece(const uint8_t *bp, int off, const uint32_t *sh, int j) {
    if constexpr (AL16) return *reinterpret_cast<const u32x4 *>(bp + off);
    else if constexpr (PH) return load16_at(bp, off, sh[j]);
    else return load16_any(bp + off);
}

__device__ __forceinline__ float f16f(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t w) {
    return __builtin_amdgcn_ubfe(v, off, w);
}

// A run of 16 x values: its digit planes (byte i of dword d = element
// 4 d + i), the scale 2^(E-22) and the float sum of the run.
struct XRun {
    u32x4 p0, p1, p2;
    float s, X;
};

__device__ __forceinline__ void make_run(const float *p, XRun &r) {
    float v[16];
    float m = 0.f;
    r.X = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = p[i];
#pragma unroll
    for (int i = 0; i < 16; ++i) r.X += v[i];
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
    int E = 0;
    (void)frexpf(m, &E);  // m = f 2^E, f in [0.5, 1): |x| < 2^E (E = 0 for m = 0)
    // a non-finite x makes the run's sum NaN
    r.s = __builtin_isfinite(m) ? ldexpf(1.0f, E - 22) : __builtin_nanf("");
    uint32_t w0[4] = {0, 0, 0, 0}, w1[4] = {0, 0, 0, 0}, w2[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int xi = __builtin_isfinite(m) ? static_cast<int>(rintf(ldexpf(v[i], 22 - E))) : 0;
        const int p2 = ((xi + 128) & 255) - 128;
        const int r1 = (xi - p2) >> 8;  // exact: xi - p2 is a multiple of 256
        const int p1 = ((r1 + 128) & 255) - 128;
        const int p0 = (r1 - p1) >> 8;
        w0[i >> 2] |= static_cast<uint32_t>(p0 & 255) << (8 * (i & 3));
        w1[i >> 2] |= static_cast<uint32_t>(p1 & 255) << (8 * (i & 3));
        w2[i >> 2] |= static_cast<uint32_t>(p2 & 255) << (8 * (i & 3));
    }
    r.p0 = u32x4{w0[0], w0[1], w0[2], w0[3]};
    r.p1 = u32x4{w1[0], w1[1], w1[2], w1[3]};
    r.p2 = u32x4{w2[0], w2[1], w2[2], w2[3]};
}

// sum over the 16 int8 codes of c (byte i of dword d = element 4 d + i)
// times the run's x, from exact int32 sums per digit plane
__device__ __forceinline__ float idot(const u32x4 &c, const XRun &x) {
    int a = 0, b = 0, e = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        a = __builtin_amdgcn_sdot4(static_cast<int>(c[d]), static_cast<int>(x.p0[d]), a, false);
        b = __builtin_amdgcn_sdot4(static_cast<int>(c[d]), static_cast<int>(x.p1[d]), b, false);
        e = __builtin_amdgcn_sdot4(static_cast<int>(c[d]), static_cast<int>(x.p2[d]), e, false);
    }
    return x.s * __builtin_fmaf(static_cast<float>(a), 65536.f,
                                __builtin_fmaf(static_cast<float>(b), 256.f, static_cast<float>(e)));
}

__device__ __forceinline__ u32x4 vmap(const u32x4 &a, uint32_t mask, uint32_t sh) {
    return u32x4{(a.x >> sh) & mask, (a.y >> sh) & mask, (a.z >> sh) & mask, (a.w >> sh) & mask};
}

// (c & cm) | (rotr(h, r) & hm) per dword: a code field merged with high bits
// rotated into place (one v_alignbit, an and and an and-or a dword; the
// rotation wraps only bits that hm drops)
__device__ __forceinline__ u32x4 merge_hi(const u32x4 &c, uint32_t cm, const u32x4 &h, uint32_t r, uint32_t hm) {
    const auto one = [&](uint32_t cv, uint32_t hv) {
        return (cv & cm) | (__builtin_amdgcn_alignbit(hv, hv, r & 31) & hm);
    };
    return u32x4{one(c.x, h.x), one(c.y, h.y), one(c.z, h.z), one(c.w, h.w)};
}

// ---- per kind: block geometry, a task's x runs, its raw loads, its sum ----

template <int KIND> struct Fmt;

// Q8_0 (dequant.rs:225-231): d f16, then 32 int8 codes; one task per block.
template <> struct Fmt<OURO_KIND_Q8_0> {
    static constexpr int BB = 34, EPB = 32, TPB = 1, G = 16, NP = 2;
    __device__ static int A(int) { return 0; }
    __device__ static int poff(int, int j) { return 2 + 16 * j; }
    struct Raw { u32x4 a, b; uint32_t d0, d1; };
    template <bool AL16, bool PH> __device__ static Raw load(const uint8_t *bp, int, const uint32_t *sh) {
        Raw r;
        r.a = piece<false, PH>(bp, 2, sh, 0);
        r.b = piece<false, PH>(bp, 18, sh, 1);
        r.d0 = bp[0];
        r.d1 = bp[1];
        return r;
    }
    __device__ static float dot(const Raw &r, int, const XRun &xa, const XRun &xb) {
        const float d = f16f(r.d0 | (r.d1 << 8));
        return d * (idot(r.a, xa) + idot(r.b, xb));
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
    static constexpr int BB = 144, EPB = 256, TPB = 8, G = 32, NP = 2;
    __device__ static int A(int u) { return 64 * (u >> 1) + 16 * (u & 1); }
    __device__ static int poff(int u, int j) { return j ? 16 + 16 * u : 0; }
    struct Raw { u32x4 h, q; };
    template <bool AL16, bool PH> __device__ static Raw load(const uint8_t *bp, int u, const uint32_t *sh) {
        return Raw{piece<AL16, PH>(bp, 0, sh, 0), piece<AL16, PH>(bp, 16 + 16 * u, sh, 1)};
    }
    __device__ static float dot(const Raw &r, int u, const XRun &xa, const XRun &xb) {
#pragma clang fp contract(off)
        const int j = u >> 1;
        uint32_t s1, m1, s2, m2;
        scale_min_k4(2 * j, r.h.y, r.h.z, r.h.w, s1, m1);
        scale_min_k4(2 * j + 1, r.h.y, r.h.z, r.h.w, s2, m2);
        const float d = f16f(r.h.x & 0xffffu), dmin = f16f(r.h.x >> 16);
        const float SA = idot(vmap(r.q, 0x0f0f0f0fu, 0), xa);
        const float SB = idot(vmap(r.q, 0x0f0f0f0fu, 4), xb);
        return (d * static_cast<float>(s1)) * SA - (dmin * static_cast<float>(m1)) * xa.X +
               ((d * static_cast<float>(s2)) * SB - (dmin * static_cast<float>(m2)) * xb.X);
    }
};

// Q5_K (dequant.rs:454-481): d, dmin, scales[12], qh[32], qs[128].  As Q4_K,
// with bit 2j (low nibble) / 2j + 1 (high nibble) of qh[16h + i] adding 16.
template <> struct Fmt<OURO_KIND_Q5K> {
    static constexpr int BB = 176, EPB = 256, TPB = 8, G = 32, NP = 3;
    __device__ static int A(int u) { return 64 * (u >> 1) + 16 * (u & 1); }
    __device__ static int poff(int u, int j) { return j == 0 ? 0 : j == 1 ? 16 + 16 * (u & 1) : 48 + 16 * u; }
    struct Raw { u32x4 h, qh, q; };
    template <bool AL16, bool PH> __device__ static Raw load(const uint8_t *bp, int u, const uint32_t *sh) {
        return Raw{piece<AL16, PH>(bp, 0, sh, 0), piece<AL16, PH>(bp, 16 + 16 * (u & 1), sh, 1),
                   piece<AL16, PH>(bp, 48 + 16 * u, sh, 2)};
    }
    __device__ static float dot(const Raw &r, int u, const XRun &xa, const XRun &xb) {
#pragma clang fp contract(off)
        const int j = u >> 1;
        uint32_t s1, m1, s2, m2;
        scale_min_k4(2 * j, r.h.y, r.h.z, r.h.w, s1, m1);
        scale_min_k4(2 * j + 1, r.h.y, r.h.z, r.h.w, s2, m2);
        const float d = f16f(r.h.x & 0xffffu), dmin = f16f(r.h.x >> 16);
        // bit 2j / 2j + 1 of qh to bit 4 of each byte
        const u32x4 lo = merge_hi(r.q, 0x0f0f0f0fu, r.qh, 2 * j - 4, 0x10101010u);
        const u32x4 hi = merge_hi(vmap(r.q, 0xffffffffu, 4), 0x0f0f0f0fu, r.qh, 2 * j - 3, 0x10101010u);
        const float SA = idot(lo, xa);
        const float SB = idot(hi, xb);
        return (d * static_cast<float>(s1)) * SA - (dmin * static_cast<float>(m1)) * xa.X +
               ((d * static_cast<float>(s2)) * SB - (dmin * static_cast<float>(m2)) * xb.X);
    }
};

// Q6_K (dequant.rs:484-510): ql[128], qh[64], scales int8[16], d.  Task u:
// half n = u / 4, l0 = 16 ((u / 2) % 2), s = u % 2: ql bytes 64n + 32s + l0 + i
// with bits 2s (low nibble) / 4 + 2s (high nibble) of qh[32n + l0 + i] give
// element 128n + 32s + l0 + i (scale 8n + l0/16 + 2s) and that + 64 (scale + 4),
// code - 32.
template <> struct Fmt<OURO_KIND_Q6K> {
    static constexpr int BB = 210, EPB = 256, TPB = 8, G = 64, NP = 2;
    __device__ static int A(int u) { return 128 * (u >> 2) + 32 * (u & 1) + 16 * ((u >> 1) & 1); }
    __device__ static int poff(int u, int j) {
        const int n = u >> 2, s = u & 1, l0 = 16 * ((u >> 1) & 1);
        return j ? 128 + 32 * n + l0 : 64 * n + 32 * s + l0;
    }
    struct Raw { u32x4 ql, qh; uint32_t sa, sb, d0, d1; };
    template <bool AL16, bool PH> __device__ static Raw load(const uint8_t *bp, int u, const uint32_t *sh) {
        const int n = u >> 2, s = u & 1, l0 = 16 * ((u >> 1) & 1);
        Raw r;
        r.ql = piece<false, PH>(bp, 64 * n + 32 * s + l0, sh, 0);
        r.qh = piece<false, PH>(bp, 128 + 32 * n + l0, sh, 1);
        const uint8_t *sc = bp + 192 + 8 * n + (l0 >> 4) + 2 * s;
        r.sa = sc[0];
        r.sb = sc[4];
        r.d0 = bp[208];
        r.d1 = bp[209];
        return r;
    }
    __device__ static float dot(const Raw &r, int u, const XRun &xa, const XRun &xb) {
#pragma clang fp contract(off)
        const int s = u & 1;
        const float d = f16f(r.d0 | (r.d1 << 8));
        // bits 2s, 2s + 1 / 4 + 2s, 5 + 2s of qh to bits 4, 5 of each byte
        const u32x4 lo = merge_hi(r.ql, 0x0f0f0f0fu, r.qh, 2 * s - 4, 0x30303030u);
        const u32x4 hi = merge_hi(vmap(r.ql, 0xffffffffu, 4), 0x0f0f0f0fu, r.qh, 2 * s, 0x30303030u);
        const float SA = idot(lo, xa) - 32.f * xa.X;
        const float SB = idot(hi, xb) - 32.f * xb.X;
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
    static constexpr int BB = 110, EPB = 256, TPB = 8, G = 32, NP = 2;
    __device__ static int A(int u) { return 128 * (u >> 2) + 64 * (u & 1) + 16 * ((u >> 1) & 1); }
    __device__ static int poff(int u, int j) {
        const int n = u >> 2, l0 = 16 * ((u >> 1) & 1);
        return j ? l0 : 32 + 32 * n + l0;
    }
    struct Raw { u32x4 q, hm; uint32_t la, ha, lb, hb, d0, d1; };
    template <bool AL16, bool PH> __device__ static Raw load(const uint8_t *bp, int u, const uint32_t *sh) {
        const int n = u >> 2, t = u & 1, l0 = 16 * ((u >> 1) & 1);
        const int ka = 8 * n + 4 * t + (l0 >> 4), kb = ka + 2;
        Raw r;
        r.q = piece<false, PH>(bp, 32 + 32 * n + l0, sh, 0);
        r.hm = piece<false, PH>(bp, l0, sh, 1);
        const uint8_t *sc = bp + 96;
        r.la = sc[ka & 7];
        r.ha = sc[8 + (ka & 3)];
        r.lb = sc[kb & 7];
        r.hb = sc[8 + (kb & 3)];
        r.d0 = bp[108];
        r.d1 = bp[109];
        return r;
    }
    __device__ static float dot(const Raw &r, int u, const XRun &xa, const XRun &xb) {
#pragma clang fp contract(off)
        const int n = u >> 2, t = u & 1, l0 = 16 * ((u >> 1) & 1);
        const int ka = 8 * n + 4 * t + (l0 >> 4), kb = ka + 2;
        const int j0 = 2 * t;
        const float d = f16f(r.d0 | (r.d1 << 8));
        const uint32_t sa = bfe(r.la, 4 * (ka >> 3), 4) | (bfe(r.ha, 2 * (ka >> 2), 2) << 4);
        const uint32_t sb = bfe(r.lb, 4 * (kb >> 3), 4) | (bfe(r.hb, 2 * (kb >> 2), 2) << 4);
        // fields j0 and j0 + 1 at bits 0-1 and 2-3 of each byte; hmask bit
        // 4n + j0 to bit 2 (code + 4 hbit) and bit 4n + j0 + 1 to bit 4 (four
        // times code + 4 hbit: the sum is scaled by 1/4, exactly)
        const u32x4 qs = vmap(r.q, 0xffffffffu, 2 * j0);
        const u32x4 ca = merge_hi(qs, 0x03030303u, r.hm, 4 * n + j0 - 2, 0x04040404u);
        const u32x4 cb = merge_hi(qs, 0x0c0c0c0cu, r.hm, 4 * n + j0 - 3, 0x10101010u);
        const float SA = idot(ca, xa) - 4.f * xa.X;
        const float SB = 0.25f * idot(cb, xb) - 4.f * xb.X;
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
__device__ __forceinline__ void load_x(const float *xc, int blk, int u, XRun &xa, XRun &xb) {
    using F = Fmt<KIND>;
    const float *p = xc + static_cast<long long>(blk) * F::EPB + F::A(u);
    make_run(p, xa);
    make_run(p + F::G, xb);
}

// Row sums meet in LDS and are added and stored once per batch of tiles, so
// no global store sits between a tile's loads and the next tile's: a store
// in the loop makes the compiler wait for every load in flight (the vector
// memory counter covers loads and stores in issue order) before it reuses the
// store's registers.
//
// Several task sets per workgroup (slots > 1): each thread's sum of each row
// of a batch of up to kBatch tiles, red[(b R + r) nt + t]; one wavefront per
// row adds a row's task sums.
constexpr int kBatch = 4;
// One task set per workgroup (slots == 1): each wavefront adds its lanes'
// sums in registers and keeps one value per row, red[(b R + r) nwaves +
// wave], for a batch of up to kBatch1 tiles.
constexpr int kBatch1 = 64;

// s_waitcnt vmcnt(0) (gfx9 encoding: expcnt and lgkmcnt left at their
// maxima) at the end of a flush: its stores are then known complete on the
// way back to the loop head, so the compiler need not drain the next tile's
// loads there before reusing the stores' registers.
__device__ __forceinline__ void vm_drain() { __builtin_amdgcn_s_waitcnt(0x0f70); }

template <int R>
__device__ __forceinline__ void stash(float *red, const float (&v)[R], int b) {
    const int t = threadIdx.x, nt = blockDim.x;
#pragma unroll
    for (int r = 0; r < R; ++r) red[(b * R + r) * nt + t] = v[r];
}

// Rows of the nb tiles tile0, tile0 + g, ... of a batch.
template <int R>
__device__ __forceinline__ void flush(const KqArgs &a, const float *red, int nb, int tile0, int g, int col) {
    const int t = threadIdx.x, nt = blockDim.x;
    const int rows_per_tile = a.slots * R;
    const int wave = t >> 6, lane = t & 63, nwaves = nt >> 6;
    __syncthreads();
    for (int o = wave; o < nb * rows_per_tile; o += nwaves) {
        const int b = o / rows_per_tile, ob = o - b * rows_per_tile;
        const int s = ob / R, r = ob - s * R;
        const float *src = red + (b * R + r) * nt + s * a.tpr;
        float acc = 0.f;
        for (int i = lane; i < a.tpr; i += 64) acc += src[i];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc += xor_shfl(acc, off);
        const int row = (tile0 + b * g) * rows_per_tile + ob;
        if (lane == 0 && row < a.out_len) a.y[static_cast<long long>(col) * a.out_len + row] = acc;
    }
    __syncthreads();
    vm_drain();
}

__device__ __forceinline__ float fbits(unsigned u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ unsigned ubits(float f) { return __builtin_bit_cast(unsigned, f); }
// x of the lane the DPP control selects (0 where it selects none)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return fbits(static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(ubits(x)), CTRL, 0xf, 0xf, false)));
}

// Row totals of R per-lane values over the 64 lanes without LDS: offsets 32
// and 16 by v_permlane32_swap / v_permlane16_swap (halving the value count
// while R allows), then a DPP shift-right scan inside 16-lane rows.  Lane L
// with L % (64 / R) == 64 / R - 1 returns the total of row L / (64 / R).
template <int R>
__device__ __forceinline__ float row_totals_f(float (&v)[R]) {
    static_assert(R == 1 || R == 2 || R == 4, "R is 1, 2 or 4");
    constexpr int span = 64 / R;
    if constexpr (R > 1) {
#pragma unroll
        for (int i = 0; i < R / 2; ++i) {
            const auto q = __builtin_amdgcn_permlane32_swap(ubits(v[i]), ubits(v[i + R / 2]), false, false);
            v[i] = fbits(q[0]) + fbits(q[1]);
        }
    } else {
        const auto q = __builtin_amdgcn_permlane32_swap(ubits(v[0]), ubits(v[0]), false, false);
        v[0] = fbits(q[0]) + fbits(q[1]);
    }
    if constexpr (R > 2) {
        const auto q = __builtin_amdgcn_permlane16_swap(ubits(v[0]), ubits(v[1]), false, false);
        v[0] = fbits(q[0]) + fbits(q[1]);
    } else {
        const auto q = __builtin_amdgcn_permlane16_swap(ubits(v[0]), ubits(v[0]), false, false);
        v[0] = fbits(q[0]) + fbits(q[1]);
    }
    constexpr int tail = span < 16 ? span : 16;
    if constexpr (tail > 1) v[0] += dpp_f<0x111>(v[0]);  // row_shr:1
    if constexpr (tail > 2) v[0] += dpp_f<0x112>(v[0]);
    if constexpr (tail > 4) v[0] += dpp_f<0x114>(v[0]);
    if constexpr (tail > 8) v[0] += dpp_f<0x118>(v[0]);
    return v[0];
}

// slots == 1: the wavefront's totals of tile b's R rows into LDS (lanes past
// the task set add 0).
template <int R>
__device__ __forceinline__ void stash1(float *red, float (&v)[R], int b, bool live) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nwaves = blockDim.x >> 6;
    if (!live) {
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = 0.f;
    }
    const float s = row_totals_f<R>(v);
    constexpr int span = 64 / R;
    if (lane % span == span - 1) red[(b * R + lane / span) * nwaves + wave] = s;
}

template <int R>
__device__ __forceinline__ void flush1(const KqArgs &a, const float *red, int nb, int tile0, int g, int col) {
    const int t = threadIdx.x, nwaves = blockDim.x >> 6;
    __syncthreads();
    for (int o = t; o < nb * R; o += blockDim.x) {
        const int b = o / R, r = o - b * R;
        float acc = 0.f;
        for (int w = 0; w < nwaves; ++w) acc += red[(b * R + r) * nwaves + w];
        const int row = (tile0 + b * g) * R + r;
        if (row < a.out_len) a.y[static_cast<long long>(col) * a.out_len + row] = acc;
    }
    __syncthreads();
    vm_drain();
}

// One workgroup walks tiles blockIdx.x, + gridDim.x, ...; the loads of the
// next tile are issued before the current one is summed (two register sets).
// Lanes past the last slot (padding to a whole wavefront) run a clamped copy
// of a real task whose sums are never read, so no load sits behind a branch.
// Wavefronts per SIMD the register allocation is held to: Q3_K fits 4
// (136 -> 128 VGPRs, no spill); the other kinds are left as the compiler
// allocates them (4 waves already; Q8_0 held to 5 ran 10 % slower, the
// others spill when pressed).
template <int KIND> constexpr int kWavesPerSimd = KIND == OURO_KIND_Q3K ? 4 : 1;

template <int KIND, int R, bool AL16, bool PH, int MAXT>
__global__ __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(kWavesPerSimd<KIND>)))
void kq_gemv_kernel(KqArgs a) {
    using F = Fmt<KIND>;
    extern __shared__ float red[];  // slots == 1: [kBatch1][R][wavefronts], else [kBatch][R][blockDim.x]
    const int t = threadIdx.x;
    const int slot = min(t / a.tpr, a.slots - 1);
    const int task = min(t - slot * a.tpr, a.tpr - 1);
    const int blk = task / F::TPB, u = task % F::TPB;
    const int col = blockIdx.y;
    XRun xa, xb;
    load_x<KIND>(a.x + static_cast<long long>(col) * a.in_len, blk, u, xa, xb);
    const int rows_per_tile = a.slots * R;
    const uint8_t *wb = a.w + static_cast<long long>(blk) * F::BB;
    // a row is under 4 GiB (the host checks), so its offset is one 32 x 32 -> 64-bit multiply-add
    const uint32_t rb32 = static_cast<uint32_t>(a.row_bytes);
    // PH: rows are whole dwords, so each piece's byte phase is the same on every row
    uint32_t sh[F::NP];
#pragma unroll
    for (int j = 0; j < F::NP; ++j) sh[j] = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(wb + F::poff(u, j)) & 3);
    auto issue = [&](typename F::Raw(&raw)[R], int tile) {
        const int row0 = min(tile, a.tiles - 1) * rows_per_tile + slot * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = static_cast<uint32_t>(min(row0 + r, a.out_len - 1));  // clamped rows are dropped
            raw[r] = F::template load<AL16, PH>(wb + static_cast<uint64_t>(row) * rb32, u, sh);
        }
    };
    const int g = gridDim.x;
    int tile = blockIdx.x;
    if (tile >= a.tiles) return;
    int tile0 = tile, nb = 0;  // the batch's first tile and its tiles so far
    // sum one tile into the batch; a full batch, or the last tile, is added up
    const bool one = a.slots == 1;          // uniform
    const bool live = t < a.tpr * a.slots;  // not a padding lane
    const int batch = one ? kBatch1 : kBatch;
    auto sum = [&](const typename F::Raw(&raw)[R]) {
        float v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = F::dot(raw[r], u, xa, xb);
        if (one) stash1<R>(red, v, nb, live);
        else stash<R>(red, v, nb);
        ++nb;
        tile += g;
        if (nb == batch || tile >= a.tiles) {  // uniform over the workgroup
            if (one) flush1<R>(a, red, nb, tile0, g, col);
            else flush<R>(a, red, nb, tile0, g, col);
            nb = 0;
            tile0 = tile;
        }
    };
    // The scheduling barriers keep each tile's loads ahead of the previous
    // tile's arithmetic: without them the compiler starts the sum first, and
    // then waits for every load in flight before issuing the next tile's.
    typename F::Raw ra[R], rb[R];
    issue(ra, tile);
    vm_drain();  // the loop head is then reached with only the loop's own loads in flight
    for (;;) {
        issue(rb, tile + g);
        __builtin_amdgcn_sched_barrier(0);
        sum(ra);
        if (tile >= a.tiles) break;
        issue(ra, tile + g);
        __builtin_amdgcn_sched_barrier(0);
        sum(rb);
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
        XRun xa, xb;
        load_x<KIND>(xc, blk, u, xa, xb);
        const uint32_t none[F::NP] = {};
        const typename F::Raw raw =
            F::template load<false, false>(a.w + row * a.row_bytes + static_cast<long long>(blk) * F::BB, u, none);
        acc += F::dot(raw, u, xa, xb);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += xor_shfl(acc, off);
    if (lane == 0) a.y[static_cast<long long>(col) * a.out_len + row] = acc;
}

// ---- Q3_K on the int8 matrix cores ----
//
// v_mfma_i32_16x16x64_i8 with x's digit planes as the A operand and the
// codes as B, so the products leave the vector ALU, which is left with the
// decode and the scales.  A wavefront takes 16 rows (the columns of D) a
// step.  Lane l = 16 g + c loads, for row c of the step, piece g of each
// block: half n = g / 2, bytes l0 = 16 (g % 2) .. l0 + 15 of qs and of
// hmask, and the scale bytes.  For run j (elements 128 n + 32 j + l0 + i,
// code bits 2j of qs, hmask bit 4n + j) its 16-byte B slice holds 32 code as
// int8: the two code bits at bits 5-6 and the inverted hmask bit at bit 7,
// whose int8 value is 32 (lo2 + 4 hbit - 4).  A row 4 g' + p holds digit
// plane p (p < 3) of run (g', j)'s 16 x values in k-slot group g' and zeros
// elsewhere, so D row 4 g + p, column c is run (g, j) of row c summed against
// plane p: lane l receives the three plane sums of its own run, adds them
// exactly in int32 (65536 S0 + 256 S1 + S2, each a multiple of 32) and
// applies the run's scale, the x exponent and, per block, d in fp32.  The
// four pieces' partial sums of a row meet by two lane swaps at the end.
//
// The x planes of a column are built once per workgroup into LDS (896 bytes
// a block: for each j the planes [g][p][16] and a 16-byte zero slot, which
// the A lanes outside their group read, then the exponents [g][j]).
//
// Loads.  When the payload and its rows are dword-aligned (Q3K_ST), a step
// is two blocks (220 bytes of each of the 16 rows) and each wavefront stages
// its rows' step segments through its own LDS area with contiguous 16-byte
// loads (a load's 16-lane quarters read 256 consecutive bytes instead of
// 16 bytes from each of 16 rows).  The even block of a segment sits on a
// 16-byte boundary in LDS, so its pieces are single 16-byte reads; the odd
// block starts 2 bytes before one, so its qs and hmask pieces are read as
// bytes 2..15 (one 16-byte read) plus bytes 0..1 (from the dword before),
// in the element order 2, .., 15, 0, 1, which is the order the odd blocks'
// x planes are stored in.  Otherwise (Q3K_ANY) each lane loads its pieces
// from global memory and shifts them into place.
constexpr int kQ3Waves = 4;          // wavefronts per workgroup, 16 rows each
constexpr int kQ3Threads = 64 * kQ3Waves;
constexpr int kQ3Rows = 16 * kQ3Waves;
constexpr int kQ3MaxBlocks = 64;     // longer rows take the task kernel
constexpr int kQ3Run = 208;          // LDS bytes of a block's run j: planes [g][p][16], then 16 zero bytes
constexpr int kQ3Unit = 4 * kQ3Run + 64;  // a block: its four runs' planes, then the exponents [g][j]
enum { Q3K_ANY = 0, Q3K_ST = 1, Q3K_STS = 2 };  // STS: staged, shared 16-row tiles (kq45_mfma_kernel's SH)
// staged (Q3K_ST): LDS bytes of a row's step segment (220 used); at 240 the
// 16-byte reads of 8 consecutive lanes (rows c .. c + 7) fall in distinct
// banks (224, rows 4 apart share them: 2-way conflicts, 2.5 % slower)
constexpr int kQ3Pitch = 240;
constexpr int kQ3Stage = 16 * kQ3Pitch;  // a wavefront's staging area

typedef int q3v4i __attribute__((ext_vector_type(4)));

// One block's pieces for one lane: qs and hmask (q4 / h4: bytes 0..1 of a
// staged odd block's pieces, in their upper halves) and the scale piece P.
struct Q3Raw {
    u32x4 q, h, P;
    uint32_t q4, h4;
};

// PAR: 0 a staged even block (P = block bytes 96..111: the scale bytes from
// P byte 0, d at 12), 1 a staged odd block (q, h = piece bytes 2..15 and two
// more; P = block bytes 94..109: the scale bytes from byte 2, d at 14), 2 a
// block loaded per lane (as 1, in natural order).
template <int PAR> constexpr int kQ3PO = PAR == 0 ? 0 : 2;

__device__ __forceinline__ void q3_load_any(Q3Raw &r, const uint8_t *bp, int g) {
    r.q = load16_any(bp + 32 + 16 * g);
    r.h = load16_any(bp + 16 * (g & 1));
    r.P = load16_any(bp + 94);
}

// Scale k = 8 n + 2 j + g % 2 of the lane's piece, minus 32: low four bits
// nibble n of scale byte 2 j + g % 2, high two bits field 2 n + j / 2 of
// byte 8 + 2 (j % 2) + g % 2 (dequant.rs:398-451).  L = 8 (g % 2) + 4 n.
// P's high-bit bytes come with the top bit of every two-bit field flipped
// (q3_flip), so the field read as a signed value is hi - 2 and the scale
// minus 32 is lo + 16 (hi - 2).
template <int PO, int J>
__device__ __forceinline__ int q3_scale(const u32x4 &P, uint32_t L) {
    constexpr int blo = PO + 2 * J, bhi = PO + 8 + 2 * (J & 1);
    const uint32_t lo = bfe(P[blo >> 2], 8 * (blo & 3) + L, 4);
    const int hi = __builtin_amdgcn_sbfe(static_cast<int>(P[bhi >> 2]), 8 * (bhi & 3) + 2 * (J >> 1) + L, 2);
    return static_cast<int>(lo) + hi * 16;
}

// P with bit 1 of every two-bit field of the high-bit bytes (scale bytes
// 8..11, P bytes PO + 8 .. PO + 11) flipped.
template <int PO>
__device__ __forceinline__ u32x4 q3_flip(u32x4 P) {
    if constexpr (PO == 0) {
        P.z ^= 0xaaaaaaaau;
    } else {
        P.z ^= 0xaaaa0000u;
        P.w ^= 0x0000aaaau;
    }
    return P;
}

// One block of the lane's row: the four runs' MFMAs, then d.  aoff: the
// lane's A slot within a run's planes; hr[j]: the rotation that brings
// hmask bit 4n + j to bit 7.
template <int PAR>
__device__ __forceinline__ float q3_block(const Q3Raw &r, const uint8_t *xlds, int b, int aoff,
                                          const uint32_t (&hr)[4], uint32_t L, int g) {
#pragma clang fp contract(off)
    constexpr int PO = kQ3PO<PAR>;
    u32x4 q = r.q, h = r.h;
    if constexpr (PAR == 1) {  // bytes 14, 15, 0, 1 in the last dword
        q.w = (q.w & 0xffffu) | (r.q4 & 0xffff0000u);
        h.w = (h.w & 0xffffu) | (r.h4 & 0xffff0000u);
    }
    const u32x4 hn = ~h;
    const u32x4 P = q3_flip<PO>(r.P);
    const uint8_t *xb = xlds + b * kQ3Unit;
    const float4 xs = *reinterpret_cast<const float4 *>(xb + 4 * kQ3Run + 16 * g);
    float blk = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const q3v4i A = *reinterpret_cast<const q3v4i *>(xb + kQ3Run * j + aoff);
        q3v4i B;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t qv = __builtin_amdgcn_alignbit(q[d], q[d], (2 * j - 5) & 31) & 0x60606060u;
            B[d] = static_cast<int>(qv | (__builtin_amdgcn_alignbit(hn[d], hn[d], hr[j]) & 0x80808080u));
        }
        const q3v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, q3v4i{0, 0, 0, 0}, 0, 0, 0);
        const int t = (D[1] << 3) + (D[2] >> 5);
        const int U = (D[0] << 11) + t;
        int s;
        if (j == 0) s = q3_scale<PO, 0>(P, L);
        else if (j == 1) s = q3_scale<PO, 1>(P, L);
        else if (j == 2) s = q3_scale<PO, 2>(P, L);
        else s = q3_scale<PO, 3>(P, L);
        const float xsj = j == 0 ? xs.x : j == 1 ? xs.y : j == 2 ? xs.z : xs.w;
        blk = __builtin_fmaf(static_cast<float>(s), xsj * static_cast<float>(U), blk);
    }
    const uint32_t dbits = PAR == 0 ? (r.P.w & 0xffffu) : (r.P.w >> 16);
    return f16f(dbits) * blk;
}

// x's digit planes of every run into LDS; rot_odd: the element order of the
// odd blocks' B slices (2: elements 2, .., 15, 0, 1).
__device__ __forceinline__ void q3_prep(const float *xc, int nb, uint8_t *xlds, int rot_odd) {
    for (int run = threadIdx.x; run < nb * 16; run += blockDim.x) {
        const int b = run >> 4, g = (run >> 2) & 3, j = run & 3;
        const float *src = xc + 256 * b + 128 * (g >> 1) + 32 * j + 16 * (g & 1);
        const int rot = (b & 1) ? rot_odd : 0;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = src[(i + rot) & 15];
        XRun xr;
        make_run(v, xr);
        uint8_t *xb = xlds + b * kQ3Unit;
        u32x4 *dst = reinterpret_cast<u32x4 *>(xb + kQ3Run * j + 48 * g);
        dst[0] = xr.p0;
        dst[1] = xr.p1;
        dst[2] = xr.p2;
        if (g == 0) *reinterpret_cast<u32x4 *>(xb + kQ3Run * j + 192) = u32x4{0u, 0u, 0u, 0u};
        reinterpret_cast<float *>(xb + 4 * kQ3Run)[4 * g + j] = xr.s;
    }
}

template <int MODE>
__global__ __launch_bounds__(kQ3Threads) void kq3_mfma_kernel(KqArgs a) {
    constexpr bool SH = MODE == Q3K_STS;
    constexpr int RT = SH ? 16 : kQ3Rows;  // rows a tile
    extern __shared__ __attribute__((aligned(16))) uint8_t xlds[];
    const int nb = a.in_len / 256;
    const int col = blockIdx.y;
    const float *xc = a.x + static_cast<long long>(col) * a.in_len;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4, n = g >> 1;
    // A slot: row c = 4 g' + p holds plane p of run (g', j) in k-slot group
    // g, zeros (the run's zero slot) unless g' = g and p < 3
    const int aoff = (c >> 2) == g && (c & 3) < 3 ? 48 * g + 16 * (c & 3) : 192;
    uint32_t hr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) hr[j] = static_cast<uint32_t>(4 * n + j - 7) & 31u;
    const uint32_t L = 8u * (g & 1) + 4u * n;
    const int tiles = (a.out_len + RT - 1) / RT;
    const int rw = SH ? 0 : 16 * wave;  // the wavefront's first row in a tile
    int tile = blockIdx.x;
    if (tile >= tiles) return;  // the whole workgroup (blockIdx.x is uniform)
    const uint32_t rb32 = static_cast<uint32_t>(a.row_bytes);
    auto row_ptr = [&](int t) {
        const int row = min(min(t, tiles - 1) * RT + rw + c, a.out_len - 1);  // clamped rows are dropped
        return a.w + static_cast<uint64_t>(static_cast<uint32_t>(row)) * rb32;
    };
    // a row's partial sums over the four pieces, added by two lane swaps;
    // lanes 0..15 store
    auto finish = [&](float acc, int t) {
        auto q1 = __builtin_amdgcn_permlane32_swap(ubits(acc), ubits(acc), false, false);
        acc = fbits(q1[0]) + fbits(q1[1]);
        auto q2 = __builtin_amdgcn_permlane16_swap(ubits(acc), ubits(acc), false, false);
        acc = fbits(q2[0]) + fbits(q2[1]);
        if constexpr (SH) {  // every wavefront, once a tile
            float(*red)[4][16] = reinterpret_cast<float(*)[4][16]>(xlds + nb * kQ3Unit + kQ3Waves * kQ3Stage);
            const int par = (t / static_cast<int>(gridDim.x)) & 1;
            if (g == 0) red[par][wave][c] = acc;
            __syncthreads();
            const int row = t * RT + c;
            if (wave == 0 && g == 0 && row < a.out_len)
                a.y[static_cast<long long>(col) * a.out_len + row] =
                    ((red[par][0][c] + red[par][1][c]) + red[par][2][c]) + red[par][3][c];
        } else {
            const int row = t * RT + rw + c;
            if (g == 0 && row < a.out_len) a.y[static_cast<long long>(col) * a.out_len + row] = acc;
        }
    };
    const int g8 = gridDim.x;
    if constexpr (MODE != Q3K_ANY) {
        // steps of two blocks (nb is even).  Each wavefront stages its 16
        // rows' 220-byte step segments through its own LDS area with
        // contiguous 16-byte loads: 14 units a row, unit 13 read from byte
        // 204 (overlapping unit 12, so no read passes the segment) and stored
        // at 208, so segment bytes from 208 on sit 4 bytes later in LDS.
        const int steps = nb / 2;
        uint8_t *wl = xlds + nb * kQ3Unit + wave * kQ3Stage;
        int urow[4], uoff[4], ulds[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int id = min(64 * i + lane, 223), un = id % 14;
            urow[i] = id / 14;
            uoff[i] = un < 13 ? 16 * un : 204;
            ulds[i] = kQ3Pitch * (id / 14) + 16 * un;
        }
        u32x4 st[4];
        auto issue = [&](int t, int s) {
            const int r0 = min(t, tiles - 1) * RT + rw;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = min(r0 + urow[i], a.out_len - 1);  // clamped rows are dropped
                st[i] = *reinterpret_cast<const u32x4_a4 *>(a.w + static_cast<uint64_t>(static_cast<uint32_t>(row)) * rb32 +
                                                           220 * s + uoff[i]);
            }
        };
        auto stage = [&]() {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i < 3 || lane < 32) *reinterpret_cast<u32x4 *>(wl + ulds[i]) = st[i];
        };
        const uint8_t *rl = wl + kQ3Pitch * c;
        // the wavefront's steps of a tile: s0, s0 + ss, .. (STS: wavefronts
        // with s0 >= steps have none, and only meet the others at the tile's end)
        const int s0 = SH ? wave : 0, ss = SH ? 4 : 1;
        const bool any = !SH || s0 < steps;
        int s = s0;
        float acc = 0.f;
        if (any) issue(tile, s0);
        q3_prep(xc, nb, xlds, 2);  // the first loads are in flight meanwhile
        __syncthreads();
        for (;;) {
            if (!any) {  // STS only
                finish(0.f, tile);
                tile += g8;
                if (tile >= tiles) break;
                continue;
            }
            stage();
            const bool last = s + ss >= steps;
            issue(last ? tile + g8 : tile, last ? s0 : s + ss);
            __builtin_amdgcn_sched_barrier(0);
            // even block: segment bytes 0..109 (scale bytes from P byte 0, d at 12)
            Q3Raw e, o;
            e.q = *reinterpret_cast<const u32x4 *>(rl + 32 + 16 * g);
            e.h = *reinterpret_cast<const u32x4 *>(rl + 16 * (g & 1));
            e.P = *reinterpret_cast<const u32x4 *>(rl + 96);
            // odd block: segment bytes 110..219; a piece's bytes 2..15 and 0..1
            // (elements 2, .., 15, 0, 1); scale bytes from P byte 2, d at 14
            o.q = *reinterpret_cast<const u32x4 *>(rl + 144 + 16 * g);
            o.q4 = *reinterpret_cast<const uint32_t *>(rl + 140 + 16 * g);
            o.h = *reinterpret_cast<const u32x4 *>(rl + 112 + 16 * (g & 1));
            o.h4 = *reinterpret_cast<const uint32_t *>(rl + 108 + 16 * (g & 1));
            o.P.x = *reinterpret_cast<const uint32_t *>(rl + 204);
            o.P.y = *reinterpret_cast<const uint32_t *>(rl + 212);
            const uint2 zw = *reinterpret_cast<const uint2 *>(rl + 216);
            o.P.z = zw.x;
            o.P.w = zw.y;
            acc += q3_block<0>(e, xlds, 2 * s, aoff, hr, L, g);
            acc += q3_block<1>(o, xlds, 2 * s + 1, aoff, hr, L, g);
            if (last) {
                finish(acc, tile);
                acc = 0.f;
                s = s0;
                tile += g8;
            } else {
                s += ss;
            }
            if (tile >= tiles) break;
        }
    } else {
        Q3Raw r0, r1;
        auto issue = [&](Q3Raw &r, int t, int b) { q3_load_any(r, row_ptr(t) + 110 * b, g); };
        int b = 0;
        float acc = 0.f;
        issue(r0, tile, 0);
        q3_prep(xc, nb, xlds, 0);
        __syncthreads();
        auto step = [&](const Q3Raw &r) {
            acc += q3_block<2>(r, xlds, b, aoff, hr, L, g);
            if (++b == nb) {
                finish(acc, tile);
                acc = 0.f;
                b = 0;
                tile += g8;
            }
        };
        for (;;) {
            issue(r1, b + 1 == nb ? tile + g8 : tile, b + 1 == nb ? 0 : b + 1);
            __builtin_amdgcn_sched_barrier(0);
            step(r0);
            if (tile >= tiles) break;
            issue(r0, b + 1 == nb ? tile + g8 : tile, b + 1 == nb ? 0 : b + 1);
            __builtin_amdgcn_sched_barrier(0);
            step(r1);
            if (tile >= tiles) break;
        }
    }
}

// ---- Q4_K and Q5_K on the int8 matrix cores ----
//
// The scheme of kq3_mfma_kernel with 16-byte-aligned blocks (144 and 176
// bytes): a step is one block of the wavefront's 16 rows, staged through
// its LDS area with contiguous 16-byte loads, and every piece is one
// 16-byte LDS read.  Lane l = 16 g + c takes pair g of row c's block (qs
// bytes 32 g .. 32 g + 31; Q5_K also the 32 qh bytes), whose runs j are
// elements 64 g + 16 j: the low nibbles of the pair's first and second 16
// bytes (sub-block 2 g), then their high nibbles (2 g + 1); Q5_K adds 16
// for bit 2 g (low) / 2 g + 1 (high) of the run's qh byte.  The codes (0..15
// or 0..31) are the B operand as they are; with |p0| <= 64 the plane sums
// combine exactly in int32, and the run adds d s 2^(E-22) U - dmin m X
// (scale_min_k4, X the run's float sum of x).
//
// SH (for matrices of few rows): a tile is 16 rows shared by the four
// wavefronts, wavefront w taking blocks w, w + 4, ..; their partial sums
// meet in LDS (double-buffered by tile, one barrier a tile) and are added in
// wavefront order.  Four times the workgroups and a quarter of the serial
// steps per tile of the 64-row tiles.
constexpr int kQ45Unit = 4 * kQ3Run + 128;  // a block's planes, then the exponents and the x sums [g][j]

// x's digit planes, exponents and sums of every run (elements 256 b + 64 g + 16 j ..)
__device__ __forceinline__ void q45_prep(const float *xc, int nb, uint8_t *xlds) {
    for (int run = threadIdx.x; run < nb * 16; run += blockDim.x) {
        const int b = run >> 4, g = (run >> 2) & 3, j = run & 3;
        XRun xr;
        make_run(xc + 256 * b + 64 * g + 16 * j, xr);
        uint8_t *xb = xlds + b * kQ45Unit;
        u32x4 *dst = reinterpret_cast<u32x4 *>(xb + kQ3Run * j + 48 * g);
        dst[0] = xr.p0;
        dst[1] = xr.p1;
        dst[2] = xr.p2;
        if (g == 0) *reinterpret_cast<u32x4 *>(xb + kQ3Run * j + 192) = u32x4{0u, 0u, 0u, 0u};
        reinterpret_cast<float *>(xb + 4 * kQ3Run)[4 * g + j] = xr.s;
        reinterpret_cast<float *>(xb + 4 * kQ3Run + 64)[4 * g + j] = xr.X;
    }
}

template <int KIND, bool SH>
__global__ __launch_bounds__(kQ3Threads) void kq45_mfma_kernel(KqArgs a) {
#pragma clang fp contract(off)
    constexpr bool Q5 = KIND == OURO_KIND_Q5K;
    constexpr int RT = SH ? 16 : kQ3Rows;  // rows a tile
    constexpr int BB = Q5 ? 176 : 144, NU = BB / 16;  // 16-byte units of a block
    constexpr int kUnits = 16 * NU, kIns = (kUnits + 63) / 64;
    extern __shared__ __attribute__((aligned(16))) uint8_t xlds[];
    const int nb = a.in_len / 256;
    const int col = blockIdx.y;
    const float *xc = a.x + static_cast<long long>(col) * a.in_len;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int aoff = (c >> 2) == g && (c & 3) < 3 ? 48 * g + 16 * (c & 3) : 192;
    const int tiles = (a.out_len + RT - 1) / RT;
    const int rw = SH ? 0 : 16 * wave;  // the wavefront's first row in a tile
    int tile = blockIdx.x;
    if (tile >= tiles) return;  // the whole workgroup (blockIdx.x is uniform)
    const uint32_t rb32 = static_cast<uint32_t>(a.row_bytes);
    const int g8 = gridDim.x;
    uint8_t *wl = xlds + nb * kQ45Unit + wave * (16 * BB);
    // SH: the wavefronts' row sums [tile parity][wavefront][row], after the staging areas
    float(*red)[4][16] = reinterpret_cast<float(*)[4][16]>(xlds + nb * kQ45Unit + 4 * 16 * BB);
    int urow[kIns], uoff[kIns];
#pragma unroll
    for (int i = 0; i < kIns; ++i) {
        const int id = min(64 * i + lane, kUnits - 1);
        urow[i] = id / NU;
        uoff[i] = 16 * (id % NU);
    }
    u32x4 st[kIns];
    auto issue = [&](int t, int b) {
        const int r0 = min(t, tiles - 1) * RT + rw;
#pragma unroll
        for (int i = 0; i < kIns; ++i) {
            const int row = min(r0 + urow[i], a.out_len - 1);  // clamped rows are dropped
            st[i] = *reinterpret_cast<const u32x4 *>(a.w + static_cast<uint64_t>(static_cast<uint32_t>(row)) * rb32 +
                                                     BB * b + uoff[i]);
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < kIns; ++i)
            if (64 * i + lane < kUnits) *reinterpret_cast<u32x4 *>(wl + BB * urow[i] + uoff[i]) = st[i];
    };
    auto finish = [&](float acc, int t) {
        auto q1 = __builtin_amdgcn_permlane32_swap(ubits(acc), ubits(acc), false, false);
        acc = fbits(q1[0]) + fbits(q1[1]);
        auto q2 = __builtin_amdgcn_permlane16_swap(ubits(acc), ubits(acc), false, false);
        acc = fbits(q2[0]) + fbits(q2[1]);
        if constexpr (SH) {  // every wavefront, once a tile
            const int par = (t / g8) & 1;
            if (g == 0) red[par][wave][c] = acc;
            __syncthreads();
            const int row = t * RT + c;
            if (wave == 0 && g == 0 && row < a.out_len)
                a.y[static_cast<long long>(col) * a.out_len + row] =
                    ((red[par][0][c] + red[par][1][c]) + red[par][2][c]) + red[par][3][c];
        } else {
            const int row = t * RT + rw + c;
            if (g == 0 && row < a.out_len) a.y[static_cast<long long>(col) * a.out_len + row] = acc;
        }
    };
    const uint8_t *rl = wl + BB * c;
    // the wavefront's blocks of a tile: b0, b0 + bs, .. (SH: wavefronts with
    // b0 >= nb have none, and only meet the others at the tile's end)
    const int b0 = SH ? wave : 0, bs = SH ? 4 : 1;
    const bool any = !SH || b0 < nb;
    int b = b0;
    float acc = 0.f;
    if (any) issue(tile, b0);
    q45_prep(xc, nb, xlds);  // the first loads are in flight meanwhile
    __syncthreads();
    for (;;) {
        if (!any) {  // SH only
            finish(0.f, tile);
            tile += g8;
            if (tile >= tiles) break;
            continue;
        }
        stage();
        const bool last = b + bs >= nb;
        issue(last ? tile + g8 : tile, last ? b0 : b + bs);
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 P = *reinterpret_cast<const u32x4 *>(rl);  // d, dmin, scales[12]
        const u32x4 q0 = *reinterpret_cast<const u32x4 *>(rl + (Q5 ? 48 : 16) + 32 * g);
        const u32x4 q1 = *reinterpret_cast<const u32x4 *>(rl + (Q5 ? 64 : 32) + 32 * g);
        u32x4 h0{}, h1{};
        if constexpr (Q5) {
            h0 = *reinterpret_cast<const u32x4 *>(rl + 16);
            h1 = *reinterpret_cast<const u32x4 *>(rl + 32);
        }
        uint32_t s0, m0, s1, m1;
        scale_min_k4(2 * g, P.y, P.z, P.w, s0, m0);
        scale_min_k4(2 * g + 1, P.y, P.z, P.w, s1, m1);
        const uint8_t *xb = xlds + b * kQ45Unit;
        const float4 xs = *reinterpret_cast<const float4 *>(xb + 4 * kQ3Run + 16 * g);
        const float4 xx = *reinterpret_cast<const float4 *>(xb + 4 * kQ3Run + 64 + 16 * g);
        float ad = 0.f, am = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const q3v4i A = *reinterpret_cast<const q3v4i *>(xb + kQ3Run * j + aoff);
            const u32x4 &q = (j & 1) ? q1 : q0;
            q3v4i Bc;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t v = (j < 2 ? q[d] : q[d] >> 4) & 0x0f0f0f0fu;
                if constexpr (Q5) {
                    const uint32_t hv = (j & 1) ? h1[d] : h0[d];
                    v |= __builtin_amdgcn_alignbit(hv, hv, static_cast<uint32_t>(2 * g + (j >> 1) - 4) & 31u) & 0x10101010u;
                }
                Bc[d] = static_cast<int>(v);
            }
            const q3v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bc, q3v4i{0, 0, 0, 0}, 0, 0, 0);
            const int U = (D[0] << 16) + (D[1] << 8) + D[2];
            const float xsj = j == 0 ? xs.x : j == 1 ? xs.y : j == 2 ? xs.z : xs.w;
            const float xxj = j == 0 ? xx.x : j == 1 ? xx.y : j == 2 ? xx.z : xx.w;
            ad = __builtin_fmaf(static_cast<float>(j < 2 ? s0 : s1), xsj * static_cast<float>(U), ad);
            am = __builtin_fmaf(static_cast<float>(j < 2 ? m0 : m1), xxj, am);
        }
        acc += f16f(P.x & 0xffffu) * ad - f16f(P.x >> 16) * am;
        if (last) {
            finish(acc, tile);
            acc = 0.f;
            b = b0;
            tile += g8;
        } else {
            b += bs;
        }
        if (tile >= tiles) break;
    }
}

// ---- Q8_0 on the int8 matrix cores ----
//
// d f16, then 32 int8 codes (dequant.rs:225-231).  With the payload on a
// 16-byte boundary and rows of a multiple of 8 blocks (272 bytes, so every
// row is on one too) a step is one 256-element chunk, 8 blocks of each of
// the tile's 16 rows, staged through LDS like kq45_mfma_kernel's blocks, in
// the shared 16-row tiles.  With q45_prep's x planes, MFMA j gives lane
// 16 g + c the run of elements 64 g + 16 j: half j % 2 of block
// 2 g + j / 2 of row c.  Block b of a segment starts at 34 b: the even
// block of a lane's pair has its codes 2 bytes past a dword (read as the
// dwords around them and shifted), the odd one on a dword (its d the upper
// half of the dword before).  The codes are the B operand as they are; the
// plane sums can pass 2^31 combined, so U is combined in fp32.
constexpr int kQ8Seg = 272;  // segment bytes of a row (8 blocks)

__global__ __launch_bounds__(kQ3Threads) void kq8_mfma_kernel(KqArgs a) {
#pragma clang fp contract(off)
    constexpr int NU = kQ8Seg / 16, kUnits = 16 * NU, kIns = (kUnits + 63) / 64;
    extern __shared__ __attribute__((aligned(16))) uint8_t xlds[];
    const int nb = a.in_len / 256;  // steps: 256-element chunks
    const int col = blockIdx.y;
    const float *xc = a.x + static_cast<long long>(col) * a.in_len;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int aoff = (c >> 2) == g && (c & 3) < 3 ? 48 * g + 16 * (c & 3) : 192;
    const int tiles = (a.out_len + 15) / 16;
    int tile = blockIdx.x;
    if (tile >= tiles) return;  // the whole workgroup (blockIdx.x is uniform)
    const uint32_t rb32 = static_cast<uint32_t>(a.row_bytes);
    const int g8 = gridDim.x;
    uint8_t *wl = xlds + nb * kQ45Unit + wave * (16 * kQ8Seg);
    // the wavefronts' row sums [tile parity][wavefront][row], after the staging areas
    float(*red)[4][16] = reinterpret_cast<float(*)[4][16]>(xlds + nb * kQ45Unit + 4 * 16 * kQ8Seg);
    int urow[kIns], uoff[kIns];
#pragma unroll
    for (int i = 0; i < kIns; ++i) {
        const int id = min(64 * i + lane, kUnits - 1);
        urow[i] = id / NU;
        uoff[i] = 16 * (id % NU);
    }
    u32x4 st[kIns];
    auto issue = [&](int t, int s) {
        const int r0 = min(t, tiles - 1) * 16;
#pragma unroll
        for (int i = 0; i < kIns; ++i) {
            const int row = min(r0 + urow[i], a.out_len - 1);  // clamped rows are dropped
            st[i] = *reinterpret_cast<const u32x4 *>(a.w + static_cast<uint64_t>(static_cast<uint32_t>(row)) * rb32 +
                                                     kQ8Seg * s + uoff[i]);
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < kIns; ++i)
            if (64 * i + lane < kUnits) *reinterpret_cast<u32x4 *>(wl + kQ8Seg * urow[i] + uoff[i]) = st[i];
    };
    auto finish = [&](float acc, int t) {  // every wavefront, once a tile
        auto q1 = __builtin_amdgcn_permlane32_swap(ubits(acc), ubits(acc), false, false);
        acc = fbits(q1[0]) + fbits(q1[1]);
        auto q2 = __builtin_amdgcn_permlane16_swap(ubits(acc), ubits(acc), false, false);
        acc = fbits(q2[0]) + fbits(q2[1]);
        const int par = (t / g8) & 1;
        if (g == 0) red[par][wave][c] = acc;
        __syncthreads();
        const int row = t * 16 + c;
        if (wave == 0 && g == 0 && row < a.out_len)
            a.y[static_cast<long long>(col) * a.out_len + row] =
                ((red[par][0][c] + red[par][1][c]) + red[par][2][c]) + red[par][3][c];
    };
    // the lane's blocks 2g (codes from segment byte 68 g + 2) and 2g + 1
    // (d at 68 g + 34, codes from 68 g + 36)
    const uint32_t *re = reinterpret_cast<const uint32_t *>(wl + kQ8Seg * c + 68 * g);
    const int s0 = wave;
    const bool any = s0 < nb;  // wavefronts without steps only meet the others at the tile's end
    int s = s0;
    float acc = 0.f;
    if (any) issue(tile, s0);
    q45_prep(xc, nb, xlds);  // the first loads are in flight meanwhile
    __syncthreads();
    for (;;) {
        if (!any) {
            finish(0.f, tile);
            tile += g8;
            if (tile >= tiles) break;
            continue;
        }
        stage();
        const bool last = s + 4 >= nb;
        issue(last ? tile + g8 : tile, last ? s0 : s + 4);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t w[17];  // the lane's 68 bytes (its two blocks)
#pragma unroll
        for (int i = 0; i < 17; ++i) w[i] = re[i];
        u32x4 ce[2], co[2];  // the even and odd block's codes, halves 0 and 1
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            ce[k >> 2][k & 3] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2);
            co[k >> 2][k & 3] = w[9 + k];
        }
        const float de = f16f(w[0] & 0xffffu), dodd = f16f(w[8] >> 16);
        const uint8_t *xb = xlds + s * kQ45Unit;
        const float4 xs = *reinterpret_cast<const float4 *>(xb + 4 * kQ3Run + 16 * g);
        float be = 0.f, bo = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const q3v4i A = *reinterpret_cast<const q3v4i *>(xb + kQ3Run * j + aoff);
            const u32x4 &q = j < 2 ? ce[j & 1] : co[j & 1];
            const q3v4i Bc{static_cast<int>(q.x), static_cast<int>(q.y), static_cast<int>(q.z), static_cast<int>(q.w)};
            const q3v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bc, q3v4i{0, 0, 0, 0}, 0, 0, 0);
            const float U = __builtin_fmaf(static_cast<float>(D[0]), 65536.f, static_cast<float>((D[1] << 8) + D[2]));
            const float xsj = j == 0 ? xs.x : j == 1 ? xs.y : j == 2 ? xs.z : xs.w;
            if (j < 2) be = __builtin_fmaf(xsj, U, be);
            else bo = __builtin_fmaf(xsj, U, bo);
        }
        acc += de * be + dodd * bo;
        if (last) {
            finish(acc, tile);
            acc = 0.f;
            s = s0;
            tile += g8;
        } else {
            s += 4;
        }
        if (tile >= tiles) break;
    }
}

// ---- Q6_K on the int8 matrix cores ----
//
// ql[128], qh[64], scales int8[16], d (dequant.rs:484-510).  Lane l = 16 g + c
// takes half n = g / 2, bytes l0 = 16 (g % 2) .. l0 + 15 of row c's block: ql
// at 64 n + l0 and 64 n + 32 + l0, qh at 128 + 32 n + l0; its run j is
// elements 128 n + 32 j + l0 (the places of Q3_K's runs): the low nibbles of
// the first / second ql piece (j = 0, 1), then their high nibbles, with bits
// 2j, 2j + 1 of the qh byte below them, scale 8 n + g % 2 + 2 j.  The B slice
// holds 4 (code - 32) as int8: the nibble at bits 2-5, the high bits at 6-7
// with the top one inverted; the plane sums are combined in fp32 (in int32
// they could reach 2^31).  With the payload and rows dword-aligned a step is
// two blocks (an even block on a dword, an odd one 2 bytes past one): each
// wavefront stages its 16 rows' 420-byte step segments at their natural
// offsets in its LDS rows (26 sixteen-byte units and one dword a row, rows 432
// bytes apart: 16-byte reads of 8 consecutive rows fall in distinct banks).
// The even block's pieces are single 16-byte reads; an odd block's piece
// starts 2 bytes past a 16-byte boundary: its bytes 0..13 are bytes 2..15 of
// the 16-byte read there, its bytes 14, 15 come from the dword that follows
// and replace the low half of the first dword (elements 14, 15, 0, .., 13,
// the order the odd blocks' x planes are stored in).
constexpr int kQ6Pitch = 432;  // LDS bytes of a staged row (420 used)

template <int PAR>  // 0: the step's even block, 1: its odd block
__device__ __forceinline__ float q6_block(const uint8_t *rl, const uint8_t *xb, int aoff, int n, int h, int g) {
#pragma clang fp contract(off)
    constexpr int B0 = PAR ? 210 : 0;  // the block's first byte in the LDS row
    u32x4 l0v, l1v, qh;
    uint2 sc;
    float d;
    if constexpr (PAR == 0) {
        l0v = *reinterpret_cast<const u32x4 *>(rl + 64 * n + 16 * h);
        l1v = *reinterpret_cast<const u32x4 *>(rl + 64 * n + 32 + 16 * h);
        qh = *reinterpret_cast<const u32x4 *>(rl + 128 + 32 * n + 16 * h);
        sc = *reinterpret_cast<const uint2 *>(rl + 192 + 8 * n);
        d = f16f(*reinterpret_cast<const uint16_t *>(rl + 208));
    } else {
        // a piece at block offset o (LDS 210 + o): bytes 0..13 from the 16-byte
        // read at 208 + o, bytes 14, 15 from the low half of the dword at 224 + o
        auto piece = [&](int o) {
            u32x4 r = *reinterpret_cast<const u32x4 *>(rl + 208 + o);
            const uint32_t nx = *reinterpret_cast<const uint32_t *>(rl + 224 + o);
            r.x = (r.x & 0xffff0000u) | (nx & 0xffffu);  // [. . b0 b1] -> [b14 b15 b0 b1]
            return r;
        };
        l0v = piece(64 * n + 16 * h);
        l1v = piece(64 * n + 32 + 16 * h);
        qh = piece(128 + 32 * n + 16 * h);
        // scale bytes 8n .. 8n + 7: block 192 + 8n .., LDS 402 + 8n .. (2 bytes past a dword)
        const uint32_t s0 = *reinterpret_cast<const uint32_t *>(rl + 400 + 8 * n);
        const uint32_t s1 = *reinterpret_cast<const uint32_t *>(rl + 404 + 8 * n);
        const uint32_t s2 = *reinterpret_cast<const uint32_t *>(rl + 408 + 8 * n);
        sc.x = __builtin_amdgcn_alignbyte(s1, s0, 2);
        sc.y = __builtin_amdgcn_alignbyte(s2, s1, 2);
        d = f16f(*reinterpret_cast<const uint16_t *>(rl + B0 + 208));
    }
    const float4 xs = *reinterpret_cast<const float4 *>(xb + 4 * kQ3Run + 16 * g);
    float blk = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const q3v4i A = *reinterpret_cast<const q3v4i *>(xb + kQ3Run * j + aoff);
        const u32x4 &ql = (j & 1) ? l1v : l0v;
        q3v4i Bc;
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            const uint32_t lo = (j < 2 ? ql[dw] << 2 : ql[dw] >> 2) & 0x3c3c3c3cu;
            const uint32_t hi = __builtin_amdgcn_alignbit(qh[dw], qh[dw], static_cast<uint32_t>(2 * j - 6) & 31u) & 0xc0c0c0c0u;
            Bc[dw] = static_cast<int>((lo | hi) ^ 0x80808080u);
        }
        const q3v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bc, q3v4i{0, 0, 0, 0}, 0, 0, 0);
        // 4 (65536 S0 + 256 S1 + S2): each plane sum a multiple of 4
        const float U = __builtin_fmaf(static_cast<float>(D[0]), 16384.f, static_cast<float>((D[1] << 6) + (D[2] >> 2)));
        const int scj = __builtin_amdgcn_sbfe(static_cast<int>(j < 2 ? sc.x : sc.y), 8 * h + 16 * (j & 1), 8);
        const float xsj = j == 0 ? xs.x : j == 1 ? xs.y : j == 2 ? xs.z : xs.w;
        blk = __builtin_fmaf(static_cast<float>(scj), xsj * U, blk);
    }
    return d * blk;
}

template <int KIND, bool SH>  // SH: the shared 16-row tiles of kq45_mfma_kernel
__global__ __launch_bounds__(kQ3Threads) void kq6_mfma_kernel(KqArgs a) {
    constexpr int kUnits = 16 * 26, kIns = (kUnits + 63) / 64;
    constexpr int RT = SH ? 16 : kQ3Rows;  // rows a tile
    extern __shared__ __attribute__((aligned(16))) uint8_t xlds[];
    const int nb = a.in_len / 256, steps = nb / 2;
    const int col = blockIdx.y;
    const float *xc = a.x + static_cast<long long>(col) * a.in_len;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4, n = g >> 1, h = g & 1;
    const int aoff = (c >> 2) == g && (c & 3) < 3 ? 48 * g + 16 * (c & 3) : 192;
    const int tiles = (a.out_len + RT - 1) / RT;
    const int rw = SH ? 0 : 16 * wave;  // the wavefront's first row in a tile
    int tile = blockIdx.x;
    if (tile >= tiles) return;  // the whole workgroup (blockIdx.x is uniform)
    const uint32_t rb32 = static_cast<uint32_t>(a.row_bytes);
    const int g8 = gridDim.x;
    uint8_t *wl = xlds + nb * kQ3Unit + wave * (16 * kQ6Pitch);
    float(*red)[4][16] = reinterpret_cast<float(*)[4][16]>(xlds + nb * kQ3Unit + 4 * 16 * kQ6Pitch);
    int urow[kIns], uoff[kIns];
#pragma unroll
    for (int i = 0; i < kIns; ++i) {
        const int id = min(64 * i + lane, kUnits - 1);
        urow[i] = id / 26;
        uoff[i] = 16 * (id % 26);
    }
    u32x4 st[kIns];
    uint32_t tail = 0;  // lanes 0..15: segment bytes 416..419 of row lane
    auto issue = [&](int t, int s) {
        const int r0 = min(t, tiles - 1) * RT + rw;
        const uint8_t *seg = a.w + 420 * s;
#pragma unroll
        for (int i = 0; i < kIns; ++i) {
            const int row = min(r0 + urow[i], a.out_len - 1);  // clamped rows are dropped
            st[i] = *reinterpret_cast<const u32x4_a4 *>(seg + static_cast<uint64_t>(static_cast<uint32_t>(row)) * rb32 + uoff[i]);
        }
        const int trow = min(r0 + (lane & 15), a.out_len - 1);
        tail = *reinterpret_cast<const uint32_t *>(seg + static_cast<uint64_t>(static_cast<uint32_t>(trow)) * rb32 + 416);
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < kIns; ++i)
            if (64 * i + lane < kUnits) *reinterpret_cast<u32x4 *>(wl + kQ6Pitch * urow[i] + uoff[i]) = st[i];
        if (lane < 16) *reinterpret_cast<uint32_t *>(wl + kQ6Pitch * lane + 416) = tail;
    };
    auto finish = [&](float acc, int t) {
        auto q1 = __builtin_amdgcn_permlane32_swap(ubits(acc), ubits(acc), false, false);
        acc = fbits(q1[0]) + fbits(q1[1]);
        auto q2 = __builtin_amdgcn_permlane16_swap(ubits(acc), ubits(acc), false, false);
        acc = fbits(q2[0]) + fbits(q2[1]);
        if constexpr (SH) {  // every wavefront, once a tile
            const int par = (t / g8) & 1;
            if (g == 0) red[par][wave][c] = acc;
            __syncthreads();
            const int row = t * RT + c;
            if (wave == 0 && g == 0 && row < a.out_len)
                a.y[static_cast<long long>(col) * a.out_len + row] =
                    ((red[par][0][c] + red[par][1][c]) + red[par][2][c]) + red[par][3][c];
        } else {
            const int row = t * RT + rw + c;
            if (g == 0 && row < a.out_len) a.y[static_cast<long long>(col) * a.out_len + row] = acc;
        }
    };
    const uint8_t *rl = wl + kQ6Pitch * c;
    // the wavefront's steps of a tile: s0, s0 + ss, .. (SH: wavefronts with
    // s0 >= steps have none, and only meet the others at the tile's end)
    const int s0 = SH ? wave : 0, ss = SH ? 4 : 1;
    const bool any = !SH || s0 < steps;
    int s = s0;
    float acc = 0.f;
    if (any) issue(tile, s0);
    q3_prep(xc, nb, xlds, 14);  // the first loads are in flight meanwhile
    __syncthreads();
    for (;;) {
        if (!any) {  // SH only
            finish(0.f, tile);
            tile += g8;
            if (tile >= tiles) break;
            continue;
        }
        stage();
        const bool last = s + ss >= steps;
        issue(last ? tile + g8 : tile, last ? s0 : s + ss);
        __builtin_amdgcn_sched_barrier(0);
        acc += q6_block<0>(rl, xlds + 2 * s * kQ3Unit, aoff, n, h, g);
        acc += q6_block<1>(rl, xlds + (2 * s + 1) * kQ3Unit, aoff, n, h, g);
        if (last) {
            finish(acc, tile);
            acc = 0.f;
            s = s0;
            tile += g8;
        } else {
            s += ss;
        }
        if (tile >= tiles) break;
    }
}

// Rows per slot per tile (two tiles' loads in flight): measured best over
// 248320x5120 and 6912x2560 (R = 1, 2, 4), with workgroups of at most 256
// threads (384- and 512-thread caps were 10-60 % slower).
template <int KIND> constexpr int kRows = KIND == OURO_KIND_Q4K ? 4 : 2;
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

// Launch shape for rows of tpr tasks: slots side by side in a workgroup of
// nt threads (up to 256 threads, the most rows side by side with the fewest
// idle lanes; a longer row is one task set of up to 1024 threads).  tpr past
// 1024: the row kernel (slots = 0).
struct KqPlan {
    int slots, nt;
};

KqPlan kq_plan(int tpr) {
    if (tpr > kMaxThreads) return KqPlan{0, 0};
    int best = 1;
    if (tpr <= kSlotCap) {
        double best_util = 0.0;
        for (int sl = 1; sl * tpr <= kSlotCap; ++sl) {
            const int nt = (sl * tpr + 63) / 64 * 64;
            if (nt > kSlotCap) break;
            const double util = static_cast<double>(sl * tpr) / nt;
            if (util > best_util + 1e-9) best_util = util, best = sl;
        }
    }
    return KqPlan{best, (best * tpr + 63) / 64 * 64};
}

// Tiling of the matrix-core kernels for a matrix of out_len rows whose x
// planes and staging areas take lds bytes of LDS and whose rows take steps
// serial steps: 0 the 64-row tiles, 1 the shared 16-row tiles (SH), -1 the
// task kernel.  Q4_K, Q5_K and Q6_K (any_sh) take SH wherever it fits, tall
// matrices included (248320x5120: 133.1 -> 121.6, 160.6 -> 147.1, 182.7 ->
// 176.1 us; 16384x5120 Q4_K 17.7 -> 12.6 us).  Q3_K keeps the 64-row tiles
// (248320x5120 109.7 against 116.4 us with SH) unless they number fewer
// than the CUs, where each workgroup walks its rows' whole length alone: SH
// then pays when the 64-row grid would leave over half the CUs idle or a
// tile is 12 steps or more (14336x4096, 8 steps: 10.4 against 11.1 us with
// SH; 8192x8192 16.5 -> 11.4; 4096x4096 9.0 -> 5.3).  Where SH does not fit
// in LDS on a matrix of few rows, and below 2048 rows, the task kernel is
// faster (Q3_K 4096x14336 20.3 against 26.4 us; 1024x5120 4.2-5.2 against
// 12.0-13.2 us).  Other Q4_K measurements: 8192x8192 23.4 -> 11.8,
// 4096x14336 38.1 -> 15.5, 6912x2560 9.1 -> 6.0 us with SH.
constexpr int kShRed = 2 * 4 * 16 * 4;  // LDS bytes of SH's row sums
int kq_tiling(int out_len, size_t lds, int steps, bool any_sh) {
    if (lds > 65536) return -1;
    const int t64 = (out_len + kQ3Rows - 1) / kQ3Rows, cus = cu_count();
    const bool sh = out_len >= 2048 && lds + kShRed <= 65536;
    if (any_sh && sh) return 1;
    if (t64 >= cus) return 0;
    if (any_sh || 2 * t64 <= cus || steps >= 12) return sh ? 1 : -1;
    return 0;
}

template <int KIND>
int launch_kind(KqArgs a, int k, bool al16, hipStream_t s) {
    const bool ph = a.row_bytes % 4 == 0;
    using F = Fmt<KIND>;
    if constexpr (KIND == OURO_KIND_Q8_0) {
        // a 16-byte-aligned payload with rows of a multiple of 8 blocks
        const int nb = a.in_len / 256;
        const size_t lds = static_cast<size_t>(nb) * kQ45Unit + kQ3Waves * 16 * kQ8Seg;
        if (al16 && a.in_len % 256 == 0 && kq_tiling(a.out_len, lds, nb, true) == 1) {
            const dim3 grid(std::min((a.out_len + 15) / 16, cu_count() * 4), k);
            hipLaunchKernelGGL(kq8_mfma_kernel, grid, dim3(kQ3Threads), lds + kShRed, s, a);
            return check_launch("kq8_mfma_kernel");
        }
    }
    if constexpr (KIND == OURO_KIND_Q6K) {
        // dword-aligned payload and rows (nb even): steps of an even and an odd block
        const int nb = a.in_len / 256;
        const size_t lds = static_cast<size_t>(nb) * kQ3Unit + kQ3Waves * 16 * kQ6Pitch;
        const int til = kq_tiling(a.out_len, lds, nb / 2, true);
        if (reinterpret_cast<uintptr_t>(a.w) % 4 == 0 && ph && til >= 0) {
            if (til == 1) {
                const dim3 grid(std::min((a.out_len + 15) / 16, cu_count() * 3), k);
                hipLaunchKernelGGL((kq6_mfma_kernel<KIND, true>), grid, dim3(kQ3Threads), lds + kShRed, s, a);
            } else {
                const dim3 grid(std::min((a.out_len + kQ3Rows - 1) / kQ3Rows, cu_count() * 3), k);
                hipLaunchKernelGGL((kq6_mfma_kernel<KIND, false>), grid, dim3(kQ3Threads), lds, s, a);
            }
            return check_launch("kq6_mfma_kernel");
        }
    }
    if constexpr (KIND == OURO_KIND_Q4K || KIND == OURO_KIND_Q5K) {
        // the matrix-core kernel on a 16-byte-aligned payload (every block and row then is)
        const int nb = a.in_len / 256;
        const size_t lds = static_cast<size_t>(nb) * kQ45Unit + kQ3Waves * 16 * F::BB;
        const int til = kq_tiling(a.out_len, lds, nb, true);
        if (al16 && til >= 0) {
            if (til == 1) {
                const dim3 grid(std::min((a.out_len + 15) / 16, cu_count() * 4), k);
                hipLaunchKernelGGL((kq45_mfma_kernel<KIND, true>), grid, dim3(kQ3Threads), lds + kShRed, s, a);
            } else {
                const dim3 grid(std::min((a.out_len + kQ3Rows - 1) / kQ3Rows, cu_count() * 4), k);
                hipLaunchKernelGGL((kq45_mfma_kernel<KIND, false>), grid, dim3(kQ3Threads), lds, s, a);
            }
            return check_launch("kq45_mfma_kernel");
        }
    }
    if constexpr (KIND == OURO_KIND_Q3K) {
        const int nb = a.in_len / 256;
        if (nb <= kQ3MaxBlocks) {
            // dword-aligned payload and rows (so nb is even): the staged loads
            const bool al = reinterpret_cast<uintptr_t>(a.w) % 4 == 0 && ph;
            const int tiles = (a.out_len + kQ3Rows - 1) / kQ3Rows;
            const dim3 grid(std::min(tiles, cu_count() * 4), k);
            const size_t lds = static_cast<size_t>(nb) * kQ3Unit;
            const size_t lds_st = lds + kQ3Waves * kQ3Stage;
            const int til = al ? kq_tiling(a.out_len, lds_st, nb / 2, false) : -1;
            if (til == 1) {
                const dim3 gs(std::min((a.out_len + 15) / 16, cu_count() * 4), k);
                hipLaunchKernelGGL(kq3_mfma_kernel<Q3K_STS>, gs, dim3(kQ3Threads), lds_st + kShRed, s, a);
                return check_launch("kq3_mfma_kernel");
            }
            if (til == 0) {
                hipLaunchKernelGGL(kq3_mfma_kernel<Q3K_ST>, grid, dim3(kQ3Threads), lds_st, s, a);
                return check_launch("kq3_mfma_kernel");
            }
            if (!al && kq_tiling(a.out_len, lds, nb, false) == 0) {  // unstaged: each lane loads its own pieces
                hipLaunchKernelGGL(kq3_mfma_kernel<Q3K_ANY>, grid, dim3(kQ3Threads), lds, s, a);
                return check_launch("kq3_mfma_kernel");
            }
        }
    }
    a.tpr = a.in_len / F::EPB * F::TPB;
    const KqPlan pl = kq_plan(a.tpr);
    if (!pl.slots) {
        dim3 grid((a.out_len + 3) / 4, k);
        hipLaunchKernelGGL(kq_row_kernel<KIND>, grid, dim3(256), 0, s, a);
        return check_launch("kq_row_kernel");
    }
    a.slots = pl.slots;
    const int nt = pl.nt;
    auto go = [&](auto rows_c, auto maxt_c) {
        constexpr int R = decltype(rows_c)::value, MAXT = decltype(maxt_c)::value;
        a.tiles = (a.out_len + a.slots * R - 1) / (a.slots * R);
        const int grid_x = std::min(a.tiles, cu_count() * std::max(1, 2048 / nt));
        const size_t lds = (a.slots == 1 ? static_cast<size_t>(kBatch1) * R * (nt / 64)
                                         : static_cast<size_t>(kBatch) * R * nt) * sizeof(float);
        dim3 grid(grid_x, k);
        if (al16) hipLaunchKernelGGL((kq_gemv_kernel<KIND, R, true, false, MAXT>), grid, dim3(nt), lds, s, a);
        else if (ph) hipLaunchKernelGGL((kq_gemv_kernel<KIND, R, false, true, MAXT>), grid, dim3(nt), lds, s, a);
        else hipLaunchKernelGGL((kq_gemv_kernel<KIND, R, false, false, MAXT>), grid, dim3(nt), lds, s, a);
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
    if (a.row_bytes >= (1LL << 32)) return fail(OURO_ERR_SHAPE, "matvec_q kind %d: in_len %zu too large", kind, in_len);
    a.out_len = static_cast<int>(out_len);
    a.in_len = static_cast<int>(in_len);
    // the 144- and 176-byte blocks keep 16-byte alignment when the payload has it
    const bool al16 = reinterpret_cast<uintptr_t>(payload) % 16 == 0;
    const hipStream_t s = as_stream(stream);
    const int kk = static_cast<int>(k);
    switch (kind) {
    case OURO_KIND_Q8_0: return launch_kind<OURO_KIND_Q8_0>(a, kk, al16, s);
    case OURO_KIND_Q3K: return launch_kind<OURO_KIND_Q3K>(a, kk, false, s);
    case OURO_KIND_Q4K: return launch_kind<OURO_KIND_Q4K>(a, kk, al16, s);
    case OURO_KIND_Q5K: return launch_kind<OURO_KIND_Q5K>(a, kk, al16, s);
    default: return launch_kind<OURO_KIND_Q6K>(a, kk, false, s);
    }
}

}  // namespace ouro
