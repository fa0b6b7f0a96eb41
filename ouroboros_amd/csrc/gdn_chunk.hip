// gdn_chunk.hip - chunked (WY / UT-transform) prefill of the gated delta-net.
//
// The reference prefills token by token (shell/src/bonsai.rs:48-52 driving
// run_delta, qwen35.rs:1048-1158; the recurrence of qwen35.rs:27-57).  This
// kernel computes the same recurrence 64 tokens at a time.  For a chunk with
// start state S0 (d_k x d_v, S(i,j) at i + j*d), raw bf16 rows K, Q, V, per
// token beta and log-decay gate, g = inclusive cumsum(gate), b = exp(g),
// nk = 1/(|k|+eps), nq = scale/(|q|+eps):
//   A[s][j] = beta_s exp(g_s - g_j) nk_s nk_j (K K^T)[s][j]   (j < s)
//   T       = (I + A)^-1                        (unit lower triangular)
//   R       = diag(beta) V - diag(beta b nk) (K S0)
//   U       = T R                               (the pseudo-values u_s)
//   O       = diag(b nq) (Q S0) + Pt U,  Pt[r][s] = exp(g_r-g_s) nq_r nk_s (Q K^T)[r][s], s <= r
//   S_end   = b_C S0 + K^T diag(nk exp(g_C - g)) U
// which is the token recurrence S_t = g_t S_{t-1} + beta_t k_t (v_t - g_t S_{t-1}^T k_t)^T,
// o_t = S_t^T q_t unrolled over the chunk.
//
// Every contraction runs on v_mfma_f32_16x16x32_bf16 with fp32 accumulate.
// Raw bf16 q, k, v are exact MFMA operands; fp32 operands (S, T, R, U, Pt)
// are split as hi + lo bf16 and multiplied in two or three passes, so the
// products carry ~16 mantissa bits.  T = (I + A)^-1 is inverted in fp32:
// the four 16x16 diagonal blocks by substitution on the VALU, the six blocks
// below them on v_mfma_f32_16x16x4f32.
//
// Two kernels.  gdn_chunk_prep_kernel runs every (chunk, v-head) in parallel
// and computes what does not depend on the state: k-row norms, g, beta and
// T, written to a workspace record (it does not read Q).
// gdn_chunk_scan_kernel then walks the chunks of a sequence in order.
// Output column j of the recurrence only touches state column j, so
// 16-column stripes of the state are independent chains: a "chain" wave
// keeps one stripe in registers and runs K S0 -> R -> U -> S update (and
// forms the q-row norms of one row tile from the Q operands it reads),
// while a paired "output" wave forms Pt from the chunk's K and Q rows and O
// for the same stripe and, with the record's beta, g and k-norms, the other
// per-row coefficients of the next chunk; two barriers per chunk.
#include "common.hpp"

#include <atomic>

namespace ouro {
namespace {

constexpr int kD = 128;           // d_k = d_v (qwen35.rs:8)
constexpr int kC = 64;            // chunk length
constexpr int kDVB = 64;          // state columns per scan workgroup (16 per wave)
constexpr int kScanThreads = 512; // 4 chain + 4 output waves
constexpr int kPrepThreads = 256; // 4 waves
constexpr int kMaxSeq = 256;      // sequences per launch (offsets by value)

constexpr int KP = kD + 8;        // bf16 row pitch of K, Q (272 B)
constexpr int KTP = kC + 4;       // bf16 row pitch of K^T (136 B; conflict-free 8-byte reads)

// T slots are (s-tile a, t-slab q) = (0,0) (1,0) (2,0) (3,0) (2,1) (3,1)
// (T is lower triangular: slab q is zero for a < 2q); the scan's Pt slots
// are (r-tile b, s-slab q) = (0,0) (1,0) (2,0) (2,1) (3,0) (3,1).  A slot
// is an A operand: lane r + 16 g holds T[16a + r][32q + 4g .. +3] ++
// T[16a + r][32q + 16 + 4g .. +3], as hi and lo bf16: its first half is
// 16x16 block (a, 2q) of T, its second half block (a, 2q + 1).  In slots
// (0,0) and (2,1) the second half lies above the diagonal and is zero; in
// a diagonal block (i, i) lane r + 16 g is zero when 4 g > r, so 40 of its
// 64 lanes carry values.
//
// Workspace record of one (chunk, v-head), 256-byte aligned, 9,472 B, in
// 16-byte units:
//   0 .. 255    the dense slots (2,0) (3,0) as [slot][hi, lo][64 lanes]
//   256 .. 383  the dense blocks (1,0) (3,2), [block][64 lanes] holding
//               (hi.xy, lo.xy) of the lane's four values
//   384 .. 543  the diagonal blocks (0,0) (1,1) (2,2) (3,3), [block][40]
//               in the same form, lane r + 16 g (4 g <= r) at diag_unit
//   8,704 B:    beta, g (inclusive cumsum of the log-decays), nk [64] fp32
// The scan forms the other per-row coefficients from these while it
// stages them (LDS vectors below), and the q-row norms nq from the Q rows
// it stages; nq is applied to the output rows last: O = nq (e^g Q S0 +
// Pt U) with nq taken out of Pt.  Each record is written once by the prep
// and read once by the scan, so its size is HBM traffic twice over: with
// all ten blocks stored whole (11,008 B) a 4 x 4096-token call (8,192
// records) moved 25 MB more.
constexpr int REC_T = 0;
constexpr int RU_HALF = 256;  // first unit of the dense blocks (1,0) (3,2)
constexpr int RU_DIAG = 384;  // first unit of the diagonal blocks
constexpr int kRecUnits = RU_DIAG + 4 * 40;
constexpr int REC_V = kRecUnits * 16;
enum { R_BETA = 0, R_G = 64, R_NK = 128, kRecVec = 192 };
constexpr size_t kRec = 9472;
static_assert(REC_V + kRecVec * 4 <= static_cast<int>(kRec) && kRec % 256 == 0, "record size");
// Unit of lane r + 16 g (4 g <= r) of diagonal block i: lanes in g-major
// order, g = 0 holding 16 rows, g = 1 12, g = 2 8, g = 3 4.
__host__ __device__ constexpr int diag_unit(int i, int r, int g) { return RU_DIAG + 40 * i + r + 2 * g * (7 - g); }
// T slot holding diagonal block i (its first half for even i, second for odd).
__host__ __device__ constexpr int diag_tslot(int i) { return i < 2 ? i : i + 2; }

// The scan's LDS vectors [64] fp32 of a chunk: beta, rk = beta e^g nk,
// w = nk e^(g_C - g), eg = e^g, g, nk, rho = e^(g - g_16floor(r/16)) and
// cb_b = e^(g_16b - g) nk for rows < 16b (b = 1..3).
enum { V_BETA = 0, V_RK = 64, V_W = 128, V_EG = 192, V_G = 256, V_NK = 320, V_RHO = 384, V_CB = 448, kVec = 640 };

// Scan kernel LDS byte offsets: K, Q, V, K^T, the vectors and the T
// operands of chunk c are staged in the second half of chunk c - 1 and read
// in the first half of chunk c (K^T in the second: it is double-buffered);
// the Pt operands are formed from K and Q in the first half of chunk c and
// read in its second half; X passes so (Q S0) and U (first half) from each
// chain wave to its output wave.
constexpr int VP = kDVB + 8;                // bf16 row pitch of the V tile (144 B)
constexpr int S_K = 0;                      // K [64][KP]
constexpr int S_Q = S_K + kC * KP * 2;      // Q [64][KP]
constexpr int S_KT = S_Q + kC * KP * 2;     // K^T [2][128][KTP]
constexpr int S_V = S_KT + 2 * kD * KTP * 2;  // V [64][VP]: the workgroup's 64 columns
constexpr int S_VEC = S_V + kC * VP * 2;    // vectors [kVec]
constexpr int S_T = S_VEC + kVec * 4;       // T operands [12][64] x 16 B
constexpr int S_P = S_T + 12 * 64 * 16;     // Pt operands [12][64] x 16 B
constexpr int S_X = S_P + 12 * 64 * 16;     // [4 waves][(so Q S0)^T 4 KiB, U hi/lo 4 KiB]
constexpr int X_WAVE = 8192;
constexpr int S_NQ = S_X + 4 * X_WAVE;      // nq [64] of the chunk (chain wave w: rows 16w.., read by the output waves)
constexpr int SCAN_LDS = S_NQ + kC * 4;
static_assert(SCAN_LDS <= 160 * 1024 && S_V % 16 == 0 && S_VEC % 16 == 0 && S_T % 16 == 0, "scan LDS layout");

// Prep kernel: one wave per (chunk, v-head), four per workgroup; each wave
// has A (then T) [64][AP] fp32 and three vectors [64] in LDS.
constexpr int kPrepWaves = kPrepThreads / 64;
constexpr int AP = kC + 4;                         // fp32 row pitch of A / T
constexpr int PW_BYTES = kC * AP * 4 + 3 * kC * 4; // per-wave LDS
constexpr int PREP_LDS = kPrepWaves * PW_BYTES;
constexpr int kPrepGrid = 512;  // prep workgroups per launch: two per CU

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

struct ChunkArgs {
    float *state;
    const uint16_t *q, *k, *v;
    const float *gate, *beta;
    float *out;
    unsigned char *ws;
    int Hk, Hv, nseq;
    unsigned flags;
    float eps;
    int cu[kMaxSeq + 1];    // token offsets of the sequences
    int coff[kMaxSeq + 1];  // chunk offsets (cumulative chunk counts)
};
// passed by value to a kernel: the host and device passes must lay it out
// alike (2144 bytes in the code object's kernel-argument metadata)
static_assert(sizeof(ChunkArgs) == 2144, "ChunkArgs: kernel argument layout");

__device__ __forceinline__ f32x4 mfma(const bf16x8 &a, const bf16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf(uint16_t u) { return bf16_bits_to_f32(u); }

__device__ __forceinline__ f32x4 ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }

__device__ __forceinline__ int khead(const ChunkArgs &a, int h) {
    return (a.flags & OURO_GDN_KHEAD_DIV) ? h / (a.Hv / a.Hk) : h % a.Hk;
}

// The j-th of the Hv / Hk v-heads that read k-head kh.
__device__ __forceinline__ int vhead(const ChunkArgs &a, int kh, int j) {
    return (a.flags & OURO_GDN_KHEAD_DIV) ? kh * (a.Hv / a.Hk) + j : kh + a.Hk * j;
}

// Sum of squares of 32 bf16 (4 x 16 B).
__device__ __forceinline__ float sumsq32(const uint4 (&w)[4]) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t ws[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x0 = __uint_as_float(ws[e] << 16), x1 = __uint_as_float(ws[e] & 0xffff0000u);
            ss += x0 * x0 + x1 * x1;
        }
    }
    return ss;
}

// x = hi + lo for two values at once: hi = bf16(x) (round to nearest even),
// lo = bf16(x - hi); packed as bf16 pairs.
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
    const float ha = __uint_as_float(h << 16), hb = __uint_as_float(h & 0xffff0000u);
    hi = h;
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a - ha, b - hb}, bf16x2));
}

// ---------------------------------------------------------------------------
// Operand layout.  v_mfma_f32_16x16x32_bf16 lane l (r = l % 16, g = l / 16)
// holds A[r][8g..8g+7], B[8g..8g+7][r] and D[4g..4g+3][r].  A 64-row D
// result (four 16-row tiles) is used directly as the B operand of the next
// contraction over those 64 rows: for the 32-row slab of tiles 2q, 2q+1 the
// lane's eight k values are rows 32q + 4g + {0..3} and 32q + 16 + 4g + {0..3}
// (tile 2q, then tile 2q+1).  The operand on the other side is read with the
// same row order (ld_perm, ld_op), so the sum runs over the same k set.  The same
// pair of D tiles of a transposed product (lane index = the other matrix
// dimension) is an A operand in that order.
// ---------------------------------------------------------------------------

// Two D tiles (rows 32q + 4g + e and 32q + 16 + 4g + e) as hi and lo operands.
__device__ __forceinline__ void split8(const f32x4 &t0, const f32x4 &t1, bf16x8 &hi, bf16x8 &lo) {
    uint4 h, l;
    split2(t0[0], t0[1], h.x, l.x);
    split2(t0[2], t0[3], h.y, l.y);
    split2(t1[0], t1[1], h.z, l.z);
    split2(t1[2], t1[3], h.w, l.w);
    hi = __builtin_bit_cast(bf16x8, h);
    lo = __builtin_bit_cast(bf16x8, l);
}

// A operand row[base + 4g .. +3] ++ row[base + 16 + 4g .. +3].
__device__ __forceinline__ bf16x8 ld_perm(const uint16_t *row, int base, int lg) {
    const uint2 x = *reinterpret_cast<const uint2 *>(row + base + 4 * lg);
    const uint2 y = *reinterpret_cast<const uint2 *>(row + base + 16 + 4 * lg);
    return __builtin_bit_cast(bf16x8, make_uint4(x.x, x.y, y.x, y.y));
}

// The K and Q rows in the scan's LDS keep each 32-column slab in operand
// order: columns 4a .. 4a+3 and 16 + 4a .. 16 + 4a + 3 side by side at
// 8a (kpos maps a column w of the slab, w % 4 == 0, to its place), so the
// operand of ld_perm is one aligned 16-byte read (ld_op): 0.324 -> 0.296 ms
// per 4 x 4096-token call.  The same order for K^T (16-byte aligned rows of
// 144 B) was slower, 0.301 ms.
__device__ __forceinline__ int kpos(int w) { return 8 * ((w & 15) >> 2) + 4 * (w >> 4); }
__device__ __forceinline__ bf16x8 ld_op(const uint16_t *row, int base, int lg) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(row + base + 8 * lg));
}
// Columns 8c .. 8c+7 of a K or Q row into that order.
__device__ __forceinline__ void st_op(uint16_t *row, int c, const uint4 &v) {
    uint16_t *slab = row + 32 * (c >> 2);
    const int w = 8 * (c & 3);
    *reinterpret_cast<uint2 *>(slab + kpos(w)) = make_uint2(v.x, v.y);
    *reinterpret_cast<uint2 *>(slab + kpos(w + 4)) = make_uint2(v.z, v.w);
}

// Pt slot of (r-tile bb, s-slab q), q <= bb / 2.
__host__ __device__ constexpr int pslot(int bb, int q) { return bb < 2 ? bb : 2 * (bb - 1) + q; }
// T slot of (s-tile aa, t-slab q), q <= aa / 2.
__host__ __device__ constexpr int tslot(int aa, int q) { return q == 0 ? aa : 2 + aa; }

// ---------------------------------------------------------------------------
// Prep: one wave per (chunk, v-head) item, no workgroup barriers.  K stays
// in registers in MFMA operand layout (lane r + 16 g holds
// K[16a + r][32kk + 8g .. +7] for row tile a and k-step kk), so K K^T needs
// no LDS; Q is not read (the scan forms the q-row norms).  A^T goes to the wave's LDS
// and T = (I + A)^-1 is solved in 16 x 16 blocks.
// ---------------------------------------------------------------------------
// Where item `item` (a (chunk, v-head) pair) lies: items of one chunk in
// k-head order, so that the v-heads reading the same K and Q rows are
// neighbours.
struct PrepItem {
    int cg, h, t0, n, kh;
};
__device__ __forceinline__ PrepItem prep_item(const ChunkArgs &a, int item) {
    PrepItem p;
    p.cg = item / a.Hv;
    p.h = vhead(a, (item % a.Hv) / (a.Hv / a.Hk), (item % a.Hv) % (a.Hv / a.Hk));
    int lo = 0, hi = a.nseq;  // sequence of chunk cg: coff[lo] <= cg < coff[lo + 1]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (a.coff[mid] <= p.cg) lo = mid; else hi = mid;
    }
    p.t0 = a.cu[lo] + (p.cg - a.coff[lo]) * kC;
    p.n = min(kC, a.cu[lo + 1] - p.t0);
    p.kh = khead(a, p.h);
    return p;
}

// K rows 16aa + lr, columns 32kk + 8lg .. +7 of an item (rows past n load
// row n - 1 and are zeroed when used).
__device__ __forceinline__ void prep_load(const ChunkArgs &a, const PrepItem &p, int lr, int lg, uint4 (&kr)[4][4]) {
#pragma unroll
    for (int aa = 0; aa < 4; ++aa) {
        const int row = min(16 * aa + lr, p.n - 1);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const long long off = (static_cast<long long>(p.t0 + row) * a.Hk + p.kh) * kD + 32 * kk + 8 * lg;
            kr[aa][kk] = *reinterpret_cast<const uint4 *>(a.k + off);
        }
    }
}

// Each wave walks items wave, wave + waves, ...; the next item's K rows are
// loaded (into the same registers, which K K^T has finished with) while the
// current one's T is solved and written.  With the grid a multiple of 8,
// workgroups are numbered XCD by XCD (workgroup b runs on XCD b % 8), so
// the v-heads of a chunk, whose beta and gate reads share 128-byte lines
// (one line per token), are served by one L2 (per 4 x 4096-token call the
// prep read 101 MB for its 71 MB of K, beta and gate with the heads of a
// chunk spread over all eight).
__global__ __launch_bounds__(kPrepThreads) void gdn_chunk_prep_kernel(ChunkArgs a, int items) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int grid = static_cast<int>(gridDim.x), b = static_cast<int>(blockIdx.x);
    const int wg = grid % 8 == 0 ? (b % 8) * (grid / 8) + b / 8 : b;
    const int stride = grid * kPrepWaves;
    int item = wg * kPrepWaves + wave;
    if (item >= items) return;  // whole wave
    float *Al = reinterpret_cast<float *>(lds + wave * PW_BYTES);
    float *nk = Al + kC * AP;
    float *gv = nk + kC;
    float *bv = gv + kC;
    const bool l2 = (a.flags & OURO_GDN_L2NORM_QK) != 0;

    PrepItem cur = prep_item(a, item);
    uint4 kr[4][4];
    prep_load(a, cur, lr, lg, kr);
    for (;;) {
    const int next = item + stride;
    const int cg = cur.cg, h = cur.h, t0 = cur.t0, n = cur.n;
    unsigned char *rec = a.ws + (static_cast<size_t>(cg) * a.Hv + h) * kRec;
#pragma unroll
    for (int aa = 0; aa < 4; ++aa) {
        const int row = 16 * aa + lr;
        if (row >= n) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) kr[aa][kk] = make_uint4(0, 0, 0, 0);
        }
        float sk = sumsq32(kr[aa]);
        sk += __shfl_xor(sk, 16, 64);
        sk += __shfl_xor(sk, 32, 64);
        if (lg == 0) nk[row] = row < n ? (l2 ? 1.0f / (sqrtf(sk) + a.eps) : 1.0f) : 0.f;
    }
    {  // inclusive scan of the log-decays, one token per lane
        float g = lane < n ? a.gate[static_cast<long long>(t0 + lane) * a.Hv + h] : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(g, off, 64);
            if (lane >= off) g += o;
        }
        gv[lane] = g;
        bv[lane] = lane < n ? a.beta[static_cast<long long>(t0 + lane) * a.Hv + h] : 0.f;
    }
    __builtin_amdgcn_wave_barrier();
    {  // per-row beta, g, nk, row = lane (zero past n: nk = beta = 0; g stays at g_{n-1})
        float *rv = reinterpret_cast<float *>(rec + REC_V);
        rv[R_BETA + lane] = bv[lane];
        rv[R_G + lane] = gv[lane];
        rv[R_NK + lane] = nk[lane];
    }

    // A[r][c] = beta_r exp(g_r - g_c) nk_r nk_c (K K^T)[r][c], c < r, stored
    // transposed (Al[c][r]); tiles on and below the diagonal only (the solve
    // never reads r <= c).
#pragma unroll
    for (int aa = 0; aa < 4; ++aa) {
        const f32x4 b4 = ld4(bv + 16 * aa + 4 * lg);
        const f32x4 g4r = ld4(gv + 16 * aa + 4 * lg);
        const f32x4 k4 = ld4(nk + 16 * aa + 4 * lg);
#pragma unroll
        for (int bb = 0; bb <= aa; ++bb) {
            f32x4 g4 = {0, 0, 0, 0};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                g4 = mfma(__builtin_bit_cast(bf16x8, kr[aa][kk]), __builtin_bit_cast(bf16x8, kr[bb][kk]), g4);
            const int c = 16 * bb + lr;
            const float gc = gv[c], kc = nk[c];
            f32x4 av;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 16 * aa + 4 * lg + e;
                av[e] = (c < r) ? b4[e] * __expf(g4r[e] - gc) * k4[e] * kc * g4[e] : 0.f;
            }
            *reinterpret_cast<f32x4 *>(Al + c * AP + 16 * aa + 4 * lg) = av;
        }
    }
    __builtin_amdgcn_wave_barrier();
    // K is consumed: the next item's rows load during the solve
    PrepItem nxt{};
    if (next < items) {
        nxt = prep_item(a, next);
        prep_load(a, nxt, lr, lg, kr);
    }

    // T = (I + A)^-1 in 16 x 16 blocks.  A sits transposed in the blocks on
    // and above the diagonal of Al (block (j, i) holds A_ij^T, i >= j); T
    // goes row-major: each diagonal block over A_ii, T_ij (i > j) into the
    // free blocks below the diagonal.
    {  // T_ii = (I + A_ii)^-1: lane (i = lg, c = lr) solves column c by
       // substitution (once t_j is final, t_s -= A_ii[s][j] t_j for s > j)
        float t[16];
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) t[s2] = (s2 == lr) ? 1.f : 0.f;
        const float *Ad = Al + 16 * lg * AP + 16 * lg;  // Ad[j * AP + s] = A[16i + s][16i + j]
#pragma unroll
        for (int j = 0; j < 15; ++j) {
            const float tj = t[j];
#pragma unroll
            for (int s4 = (j + 1) & ~3; s4 < 16; s4 += 4) {
                const f32x4 a4 = ld4(Ad + j * AP + s4);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (s4 + e > j) t[s4 + e] -= a4[e] * tj;
            }
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) Al[(16 * lg + s2) * AP + 16 * lg + lr] = t[s2];
        __builtin_amdgcn_wave_barrier();
    }
    // T_ij = -T_ii (sum over k = j .. i-1 of A_ik T_kj) on fp32 MFMA, level
    // by level (i - j = 1, 2, 3; the blocks of a level are independent, so
    // their products interleave and a level ends with one barrier).  The sum
    // Y in D layout (lane l, register e: row 4 (l / 16) + e, column l % 16)
    // is the B operand of the second product as it stands, with the k index
    // of step e taken as 4 (l / 16) + e.
    auto offdiag_y = [&](int i, int j) {
        f32x4 y = {0.f, 0.f, 0.f, 0.f};
        for (int k = j; k < i; ++k)
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int kk = 16 * k + 4 * s4 + lg;  // A[16i + lr][kk] T[kk][16j + lr]
                y = __builtin_amdgcn_mfma_f32_16x16x4f32(Al[kk * AP + 16 * i + lr], Al[kk * AP + 16 * j + lr], y, 0, 0,
                                                         0);
            }
        return y;
    };
    auto offdiag_x = [&](int i, const f32x4 &y) {  // T_ii Y
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            x = __builtin_amdgcn_mfma_f32_16x16x4f32(Al[(16 * i + lr) * AP + 16 * i + 4 * lg + e], y[e], x, 0, 0, 0);
        return x;
    };
    auto put = [&](int i, int j, const f32x4 &x) {
#pragma unroll
        for (int e = 0; e < 4; ++e) Al[(16 * i + 4 * lg + e) * AP + 16 * j + lr] = -x[e];
    };
    {
        const f32x4 y10 = offdiag_y(1, 0), y21 = offdiag_y(2, 1), y32 = offdiag_y(3, 2);
        const f32x4 x10 = offdiag_x(1, y10), x21 = offdiag_x(2, y21), x32 = offdiag_x(3, y32);
        put(1, 0, x10);
        put(2, 1, x21);
        put(3, 2, x32);
        __builtin_amdgcn_wave_barrier();
    }
    {
        const f32x4 y20 = offdiag_y(2, 0), y31 = offdiag_y(3, 1);
        const f32x4 x20 = offdiag_x(2, y20), x31 = offdiag_x(3, y31);
        put(2, 0, x20);
        put(3, 1, x31);
        __builtin_amdgcn_wave_barrier();
    }
    put(3, 0, offdiag_x(3, offdiag_y(3, 0)));
    __builtin_amdgcn_wave_barrier();

    // T operands, split hi/lo: lane (lr, lg) of block (i, j) holds
    // T[16i + lr][16j + 4lg .. +3]
    {
        uint4 *rt = reinterpret_cast<uint4 *>(rec + REC_T);
        const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int aa = 2; aa < 4; ++aa) {  // dense slots (2,0), (3,0)
            const float *row = Al + (16 * aa + lr) * AP + 4 * lg;
            bf16x8 th, tl;
            split8(ld4(row), ld4(row + 16), th, tl);
            rt[(2 * (aa - 2)) * 64 + lane] = __builtin_bit_cast(uint4, th);
            rt[(2 * (aa - 2) + 1) * 64 + lane] = __builtin_bit_cast(uint4, tl);
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {  // dense blocks (1,0), (3,2)
            const float *row = Al + (16 * (2 * k + 1) + lr) * AP + 32 * k + 4 * lg;
            bf16x8 th, tl;
            split8(ld4(row), z4, th, tl);
            const uint4 h = __builtin_bit_cast(uint4, th), l = __builtin_bit_cast(uint4, tl);
            rt[RU_HALF + 64 * k + lane] = make_uint4(h.x, h.y, l.x, l.y);
        }
        if (4 * lg <= lr) {  // the diagonal blocks' non-zero lanes
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float *row = Al + (16 * i + lr) * AP + 16 * i + 4 * lg;
                bf16x8 th, tl;
                split8(ld4(row), z4, th, tl);
                const uint4 h = __builtin_bit_cast(uint4, th), l = __builtin_bit_cast(uint4, tl);
                rt[diag_unit(i, lr, lg)] = make_uint4(h.x, h.y, l.x, l.y);
            }
        }
    }
    if (next >= items) break;
    item = next;
    cur = nxt;
    __builtin_amdgcn_wave_barrier();
    }
}

// ---------------------------------------------------------------------------
// Scan: one 512-thread workgroup per (sequence, v-head, 64 state columns).
// Chain wave w (0..3) owns state columns jb + 16w .. +15, all 128 rows, in
// registers and runs the recurrence for them: K S0 and (beside it, on the
// same B operands) Q S0, R, U = T R, and S = b_C S0 + K^T U~, every
// contraction an MFMA whose operands are its own accumulators or chunk rows
// in LDS; after the state update it stages the next chunk's K and K^T,
// whose loads it issued at the start of the chunk.  Output wave 4 + w
// finishes O of the same chunk for the same stripe: in the first half it
// forms its share of the Pt operands from the K and Q rows in LDS; in the
// second half it takes so (Q S0) and U from chain wave w (through LDS),
// adds Pt U, stores O and stages the next chunk's Q, V, vectors and T
// operands (loads also issued at the start of the chunk).  Staging K and
// K^T on the chain waves, whose second half is the shorter one, took a
// 4 x 4096-token call from 0.299 to 0.291 ms; Q as well was slower
// (0.350 ms).  O is formed transposed (O^T = S0^T Q^T + U^T Pt^T,
// the same operands with A and B swapped), so a lane holds four adjacent
// columns of a row and stores them as one 16-byte write.
// ---------------------------------------------------------------------------

// Loads of the next chunk.  The chain waves stage K and K^T (their second
// half is short), the output waves Q, V, the vectors and the T operands.
// Thread to (0..255 within its role), item it (0, 1): id = to + 256 it
// covers K rows 2p, 2p+1 (p = id % 32) and bf16 columns 8c .. 8c+7
// (c = id / 32); V item i is row id / 8, columns 8 (id % 8) .. of the
// workgroup's 64.
struct NextRegs {
    uint4 q[4], t[3], v[2];
    float vec[8];  // threads 0..63: row's beta, g, nk; g_{n-1}, g_16floor(r/16), g_16, g_32, g_48
};
struct NextK {
    uint4 k[2][2];
};

// base + a 32-bit byte offset (lets the loads use a uniform base address)
template <typename T>
__device__ __forceinline__ const T &at(const void *base, unsigned byte_off) {
    return *reinterpret_cast<const T *>(static_cast<const char *>(base) + byte_off);
}

// Rows at or past n load row n - 1 (always valid, n >= 1) and are zeroed
// when staged into LDS, so the loads carry no branches and nothing waits
// for them before the stage.
__device__ __forceinline__ uint4 zero_if(bool z, uint4 v) {
    return z ? make_uint4(0, 0, 0, 0) : v;
}

__device__ __forceinline__ void load_next(const ChunkArgs &a, NextRegs &r, int to, int t0, int n, int kh, int h,
                                          int jb, const unsigned char *rec) {
    // uniform chunk bases, 32-bit lane offsets
    const uint16_t *qb = a.q + (static_cast<long long>(t0) * a.Hk + kh) * kD;
    const uint16_t *vb = a.v + (static_cast<long long>(t0) * a.Hv + h) * kD + jb;
    const unsigned ks = static_cast<unsigned>(a.Hk) * kD, vs = static_cast<unsigned>(a.Hv) * kD;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int id = to + 256 * it;
        const unsigned vrow = static_cast<unsigned>(min(id >> 3, n - 1));
        r.v[it] = at<uint4>(vb, 2u * (vrow * vs + 8u * (id & 7)));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = to + 256 * i;
        const unsigned row = static_cast<unsigned>(min(idx >> 4, n - 1));
        r.q[i] = at<uint4>(qb, 2u * (row * ks + 8u * (idx & 15)));
    }
    {
        const float *rv = reinterpret_cast<const float *>(rec + REC_V);
        const int row = to & 63;
        r.vec[0] = rv[R_BETA + row];
        r.vec[1] = rv[R_G + row];
        r.vec[2] = rv[R_NK + row];
        r.vec[3] = rv[R_G + n - 1];
        r.vec[4] = rv[R_G + (row & ~15)];
#pragma unroll
        for (int bb = 1; bb < 4; ++bb) r.vec[4 + bb] = rv[R_G + 16 * bb];
    }
    const uint4 *rt = reinterpret_cast<const uint4 *>(rec + REC_T);
    r.t[0] = rt[to];
    r.t[1] = rt[to + 256];
    r.t[2] = rt[min(to + 512, kRecUnits - 1)];  // threads 0..31
}

// The next chunk's K rows (chain waves).
__device__ __forceinline__ void load_next_k(const ChunkArgs &a, NextK &r, int to, int t0, int n, int kh) {
    const uint16_t *kb = a.k + (static_cast<long long>(t0) * a.Hk + kh) * kD;
    const unsigned ks = static_cast<unsigned>(a.Hk) * kD;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int id = to + 256 * it;
        const int p = id & 31, c = id >> 5;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const unsigned row = static_cast<unsigned>(min(2 * p + w, n - 1));
            r.k[it][w] = at<uint4>(kb, 2u * (row * ks + 8u * c));
        }
    }
}

// Stage the next chunk's K and K^T (into buffer buf); nothing reads K in
// a chunk's second half, and K^T buffer buf is the one the current chunk
// does not use.
__device__ __forceinline__ void store_next_k(const NextK &r, unsigned char *lds, int buf, int to, int n) {
    uint16_t *K = reinterpret_cast<uint16_t *>(lds + S_K);
    uint32_t *KT = reinterpret_cast<uint32_t *>(lds + S_KT + buf * kD * KTP * 2);
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int id = to + 256 * it;
        const int p = id & 31, c = id >> 5;
        const uint4 k0 = zero_if(2 * p >= n, r.k[it][0]), k1 = zero_if(2 * p + 1 >= n, r.k[it][1]);
        st_op(K + (2 * p) * KP, c, k0);
        st_op(K + (2 * p + 1) * KP, c, k1);
        // K^T[8c + e][2p .. 2p+1]: one 32-bit store per column e
        const uint32_t x0[4] = {k0.x, k0.y, k0.z, k0.w};
        const uint32_t x1[4] = {k1.x, k1.y, k1.z, k1.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            KT[((8 * c + 2 * e) * KTP + 2 * p) >> 1] = (x0[e] & 0xffffu) | (x1[e] << 16);
            KT[((8 * c + 2 * e + 1) * KTP + 2 * p) >> 1] = (x0[e] >> 16) | (x1[e] & 0xffff0000u);
        }
    }
}

// Stage the next chunk's Q, V, vectors and T operands (output waves).
__device__ __forceinline__ void store_next(const NextRegs &r, unsigned char *lds, int to, int n) {
    uint16_t *Q = reinterpret_cast<uint16_t *>(lds + S_Q);
    uint16_t *V = reinterpret_cast<uint16_t *>(lds + S_V);
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int id = to + 256 * it;
        *reinterpret_cast<uint4 *>(V + (id >> 3) * VP + 8 * (id & 7)) = zero_if((id >> 3) >= n, r.v[it]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = to + 256 * i;
        st_op(Q + (idx >> 4) * KP, idx & 15, zero_if((idx >> 4) >= n, r.q[i]));
    }
    {  // the coefficients of row to % 64, split over the four waves (wave-uniform branches)
        float *cv = reinterpret_cast<float *>(lds + S_VEC);
        const int row = to & 63, part = to >> 6;
        const float b = r.vec[0], g = r.vec[1], kn = r.vec[2];
        if (part == 0) {
            const float eg = __expf(g);
            cv[V_BETA + row] = b;
            cv[V_RK + row] = b * eg * kn;
            cv[V_EG + row] = eg;
            cv[V_G + row] = g;
        } else if (part == 1) {
            cv[V_W + row] = kn * __expf(r.vec[3] - g);
            cv[V_NK + row] = kn;
        } else if (part == 2) {
            // Pt's decay e^(g_r - g_s) as e^(g_r - g_16b) e^(g_16b - g_s) off the
            // diagonal tiles (both factors <= 1)
            cv[V_RHO + row] = __expf(g - r.vec[4]);
            cv[V_CB + row] = row < 16 ? __expf(r.vec[5] - g) * kn : 0.f;
        } else {
#pragma unroll
            for (int bb = 2; bb < 4; ++bb)
                cv[V_CB + 64 * (bb - 1) + row] = row < 16 * bb ? __expf(r.vec[4 + bb] - g) * kn : 0.f;
        }
    }
    // T operands [slot][hi, lo][lane] x 16 B; the positions that are always
    // zero were cleared by zero_t and are not written here
    uint4 *T = reinterpret_cast<uint4 *>(lds + S_T);
    uint2 *T2 = reinterpret_cast<uint2 *>(lds + S_T);  // the same in 8-byte halves
    // units 0..255: dense slots 2, 3
    T[(2 * (2 + (to >> 7)) + ((to >> 6) & 1)) * 64 + (to & 63)] = r.t[0];
    // one unit (hi.xy, lo.xy) into half hf of lane ln of slot ts
    const auto put_half = [&](const uint4 &v, int ts, int hf, int ln) {
        T2[((2 * ts) * 64 + ln) * 2 + hf] = make_uint2(v.x, v.y);
        T2[((2 * ts + 1) * 64 + ln) * 2 + hf] = make_uint2(v.z, v.w);
    };
    // the unit of diagonal-block index d (0 .. 159): block d / 40, lane in g-major order
    const auto put_diag = [&](const uint4 &v, int d) {
        const int i = d / 40, x = d % 40;
        const int g = x < 16 ? 0 : x < 28 ? 1 : x < 36 ? 2 : 3;
        put_half(v, diag_tslot(i), i & 1, x - 2 * g * (7 - g) + 16 * g);
    };
    if (to < 128) {  // units 256..383: blocks (1,0), (3,2), first half of slots 1, 5
        put_half(r.t[1], to < 64 ? 1 : 5, 0, to & 63);
    } else {         // units 384..511
        put_diag(r.t[1], to - 128);
    }
    if (to < 32) put_diag(r.t[2], to + 128);  // units 512..543
}

// The T operand positions no record unit covers, cleared once before the
// first chunk is staged (store_next never writes them): the second halves
// of slots 0 and 4 (blocks above the diagonal) and, in each diagonal
// block, the lanes r + 16 g with 4 g > r.
__device__ __forceinline__ void zero_t(unsigned char *lds, int to) {
    uint2 *T2 = reinterpret_cast<uint2 *>(lds + S_T);
    const int i = to >> 6, ln = to & 63, r = ln & 15, g = ln >> 4;
    const uint2 z = make_uint2(0u, 0u);
    if (4 * g > r) {
        const int ts = diag_tslot(i), hf = i & 1;
        T2[((2 * ts) * 64 + ln) * 2 + hf] = z;
        T2[((2 * ts + 1) * 64 + ln) * 2 + hf] = z;
    }
    if (i < 2) {
        const int ts = i == 0 ? 0 : 4;
        T2[((2 * ts) * 64 + ln) * 2 + 1] = z;
        T2[((2 * ts + 1) * 64 + ln) * 2 + 1] = z;
    }
}

// Pt slot (r-tile bb, s-slab q) of the chunk in LDS: the P^T tiles
// (s-tile aa = 2q, 2q + 1) = K Q^T scaled by e^(g_r - g_s) nk_s for s <= r
// (nq_r is applied to the output rows), as hi/lo A operands of Pt U (lane
// r + 16 g: row 16 bb + r).
__device__ __forceinline__ void pt_slot(unsigned char *lds, int bb, int q, int lane, int lr, int lg) {
    const uint16_t *K = reinterpret_cast<const uint16_t *>(lds + S_K);
    const uint16_t *Q = reinterpret_cast<const uint16_t *>(lds + S_Q);
    const float *cv = reinterpret_cast<const float *>(lds + S_VEC);
    const int r = 16 * bb + lr;
    const float rr = cv[V_RHO + r], gr = cv[V_G + r];
    f32x4 ps[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int aa = 2 * q + t;
        ps[t] = f32x4{0, 0, 0, 0};
        if (aa > bb) continue;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            ps[t] = mfma(ld_op(K + (16 * aa + lr) * KP, 32 * kk, lg), ld_op(Q + r * KP, 32 * kk, lg), ps[t]);
        if (aa < bb) {  // s < 16 bb <= r: e^(g_r - g_16b) * e^(g_16b - g_s) nk_s
            const f32x4 c4 = ld4(cv + V_CB + 64 * (bb - 1) + 16 * aa + 4 * lg);
#pragma unroll
            for (int e = 0; e < 4; ++e) ps[t][e] *= rr * c4[e];
        } else {  // diagonal tile: s <= r only
            const f32x4 gs = ld4(cv + V_G + 16 * aa + 4 * lg), kn = ld4(cv + V_NK + 16 * aa + 4 * lg);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int sr = 16 * aa + 4 * lg + e;
                const float ev = __expf(sr <= r ? gr - gs[e] : 0.f);
                ps[t][e] = sr <= r ? ev * kn[e] * ps[t][e] : 0.f;
            }
        }
    }
    bf16x8 ph, pl;
    split8(ps[0], ps[1], ph, pl);
    uint4 *P = reinterpret_cast<uint4 *>(lds + S_P);
    P[(2 * pslot(bb, q)) * 64 + lane] = __builtin_bit_cast(uint4, ph);
    P[(2 * pslot(bb, q) + 1) * 64 + lane] = __builtin_bit_cast(uint4, pl);
}

__global__ __launch_bounds__(kScanThreads) void gdn_chunk_scan_kernel(ChunkArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const bool chain = wave < 4;                      // wave-uniform role
    const int tr = tid & 255;                         // thread index within the role
    // Workgroups that read the same K, Q rows (the column halves of the
    // v-heads of one k-head: G = 2 Hv / Hk of them) form a group, and a
    // group is placed on one XCD (workgroup i runs on XCD i % 8) so that
    // they share its L2.
    const int G = 2 * (a.Hv / a.Hk);
    const int groups = a.nseq * a.Hk;
    int grp, mem;
    if (groups % 8 == 0) {
        const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
        grp = (slot / G) * 8 + xcd;
        mem = slot % G;
    } else {
        grp = blockIdx.x / G;
        mem = blockIdx.x % G;
    }
    const int seq = grp / a.Hk, kh = grp % a.Hk;
    const int h = vhead(a, kh, mem >> 1);
    const int jb = (mem & 1) * kDVB;    // first state column of the workgroup
    const int jw = jb + 16 * (wave & 3);  // first state column of this stripe
    const int t_begin = a.cu[seq], t_end = a.cu[seq + 1];
    if (t_end <= t_begin) return;  // empty sequence: state unchanged (uniform per block)
    const int nchunks = (t_end - t_begin + kC - 1) / kC;
    auto record = [&](int c) { return a.ws + (static_cast<size_t>(a.coff[seq] + c) * a.Hv + h) * kRec; };
    uint4 *X = reinterpret_cast<uint4 *>(lds + S_X + (wave & 3) * X_WAVE);  // [slot][lane]: O^T 0..3, U 4..7
    const uint16_t *K = reinterpret_cast<const uint16_t *>(lds + S_K);
    const uint16_t *Q = reinterpret_cast<const uint16_t *>(lds + S_Q);
    const float *cv = reinterpret_cast<const float *>(lds + S_VEC);

    // Both roles run the same barriers: two per chunk.
    if (chain) {
        // state tile t holds S[16t + 4g + e][jw + r]
        float *S = a.state + (static_cast<long long>(seq) * a.Hv + h) * kD * kD + static_cast<long long>(jw + lr) * kD;
        f32x4 st[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) st[t] = ld4(S + 16 * t + 4 * lg);
        bf16x8 sh[4], sl[4];  // S0 of the chunk as hi/lo B operands, slab q = tiles 2q, 2q+1
#pragma unroll
        for (int q = 0; q < 4; ++q) split8(st[2 * q], st[2 * q + 1], sh[q], sl[q]);
        const uint16_t *Vl = reinterpret_cast<const uint16_t *>(lds + S_V) + 16 * (wave & 3) + lr;
        const uint4 *Tl = reinterpret_cast<const uint4 *>(lds + S_T);  // [slot][lane]
        NextK nk;
        {
            const int n0 = min(kC, t_end - t_begin);
            load_next_k(a, nk, tr, t_begin, n0, kh);
            store_next_k(nk, lds, 0, tr, n0);
        }

        for (int c = 0; c < nchunks; ++c) {
            const int n = min(kC, t_end - t_begin - c * kC);
            const bool more = c + 1 < nchunks;
            const int n1 = more ? min(kC, t_end - t_begin - (c + 1) * kC) : 0;
            __syncthreads();  // chunk c staged (K, Q, V, vectors, T); X is free
            if (more) load_next_k(a, nk, tr, t_begin + (c + 1) * kC, n1, kh);

            // ---- first half: KS and (Q S0)^T, R, U -> X, U~ -----------------
            const float bC = __expf(cv[V_G + n - 1]);
            f32x4 ks[4], rr[4], ot[4];
#pragma unroll
            for (int aa = 0; aa < 4; ++aa) ks[aa] = ot[aa] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                bf16x8 ka[4];
#pragma unroll
                for (int aa = 0; aa < 4; ++aa) ka[aa] = ld_op(K + (16 * aa + lr) * KP, 32 * q, lg);
#pragma unroll
                for (int aa = 0; aa < 4; ++aa) ks[aa] = mfma(ka[aa], sh[q], ks[aa]);
#pragma unroll
                for (int aa = 0; aa < 4; ++aa) ks[aa] = mfma(ka[aa], sl[q], ks[aa]);
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) ka[bb] = ld_op(Q + (16 * bb + lr) * KP, 32 * q, lg);
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) ot[bb] = mfma(sh[q], ka[bb], ot[bb]);
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) ot[bb] = mfma(sl[q], ka[bb], ot[bb]);
            }
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {  // ot[bb][e] = (Q S0)[16 bb + r][jw + 4 g + e], scaled by e^g of row 16 bb + r
                const float eg = cv[V_EG + 16 * bb + lr];
#pragma unroll
                for (int e = 0; e < 4; ++e) ot[bb][e] *= eg;
                X[bb * 64 + lane] = __builtin_bit_cast(uint4, ot[bb]);
            }
#pragma unroll
            for (int aa = 0; aa < 4; ++aa) {
                const f32x4 b4 = ld4(cv + V_BETA + 16 * aa + 4 * lg);
                const f32x4 r4 = ld4(cv + V_RK + 16 * aa + 4 * lg);
#pragma unroll
                for (int e = 0; e < 4; ++e)  // V rows past n are zero in LDS
                    rr[aa][e] = b4[e] * bf(Vl[(16 * aa + 4 * lg + e) * VP]) - r4[e] * ks[aa][e];
            }
            bf16x8 rh[2], rl[2];
            split8(rr[0], rr[1], rh[0], rl[0]);
            split8(rr[2], rr[3], rh[1], rl[1]);
            f32x4 u[4];
#pragma unroll
            for (int aa = 0; aa < 4; ++aa) u[aa] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 2; ++q) {  // T is lower triangular: s-tile aa needs slabs q <= aa / 2
#pragma unroll
                for (int aa = 2 * q; aa < 4; ++aa)
                    u[aa] = mfma(__builtin_bit_cast(bf16x8, Tl[(2 * tslot(aa, q)) * 64 + lane]), rh[q], u[aa]);
#pragma unroll
                for (int aa = 2 * q; aa < 4; ++aa)
                    u[aa] = mfma(__builtin_bit_cast(bf16x8, Tl[(2 * tslot(aa, q)) * 64 + lane]), rl[q], u[aa]);
#pragma unroll
                for (int aa = 2 * q; aa < 4; ++aa)
                    u[aa] = mfma(__builtin_bit_cast(bf16x8, Tl[(2 * tslot(aa, q) + 1) * 64 + lane]), rh[q], u[aa]);
            }
            bf16x8 wh[2], wl[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                bf16x8 uh, ul;
                split8(u[2 * q], u[2 * q + 1], uh, ul);
                X[256 + (2 * q) * 64 + lane] = __builtin_bit_cast(uint4, uh);
                X[256 + (2 * q + 1) * 64 + lane] = __builtin_bit_cast(uint4, ul);
                f32x4 w0 = u[2 * q], w1 = u[2 * q + 1];
                const f32x4 c0 = ld4(cv + V_W + 32 * q + 4 * lg), c1 = ld4(cv + V_W + 32 * q + 16 + 4 * lg);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w0[e] *= c0[e];
                    w1[e] *= c1[e];
                }
                split8(w0, w1, wh[q], wl[q]);
            }
            {  // nq of row 16 wave + r: l2_norm and the 1/sqrt(d) scale (qwen35.rs:73-79, 1103-1107),
               // from the row's Q operands read once more (after the chain's products, where the
               // chain waits for the output waves anyway)
                const bool l2 = (a.flags & OURO_GDN_L2NORM_QK) != 0;
                const float qscale = (a.flags & OURO_GDN_SCALE_Q) ? 1.0f / sqrtf(static_cast<float>(kD)) : 1.0f;
                float sq = 0.f;
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const uint4 w = __builtin_bit_cast(uint4, ld_op(Q + (16 * wave + lr) * KP, 32 * kk, lg));
                    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x0 = __uint_as_float(ws[e] << 16), x1 = __uint_as_float(ws[e] & 0xffff0000u);
                        sq += x0 * x0 + x1 * x1;
                    }
                }
                sq += __shfl_xor(sq, 16, 64);
                sq += __shfl_xor(sq, 32, 64);
                const int row = 16 * wave + lr;
                if (lg == 0)
                    reinterpret_cast<float *>(lds + S_NQ)[row] =
                        row < n ? (l2 ? 1.0f / (sqrtf(sq) + a.eps) : 1.0f) * qscale : 0.f;
            }

            __syncthreads();  // X holds (Q S0)^T and U of chunk c; K, Q, V, T may be refilled

            // ---- second half: S = b_C S0 + K^T U~ ----------------------------
            const uint16_t *KT = reinterpret_cast<const uint16_t *>(lds + S_KT + (c & 1) * kD * KTP * 2);
#pragma unroll
            for (int t = 0; t < 8; ++t) st[t] = st[t] * bC;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                bf16x8 kt[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) kt[t] = ld_perm(KT + (16 * t + lr) * KTP, 32 * q, lg);
#pragma unroll
                for (int t = 0; t < 8; ++t) st[t] = mfma(kt[t], wh[q], st[t]);
#pragma unroll
                for (int t = 0; t < 8; ++t) st[t] = mfma(kt[t], wl[q], st[t]);
            }
            if (more) {
                store_next_k(nk, lds, (c + 1) & 1, tr, n1);
#pragma unroll
                for (int q = 0; q < 4; ++q) split8(st[2 * q], st[2 * q + 1], sh[q], sl[q]);
            }
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) *reinterpret_cast<f32x4 *>(S + 16 * t + 4 * lg) = st[t];
    } else {
        const int ow = wave - 4;
        NextRegs nx;
        {
            const int n0 = min(kC, t_end - t_begin);
            load_next(a, nx, tr, t_begin, n0, kh, h, jb, record(0));
            zero_t(lds, tr);
            store_next(nx, lds, tr, n0);
        }
        float *ob = a.out + static_cast<long long>(h) * kD + jw + 4 * lg;
        const long long os = static_cast<long long>(a.Hv) * kD;

        for (int c = 0; c < nchunks; ++c) {
            const int t0 = t_begin + c * kC;
            const int n = min(kC, t_end - t0);
            const bool more = c + 1 < nchunks;
            const int n1 = more ? min(kC, t_end - t0 - kC) : 0;
            __syncthreads();  // chunk c staged

            // ---- first half: next loads, Pt -----------------------------------
            if (more) load_next(a, nx, tr, t0 + kC, n1, kh, h, jb, record(c + 1));
            // this wave's Pt slots (two off-diagonal tiles and a diagonal one,
            // or one of each; the diagonal tiles carry the exponentials):
            // (3,0), (0,0) | (2,0), (2,1) | (1,0) | (3,1)
            if (ow == 0) {
                pt_slot(lds, 3, 0, lane, lr, lg);
                pt_slot(lds, 0, 0, lane, lr, lg);
            }
            if (ow == 1) {
                pt_slot(lds, 2, 0, lane, lr, lg);
                pt_slot(lds, 2, 1, lane, lr, lg);
            }
            if (ow == 2) pt_slot(lds, 1, 0, lane, lr, lg);
            if (ow == 3) pt_slot(lds, 3, 1, lane, lr, lg);

            __syncthreads();  // X holds (Q S0)^T and U of chunk c; the Pt operands are complete

            // ---- second half: O^T = (so Q S0)^T + U^T Pt^T, store O, stage chunk c + 1
            {
                const uint4 *P = reinterpret_cast<const uint4 *>(lds + S_P);  // [slot][lane]
                f32x4 ot[4];
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) ot[bb] = __builtin_bit_cast(f32x4, X[bb * 64 + lane]);
                bf16x8 uh[2], ul[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    uh[q] = __builtin_bit_cast(bf16x8, X[256 + (2 * q) * 64 + lane]);
                    ul[q] = __builtin_bit_cast(bf16x8, X[256 + (2 * q + 1) * 64 + lane]);
                }
#pragma unroll
                for (int pass = 0; pass < 3; ++pass) {
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb) {
#pragma unroll
                        for (int q = 0; q <= bb / 2; ++q) {
                            const bf16x8 ph = __builtin_bit_cast(bf16x8, P[(2 * pslot(bb, q)) * 64 + lane]);
                            const bf16x8 pl = __builtin_bit_cast(bf16x8, P[(2 * pslot(bb, q) + 1) * 64 + lane]);
                            if (pass == 0) ot[bb] = mfma(uh[q], ph, ot[bb]);
                            if (pass == 1) ot[bb] = mfma(ul[q], ph, ot[bb]);
                            if (pass == 2) ot[bb] = mfma(uh[q], pl, ot[bb]);
                        }
                    }
                }
                // ot[bb][e] = O[16 bb + r][jw + 4 g + e] / nq_r
                float *obc = ob + static_cast<long long>(t0) * os;
                const float *nqs = reinterpret_cast<const float *>(lds + S_NQ);
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) {
                    const int row = 16 * bb + lr;
                    const float nq = nqs[row];
#pragma unroll
                    for (int e = 0; e < 4; ++e) ot[bb][e] *= nq;
                    if (row < n) *reinterpret_cast<f32x4 *>(obc + row * os) = ot[bb];
                }
            }
            if (more) store_next(nx, lds, tr, n1);
        }
    }
}

int set_lds(const void *kern, int bytes) {
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess)
        return fail(OURO_ERR_HIP, "gdn chunk prefill: %d B of LDS refused: %s", bytes, hipGetErrorString(e));
    return OURO_OK;
}

}  // namespace

size_t gdn_chunk_ws_bytes(size_t T, size_t N, size_t Hv) {
    const size_t ns = N < static_cast<size_t>(kMaxSeq) ? N : static_cast<size_t>(kMaxSeq);
    return (T / kC + ns + 1) * Hv * kRec;
}

int gdn_chunk_prefill(float *state, const void *q, const void *k, const void *v, const float *gate,
                      const float *beta, float *out, const int32_t *cu_host, size_t N, size_t T,
                      size_t Hk, size_t Hv, size_t d, size_t chunk, unsigned flags, float eps,
                      void *workspace, void *stream) {
    if (!state || !q || !k || !v || !gate || !beta || !out)
        return fail(OURO_ERR_INVALID_ARG, "gdn chunk prefill: NULL argument");
    if (d != static_cast<size_t>(kD)) return fail(OURO_ERR_SHAPE, "gdn chunk prefill: d = %zu, only 128", d);
    if (chunk != static_cast<size_t>(kC)) return fail(OURO_ERR_SHAPE, "gdn chunk prefill: chunk = %zu, only 64", chunk);
    if (!Hk || !Hv || Hv % Hk || Hv > 4096) return fail(OURO_ERR_SHAPE, "gdn chunk prefill: bad heads Hk=%zu Hv=%zu", Hk, Hv);
    if (flags & ~(OURO_GDN_L2NORM_QK | OURO_GDN_SCALE_Q | OURO_GDN_KHEAD_DIV))
        return fail(OURO_ERR_INVALID_ARG, "gdn chunk prefill: bad flags 0x%x", flags);
    if (T > 0x7fffffffULL / (Hv * kD)) return fail(OURO_ERR_SHAPE, "gdn chunk prefill: too many tokens");
    if (!N) return fail(OURO_ERR_SHAPE, "gdn chunk prefill: no sequences");
    const uintptr_t mis = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(state) |
                          reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(workspace);
    if (mis % 16) return fail(OURO_ERR_ALIGN, "gdn chunk prefill: q, k, v, state, out, workspace need 16-byte alignment");
    // Validate the offsets on the host before any launch.
    if (cu_host) {
        if (cu_host[0] != 0 || static_cast<size_t>(cu_host[N]) != T)
            return fail(OURO_ERR_SHAPE, "gdn chunk prefill: cu_seqlens must run 0..T");
        for (size_t i = 0; i < N; ++i)
            if (cu_host[i + 1] < cu_host[i]) return fail(OURO_ERR_SHAPE, "gdn chunk prefill: cu_seqlens decreasing");
    } else if (N != 1) {
        return fail(OURO_ERR_SHAPE, "gdn chunk prefill: cu_seqlens NULL needs N == 1");
    }
    unsigned char *ws = static_cast<unsigned char *>(workspace);
    if (!ws) {
        ws = static_cast<unsigned char *>(ouro::workspace(gdn_chunk_ws_bytes(T, N, Hv), stream));
        if (!ws) return OURO_ERR_HIP;
    }
    // LDS opt-in once per process (an idempotent call; threads that race
    // here both make it)
    static std::atomic<bool> attr_set{false};
    if (!attr_set.load(std::memory_order_acquire)) {
        int st = set_lds(reinterpret_cast<const void *>(gdn_chunk_scan_kernel), SCAN_LDS);
        if (!st) st = set_lds(reinterpret_cast<const void *>(gdn_chunk_prep_kernel), PREP_LDS);
        if (st) return st;
        attr_set.store(true, std::memory_order_release);
    }
    ChunkArgs a{};
    a.q = static_cast<const uint16_t *>(q);
    a.k = static_cast<const uint16_t *>(k);
    a.v = static_cast<const uint16_t *>(v);
    a.gate = gate;
    a.beta = beta;
    a.out = out;
    a.ws = ws;
    a.Hk = static_cast<int>(Hk);
    a.Hv = static_cast<int>(Hv);
    a.flags = flags;
    a.eps = eps;
    // Slices of up to kMaxSeq sequences; each slice reuses the workspace
    // after the previous slice's scan (stream order).
    for (size_t s0 = 0; s0 < N; s0 += kMaxSeq) {
        const size_t ns = N - s0 < static_cast<size_t>(kMaxSeq) ? N - s0 : kMaxSeq;
        a.nseq = static_cast<int>(ns);
        a.state = state + s0 * Hv * kD * kD;
        a.coff[0] = 0;
        for (size_t i = 0; i <= ns; ++i) {
            a.cu[i] = cu_host ? cu_host[s0 + i] : (i == 0 ? 0 : static_cast<int>(T));
            if (i) a.coff[i] = a.coff[i - 1] + (a.cu[i] - a.cu[i - 1] + kC - 1) / kC;
        }
        const int chunks = a.coff[ns];
        if (chunks == 0) continue;
        const int items = chunks * static_cast<int>(Hv);
        // resident workgroups only (two per CU by their LDS); each wave
        // walks items with a stride of the whole grid
        int wgs = std::min((items + kPrepWaves - 1) / kPrepWaves, kPrepGrid);
        if (wgs > 8) wgs -= wgs % 8;  // XCD-ordered numbering (waves stride over the rest)
        hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(static_cast<unsigned>(wgs)), dim3(kPrepThreads), PREP_LDS,
                           as_stream(stream), a, items);
        int st = check_launch("gdn_chunk_prep_kernel");
        if (st) return st;
        hipLaunchKernelGGL(gdn_chunk_scan_kernel, dim3(static_cast<unsigned>(ns * Hv * 2)), dim3(kScanThreads),
                           SCAN_LDS, as_stream(stream), a);
        st = check_launch("gdn_chunk_scan_kernel");
        if (st) return st;
    }
    return OURO_OK;
}

}  // namespace ouro

using namespace ouro;

extern "C" {

size_t ouro_gdn_chunk_workspace_bytes(size_t T, size_t N, size_t Hv, size_t d, size_t chunk) {
    if (d != static_cast<size_t>(kD) || chunk != static_cast<size_t>(kC)) return 0;
    return gdn_chunk_ws_bytes(T, N, Hv);
}

int ouro_gdn_chunk_prefill(float *state, const void *q, const void *k, const void *v, const float *gate,
                           const float *beta, float *out, const int32_t *cu_seqlens_host, size_t N,
                           size_t T, size_t Hk, size_t Hv, size_t d, size_t chunk, unsigned flags,
                           float eps, void *workspace, void *stream) {
    OURO_REQUIRE_INIT();
    return gdn_chunk_prefill(state, q, k, v, gate, beta, out, cu_seqlens_host, N, T, Hk, Hv, d, chunk,
                             flags, eps, workspace, stream);
}

}  // extern "C"
