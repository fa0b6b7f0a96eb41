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
// products carry ~16 mantissa bits.  T is solved in fp32 on the VALU.
//
// Two kernels.  gdn_chunk_prep_kernel runs every (chunk, v-head) in parallel
// and computes what does not depend on the state: row norms, g, A and T,
// written to a workspace record (T as hi/lo bf16 plus the vectors).
// gdn_chunk_scan_kernel then walks the chunks of a sequence in order: one
// 512-thread workgroup owns (sequence, v-head, 64 of the 128 state columns)
// -- output column j of the recurrence only touches state column j, so the
// two column halves of a head are independent chains -- and does only the
// state-dependent contractions, four barriers per chunk, with the next
// chunk's rows loaded into registers while the current one computes.
#include "common.hpp"

namespace ouro {
namespace {

constexpr int kD = 128;           // d_k = d_v (qwen35.rs:8)
constexpr int kC = 64;            // chunk length
constexpr int kDVB = 64;          // state columns per scan workgroup
constexpr int kScanThreads = 512; // 8 waves
constexpr int kPrepThreads = 256; // 4 waves
constexpr int kMaxSeq = 256;      // sequences per launch (offsets by value)

constexpr int KP = kD + 8;        // bf16 row pitch of K, Q, S^T (272 B)
constexpr int VP = kDVB + 8;      // bf16 row pitch of V (144 B)
constexpr int FP = kC + 8;        // pitch of 64x64 matrices: fp32 (288 B) or bf16 planes (144 B)
constexpr int HL = kC * FP;       // elements of one bf16 plane (hi or lo) of a 64x64 matrix
constexpr int MAT = kC * FP * 4;  // bytes of a 64x64 fp32 (= hi+lo bf16) slot

// Workspace record of one (chunk, v-head): T hi [64][64] bf16, T lo, then
// nk, nq, g [64] fp32 each, padded to a multiple of 256 B.
constexpr int REC_T = 2 * kC * kC * 2;
constexpr size_t kRec = 17408;
static_assert(REC_T + 3 * kC * 4 <= static_cast<int>(kRec), "record size");

// Scan kernel LDS byte offsets.
constexpr int OFF_K = 0;
constexpr int OFF_Q = OFF_K + kC * KP * 2;        // Q, then U~^T hi/lo
constexpr int OFF_V = OFF_Q + MAT;
constexpr int OFF_T = OFF_V + kC * VP * 2;        // T hi/lo
constexpr int OFF_R = OFF_T + MAT;                // R^T hi/lo
constexpr int OFF_P = OFF_R + MAT;                // Pt hi/lo
constexpr int OFF_SHI = OFF_P + MAT;              // S0 hi, [j][i]
constexpr int OFF_SLO = OFF_SHI + kDVB * KP * 2;  // S0 lo
constexpr int OFF_U = OFF_SLO + kDVB * KP * 2;    // U^T hi/lo
constexpr int OFF_VEC = OFF_U + MAT;              // nk, nq, g, beta
constexpr int SCAN_LDS = OFF_VEC + 4 * kC * 4;
static_assert(SCAN_LDS <= 160 * 1024, "LDS budget of a gfx950 workgroup");

// Prep kernel LDS byte offsets.
constexpr int PO_K = 0;
constexpr int PO_A = PO_K + kC * KP * 2;
constexpr int PO_T = PO_A + MAT;
constexpr int PO_RT = PO_T + MAT;                 // 3 x 16 x 17 fp32
constexpr int PO_VEC = PO_RT + 3 * 16 * 17 * 4;   // nk, nq, g, beta
constexpr int PREP_LDS = PO_VEC + 4 * kC * 4;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

__device__ __forceinline__ f32x4 mfma(const bf16x8 &a, const bf16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf(uint16_t u) { return bf16_bits_to_f32(u); }

// 8 bf16 from LDS (16-byte aligned) as an MFMA operand.
__device__ __forceinline__ bf16x8 ld_bf8(const uint16_t *p) {
    return *reinterpret_cast<const bf16x8 *>(p);
}

// x = hi + lo with hi = bf16(x), lo = bf16(x - hi): ~16 significant bits.
__device__ __forceinline__ void split(float x, uint16_t &hi, uint16_t &lo) {
    const __bf16 h = static_cast<__bf16>(x);
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, static_cast<__bf16>(x - static_cast<float>(h)));
}

__device__ __forceinline__ uint32_t pack2(uint16_t a, uint16_t b) {
    return a | (static_cast<uint32_t>(b) << 16);
}

// Store 4 consecutive values (along the contiguous axis) of a hi/lo matrix.
__device__ __forceinline__ void st_split4(uint16_t *hl, int off, const f32x4 &v) {
    uint16_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split(v[e], h[e], l[e]);
    *reinterpret_cast<uint2 *>(hl + off) = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
    *reinterpret_cast<uint2 *>(hl + HL + off) = make_uint2(pack2(l[0], l[1]), pack2(l[2], l[3]));
}

__device__ __forceinline__ int khead(const ChunkArgs &a, int h) {
    return (a.flags & OURO_GDN_KHEAD_DIV) ? h / (a.Hv / a.Hk) : h % a.Hk;
}

// Sum of squares of 32 bf16 (4 x 16 B) at p.
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

// ---------------------------------------------------------------------------
// Prep: one 256-thread workgroup per (chunk, v-head).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kPrepThreads) void gdn_chunk_prep_kernel(ChunkArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    uint16_t *Kl = reinterpret_cast<uint16_t *>(lds + PO_K);
    float *Al = reinterpret_cast<float *>(lds + PO_A);
    float *Tl = reinterpret_cast<float *>(lds + PO_T);
    float *Rt = reinterpret_cast<float *>(lds + PO_RT);
    float *nk = reinterpret_cast<float *>(lds + PO_VEC);
    float *nq = nk + kC;
    float *gv = nq + kC;
    float *bv = gv + kC;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int cg = blockIdx.x, h = blockIdx.y;
    int lo = 0, hi = a.nseq;  // sequence of chunk cg: largest s with coff[s] <= cg
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (a.coff[mid] <= cg) lo = mid; else hi = mid;
    }
    const int seq = lo;
    const int t0 = a.cu[seq] + (cg - a.coff[seq]) * kC;
    const int n = min(kC, a.cu[seq + 1] - t0);
    const int kh = khead(a, h);
    const bool l2 = (a.flags & OURO_GDN_L2NORM_QK) != 0;
    const float qscale = (a.flags & OURO_GDN_SCALE_Q) ? 1.0f / sqrtf(static_cast<float>(kD)) : 1.0f;

    // K rows to LDS (zero beyond n); row norms of K and Q, 4 lanes per row.
    for (int idx = tid; idx < kC * 16; idx += kPrepThreads) {
        const int r = idx >> 4, c16 = idx & 15;
        uint4 kv = make_uint4(0, 0, 0, 0);
        if (r < n) kv = *reinterpret_cast<const uint4 *>(a.k + (static_cast<long long>(t0 + r) * a.Hk + kh) * kD + 8 * c16);
        *reinterpret_cast<uint4 *>(Kl + r * KP + 8 * c16) = kv;
    }
    {
        const int r = tid >> 2, qq = tid & 3;
        uint4 w[4] = {};
        if (r < n) {
            const uint4 *qp = reinterpret_cast<const uint4 *>(a.q + (static_cast<long long>(t0 + r) * a.Hk + kh) * kD + 32 * qq);
#pragma unroll
            for (int c = 0; c < 4; ++c) w[c] = qp[c];
        }
        float ss = sumsq32(w);
        ss += __shfl_xor(ss, 1, 64);
        ss += __shfl_xor(ss, 2, 64);
        if (qq == 0) nq[r] = r < n ? (l2 ? 1.0f / (sqrtf(ss) + a.eps) : 1.0f) * qscale : 0.f;
    }
    if (wave == 0) {  // inclusive scan of the log-decays
        float g = lane < n ? a.gate[static_cast<long long>(t0 + lane) * a.Hv + h] : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(g, off, 64);
            if (lane >= off) g += o;
        }
        gv[lane] = g;
    }
    if (wave == 1) bv[lane] = lane < n ? a.beta[static_cast<long long>(t0 + lane) * a.Hv + h] : 0.f;
    __syncthreads();
    {
        const int r = tid >> 2, qq = tid & 3;
        uint4 w[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) w[c] = *reinterpret_cast<const uint4 *>(Kl + r * KP + 32 * qq + 8 * c);
        float ss = sumsq32(w);
        ss += __shfl_xor(ss, 1, 64);
        ss += __shfl_xor(ss, 2, 64);
        if (qq == 0) nk[r] = r < n ? (l2 ? 1.0f / (sqrtf(ss) + a.eps) : 1.0f) : 0.f;
    }
    __syncthreads();

    // A = strictly lower (beta_s exp(g_s - g_j) nk_s nk_j K K^T); 4 tiles per wave.
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int id = 4 * wave + u;
        const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
        f32x4 g4 = {0, 0, 0, 0};
        if (n0 <= m0) {  // tiles above the diagonal are zero (uniform per wave)
#pragma unroll
            for (int kk = 0; kk < kD / 32; ++kk) {
                const int kc = kk * 32 + 8 * lg;
                g4 = mfma(ld_bf8(Kl + (m0 + lr) * KP + kc), ld_bf8(Kl + (n0 + lr) * KP + kc), g4);
            }
        }
        const int c = n0 + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = m0 + 4 * lg + e;
            Al[r * FP + c] = (c < r) ? bv[r] * __expf(gv[r] - gv[c]) * nk[r] * nk[c] * g4[e] : 0.f;
        }
    }
    __syncthreads();

    // T = (I + A)^-1: 16x16 diagonal blocks by forward substitution, then
    // T_ij = -T_ii sum_{k=j..i-1} A_ik T_kj in order of i - j.
    if (wave == 0) {
        const int blk = lg, c = lr;
        float t[16];
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            float acc = (s == c) ? 1.f : 0.f;
            const float *arow = Al + (16 * blk + s) * FP + 16 * blk;
#pragma unroll
            for (int j = 0; j < s; ++j) acc -= arow[j] * t[j];
            t[s] = acc;
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) Tl[(16 * blk + s) * FP + 16 * blk + c] = t[s];
    } else {
        for (int e = tid - 64; e < kC * kC; e += kPrepThreads - 64) {
            const int r = e / kC, c = e % kC;
            if ((c >> 4) > (r >> 4)) Tl[r * FP + c] = 0.f;
        }
    }
    __syncthreads();
    for (int dd = 1; dd <= 3; ++dd) {
        const int nblk = 4 - dd;
        for (int e = tid; e < nblk * 256; e += kPrepThreads) {
            const int bi = e >> 8, ar = (e >> 4) & 15, bc = e & 15;
            const int i = dd + bi, j = bi;
            float acc = 0.f;
            for (int kb = j; kb < i; ++kb) {
                const float *arow = Al + (16 * i + ar) * FP + 16 * kb;
                const float *tcol = Tl + (16 * kb) * FP + 16 * j + bc;
#pragma unroll
                for (int m = 0; m < 16; ++m) acc += arow[m] * tcol[m * FP];
            }
            Rt[bi * 272 + ar * 17 + bc] = acc;
        }
        __syncthreads();
        for (int e = tid; e < nblk * 256; e += kPrepThreads) {
            const int bi = e >> 8, ar = (e >> 4) & 15, bc = e & 15;
            const int i = dd + bi, j = bi;
            const float *trow = Tl + (16 * i + ar) * FP + 16 * i;
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < 16; ++m) acc += trow[m] * Rt[bi * 272 + m * 17 + bc];
            Tl[(16 * i + ar) * FP + 16 * j + bc] = -acc;
        }
        __syncthreads();
    }

    // Record: T hi/lo row-major [64][64], then nk, nq, g.
    unsigned char *rec = a.ws + (static_cast<size_t>(cg) * a.Hv + h) * kRec;
    {
        const int r = tid >> 2, c0 = 16 * (tid & 3);
        uint32_t hw[8], lw[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint16_t h0, l0, h1, l1;
            split(Tl[r * FP + c0 + 2 * e], h0, l0);
            split(Tl[r * FP + c0 + 2 * e + 1], h1, l1);
            hw[e] = pack2(h0, h1);
            lw[e] = pack2(l0, l1);
        }
        uint4 *th = reinterpret_cast<uint4 *>(rec + (r * kC + c0) * 2);
        uint4 *tlo = reinterpret_cast<uint4 *>(rec + kC * kC * 2 + (r * kC + c0) * 2);
        th[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        th[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
        tlo[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        tlo[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
    }
    if (tid < 3 * kC) reinterpret_cast<float *>(rec + REC_T)[tid] = nk[tid];  // nk, nq, g are contiguous
}

// ---------------------------------------------------------------------------
// Scan: one 512-thread workgroup per (sequence, v-head, 64 state columns).
// ---------------------------------------------------------------------------

// The rows of one chunk, in registers between their load and their LDS store.
struct ChunkRegs {
    uint4 k[2], q[2], v, t[2];
    float vec;
};

__device__ __forceinline__ void load_chunk(const ChunkArgs &a, ChunkRegs &r, int tid, int t0, int n, int kh,
                                           int h, int jb, const unsigned char *rec) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int idx = tid + kScanThreads * p;
        const int row = idx >> 4, c16 = idx & 15;
        r.k[p] = r.q[p] = make_uint4(0, 0, 0, 0);
        if (row < n) {
            const long long off = (static_cast<long long>(t0 + row) * a.Hk + kh) * kD + 8 * c16;
            r.k[p] = *reinterpret_cast<const uint4 *>(a.k + off);
            r.q[p] = *reinterpret_cast<const uint4 *>(a.q + off);
        }
        r.t[p] = reinterpret_cast<const uint4 *>(rec)[idx];
    }
    {
        const int row = tid >> 3, c8 = tid & 7;
        r.v = make_uint4(0, 0, 0, 0);
        if (row < n) r.v = *reinterpret_cast<const uint4 *>(a.v + (static_cast<long long>(t0 + row) * a.Hv + h) * kD + jb + 8 * c8);
    }
    r.vec = 0.f;
    if (tid < 3 * kC) {
        r.vec = reinterpret_cast<const float *>(rec + REC_T)[tid];
    } else if (tid < 4 * kC) {
        const int row = tid - 3 * kC;
        if (row < n) r.vec = a.beta[static_cast<long long>(t0 + row) * a.Hv + h];
    }
}

__global__ __launch_bounds__(kScanThreads) void gdn_chunk_scan_kernel(ChunkArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    uint16_t *Kl = reinterpret_cast<uint16_t *>(lds + OFF_K);
    uint16_t *Ql = reinterpret_cast<uint16_t *>(lds + OFF_Q);
    uint16_t *UWl = reinterpret_cast<uint16_t *>(lds + OFF_Q);  // U~^T hi/lo once Q is consumed
    uint16_t *Vl = reinterpret_cast<uint16_t *>(lds + OFF_V);
    uint16_t *Tl = reinterpret_cast<uint16_t *>(lds + OFF_T);
    uint16_t *Rl = reinterpret_cast<uint16_t *>(lds + OFF_R);
    uint16_t *Pl = reinterpret_cast<uint16_t *>(lds + OFF_P);
    uint16_t *Shi = reinterpret_cast<uint16_t *>(lds + OFF_SHI);
    uint16_t *Slo = reinterpret_cast<uint16_t *>(lds + OFF_SLO);
    uint16_t *Ul = reinterpret_cast<uint16_t *>(lds + OFF_U);
    float *vec = reinterpret_cast<float *>(lds + OFF_VEC);
    const float *nk = vec, *nq = vec + kC, *gv = vec + 2 * kC, *bv = vec + 3 * kC;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;  // MFMA row/col and k-group of this lane
    const int seq = blockIdx.x / (a.Hv * 2);
    const int h = (blockIdx.x / 2) % a.Hv;
    const int jb = (blockIdx.x % 2) * kDVB;
    const int kh = khead(a, h);
    const int t_begin = a.cu[seq], t_end = a.cu[seq + 1];
    if (t_end <= t_begin) return;  // empty sequence: state unchanged (uniform per block)
    const int nchunks = (t_end - t_begin + kC - 1) / kC;
    auto record = [&](int c) { return a.ws + (static_cast<size_t>(a.coff[seq] + c) * a.Hv + h) * kRec; };

    float *S = a.state + (static_cast<long long>(seq) * a.Hv + h) * kD * kD;

    // State tiles of this wave: 4 tiles of the 128 x 64 block, tile id
    // 4*wave + u, rows i from (id / 4) * 16, columns j from (id % 4) * 16.
    f32x4 st[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int id = 4 * wave + u;
        const int i0 = (id >> 2) * 16 + 4 * lg, j = (id & 3) * 16 + lr;
        st[u] = *reinterpret_cast<const f32x4 *>(S + (jb + j) * kD + i0);
    }

    ChunkRegs cr;
    load_chunk(a, cr, tid, t_begin, min(kC, t_end - t_begin), kh, h, jb, record(0));

    for (int c = 0; c < nchunks; ++c) {
        const int t0 = t_begin + c * kC;
        const int n = min(kC, t_end - t0);
        __syncthreads();  // the previous chunk is done with every LDS buffer

        // ---- rows of this chunk and S0 hi/lo into LDS ---------------------
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int idx = tid + kScanThreads * p;
            const int row = idx >> 4, c16 = idx & 15;
            *reinterpret_cast<uint4 *>(Kl + row * KP + 8 * c16) = cr.k[p];
            *reinterpret_cast<uint4 *>(Ql + row * KP + 8 * c16) = cr.q[p];
            const int plane = idx >> 9, e = idx & 511;  // T hi then lo, 8 bf16 per uint4
            *reinterpret_cast<uint4 *>(Tl + plane * HL + (e >> 3) * FP + 8 * (e & 7)) = cr.t[p];
        }
        *reinterpret_cast<uint4 *>(Vl + (tid >> 3) * VP + 8 * (tid & 7)) = cr.v;
        if (tid < 4 * kC) vec[tid] = cr.vec;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int id = 4 * wave + u;
            const int i0 = (id >> 2) * 16 + 4 * lg, j = (id & 3) * 16 + lr;
            uint16_t hh[4], ll[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) split(st[u][e], hh[e], ll[e]);
            *reinterpret_cast<uint2 *>(Shi + j * KP + i0) = make_uint2(pack2(hh[0], hh[1]), pack2(hh[2], hh[3]));
            *reinterpret_cast<uint2 *>(Slo + j * KP + i0) = make_uint2(pack2(ll[0], ll[1]), pack2(ll[2], ll[3]));
        }
        __syncthreads();

        // next chunk's rows: the loads fly while this chunk computes
        if (c + 1 < nchunks)
            load_chunk(a, cr, tid, t0 + kC, min(kC, t_end - t0 - kC), kh, h, jb, record(c + 1));

        // ---- phase A: P^T = K Q^T, KS = K S0, QS^T = S0^T Q^T -------------
        f32x4 qs[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
            f32x4 p4 = {0, 0, 0, 0}, k4 = p4, q4 = p4;
#pragma unroll 2
            for (int kk = 0; kk < kD / 32; ++kk) {
                const int kc = kk * 32 + 8 * lg;
                const bf16x8 ka = ld_bf8(Kl + (m0 + lr) * KP + kc);
                const bf16x8 qb = ld_bf8(Ql + (n0 + lr) * KP + kc);
                const bf16x8 sh = ld_bf8(Shi + (n0 + lr) * KP + kc), sl = ld_bf8(Slo + (n0 + lr) * KP + kc);
                const bf16x8 sha = ld_bf8(Shi + (m0 + lr) * KP + kc), sla = ld_bf8(Slo + (m0 + lr) * KP + kc);
                p4 = mfma(ka, qb, p4);
                k4 = mfma(ka, sh, k4);
                k4 = mfma(ka, sl, k4);
                q4 = mfma(sha, qb, q4);
                q4 = mfma(sla, qb, q4);
            }
            qs[u] = q4;
            // lane holds rows s = m0 + 4*lg + e of column n0 + lr
            const int col = n0 + lr;
            f32x4 pt, rv;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int sr = m0 + 4 * lg + e;
                // Pt[r][s] with r = col: exp(g_r - g_s) nq_r nk_s P[r][s], s <= r
                pt[e] = (sr <= col) ? __expf(gv[col] - gv[sr]) * nq[col] * nk[sr] * p4[e] : 0.f;
                // R[s][j] with j = col: beta_s V[s][j] - beta_s b_s nk_s KS[s][j]
                rv[e] = bv[sr] * bf(Vl[sr * VP + col]) - bv[sr] * __expf(gv[sr]) * nk[sr] * k4[e];
            }
            st_split4(Pl, col * FP + m0 + 4 * lg, pt);  // Pt row-major [r][s]
            st_split4(Rl, col * FP + m0 + 4 * lg, rv);  // R^T [j][s]
        }
        __syncthreads();

        // ---- phase B: U = T R; store U^T and U~^T = (w o U)^T as hi/lo ------
        const float gC = gv[n - 1];
        const float bC = __expf(gC);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
            f32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kk = 0; kk < kC / 32; ++kk) {
                const int kc = kk * 32 + 8 * lg;
                const bf16x8 ah = ld_bf8(Tl + (m0 + lr) * FP + kc), al = ld_bf8(Tl + HL + (m0 + lr) * FP + kc);
                const bf16x8 bh = ld_bf8(Rl + (n0 + lr) * FP + kc), bl = ld_bf8(Rl + HL + (n0 + lr) * FP + kc);
                acc = mfma(ah, bh, acc);
                acc = mfma(ah, bl, acc);
                acc = mfma(al, bh, acc);
            }
            const int off = (n0 + lr) * FP + m0 + 4 * lg;  // U^T[j][s], s = m0 + 4*lg + e
            st_split4(Ul, off, acc);
            f32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int sr = m0 + 4 * lg + e;
                w[e] = acc[e] * (nk[sr] * __expf(gC - gv[sr]));
            }
            st_split4(UWl, off, w);
        }
        __syncthreads();

        // ---- phase C: O^T = U^T Pt^T + diag-scaled QS^T;  S = b_C S + K^T U~ --
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;  // m0: j block, n0: r block
            f32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kk = 0; kk < kC / 32; ++kk) {
                const int kc = kk * 32 + 8 * lg;
                const bf16x8 ah = ld_bf8(Ul + (m0 + lr) * FP + kc), al = ld_bf8(Ul + HL + (m0 + lr) * FP + kc);
                const bf16x8 bh = ld_bf8(Pl + (n0 + lr) * FP + kc), bl = ld_bf8(Pl + HL + (n0 + lr) * FP + kc);
                acc = mfma(ah, bh, acc);
                acc = mfma(ah, bl, acc);
                acc = mfma(al, bh, acc);
            }
            const int r = n0 + lr;
            if (r < n) {
                const float sc = __expf(gv[r]) * nq[r];
                f32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = sc * qs[u][e] + acc[e];
                *reinterpret_cast<f32x4 *>(a.out + (static_cast<long long>(t0 + r) * a.Hv + h) * kD + jb + m0 + 4 * lg) = o;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) st[u] = st[u] * bC;
#pragma unroll
        for (int kk = 0; kk < kC / 32; ++kk) {
            const int kc = kk * 32 + 8 * lg;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int id = 4 * wave + u;
                const int i0 = (id >> 2) * 16, j0 = (id & 3) * 16;
                bf16x8 ka;  // K^T[i][s-run]: 8 strided bf16 of column i
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    ka[e] = __builtin_bit_cast(__bf16, Kl[(kc + e) * KP + i0 + lr]);
                const bf16x8 bh = ld_bf8(UWl + (j0 + lr) * FP + kc), bl = ld_bf8(UWl + HL + (j0 + lr) * FP + kc);
                st[u] = mfma(ka, bh, st[u]);
                st[u] = mfma(ka, bl, st[u]);
            }
        }
    }

    // final state back to HBM
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int id = 4 * wave + u;
        const int i0 = (id >> 2) * 16 + 4 * lg, j = (id & 3) * 16 + lr;
        *reinterpret_cast<f32x4 *>(S + (jb + j) * kD + i0) = st[u];
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
    static bool attr_set = false;
    if (!attr_set) {
        int st = set_lds(reinterpret_cast<const void *>(gdn_chunk_scan_kernel), SCAN_LDS);
        if (!st) st = set_lds(reinterpret_cast<const void *>(gdn_chunk_prep_kernel), PREP_LDS);
        if (st) return st;
        attr_set = true;
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
        hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(Hv)),
                           dim3(kPrepThreads), PREP_LDS, as_stream(stream), a);
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
