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
// One 512-thread workgroup owns (sequence, v-head, 64 of the 128 state
// columns): output column j of the recurrence only touches state column j,
// so the two column halves of a head are independent chains.  The chunk
// loop is sequential; everything inside a chunk is spread over 8 waves.
#include "common.hpp"

namespace ouro {
namespace {

constexpr int kD = 128;        // d_k = d_v (qwen35.rs:8)
constexpr int kC = 64;         // chunk length
constexpr int kDVB = 64;       // state columns per workgroup
constexpr int kThreads = 512;  // 8 waves
constexpr int kMaxSeq = 256;   // sequences per launch (cu_seqlens by value)

constexpr int KP = kD + 8;     // bf16 row pitch of K, Q, S^T (272 B)
constexpr int VP = kDVB + 8;   // bf16 row pitch of V (144 B)
constexpr int FP = kC + 8;     // pitch of 64x64 matrices: fp32 (288 B) or bf16 hi/lo (144 B)
constexpr int HL = kC * FP;    // elements of one bf16 plane (hi or lo) of a 64x64 matrix

// LDS byte offsets.
constexpr int MAT = kC * FP * 4;                  // bytes of a 64x64 fp32 (= hi+lo bf16) slot
constexpr int OFF_K = 0;
constexpr int OFF_Q = OFF_K + kC * KP * 2;        // Q, then U~^T hi/lo
constexpr int OFF_V = OFF_Q + MAT;
constexpr int OFF_A = OFF_V + kC * VP * 2;        // A fp32, then R^T hi/lo
constexpr int OFF_T = OFF_A + MAT;                // T fp32, then T hi/lo
constexpr int OFF_P = OFF_T + MAT;                // Pt hi/lo
constexpr int OFF_SHI = OFF_P + MAT;              // S0 hi, [j][i]
constexpr int OFF_SLO = OFF_SHI + kDVB * KP * 2;  // S0 lo
constexpr int OFF_U = OFF_SLO + kDVB * KP * 2;    // U^T hi/lo
constexpr int OFF_RT = OFF_U + MAT;               // 3 x 16 x 17 fp32 scratch
constexpr int OFF_VEC = OFF_RT + 3 * 16 * 17 * 4; // nk, nq, g, beta
constexpr int LDS_BYTES = OFF_VEC + 4 * kC * 4;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of a gfx950 workgroup");

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct ChunkArgs {
    float *state;
    const uint16_t *q, *k, *v;
    const float *gate, *beta;
    float *out;
    int Hk, Hv, nseq;
    unsigned flags;
    float eps;
    int cu[kMaxSeq + 1];
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

// Store 4 consecutive values (along the contiguous axis) of a hi/lo matrix.
__device__ __forceinline__ void st_split4(uint16_t *hl, int off, const f32x4 &v) {
    uint16_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split(v[e], h[e], l[e]);
    *reinterpret_cast<uint2 *>(hl + off) =
        make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
    *reinterpret_cast<uint2 *>(hl + HL + off) =
        make_uint2(l[0] | (static_cast<uint32_t>(l[1]) << 16), l[2] | (static_cast<uint32_t>(l[3]) << 16));
}

__global__ __launch_bounds__(kThreads) void gdn_chunk_kernel(ChunkArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    uint16_t *Kl = reinterpret_cast<uint16_t *>(lds + OFF_K);
    uint16_t *Ql = reinterpret_cast<uint16_t *>(lds + OFF_Q);
    uint16_t *UWl = reinterpret_cast<uint16_t *>(lds + OFF_Q);  // U~^T hi/lo after phase 2
    uint16_t *Vl = reinterpret_cast<uint16_t *>(lds + OFF_V);
    float *Al = reinterpret_cast<float *>(lds + OFF_A);
    uint16_t *Rl = reinterpret_cast<uint16_t *>(lds + OFF_A);   // R^T hi/lo after the solve
    float *Tl = reinterpret_cast<float *>(lds + OFF_T);
    uint16_t *Thl = reinterpret_cast<uint16_t *>(lds + OFF_T);  // T hi/lo after the solve
    uint16_t *Pl = reinterpret_cast<uint16_t *>(lds + OFF_P);
    uint16_t *Shi = reinterpret_cast<uint16_t *>(lds + OFF_SHI);
    uint16_t *Slo = reinterpret_cast<uint16_t *>(lds + OFF_SLO);
    uint16_t *Ul = reinterpret_cast<uint16_t *>(lds + OFF_U);
    float *Rt = reinterpret_cast<float *>(lds + OFF_RT);
    float *nk = reinterpret_cast<float *>(lds + OFF_VEC);
    float *nq = nk + kC;
    float *gv = nq + kC;
    float *bv = gv + kC;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;  // MFMA row/col and k-group of this lane
    const int seq = blockIdx.x / (a.Hv * 2);
    const int h = (blockIdx.x / 2) % a.Hv;
    const int jb = (blockIdx.x % 2) * kDVB;
    const int kh = (a.flags & OURO_GDN_KHEAD_DIV) ? h / (a.Hv / a.Hk) : h % a.Hk;
    const int t_begin = a.cu[seq], t_end = a.cu[seq + 1];
    if (t_end <= t_begin) return;  // empty sequence: state unchanged (uniform per block)

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

    const float qscale = (a.flags & OURO_GDN_SCALE_Q) ? 1.0f / sqrtf(static_cast<float>(kD)) : 1.0f;
    const bool l2 = (a.flags & OURO_GDN_L2NORM_QK) != 0;

    for (int t0 = t_begin; t0 < t_end; t0 += kC) {
        const int n = min(kC, t_end - t0);
        __syncthreads();  // the previous chunk is done with every LDS buffer

        // ---- phase 0: chunk rows and S0 hi/lo into LDS -----------------
        for (int idx = tid; idx < kC * 16; idx += kThreads) {
            const int r = idx >> 4, c16 = idx & 15;
            uint4 kv = make_uint4(0, 0, 0, 0), qv = kv;
            if (r < n) {
                const long long off = (static_cast<long long>(t0 + r) * a.Hk + kh) * kD + 8 * c16;
                kv = *reinterpret_cast<const uint4 *>(a.k + off);
                qv = *reinterpret_cast<const uint4 *>(a.q + off);
            }
            *reinterpret_cast<uint4 *>(Kl + r * KP + 8 * c16) = kv;
            *reinterpret_cast<uint4 *>(Ql + r * KP + 8 * c16) = qv;
        }
        {
            const int r = tid >> 3, c8 = tid & 7;
            uint4 vv = make_uint4(0, 0, 0, 0);
            if (r < n)
                vv = *reinterpret_cast<const uint4 *>(
                    a.v + (static_cast<long long>(t0 + r) * a.Hv + h) * kD + jb + 8 * c8);
            *reinterpret_cast<uint4 *>(Vl + r * VP + 8 * c8) = vv;
        }
        if (wave == 2) {  // inclusive scan of the log-decays over the chunk
            float g = lane < n ? a.gate[static_cast<long long>(t0 + lane) * a.Hv + h] : 0.f;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const float o = __shfl_up(g, off, 64);
                if (lane >= off) g += o;
            }
            gv[lane] = g;
        }
        if (wave == 3) bv[lane] = lane < n ? a.beta[static_cast<long long>(t0 + lane) * a.Hv + h] : 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int id = 4 * wave + u;
            const int i0 = (id >> 2) * 16 + 4 * lg, j = (id & 3) * 16 + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) split(st[u][e], Shi[j * KP + i0 + e], Slo[j * KP + i0 + e]);
        }
        __syncthreads();

        // ---- phase 1: row norms, 4 lanes per row ------------------------
        {
            const int row = tid >> 2, qq = tid & 3;  // rows 0..63 of K, 64..127 of Q
            const uint16_t *rp = (row < kC ? Kl + row * KP : Ql + (row - kC) * KP) + 32 * qq;
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4 w = *reinterpret_cast<const uint4 *>(rp + 8 * c);
                const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x0 = __uint_as_float(ws[e] << 16), x1 = __uint_as_float(ws[e] & 0xffff0000u);
                    ss += x0 * x0 + x1 * x1;
                }
            }
            ss += __shfl_xor(ss, 1, 64);
            ss += __shfl_xor(ss, 2, 64);
            if (qq == 0) {
                const int r = row & (kC - 1);
                float sc = l2 ? 1.0f / (sqrtf(ss) + a.eps) : 1.0f;
                if (row >= kC) sc *= qscale;
                if (r >= n) sc = 0.f;
                (row < kC ? nk : nq)[r] = sc;
            }
        }
        __syncthreads();

        // ---- phase 2: G = K K^T, P = Q K^T, KS = K S0, QS = Q S0 ---------
        f32x4 qs[2];
        float *Rf = reinterpret_cast<float *>(lds + OFF_U);  // R fp32 [r][c] until phase 4
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
            f32x4 g4 = {0, 0, 0, 0}, p4 = g4, k4 = g4, q4 = g4;
#pragma unroll 2
            for (int kk = 0; kk < kD / 32; ++kk) {
                const int kc = kk * 32 + 8 * lg;
                const bf16x8 ka = ld_bf8(Kl + (m0 + lr) * KP + kc);
                const bf16x8 qa = ld_bf8(Ql + (m0 + lr) * KP + kc);
                const bf16x8 kb = ld_bf8(Kl + (n0 + lr) * KP + kc);
                const bf16x8 sh = ld_bf8(Shi + (n0 + lr) * KP + kc);
                const bf16x8 sl = ld_bf8(Slo + (n0 + lr) * KP + kc);
                g4 = mfma(ka, kb, g4);
                p4 = mfma(qa, kb, p4);
                k4 = mfma(ka, sh, k4);
                k4 = mfma(ka, sl, k4);
                q4 = mfma(qa, sh, q4);
                q4 = mfma(qa, sl, q4);
            }
            qs[u] = q4;
            const int c = n0 + lr;
            const float gc = gv[c], nkc = nk[c];
            f32x4 pt;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = m0 + 4 * lg + e;
                const float gr = gv[r];
                const float dec = (c <= r) ? __expf(gr - gc) : 0.f;
                Al[r * FP + c] = (c < r) ? bv[r] * dec * nk[r] * nkc * g4[e] : 0.f;
                pt[e] = dec * nq[r] * nkc * p4[e];
                // R[r][c] = beta_r V[r][c] - beta_r b_r nk_r KS[r][c]
                Rf[r * FP + c] = bv[r] * bf(Vl[r * VP + c]) - bv[r] * __expf(gr) * nk[r] * k4[e];
            }
            // Pt is read row-major [r][s] as an A operand: 4 rows at column c
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = m0 + 4 * lg + e;
                split(pt[e], Pl[r * FP + c], Pl[HL + r * FP + c]);
            }
        }
        __syncthreads();

        // ---- phase 3: T = (I + A)^-1, blocked forward substitution --------
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
            // upper off-diagonal blocks are zero
            for (int e = tid - 64; e < kC * kC; e += kThreads - 64) {
                const int r = e / kC, c = e % kC;
                if ((c >> 4) > (r >> 4)) Tl[r * FP + c] = 0.f;
            }
        }
        __syncthreads();
        for (int dd = 1; dd <= 3; ++dd) {
            const int nblk = 4 - dd;
            for (int e = tid; e < nblk * 256; e += kThreads) {
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
            for (int e = tid; e < nblk * 256; e += kThreads) {
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

        // ---- phase 4: T and R^T to hi/lo bf16 (each value split once) -------
        {
            // T: 8 values per thread, row r, columns 8*cq .. 8*cq+7
            const int r = tid >> 3, cq = tid & 7;
            const f32x4 t0v = *reinterpret_cast<const f32x4 *>(Tl + r * FP + 8 * cq);
            const f32x4 t1v = *reinterpret_cast<const f32x4 *>(Tl + r * FP + 8 * cq + 4);
            // R^T[j][s] hi/lo into the A slot (A is dead): this thread takes
            // column j = tid / 8 and rows s = 8*(tid % 8) .. +7 of R.
            const int j = tid >> 3, s0 = 8 * (tid & 7);
            f32x4 r0, r1;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                r0[e] = Rf[(s0 + e) * FP + j];
                r1[e] = Rf[(s0 + 4 + e) * FP + j];
            }
            st_split4(Rl, j * FP + s0, r0);
            st_split4(Rl, j * FP + s0 + 4, r1);
            __syncthreads();
            st_split4(Thl, r * FP + 8 * cq, t0v);
            st_split4(Thl, r * FP + 8 * cq + 4, t1v);
        }
        __syncthreads();

        // ---- phase 5: U = T R; store U^T and U~^T = (w o U)^T as hi/lo ------
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
                const bf16x8 ah = ld_bf8(Thl + (m0 + lr) * FP + kc), al = ld_bf8(Thl + HL + (m0 + lr) * FP + kc);
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
                const int sidx = m0 + 4 * lg + e;
                w[e] = acc[e] * (nk[sidx] * __expf(gC - gv[sidx]));
            }
            st_split4(UWl, off, w);
        }
        __syncthreads();

        // ---- phase 6: O = diag(b nq) QS + Pt U;  S = b_C S + K^T U~ ----------
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
            f32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kk = 0; kk < kC / 32; ++kk) {
                const int kc = kk * 32 + 8 * lg;
                const bf16x8 ah = ld_bf8(Pl + (m0 + lr) * FP + kc), al = ld_bf8(Pl + HL + (m0 + lr) * FP + kc);
                const bf16x8 bh = ld_bf8(Ul + (n0 + lr) * FP + kc), bl = ld_bf8(Ul + HL + (n0 + lr) * FP + kc);
                acc = mfma(ah, bh, acc);
                acc = mfma(ah, bl, acc);
                acc = mfma(al, bh, acc);
            }
            const int c = n0 + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = m0 + 4 * lg + e;
                if (r < n) {
                    const float o = __expf(gv[r]) * nq[r] * qs[u][e] + acc[e];
                    a.out[(static_cast<long long>(t0 + r) * a.Hv + h) * kD + jb + c] = o;
                }
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

}  // namespace

int gdn_chunk_prefill(float *state, const void *q, const void *k, const void *v, const float *gate,
                      const float *beta, float *out, const int32_t *cu_host, size_t N, size_t T,
                      size_t Hk, size_t Hv, size_t d, size_t chunk, unsigned flags, float eps,
                      void *stream) {
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
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(state);
    if (mis % 16) return fail(OURO_ERR_ALIGN, "gdn chunk prefill: q, k, v, state need 16-byte alignment");
    // Validate the offsets on the host before any launch.
    if (cu_host) {
        if (cu_host[0] != 0 || static_cast<size_t>(cu_host[N]) != T)
            return fail(OURO_ERR_SHAPE, "gdn chunk prefill: cu_seqlens must run 0..T");
        for (size_t i = 0; i < N; ++i)
            if (cu_host[i + 1] < cu_host[i]) return fail(OURO_ERR_SHAPE, "gdn chunk prefill: cu_seqlens decreasing");
    } else if (N != 1) {
        return fail(OURO_ERR_SHAPE, "gdn chunk prefill: cu_seqlens NULL needs N == 1");
    }
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(gdn_chunk_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
        if (e != hipSuccess)
            return fail(OURO_ERR_HIP, "gdn chunk prefill: %d B of LDS refused: %s", LDS_BYTES, hipGetErrorString(e));
        attr_set = true;
    }
    ChunkArgs a{};
    a.q = static_cast<const uint16_t *>(q);
    a.k = static_cast<const uint16_t *>(k);
    a.v = static_cast<const uint16_t *>(v);
    a.gate = gate;
    a.beta = beta;
    a.out = out;
    a.Hk = static_cast<int>(Hk);
    a.Hv = static_cast<int>(Hv);
    a.flags = flags;
    a.eps = eps;
    // Launch in slices of up to kMaxSeq sequences; each slice is independent.
    for (size_t s0 = 0; s0 < N; s0 += kMaxSeq) {
        const size_t ns = N - s0 < static_cast<size_t>(kMaxSeq) ? N - s0 : kMaxSeq;
        a.nseq = static_cast<int>(ns);
        a.state = state + s0 * Hv * kD * kD;
        for (size_t i = 0; i <= ns; ++i) a.cu[i] = cu_host ? cu_host[s0 + i] : (i == 0 ? 0 : static_cast<int>(T));
        const unsigned blocks = static_cast<unsigned>(ns * Hv * 2);
        hipLaunchKernelGGL(gdn_chunk_kernel, dim3(blocks), dim3(kThreads), LDS_BYTES, as_stream(stream), a);
        int st = check_launch("gdn_chunk_kernel");
        if (st) return st;
    }
    return OURO_OK;
}

}  // namespace ouro

using namespace ouro;

extern "C" {

int ouro_gdn_chunk_prefill(float *state, const void *q, const void *k, const void *v, const float *gate,
                           const float *beta, float *out, const int32_t *cu_seqlens_host, size_t N,
                           size_t T, size_t Hk, size_t Hv, size_t d, size_t chunk, unsigned flags,
                           float eps, void *stream) {
    OURO_REQUIRE_INIT();
    return gdn_chunk_prefill(state, q, k, v, gate, beta, out, cu_seqlens_host, N, T, Hk, Hv, d, chunk,
                             flags, eps, stream);
}

}  // extern "C"
