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
constexpr int FP = kC + 4;     // fp32 row pitch of 64x64 matrices (272 B)

// LDS byte offsets.
constexpr int OFF_K = 0;
constexpr int OFF_Q = OFF_K + kC * KP * 2;
constexpr int OFF_V = OFF_Q + kC * KP * 2;
constexpr int OFF_A = OFF_V + kC * VP * 2;        // A, then R^T [j][s]
constexpr int OFF_T = OFF_A + kC * FP * 4;
constexpr int OFF_P = OFF_T + kC * FP * 4;        // Pt
constexpr int OFF_SHI = OFF_P + kC * FP * 4;      // S0 hi, [j][i]
constexpr int OFF_SLO = OFF_SHI + kDVB * KP * 2;  // S0 lo
constexpr int OFF_U = OFF_SLO + kDVB * KP * 2;    // U^T [j][s]
constexpr int OFF_RT = OFF_U + kDVB * FP * 4;     // 3 x 16 x 17 fp32 scratch
constexpr int OFF_VEC = OFF_RT + 3 * 16 * 17 * 4; // nk, nq, g, beta
constexpr int LDS_BYTES = OFF_VEC + 4 * kC * 4;

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

// 8 fp32 from LDS, scaled per element, split into hi + lo bf16 operands.
__device__ __forceinline__ void ld_split8(const float *p, const float *scale, bf16x8 &hi, bf16x8 &lo) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(p);
    const f32x4 b = *reinterpret_cast<const f32x4 *>(p + 4);
    float f[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x = scale ? f[e] * scale[e] : f[e];
        const __bf16 h = static_cast<__bf16>(x);
        hi[e] = h;
        lo[e] = static_cast<__bf16>(x - static_cast<float>(h));
    }
}

__global__ __launch_bounds__(kThreads) void gdn_chunk_kernel(ChunkArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    uint16_t *Kl = reinterpret_cast<uint16_t *>(lds + OFF_K);
    uint16_t *Ql = reinterpret_cast<uint16_t *>(lds + OFF_Q);
    uint16_t *Vl = reinterpret_cast<uint16_t *>(lds + OFF_V);
    float *Al = reinterpret_cast<float *>(lds + OFF_A);
    float *Tl = reinterpret_cast<float *>(lds + OFF_T);
    float *Pl = reinterpret_cast<float *>(lds + OFF_P);
    uint16_t *Shi = reinterpret_cast<uint16_t *>(lds + OFF_SHI);
    uint16_t *Slo = reinterpret_cast<uint16_t *>(lds + OFF_SLO);
    float *Ul = reinterpret_cast<float *>(lds + OFF_U);
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

    // Upper off-diagonal 16x16 blocks of T are never written: zero once.
    for (int e = tid; e < kC * kC; e += kThreads) {
        const int r = e / kC, c = e % kC;
        if ((c >> 4) > (r >> 4)) Tl[r * FP + c] = 0.f;
    }

    // State tiles of this wave: 4 tiles of the 128 x 64 block, (ti, tj) with
    // tile id 4*wave + u, ti = id / 4 (i rows), tj = id % 4 (j columns).
    f32x4 st[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int id = 4 * wave + u;
        const int i0 = (id >> 2) * 16 + 4 * lg, j = (id & 3) * 16 + lr;
        st[u] = *reinterpret_cast<const f32x4 *>(S + (jb + j) * kD + i0);
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const __bf16 hb = static_cast<__bf16>(st[u][e]);
            const __bf16 lb = static_cast<__bf16>(st[u][e] - static_cast<float>(hb));
            hi[e] = __builtin_bit_cast(uint16_t, hb);
            lo[e] = __builtin_bit_cast(uint16_t, lb);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            Shi[j * KP + i0 + e] = hi[e];
            Slo[j * KP + i0 + e] = lo[e];
        }
    }

    const float qscale = (a.flags & OURO_GDN_SCALE_Q) ? 1.0f / sqrtf(static_cast<float>(kD)) : 1.0f;
    const bool l2 = (a.flags & OURO_GDN_L2NORM_QK) != 0;

    for (int t0 = t_begin; t0 < t_end; t0 += kC) {
        const int n = min(kC, t_end - t0);
        __syncthreads();  // previous chunk fully consumed K, Q, V, U

        // ---- phase 0: chunk rows into LDS (rows >= n are zero) ----------
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
        float gate_l = 0.f;
        if (wave == 2 && lane < n) gate_l = a.gate[static_cast<long long>(t0 + lane) * a.Hv + h];
        if (wave == 3) bv[lane] = lane < n ? a.beta[static_cast<long long>(t0 + lane) * a.Hv + h] : 0.f;
        __syncthreads();

        // ---- phase 1: row norms and cumulative log-decay -----------------
        if (wave < 2) {
            const uint16_t *row = (wave == 0 ? Kl : Ql) + lane * KP;
            float ss = 0.f;
            for (int i = 0; i < kD; ++i) {
                const float x = bf(row[i]);
                ss += x * x;
            }
            float sc = l2 ? 1.0f / (sqrtf(ss) + a.eps) : 1.0f;
            if (wave == 1) sc *= qscale;
            if (lane >= n) sc = 0.f;
            (wave == 0 ? nk : nq)[lane] = sc;
        } else if (wave == 2) {
            float g = gate_l;  // inclusive scan over the 64 lanes
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const float o = __shfl_up(g, off, 64);
                if (lane >= off) g += o;
            }
            gv[lane] = g;
        }
        __syncthreads();

        // ---- phase 2: G = K K^T, P = Q K^T, KS = K S0, QS = Q S0 ---------
        f32x4 ks[2], qs[2];
        f32x4 rr[2];  // R of the KS tiles, written after T is solved
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
            f32x4 g4 = {0, 0, 0, 0}, p4 = g4, k4 = g4, q4 = g4;
#pragma unroll
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
            ks[u] = k4;
            qs[u] = q4;
            const int c = n0 + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = m0 + 4 * lg + e;
                float av = 0.f, pv = 0.f;
                if (c < r) av = bv[r] * expf(gv[r] - gv[c]) * nk[r] * nk[c] * g4[e];
                if (c <= r) pv = expf(gv[r] - gv[c]) * nq[r] * nk[c] * p4[e];
                Al[r * FP + c] = av;
                Pl[r * FP + c] = pv;
                // R[r][c] = beta_r V[r][c] - beta_r b_r nk_r KS[r][c]
                rr[u][e] = bv[r] * bf(Vl[r * VP + c]) - bv[r] * expf(gv[r]) * nk[r] * k4[e];
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

        // ---- phase 4: R^T into the A buffer -------------------------------
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
            *reinterpret_cast<f32x4 *>(Al + (n0 + lr) * FP + m0 + 4 * lg) = rr[u];
        }
        __syncthreads();

        // ---- phase 5: U = T R ---------------------------------------------
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
            f32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kk = 0; kk < kC / 32; ++kk) {
                const int kc = kk * 32 + 8 * lg;
                bf16x8 ah, al, bh, bl;
                ld_split8(Tl + (m0 + lr) * FP + kc, nullptr, ah, al);
                ld_split8(Al + (n0 + lr) * FP + kc, nullptr, bh, bl);
                acc = mfma(ah, bh, acc);
                acc = mfma(ah, bl, acc);
                acc = mfma(al, bh, acc);
            }
            *reinterpret_cast<f32x4 *>(Ul + (n0 + lr) * FP + m0 + 4 * lg) = acc;
        }
        __syncthreads();

        // ---- phase 6: O = diag(b nq) QS + Pt U;  S = b_C S + K^T (w o U) ----
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int id = 2 * wave + u;
            const int m0 = (id >> 2) * 16, n0 = (id & 3) * 16;
            f32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int kk = 0; kk < kC / 32; ++kk) {
                const int kc = kk * 32 + 8 * lg;
                bf16x8 ah, al, bh, bl;
                ld_split8(Pl + (m0 + lr) * FP + kc, nullptr, ah, al);
                ld_split8(Ul + (n0 + lr) * FP + kc, nullptr, bh, bl);
                acc = mfma(ah, bh, acc);
                acc = mfma(ah, bl, acc);
                acc = mfma(al, bh, acc);
            }
            const int c = n0 + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = m0 + 4 * lg + e;
                if (r < n) {
                    const float o = expf(gv[r]) * nq[r] * qs[u][e] + acc[e];
                    a.out[(static_cast<long long>(t0 + r) * a.Hv + h) * kD + jb + c] = o;
                }
            }
        }
        const float gC = gv[n - 1];
        const float bC = expf(gC);
        float wsc[8];  // per-token weight nk_s exp(g_C - g_s) of this lane's k-run
#pragma unroll
        for (int kk = 0; kk < kC / 32; ++kk) {
            const int kc = kk * 32 + 8 * lg;
#pragma unroll
            for (int e = 0; e < 8; ++e) wsc[e] = nk[kc + e] * expf(gC - gv[kc + e]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int id = 4 * wave + u;
                const int i0 = (id >> 2) * 16, j0 = (id & 3) * 16;
                if (kk == 0) st[u] = st[u] * bC;
                bf16x8 ka;  // K^T[i][s-run]: 8 strided bf16 of column i
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    ka[e] = __builtin_bit_cast(__bf16, Kl[(kc + e) * KP + i0 + lr]);
                bf16x8 bh, bl;
                ld_split8(Ul + (j0 + lr) * FP + kc, wsc, bh, bl);
                st[u] = mfma(ka, bh, st[u]);
                st[u] = mfma(ka, bl, st[u]);
            }
        }
        __syncthreads();  // everyone is done reading S hi/lo of this chunk

        // new S0 hi/lo for the next chunk
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int id = 4 * wave + u;
            const int i0 = (id >> 2) * 16 + 4 * lg, j = (id & 3) * 16 + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const __bf16 hb = static_cast<__bf16>(st[u][e]);
                const __bf16 lb = static_cast<__bf16>(st[u][e] - static_cast<float>(hb));
                Shi[j * KP + i0 + e] = __builtin_bit_cast(uint16_t, hb);
                Slo[j * KP + i0 + e] = __builtin_bit_cast(uint16_t, lb);
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
