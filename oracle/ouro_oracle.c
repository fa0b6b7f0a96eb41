/*
 * ouro_oracle.c - CPU oracle (test infrastructure only; see ouro_oracle.h).
 *
 * Plain-C restatement of the reference Rust CPU arithmetic.  Each function
 * cites the reference file:line it follows.  Summation orders follow the
 * reference loops exactly; the file is compiled with -ffp-contract=off so
 * that a*b+c is never fused (Rust does not fuse either).
 */
#include "ouro_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <smmintrin.h>

/* ------------------------------------------------------------------------ */
/* threading: row-split workers, as ops.rs:104-126 / 298-320 do with        */
/* std::thread::scope over out_len.div_ceil(nt) chunks.                      */
/* ------------------------------------------------------------------------ */

int orc_mt_threads(void) /* ops.rs:62-73 */
{
    const char *e = getenv("OURO_N_THREADS");
    if (e && *e) {
        int n = atoi(e);
        if (n > 0) return n;
    }
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

typedef void (*orc_range_fn)(void *ctx, size_t lo, size_t hi);

struct orc_job {
    orc_range_fn fn;
    void *ctx;
    size_t lo, hi;
};

static void *orc_job_run(void *p)
{
    struct orc_job *j = (struct orc_job *)p;
    j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}

/* Run fn over [0,n) split into nt contiguous chunks of n.div_ceil(nt). */
static void orc_parallel_for(size_t n, int nthreads, orc_range_fn fn, void *ctx)
{
    if (nthreads <= 0) nthreads = orc_mt_threads();
    size_t nt = (size_t)nthreads;
    if (nt > n) nt = n;
    if (nt <= 1) {
        if (n) fn(ctx, 0, n);
        return;
    }
    size_t chunk = (n + nt - 1) / nt;
    pthread_t th[256];
    struct orc_job jobs[256];
    if (nt > 256) nt = 256, chunk = (n + nt - 1) / nt;
    size_t used = 0;
    for (size_t t = 0; t < nt; ++t) {
        size_t lo = t * chunk, hi = lo + chunk;
        if (lo >= n) break;
        if (hi > n) hi = n;
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].lo = lo;
        jobs[t].hi = hi;
        if (pthread_create(&th[t], NULL, orc_job_run, &jobs[t]) != 0) {
            orc_job_run(&jobs[t]);
            th[t] = 0;
        }
        used = t + 1;
    }
    for (size_t t = 0; t < used; ++t)
        if (th[t]) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* dequant.rs                                                                */
/* ------------------------------------------------------------------------ */

static float bits_f32(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t f32_bits(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

float orc_f16_to_f32(uint16_t bits) /* dequant.rs:21-47 */
{
    uint32_t sign = (bits >> 15) & 1u;
    int32_t exp = (bits >> 10) & 0x1f;
    uint32_t frac = bits & 0x3ffu;
    uint32_t out;
    if (exp == 0) {
        if (frac == 0) {
            out = sign << 31;
        } else {
            int32_t e = -1;
            uint32_t f = frac;
            while ((f & 0x400u) == 0) {
                f <<= 1;
                e += 1;
            }
            f &= 0x3ffu;
            int32_t exp32 = 127 - 15 - e;
            out = (sign << 31) | ((uint32_t)exp32 << 23) | (f << 13);
        }
    } else if (exp == 0x1f) {
        out = (sign << 31) | (0xffu << 23) | (frac << 13);
    } else {
        out = (sign << 31) | ((uint32_t)(exp + 127 - 15) << 23) | (frac << 13);
    }
    return bits_f32(out);
}

float orc_bf16_to_f32(uint16_t bits) /* dequant.rs:197-199 */
{
    return bits_f32((uint32_t)bits << 16);
}

uint16_t orc_f32_to_bf16_rne(float x)
{
    uint32_t u = f32_bits(x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) /* NaN: keep quiet */
        return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/* PTQ1_POW3 (dequant.rs:130) and the digit magic of ptq1_digit (134-138). */
static const uint8_t PTQ1_POW3[6] = {1, 3, 9, 27, 81, 243};

static inline int ptq1_digit_i(uint8_t byte, int n)
{
    uint8_t q = (uint8_t)(byte * PTQ1_POW3[n]); /* u8 wrapping_mul */
    uint16_t xi = (uint16_t)(((uint16_t)q * 3u) >> 8);
    return (int)(int8_t)xi - 1;
}

void orc_tl1_group(const uint8_t *bytes, float *out) /* dequant.rs:146-171 */
{
    float d = orc_f16_to_f32((uint16_t)(bytes[26] | (bytes[27] << 8)));
    const uint8_t *qs = bytes;
    const uint8_t *qh = bytes + 24;
    size_t o = 0;
    for (int n = 0; n < 5; ++n)
        for (int m = 0; m < 16; ++m) out[o++] = (float)ptq1_digit_i(qs[m], n) * d;
    for (int n = 0; n < 5; ++n)
        for (int m = 16; m < 24; ++m) out[o++] = (float)ptq1_digit_i(qs[m], n) * d;
    for (int n = 0; n < 4; ++n)
        for (int h = 0; h < 2; ++h) out[o++] = (float)ptq1_digit_i(qh[h], n) * d;
}

void orc_dequant_tl1_row(const uint8_t *payload, size_t row, size_t row_elems,
                         float *out) /* dequant.rs:185-195 */
{
    size_t gpr = row_elems / 128;
    for (size_t g = 0; g < gpr; ++g)
        orc_tl1_group(payload + (row * gpr + g) * 28, out + g * 128);
}

static const uint8_t TQ1_POW3[5] = {1, 3, 9, 27, 81}; /* dequant.rs:18 */

static inline float tq1_trit(uint8_t byte, int n, float d) /* dequant.rs:55-59 */
{
    uint8_t q = (uint8_t)(byte * TQ1_POW3[n]);
    uint16_t xi = (uint16_t)(((uint16_t)q * 3u) >> 8);
    return ((float)xi - 1.0f) * d;
}

void orc_tq1_block(const uint8_t *bytes, float *out) /* dequant.rs:50-80 */
{
    const uint8_t *qs = bytes;
    const uint8_t *qh = bytes + 48;
    float d = orc_f16_to_f32((uint16_t)(bytes[52] | (bytes[53] << 8)));
    size_t o = 0;
    for (int n = 0; n < 5; ++n)
        for (int m = 0; m < 32; ++m) out[o++] = tq1_trit(qs[m], n, d);
    for (int n = 0; n < 5; ++n)
        for (int m = 32; m < 48; ++m) out[o++] = tq1_trit(qs[m], n, d);
    for (int n = 0; n < 4; ++n)
        for (int m = 0; m < 4; ++m) out[o++] = tq1_trit(qh[m], n, d);
}

void orc_dequant_tq1_row(const uint8_t *payload, size_t row, size_t row_bytes,
                         float *out) /* dequant.rs:96-105 */
{
    size_t start = row * row_bytes;
    size_t blocks = row_bytes / 54;
    for (size_t b = 0; b < blocks; ++b)
        orc_tq1_block(payload + start + b * 54, out + b * 256);
}

/* ---- the K-quant and Q8_0 blocks (dequant.rs:218-310, 390-560) ---------- */

static float f16_at(const uint8_t *b) { return orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

void orc_q8_block(const uint8_t *bytes, float *out) /* dequant.rs:225-231 */
{
    float d = f16_at(bytes);
    for (int j = 0; j < 32; ++j) out[j] = (float)(int8_t)bytes[2 + j] * d;
}

/* scale_min_k4 (dequant.rs:245-254) */
static void scale_min_k4(int j, const uint8_t *sc, uint8_t *d, uint8_t *m)
{
    if (j < 4) {
        *d = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *d = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
        *m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
}

void orc_q4k_block(const uint8_t *bytes, float *out) /* dequant.rs:257-282 */
{
    float d = f16_at(bytes), min = f16_at(bytes + 2);
    const uint8_t *scales = bytes + 4, *q = bytes + 16;
    int is = 0, o = 0;
    for (int blk = 0; blk < 4; ++blk) {
        uint8_t s1, m1, s2, m2;
        scale_min_k4(is, scales, &s1, &m1);
        scale_min_k4(is + 1, scales, &s2, &m2);
        float d1 = d * (float)s1, d2 = d * (float)s2;
        float mm1 = min * (float)m1, mm2 = min * (float)m2;
        for (int l = 0; l < 32; ++l) out[o + l] = d1 * (float)(q[l] & 0xF) - mm1;
        for (int l = 0; l < 32; ++l) out[o + 32 + l] = d2 * (float)(q[l] >> 4) - mm2;
        o += 64;
        q += 32;
        is += 2;
    }
}

void orc_q3k_block(const uint8_t *bytes, float *out) /* dequant.rs:398-451 */
{
    const uint8_t *hm = bytes, *q = bytes + 32, *sc = bytes + 96;
    float d_all = f16_at(bytes + 108);
    uint32_t aux[4];
    for (int i = 0; i < 3; ++i)
        aux[i] = (uint32_t)sc[4 * i] | ((uint32_t)sc[4 * i + 1] << 8) |
                 ((uint32_t)sc[4 * i + 2] << 16) | ((uint32_t)sc[4 * i + 3] << 24);
    const uint32_t K1 = 0x03030303u, K2 = 0x0f0f0f0fu, tmp = aux[2];
    uint32_t na[4];
    na[0] = (aux[0] & K2) | ((tmp & K1) << 4);
    na[1] = (aux[1] & K2) | (((tmp >> 2) & K1) << 4);
    na[2] = ((aux[0] >> 4) & K2) | (((tmp >> 4) & K1) << 4);
    na[3] = ((aux[1] >> 4) & K2) | (((tmp >> 6) & K1) << 4);
    int8_t scales[16];
    for (int i = 0; i < 16; ++i) scales[i] = (int8_t)(uint8_t)(na[i / 4] >> (8 * (i % 4)));
    int o = 0, is = 0;
    uint8_t m = 1;
    for (int n = 0; n < 2; ++n) {
        int shift = 0;
        for (int j = 0; j < 4; ++j) {
            float dl = d_all * ((float)scales[is] - 32.0f);
            ++is;
            for (int l = 0; l < 16; ++l) {
                int8_t bit = (hm[l] & m) ? 0 : 4;
                int8_t qi = (int8_t)((q[l] >> shift) & 3);
                out[o + l] = dl * (float)(int8_t)(qi - bit);
            }
            float dl2 = d_all * ((float)scales[is] - 32.0f);
            ++is;
            for (int l = 0; l < 16; ++l) {
                int8_t bit = (hm[l + 16] & m) ? 0 : 4;
                int8_t qi = (int8_t)((q[l + 16] >> shift) & 3);
                out[o + 16 + l] = dl2 * (float)(int8_t)(qi - bit);
            }
            o += 32;
            shift += 2;
            m = (uint8_t)(m << 1);
        }
        q += 32;
    }
}

void orc_q5k_block(const uint8_t *bytes, float *out) /* dequant.rs:454-481 */
{
    float d = f16_at(bytes), min = f16_at(bytes + 2);
    const uint8_t *sc = bytes + 4, *qh = bytes + 16, *ql = bytes + 48;
    int o = 0, is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < 4; ++j) {
        uint8_t s1, m1, s2, m2;
        scale_min_k4(is, sc, &s1, &m1);
        scale_min_k4(is + 1, sc, &s2, &m2);
        float d1 = d * (float)s1, m1f = min * (float)m1;
        float d2 = d * (float)s2, m2f = min * (float)m2;
        for (int l = 0; l < 32; ++l)
            out[o + l] = d1 * ((float)(ql[l] & 0xF) + ((qh[l] & u1) ? 16.0f : 0.0f)) - m1f;
        for (int l = 0; l < 32; ++l)
            out[o + 32 + l] = d2 * ((float)(ql[l] >> 4) + ((qh[l] & u2) ? 16.0f : 0.0f)) - m2f;
        o += 64;
        ql += 32;
        is += 2;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

void orc_q6k_block(const uint8_t *bytes, float *out) /* dequant.rs:484-510 */
{
    const uint8_t *ql = bytes, *qh = bytes + 128;
    const int8_t *sc = (const int8_t *)(bytes + 192);
    float d = f16_at(bytes + 208);
    int o = 0, qlo = 0, qho = 0, sco = 0;
    for (int n = 0; n < 2; ++n) {
        for (int l = 0; l < 32; ++l) {
            int is = l / 16;
            int h = qh[qho + l];
            int8_t q1 = (int8_t)((int8_t)((ql[qlo + l] & 0xF) | (((h >> 0) & 3) << 4)) - 32);
            int8_t q2 = (int8_t)((int8_t)((ql[qlo + l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32);
            int8_t q3 = (int8_t)((int8_t)((ql[qlo + l] >> 4) | (((h >> 4) & 3) << 4)) - 32);
            int8_t q4 = (int8_t)((int8_t)((ql[qlo + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32);
            out[o + l] = d * (float)sc[sco + is] * (float)q1;
            out[o + l + 32] = d * (float)sc[sco + is + 2] * (float)q2;
            out[o + l + 64] = d * (float)sc[sco + is + 4] * (float)q3;
            out[o + l + 96] = d * (float)sc[sco + is + 6] * (float)q4;
        }
        o += 128;
        qlo += 64;
        qho += 32;
        sco += 8;
    }
}

/* Bytes and elements of one block of a block-quantised kind (QuantKind::
 * block_bytes / block_elems, dequant.rs:350-372); 0 for other kinds. */
static int qblock_geometry(int kind, size_t *bb, size_t *be, void (**fn)(const uint8_t *, float *))
{
    switch (kind) {
    case ORC_KIND_TQ1_0: *bb = 54; *be = 256; *fn = orc_tq1_block; return 1;
    case ORC_KIND_Q8_0: *bb = 34; *be = 32; *fn = orc_q8_block; return 1;
    case ORC_KIND_Q3K: *bb = 110; *be = 256; *fn = orc_q3k_block; return 1;
    case ORC_KIND_Q4K: *bb = 144; *be = 256; *fn = orc_q4k_block; return 1;
    case ORC_KIND_Q5K: *bb = 176; *be = 256; *fn = orc_q5k_block; return 1;
    case ORC_KIND_Q6K: *bb = 210; *be = 256; *fn = orc_q6k_block; return 1;
    default: return 0;
    }
}

/* dequant_{q8,q3k,q4k,q5k,q6k}_row (dequant.rs:285-310, 532-560): the
 * row's whole blocks, row_bytes / block_bytes of them.  -1 for a kind that
 * is not block-quantised. */
int orc_dequant_qblock_row(int kind, const uint8_t *payload, size_t row, size_t row_bytes, float *out)
{
    size_t bb, be;
    void (*fn)(const uint8_t *, float *);
    if (!qblock_geometry(kind, &bb, &be, &fn)) return -1;
    size_t start = row * row_bytes, blocks = row_bytes / bb;
    for (size_t b = 0; b < blocks; ++b) fn(payload + start + b * bb, out + b * be);
    return 0;
}

size_t orc_row_bytes(int kind, size_t k) /* dequant.rs:350-387 */
{
    switch (kind) {
    case ORC_KIND_F32: return k * 4;
    case ORC_KIND_F16:
    case ORC_KIND_BF16: return k * 2;
    case ORC_KIND_TQ1_0: return k / 256 * 54;
    case ORC_KIND_TL1: return (k / 128) * 28;
    case ORC_KIND_Q8_0: return k / 32 * 34;
    case ORC_KIND_Q3K: return k / 256 * 110;
    case ORC_KIND_Q4K: return k / 256 * 144;
    case ORC_KIND_Q5K: return k / 256 * 176;
    case ORC_KIND_Q6K: return k / 256 * 210;
    case ORC_KIND_I2: return k / 4;
    case ORC_KIND_I2_S: return k / 128 * 32; /* codes; one fp32 scale per tensor */
    default: return 0;
    }
}

int orc_kind_supported(uint32_t id) /* dequant.rs:334-348 */
{
    switch (id) {
    case 0: case 1: case 30: case 8: case 11: case 12: case 13: case 14:
    case 34: case 143:
        return 1;
    default:
        return 0;
    }
}

/* ------------------------------------------------------------------------ */
/* ops.rs                                                                    */
/* ------------------------------------------------------------------------ */

float orc_dot(const float *a, const float *b, size_t n) /* ops.rs:53-60 */
{
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}

static inline float tl1_t(uint8_t byte, int n, float d) /* ops.rs:339-340 */
{
    return (float)ptq1_digit_i(byte, n) * d;
}

/* tl1_rows_scalar (ops.rs:324-363). */
static float tl1_row_scalar(const uint8_t *payload, size_t row, size_t gpr,
                            const float *x)
{
    size_t row_base = row * gpr * 28;
    float sum = 0.0f;
    for (size_t g = 0; g < gpr; ++g) {
        const uint8_t *gb = payload + row_base + g * 28;
        float d = orc_f16_to_f32((uint16_t)(gb[26] | (gb[27] << 8)));
        const uint8_t *qs = gb, *qh = gb + 24;
        size_t xb = g * 128;
        for (int n = 0; n < 5; ++n)
            for (int m = 0; m < 16; ++m) sum += tl1_t(qs[m], n, d) * x[xb + n * 16 + m];
        for (int n = 0; n < 5; ++n)
            for (int m = 0; m < 8; ++m) sum += tl1_t(qs[16 + m], n, d) * x[xb + 80 + n * 8 + m];
        for (int n = 0; n < 4; ++n)
            for (int m = 0; m < 2; ++m) sum += tl1_t(qh[m], n, d) * x[xb + 120 + n * 2 + m];
    }
    return sum;
}

/* digits8 + hsum of tl1_rows_avx2 (ops.rs:513-549), real SSE4.1. */
static inline __m128 tl1_digits8(const uint8_t *p, int pn, __m128 d,
                                 const float *xp, __m128 acc)
{
    __m128i b = _mm_loadl_epi64((const __m128i *)p);
    __m128i w = _mm_unpacklo_epi8(b, _mm_setzero_si128());
    __m128i q = _mm_mullo_epi16(w, _mm_set1_epi16((short)pn));
    q = _mm_and_si128(q, _mm_set1_epi16(0xFF));
    q = _mm_mullo_epi16(q, _mm_set1_epi16(3));
    q = _mm_srli_epi16(q, 8);
    q = _mm_sub_epi16(q, _mm_set1_epi16(1));
    __m128 flo = _mm_cvtepi32_ps(_mm_cvtepi16_epi32(q));
    __m128 fhi = _mm_cvtepi32_ps(_mm_cvtepi16_epi32(_mm_unpackhi_epi64(q, q)));
    acc = _mm_add_ps(_mm_mul_ps(_mm_mul_ps(flo, d), _mm_loadu_ps(xp)), acc);
    return _mm_add_ps(_mm_mul_ps(_mm_mul_ps(fhi, d), _mm_loadu_ps(xp + 4)), acc);
}

static inline float tl1_hsum(__m128 v) /* ops.rs:545-549 */
{
    __m128 s = _mm_add_ps(v, _mm_movehl_ps(v, v));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

/* tl1_rows_avx2 (ops.rs:499-584). */
static float tl1_row_sse(const uint8_t *payload, size_t row, size_t gpr,
                         const float *x)
{
    size_t row_base = row * gpr * 28;
    float sum = 0.0f;
    for (size_t g = 0; g < gpr; ++g) {
        const uint8_t *qs = payload + row_base + g * 28;
        float d = orc_f16_to_f32((uint16_t)(qs[26] | (qs[27] << 8)));
        __m128 dv = _mm_set1_ps(d);
        const float *xp = x + g * 128;
        __m128 acc = _mm_setzero_ps();
        for (int n = 0; n < 5; ++n) {
            int pn = PTQ1_POW3[n];
            acc = tl1_digits8(qs + 0, pn, dv, xp + n * 16, acc);
            acc = tl1_digits8(qs + 8, pn, dv, xp + n * 16 + 8, acc);
            acc = tl1_digits8(qs + 16, pn, dv, xp + 80 + n * 8, acc);
        }
        const uint8_t *qh = qs + 24;
        for (int n = 0; n < 4; ++n)
            for (int m = 0; m < 2; ++m) sum += tl1_t(qh[m], n, d) * xp[120 + n * 2 + m];
        sum += tl1_hsum(acc);
    }
    return sum;
}

struct tl1_ctx {
    const uint8_t *payload;
    size_t gpr, in_len, out_len, k;
    const float *x;
    float *y;
    int simd;
};

static void tl1_mv_range(void *p, size_t lo, size_t hi)
{
    struct tl1_ctx *c = (struct tl1_ctx *)p;
    for (size_t r = lo; r < hi; ++r)
        c->y[r] = c->simd ? tl1_row_sse(c->payload, r, c->gpr, c->x)
                          : tl1_row_scalar(c->payload, r, c->gpr, c->x);
}

void orc_matvec_tl1(const uint8_t *payload, size_t out_len, size_t in_len,
                    const float *x, float *y, int simd, int nthreads)
{ /* ops.rs:294-321 */
    struct tl1_ctx c = {payload, in_len / 128, in_len, out_len, 1, x, y, simd};
    orc_parallel_for(out_len, nthreads, tl1_mv_range, &c);
}

/* tl1_rows_scalar_k (ops.rs:244-286): per column the scalar order. */
static void tl1_row_scalar_k(const struct tl1_ctx *c, size_t row, float *sums)
{
    size_t k = c->k;
    for (size_t cc = 0; cc < k; ++cc) sums[cc] = 0.0f;
    size_t row_base = row * c->gpr * 28;
    for (size_t g = 0; g < c->gpr; ++g) {
        const uint8_t *gb = c->payload + row_base + g * 28;
        float d = orc_f16_to_f32((uint16_t)(gb[26] | (gb[27] << 8)));
        const uint8_t *qs = gb, *qh = gb + 24;
        size_t xb = g * 128;
        for (size_t cc = 0; cc < k; ++cc) {
            const float *xc = c->x + cc * c->in_len;
            float acc = sums[cc];
            for (int n = 0; n < 5; ++n) {
                for (int m = 0; m < 16; ++m) acc += tl1_t(qs[m], n, d) * xc[xb + n * 16 + m];
                for (int m = 0; m < 8; ++m) acc += tl1_t(qs[16 + m], n, d) * xc[xb + 80 + n * 8 + m];
            }
            for (int n = 0; n < 4; ++n)
                for (int m = 0; m < 2; ++m) acc += tl1_t(qh[m], n, d) * xc[xb + 120 + n * 2 + m];
            sums[cc] = acc;
        }
    }
}

/* tl1_rows_avx2_k (ops.rs:381-473): two 4-lane accumulators per column that
 * persist over the whole row, scalar qh tail added straight into the output,
 * then hsum(lo) + hsum(hi). */
static void tl1_row_sse_k(const struct tl1_ctx *c, size_t row, float *out)
{
    size_t k = c->k;
    __m128 *acc = (__m128 *)aligned_alloc(16, sizeof(__m128) * 2 * k);
    for (size_t i = 0; i < 2 * k; ++i) acc[i] = _mm_setzero_ps();
    for (size_t cc = 0; cc < k; ++cc) out[cc] = 0.0f;
    size_t row_base = row * c->gpr * 28;
    for (size_t g = 0; g < c->gpr; ++g) {
        const uint8_t *qs = c->payload + row_base + g * 28;
        float d = orc_f16_to_f32((uint16_t)(qs[26] | (qs[27] << 8)));
        __m128 dv = _mm_set1_ps(d);
        size_t xg = g * 128;
        for (int n = 0; n < 5; ++n) {
            __m128 lo[3], hi[3];
            for (int s = 0; s < 3; ++s) {
                __m128i b = _mm_loadl_epi64((const __m128i *)(qs + 8 * s));
                __m128i w = _mm_unpacklo_epi8(b, _mm_setzero_si128());
                __m128i q = _mm_mullo_epi16(w, _mm_set1_epi16((short)PTQ1_POW3[n]));
                q = _mm_and_si128(q, _mm_set1_epi16(0xFF));
                q = _mm_mullo_epi16(q, _mm_set1_epi16(3));
                q = _mm_srli_epi16(q, 8);
                q = _mm_sub_epi16(q, _mm_set1_epi16(1));
                lo[s] = _mm_cvtepi32_ps(_mm_cvtepi16_epi32(q));
                hi[s] = _mm_cvtepi32_ps(_mm_cvtepi16_epi32(_mm_unpackhi_epi64(q, q)));
            }
            for (size_t cc = 0; cc < k; ++cc) {
                const float *xp = c->x + cc * c->in_len + xg;
                acc[2 * cc] = _mm_add_ps(_mm_mul_ps(_mm_mul_ps(lo[0], dv), _mm_loadu_ps(xp + n * 16)), acc[2 * cc]);
                acc[2 * cc + 1] = _mm_add_ps(_mm_mul_ps(_mm_mul_ps(hi[0], dv), _mm_loadu_ps(xp + n * 16 + 4)), acc[2 * cc + 1]);
                acc[2 * cc] = _mm_add_ps(_mm_mul_ps(_mm_mul_ps(lo[1], dv), _mm_loadu_ps(xp + n * 16 + 8)), acc[2 * cc]);
                acc[2 * cc + 1] = _mm_add_ps(_mm_mul_ps(_mm_mul_ps(hi[1], dv), _mm_loadu_ps(xp + n * 16 + 12)), acc[2 * cc + 1]);
                acc[2 * cc] = _mm_add_ps(_mm_mul_ps(_mm_mul_ps(lo[2], dv), _mm_loadu_ps(xp + 80 + n * 8)), acc[2 * cc]);
                acc[2 * cc + 1] = _mm_add_ps(_mm_mul_ps(_mm_mul_ps(hi[2], dv), _mm_loadu_ps(xp + 80 + n * 8 + 4)), acc[2 * cc + 1]);
            }
        }
        const uint8_t *qh = qs + 24;
        for (int n = 0; n < 4; ++n)
            for (int m = 0; m < 2; ++m) {
                float t = tl1_t(qh[m], n, d);
                for (size_t cc = 0; cc < k; ++cc)
                    out[cc] += t * c->x[cc * c->in_len + xg + 120 + n * 2 + m];
            }
    }
    for (size_t cc = 0; cc < k; ++cc)
        out[cc] += tl1_hsum(acc[2 * cc]) + tl1_hsum(acc[2 * cc + 1]);
    free(acc);
}

static void tl1_mm_range(void *p, size_t lo, size_t hi)
{
    struct tl1_ctx *c = (struct tl1_ctx *)p;
    float *tmp = (float *)malloc(sizeof(float) * c->k);
    for (size_t r = lo; r < hi; ++r) {
        if (c->simd)
            tl1_row_sse_k(c, r, tmp);
        else
            tl1_row_scalar_k(c, r, tmp);
        for (size_t cc = 0; cc < c->k; ++cc) c->y[cc * c->out_len + r] = tmp[cc];
    }
    free(tmp);
}

void orc_matmul_tl1(const uint8_t *payload, size_t out_len, size_t in_len,
                    const float *x, size_t k, float *y, int simd, int nthreads)
{ /* ops.rs:162-215 */
    struct tl1_ctx c = {payload, in_len / 128, in_len, out_len, k, x, y, simd};
    orc_parallel_for(out_len, nthreads, tl1_mm_range, &c);
}

struct qblock_ctx {
    const uint8_t *payload;
    int kind;
    size_t in_len, rb;
    const float *x;
    float *y;
};

/* matvec_qblock's worker (ops.rs:104-124): a zeroed row of in_len floats per
 * worker, the row's blocks decoded into it, then dot with x. */
static void qblock_range(void *p, size_t lo, size_t hi)
{
    struct qblock_ctx *c = (struct qblock_ctx *)p;
    float *row = (float *)calloc(c->in_len ? c->in_len : 1, sizeof(float));
    for (size_t r = lo; r < hi; ++r) {
        orc_dequant_qblock_row(c->kind, c->payload, r, c->rb, row);
        c->y[r] = orc_dot(row, c->x, c->in_len);
    }
    free(row);
}

int orc_matvec_qblock(const uint8_t *payload, int kind, size_t out_len, size_t in_len,
                      const float *x, float *y, int nthreads)
{ /* ops.rs:101-128 */
    size_t bb, be;
    void (*fn)(const uint8_t *, float *);
    if (!qblock_geometry(kind, &bb, &be, &fn)) return -1;
    struct qblock_ctx c = {payload, kind, in_len, orc_row_bytes(kind, in_len), x, y};
    orc_parallel_for(out_len, nthreads, qblock_range, &c);
    return 0;
}

void orc_matvec_tq1(const uint8_t *payload, size_t out_len, size_t in_len,
                    const float *x, float *y, int nthreads)
{ /* ops.rs:101-128 */
    orc_matvec_qblock(payload, ORC_KIND_TQ1_0, out_len, in_len, x, y, nthreads);
}

void orc_matvec_dense(const uint8_t *payload, int kind, size_t out_len,
                      size_t in_len, const float *x, float *y)
{ /* ops.rs:87-98 (f32), 131-154 (f16), 600-623 (bf16) */
    for (size_t o = 0; o < out_len; ++o) {
        float s = 0.0f;
        for (size_t i = 0; i < in_len; ++i) {
            float w;
            if (kind == ORC_KIND_F32) {
                uint32_t u;
                memcpy(&u, payload + (o * in_len + i) * 4, 4);
                w = bits_f32(u);
            } else {
                const uint8_t *b = payload + (o * in_len + i) * 2;
                uint16_t bits = (uint16_t)(b[0] | (b[1] << 8));
                w = kind == ORC_KIND_F16 ? orc_f16_to_f32(bits) : orc_bf16_to_f32(bits);
            }
            s += w * x[i];
        }
        y[o] = s;
    }
}

int orc_matvec_q(const uint8_t *payload, int kind, size_t out_len,
                 size_t in_len, const float *x, float *y, int nthreads)
{ /* ops.rs:76-84 */
    switch (kind) {
    case ORC_KIND_F16:
    case ORC_KIND_BF16:
    case ORC_KIND_F32:
        orc_matvec_dense(payload, kind, out_len, in_len, x, y);
        return 0;
    case ORC_KIND_TL1:
        orc_matvec_tl1(payload, out_len, in_len, x, y, 1, nthreads);
        return 0;
    case ORC_KIND_TQ1_0:
    case ORC_KIND_Q8_0:
    case ORC_KIND_Q3K:
    case ORC_KIND_Q4K:
    case ORC_KIND_Q5K:
    case ORC_KIND_Q6K:
        return orc_matvec_qblock(payload, kind, out_len, in_len, x, y, nthreads);
    case ORC_KIND_I2_S: { /* x quantised by quantize_row_i8_s, then the I2_S mul_mat */
        if ((out_len * in_len) % 128) return -1;
        int8_t *q = (int8_t *)malloc(in_len ? in_len : 1);
        if (!q) return -1;
        float s;
        orc_quantize_row_i8_s(x, in_len, q, &s, NULL);
        orc_gemm_i2s(payload, out_len, in_len, q, &s, 1, NULL, y, nthreads);
        free(q);
        return 0;
    }
    default:
        return -1;
    }
}

int orc_matmul_q(const uint8_t *payload, int kind, size_t out_len,
                 size_t in_len, const float *x, size_t k, float *y,
                 int nthreads)
{ /* ops.rs:219-230 */
    if (kind == ORC_KIND_TL1) {
        orc_matmul_tl1(payload, out_len, in_len, x, k, y, 1, nthreads);
        return 0;
    }
    for (size_t c = 0; c < k; ++c)
        if (orc_matvec_q(payload, kind, out_len, in_len, x + c * in_len,
                         y + c * out_len, nthreads) != 0)
            return -1;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* This library's canonical 2-bit layout (a repack of the I2_S codes).       */
/* ------------------------------------------------------------------------ */

int orc_i2_pack(const int8_t *w, size_t out_len, size_t in_len, uint8_t *packed)
{
    if (in_len % 4) return -1;
    size_t rb = in_len / 4;
    for (size_t r = 0; r < out_len; ++r)
        for (size_t b = 0; b < rb; ++b) {
            uint8_t byte = 0;
            for (int f = 0; f < 4; ++f) {
                int v = w[r * in_len + b * 4 + f];
                if (v < -1 || v > 1) return -1;
                byte |= (uint8_t)((v + 1) << (2 * f));
            }
            packed[r * rb + b] = byte;
        }
    return 0;
}

void orc_i2_unpack(const uint8_t *packed, size_t out_len, size_t in_len,
                   int8_t *w)
{
    size_t rb = in_len / 4;
    for (size_t r = 0; r < out_len; ++r)
        for (size_t k = 0; k < in_len; ++k)
            w[r * in_len + k] =
                (int8_t)(((packed[r * rb + k / 4] >> (2 * (k % 4))) & 3) - 1);
}

size_t orc_i2_tiled_bytes(size_t out_len, size_t in_len)
{
    if (in_len == 0 || in_len % 256) return 0;
    return (out_len + 7) / 8 * 8 * (in_len / 4);
}

size_t orc_i2_tile(const uint8_t *canonical, size_t out_len, size_t in_len,
                   uint8_t *tiled)
{
    size_t bytes = orc_i2_tiled_bytes(out_len, in_len);
    if (!bytes) return 0;
    const size_t R = 8, G = in_len / 256, rb = in_len / 4;
    const size_t unit = G % 2 ? 8 : 16, wu = unit / 4;
    const size_t n4 = G / 4 * 4, n2 = n4 + (G % 4 >= 2 ? 2 : 0);
    size_t tiles = (out_len + R - 1) / R, tile_bytes = R * rb;
    for (size_t t = 0; t < tiles; ++t)
        for (size_t lane = 0; lane < 64; ++lane)
            for (size_t d = 0; d < R * G / 4; ++d) {
                uint32_t word = 0;
                for (int f = 0; f < 4; ++f) {
                    size_t gi = 4 * d + (size_t)f, r = gi / G, g = gi % G;
                    size_t row = t * R + r;
                    /* chunk of local group g: start o, size sz */
                    size_t o = g < n4 ? g / 4 * 4 : (g < n2 ? n4 : G - 1);
                    size_t sz = g < n4 ? 4 : (g < n2 ? 2 : 1);
                    size_t kg = 64 * o + sz * lane + (g - o);
                    uint8_t byte = row < out_len ? canonical[row * rb + kg] : 0x55;
                    for (int b = 0; b < 4; ++b)
                        word |= (uint32_t)((byte >> (2 * b)) & 3u) << (8 * b + 2 * f);
                }
                size_t off = t * tile_bytes + (d / wu) * 64 * unit + lane * unit + (d % wu) * 4;
                memcpy(tiled + off, &word, 4);
            }
    return bytes;
}

size_t orc_i2_mfma_bytes(size_t out_len, size_t in_len)
{
    if (in_len == 0 || in_len % 256) return 0;
    return (out_len + 15) / 16 * (in_len / 256) * 1024;
}

size_t orc_i2_tile_mfma(const uint8_t *canonical, size_t out_len, size_t in_len,
                        uint8_t *dst)
{
    size_t bytes = orc_i2_mfma_bytes(out_len, in_len);
    if (!bytes) return 0;
    const size_t nkb = in_len / 256, rb = in_len / 4, tiles = (out_len + 15) / 16;
    for (size_t rt = 0; rt < tiles; ++rt)
        for (size_t kb = 0; kb < nkb; ++kb)
            for (size_t l = 0; l < 64; ++l)
                for (size_t s = 0; s < 4; ++s) {
                    uint32_t word = 0;
                    size_t row = rt * 16 + l % 16;
                    for (size_t j = 0; j < 4; ++j)
                        for (size_t i = 0; i < 4; ++i) {
                            size_t k = 256 * kb + 64 * s + 16 * (l / 16) + 4 * j + i;
                            uint32_t code = row < out_len ? (canonical[row * rb + k / 4] >> (2 * (k % 4))) & 3u : 1u;
                            word |= ((1u - code) & 3u) << (8 * i + 2 * j);
                        }
                    memcpy(dst + ((rt * nkb + kb) * 64 + l) * 16 + 4 * s, &word, 4);
                }
    return bytes;
}

/* ---- bitnet.cpp I2_S / I8_S (src/ggml-bitnet-mad.cpp) ------------------ */

size_t orc_i2s_bytes(size_t nrow, size_t n_per_row)
{
    return nrow * n_per_row / 4 + 32;
}

int orc_quantize_i2_s(const float *src, size_t nrow, size_t n_per_row,
                      uint8_t *dst)
{ /* quantize_i2_s */
    const size_t n = nrow * n_per_row;
    if (n % 128) return -1;
    double max = 0;
    for (size_t i = 0; i < n; ++i) max = fmax(max, fabs((double)src[i]));
    const double i2_scale = max;
    memset(dst, 0, orc_i2s_bytes(nrow, n_per_row));
    for (size_t i = 0; i < n / 128; ++i)
        for (size_t j = 0; j < 128; ++j) {
            const float v = src[i * 128 + j];
            uint8_t q8;
            if (fabs((double)v) < 1e-6)
                q8 = 1;
            else
                q8 = (double)v * i2_scale > 0 ? 2 : 0;
            dst[i * 32 + j % 32] |= (uint8_t)(q8 << (6 - 2 * (j / 32)));
        }
    const float s = (float)i2_scale;
    memcpy(dst + n / 4, &s, 4);
    return 0;
}

int orc_i2s_pack(const int8_t *w, size_t nrow, size_t n_per_row,
                 float w_scale, uint8_t *dst)
{
    const size_t n = nrow * n_per_row;
    if (n % 128 || !(w_scale > 0)) return -1;
    float *src = (float *)malloc(n * sizeof(float));
    if (!src) return -1;
    int bad = 0;
    for (size_t i = 0; i < n; ++i) {
        if (w[i] < -1 || w[i] > 1) bad = 1;
        src[i] = (float)w[i] * w_scale;
    }
    int st = bad ? -1 : orc_quantize_i2_s(src, nrow, n_per_row, dst);
    free(src);
    return st;
}

int orc_i2s_code(const uint8_t *i2s, size_t n_per_row, size_t r, size_t k)
{
    const size_t e = r * n_per_row + k, i = e / 128, j = e % 128;
    return (i2s[i * 32 + j % 32] >> (6 - 2 * (j / 32))) & 3;
}

float orc_i2s_scale(const uint8_t *i2s, size_t nrow, size_t n_per_row)
{
    float s;
    memcpy(&s, i2s + nrow * n_per_row / 4, 4);
    return s;
}

void orc_quantize_row_i8_s(const float *x, size_t n, int8_t *q,
                           float *act_scale, int32_t *act_sum)
{ /* quantize_row_i8_s */
    double max = 0.00001;
    for (size_t i = 0; i < n; ++i) max = fmax(max, fabs((double)x[i]));
    const float s = (float)(127 / max);
    int32_t sum = 0;
    for (size_t i = 0; i < n; ++i) {
        float t = (float)round((double)(x[i] * s));
        if (t > 127) t = 127;
        if (t < -128) t = -128;
        q[i] = (int8_t)t;
        sum += q[i];
    }
    *act_scale = s;
    if (act_sum) *act_sum = sum;
}

void orc_act_quant_i8(const float *x, size_t rows, size_t n, int8_t *q,
                      float *act_scale)
{
    for (size_t r = 0; r < rows; ++r)
        orc_quantize_row_i8_s(x + r * n, n, q + r * n, act_scale + r, NULL);
}

int32_t orc_vec_dot_i2_i8_s(const uint8_t *i2s, size_t n_per_row, size_t r,
                            const int8_t *q)
{ /* ggml_vec_dot_i2_i8_s: codes (0..2) times int8, summed exactly */
    int32_t sumi = 0;
    for (size_t k = 0; k < n_per_row; ++k)
        sumi += orc_i2s_code(i2s, n_per_row, r, k) * (int32_t)q[k];
    return sumi;
}

struct i2s_ctx {
    const uint8_t *i2s;
    size_t out_len, in_len, ncols;
    const int8_t *xq;
    const float *act_scale;
    const int32_t *act_sum;
    float scale;
    int32_t *acc;
    float *y;
};

static void i2s_range(void *p, size_t lo, size_t hi)
{
    struct i2s_ctx *c = (struct i2s_ctx *)p;
    for (size_t r = lo; r < hi; ++r)
        for (size_t col = 0; col < c->ncols; ++col) {
            const int32_t sumi = orc_vec_dot_i2_i8_s(c->i2s, c->in_len, r, c->xq + col * c->in_len);
            float t = (float)sumi;
            t = t - (float)c->act_sum[col];
            t = t / c->act_scale[col];
            t = t * c->scale;
            c->y[col * c->out_len + r] = t;
            if (c->acc) c->acc[col * c->out_len + r] = sumi - c->act_sum[col];
        }
}

void orc_gemm_i2s(const uint8_t *i2s, size_t out_len, size_t in_len,
                  const int8_t *xq, const float *act_scale, size_t ncols,
                  int32_t *acc, float *y, int nthreads)
{ /* the I2_S branch of the ggml fork's mul_mat: quantized rows times codes */
    int32_t *sums = (int32_t *)malloc((ncols ? ncols : 1) * sizeof(int32_t));
    if (!sums) return;
    for (size_t col = 0; col < ncols; ++col) {
        int32_t s = 0;
        for (size_t k = 0; k < in_len; ++k) s += xq[col * in_len + k];
        sums[col] = s;
    }
    struct i2s_ctx c = {i2s, out_len, in_len, ncols, xq, act_scale, sums,
                        orc_i2s_scale(i2s, out_len, in_len), acc, y};
    orc_parallel_for(out_len, nthreads, i2s_range, &c);
    free(sums);
}

int orc_i2s_to_canonical(const uint8_t *i2s, size_t out_len, size_t in_len,
                         uint8_t *canonical)
{
    if (in_len % 4 || (out_len * in_len) % 128) return -1;
    const size_t rb = in_len / 4;
    for (size_t r = 0; r < out_len; ++r)
        for (size_t b = 0; b < rb; ++b) {
            uint8_t byte = 0;
            for (size_t f = 0; f < 4; ++f)
                byte |= (uint8_t)(orc_i2s_code(i2s, in_len, r, 4 * b + f) << (2 * f));
            canonical[r * rb + b] = byte;
        }
    return 0;
}

struct i2_ctx {
    const uint8_t *packed;
    size_t out_len, in_len, ncols;
    const int8_t *xq;
    const float *act_scale;
    float w_scale;
    int32_t *acc;
    float *y;
};

static void i2_range(void *p, size_t lo, size_t hi)
{
    struct i2_ctx *c = (struct i2_ctx *)p;
    size_t rb = c->in_len / 4;
    for (size_t r = lo; r < hi; ++r) {
        const uint8_t *row = c->packed + r * rb;
        for (size_t col = 0; col < c->ncols; ++col) {
            const int8_t *x = c->xq + col * c->in_len;
            int32_t a = 0;
            for (size_t k = 0; k < c->in_len; ++k)
                a += (((row[k / 4] >> (2 * (k % 4))) & 3) - 1) * (int32_t)x[k];
            if (c->acc) c->acc[col * c->out_len + r] = a;
            float t = (float)a / c->act_scale[col];
            c->y[col * c->out_len + r] = t * c->w_scale;
        }
    }
}

void orc_gemm_i2(const uint8_t *packed, size_t out_len, size_t in_len,
                 const int8_t *xq, const float *act_scale, size_t ncols,
                 float w_scale, int32_t *acc, float *y, int nthreads)
{
    struct i2_ctx c = {packed, out_len, in_len, ncols, xq, act_scale, w_scale, acc, y};
    orc_parallel_for(out_len, nthreads, i2_range, &c);
}

/* ------------------------------------------------------------------------ */
/* hadamard.rs                                                               */
/* ------------------------------------------------------------------------ */

void orc_wht_inplace(float *x, size_t n) /* hadamard.rs:15-31 */
{
    for (size_t h = 1; h < n; h *= 2)
        for (size_t c = 0; c < n; c += 2 * h)
            for (size_t i = c; i < c + h; ++i) {
                float a = x[i], b = x[i + h];
                x[i] = a + b;
                x[i + h] = a - b;
            }
}

static int check_args(size_t n, size_t block) /* hadamard.rs:33-37 */
{
    if (block == 0 || (block & (block - 1))) return -1;
    if (n % block) return -1;
    return 0;
}

int orc_rotate_fwd(float *x, const float *signs, size_t n, size_t block)
{ /* hadamard.rs:41-53 */
    if (check_args(n, block)) return -1;
    float scale = 1.0f / sqrtf((float)block);
    for (size_t i = 0; i < n; ++i) x[i] *= signs[i];
    for (size_t b = 0; b < n; b += block) orc_wht_inplace(x + b, block);
    for (size_t i = 0; i < n; ++i) x[i] *= scale;
    return 0;
}

int orc_rotate_inv(float *x, const float *signs, size_t n, size_t block)
{ /* hadamard.rs:57-66 */
    if (check_args(n, block)) return -1;
    float scale = 1.0f / sqrtf((float)block);
    for (size_t b = 0; b < n; b += block) orc_wht_inplace(x + b, block);
    for (size_t i = 0; i < n; ++i) x[i] *= signs[i] * scale;
    return 0;
}

struct rot_ctx {
    float *x;
    const float *signs;
    size_t n, block;
    int inverse;
};

static void rot_range(void *p, size_t lo, size_t hi)
{
    struct rot_ctx *c = (struct rot_ctx *)p;
    for (size_t r = lo; r < hi; ++r) {
        if (c->inverse)
            orc_rotate_inv(c->x + r * c->n, c->signs, c->n, c->block);
        else
            orc_rotate_fwd(c->x + r * c->n, c->signs, c->n, c->block);
    }
}

int orc_rotate_rows(float *x, const float *signs, size_t rows, size_t n,
                    size_t block, int inverse, int nthreads)
{
    if (check_args(n, block)) return -1;
    struct rot_ctx c = {x, signs, n, block, inverse};
    orc_parallel_for(rows, nthreads, rot_range, &c);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* qwen35.rs                                                                 */
/* ------------------------------------------------------------------------ */

void orc_delta_head_dim(float *state, size_t sdim, const float *q,
                        const float *k, const float *v, float gate, float beta,
                        float *out)
{ /* qwen35.rs:27-57 */
    float decay = expf(gate);
    float sk[512];
    float *skp = sdim <= 512 ? sk : (float *)malloc(sizeof(float) * sdim);
    for (size_t j = 0; j < sdim; ++j) {
        float acc = 0.0f;
        for (size_t i = 0; i < sdim; ++i) acc += state[i + j * sdim] * k[i];
        skp[j] = acc * decay;
    }
    for (size_t j = 0; j < sdim; ++j) {
        float dj = beta * (v[j] - skp[j]);
        for (size_t i = 0; i < sdim; ++i)
            state[i + j * sdim] = state[i + j * sdim] * decay + k[i] * dj;
    }
    for (size_t j = 0; j < sdim; ++j) {
        float acc = 0.0f;
        for (size_t i = 0; i < sdim; ++i) acc += state[i + j * sdim] * q[i];
        out[j] = acc;
    }
    if (skp != sk) free(skp);
}

void orc_l2_norm(float *v, size_t n, float eps) /* qwen35.rs:73-79 */
{
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) sum += v[i] * v[i];
    float inv = 1.0f / (sqrtf(sum) + eps);
    for (size_t i = 0; i < n; ++i) v[i] *= inv;
}

float orc_softplus(float x) /* qwen35.rs:1241-1243 */
{
    return x > 20.0f ? x : logf(1.0f + expf(x));
}

float orc_sigmoid(float x) /* qwen35.rs:1067 */
{
    return 1.0f / (1.0f + expf(-x));
}

float orc_silu(float x) /* ops.rs:34-36 */
{
    return x / (1.0f + expf(-x));
}

float orc_conv_step(float ring[3], const float w[4], float x) /* qwen35.rs:64-70 */
{
    float y = w[0] * ring[0] + w[1] * ring[1] + w[2] * ring[2] + w[3] * x;
    ring[0] = ring[1];
    ring[1] = ring[2];
    ring[2] = x;
    return y;
}

void orc_gated_norm_rms(const float *x, const float *w, const float *gate,
                        size_t n, float eps, float *y)
{ /* qwen35.rs:82-92 */
    float ms = 0.0f;
    for (size_t i = 0; i < n; ++i) ms += x[i] * x[i];
    ms = ms / (float)n;
    float inv = 1.0f / sqrtf(ms + eps);
    for (size_t i = 0; i < n; ++i) {
        float g = gate[i] / (1.0f + expf(-gate[i]));
        y[i] = x[i] * inv * w[i] * g;
    }
}

float orc_delta_q_scale(size_t d) /* qwen35.rs:108-110 */
{
    return 1.0f / sqrtf((float)d);
}

/* One (sequence, v-head) of run_delta's per-head loop (qwen35.rs:1096-1112). */
static void gdn_one_head(float *st, const float *qh_raw, const float *kh_raw,
                         const float *vh, float gate, float beta, float *out,
                         size_t d, unsigned flags, float eps)
{
    float qb[512], kb[512];
    float *qh = d <= 512 ? qb : (float *)malloc(sizeof(float) * d);
    float *kh = d <= 512 ? kb : (float *)malloc(sizeof(float) * d);
    memcpy(qh, qh_raw, sizeof(float) * d);
    memcpy(kh, kh_raw, sizeof(float) * d);
    if (flags & ORC_GDN_L2NORM_QK) {
        orc_l2_norm(qh, d, eps);
        orc_l2_norm(kh, d, eps);
    }
    if (flags & ORC_GDN_SCALE_Q) {
        float scale = 1.0f / sqrtf((float)d);
        for (size_t i = 0; i < d; ++i) qh[i] = qh[i] * scale;
    }
    orc_delta_head_dim(st, d, qh, kh, vh, gate, beta, out);
    if (qh != qb) free(qh);
    if (kh != kb) free(kh);
}

static size_t gdn_khead(size_t vh, size_t Hk, size_t Hv, unsigned flags)
{
    return (flags & ORC_GDN_KHEAD_DIV) ? vh / (Hv / Hk) : vh % Hk;
}

struct gdn_ctx {
    float *state;
    const float *q, *k, *v, *gate, *beta;
    float *out;
    size_t B, Hk, Hv, d, T;
    unsigned flags;
    float eps;
};

static void gdn_decode_range(void *p, size_t lo, size_t hi)
{
    struct gdn_ctx *c = (struct gdn_ctx *)p;
    size_t d = c->d;
    for (size_t bh = lo; bh < hi; ++bh) {
        size_t b = bh / c->Hv, h = bh % c->Hv;
        size_t kh = gdn_khead(h, c->Hk, c->Hv, c->flags);
        gdn_one_head(c->state + bh * d * d, c->q + (b * c->Hk + kh) * d,
                     c->k + (b * c->Hk + kh) * d, c->v + bh * d, c->gate[bh],
                     c->beta[bh], c->out + bh * d, d, c->flags, c->eps);
    }
}

void orc_gdn_decode(float *state, const float *q, const float *k,
                    const float *v, const float *gate, const float *beta,
                    float *out, size_t B, size_t Hk, size_t Hv, size_t d,
                    unsigned flags, float eps, int nthreads)
{
    struct gdn_ctx c = {state, q, k, v, gate, beta, out, B, Hk, Hv, d, 1, flags, eps};
    orc_parallel_for(B * Hv, nthreads, gdn_decode_range, &c);
}

static void gdn_prefill_range(void *p, size_t lo, size_t hi)
{
    struct gdn_ctx *c = (struct gdn_ctx *)p;
    size_t d = c->d;
    for (size_t h = lo; h < hi; ++h) {
        size_t kh = gdn_khead(h, c->Hk, c->Hv, c->flags);
        for (size_t t = 0; t < c->T; ++t) {
            size_t th = t * c->Hv + h;
            gdn_one_head(c->state + h * d * d, c->q + (t * c->Hk + kh) * d,
                         c->k + (t * c->Hk + kh) * d, c->v + th * d, c->gate[th],
                         c->beta[th], c->out + th * d, d, c->flags, c->eps);
        }
    }
}

void orc_gdn_prefill_tokens(float *state, const float *q, const float *k,
                            const float *v, const float *gate,
                            const float *beta, float *out, size_t T,
                            size_t Hk, size_t Hv, size_t d, unsigned flags,
                            float eps, int nthreads)
{
    struct gdn_ctx c = {state, q, k, v, gate, beta, out, 1, Hk, Hv, d, T, flags, eps};
    orc_parallel_for(Hv, nthreads, gdn_prefill_range, &c);
}

struct gdn_varlen_ctx {
    struct gdn_ctx base;
    const int32_t *cu;
};

static void gdn_varlen_range(void *p, size_t lo, size_t hi)
{
    struct gdn_varlen_ctx *c = (struct gdn_varlen_ctx *)p;
    const size_t d = c->base.d, Hv = c->base.Hv, Hk = c->base.Hk;
    for (size_t sh = lo; sh < hi; ++sh) {
        const size_t s = sh / Hv, h = sh % Hv;
        const size_t kh = gdn_khead(h, Hk, Hv, c->base.flags);
        for (size_t t = (size_t)c->cu[s]; t < (size_t)c->cu[s + 1]; ++t) {
            const size_t th = t * Hv + h;
            gdn_one_head(c->base.state + sh * d * d, c->base.q + (t * Hk + kh) * d,
                         c->base.k + (t * Hk + kh) * d, c->base.v + th * d, c->base.gate[th],
                         c->base.beta[th], c->base.out + th * d, d, c->base.flags, c->base.eps);
        }
    }
}

void orc_gdn_prefill_varlen(float *state, const float *q, const float *k,
                            const float *v, const float *gate,
                            const float *beta, float *out,
                            const int32_t *cu_seqlens, size_t N, size_t Hk,
                            size_t Hv, size_t d, unsigned flags, float eps,
                            int nthreads)
{ /* the reference prefill (shell/src/bonsai.rs:48-52): each sequence token by
     token through the recurrence, (sequence, v-head) pairs over threads */
    struct gdn_varlen_ctx c = {{state, q, k, v, gate, beta, out, 1, Hk, Hv, d, 0, flags, eps}, cu_seqlens};
    orc_parallel_for(N * Hv, nthreads, gdn_varlen_range, &c);
}

/* ---- run_delta's layer block (qwen35.rs:1066-1140) ---------------------- */

struct layer_ctx {
    const float *qkv, *z, *beta_raw, *alpha_raw, *dt_bias, *a_log, *conv_w, *norm_w;
    float *conv, *state, *out;
    size_t Hk, Hv, d;
    unsigned flags;
    float eps;
};

static void layer_range(void *p, size_t lo, size_t hi)
{
    struct layer_ctx *c = (struct layer_ctx *)p;
    const size_t d = c->d, Hk = c->Hk, Hv = c->Hv;
    const size_t di = Hk * d, ch = 2 * di + Hv * d;
    float *conv_out = (float *)malloc(sizeof(float) * ch);
    float *o = (float *)malloc(sizeof(float) * Hv * d);
    float *y = (float *)malloc(sizeof(float) * d);
    for (size_t b = lo; b < hi; ++b) {
        const float *qkv = c->qkv + b * ch;
        float *ring = c->conv + b * ch * 3;
        for (size_t i = 0; i < ch; ++i) /* qwen35.rs:1080-1088 */
            conv_out[i] = orc_silu(orc_conv_step(ring + 3 * i, c->conv_w + 4 * i, qkv[i]));
        for (size_t h = 0; h < Hv; ++h) { /* qwen35.rs:1096-1112 */
            const float beta = orc_sigmoid(c->beta_raw[b * Hv + h]);
            const float gate = c->a_log[h] * orc_softplus(c->alpha_raw[b * Hv + h] + c->dt_bias[h]);
            const size_t kh = gdn_khead(h, Hk, Hv, c->flags);
            gdn_one_head(c->state + (b * Hv + h) * d * d, conv_out + kh * d, conv_out + di + kh * d,
                         conv_out + 2 * di + h * d, gate, beta, o + h * d, d,
                         ORC_GDN_L2NORM_QK | ORC_GDN_SCALE_Q, c->eps);
        }
        for (size_t h = 0; h < Hv; ++h) { /* qwen35.rs:1119-1138 */
            orc_gated_norm_rms(o + h * d, c->norm_w, c->z + b * Hv * d + h * d, d, c->eps, y);
            size_t dst = h;
            if (c->flags & ORC_GDN_V_GROUPED) {
                const size_t rep = Hv / Hk, k = h % Hk, r = h / Hk;
                dst = k * rep + r;
            }
            memcpy(c->out + b * Hv * d + dst * d, y, sizeof(float) * d);
        }
    }
    free(conv_out);
    free(o);
    free(y);
}

void orc_gdn_layer_decode(const float *qkv, const float *z,
                          const float *beta_raw, const float *alpha_raw,
                          const float *dt_bias, const float *a_log,
                          const float *conv_w, const float *norm_w,
                          float *conv, float *state, float *out, size_t B,
                          size_t Hk, size_t Hv, size_t d, unsigned flags,
                          float eps, int nthreads)
{
    struct layer_ctx c = {qkv, z, beta_raw, alpha_raw, dt_bias, a_log, conv_w, norm_w,
                          conv, state, out, Hk, Hv, d, flags, eps};
    orc_parallel_for(B, nthreads, layer_range, &c);
}

size_t orc_finite_argmax(const float *l, size_t n) /* infer/mod.rs:70-83 */
{
    size_t best = 0;
    int found = 0;
    for (size_t i = 0; i < n; ++i) {
        float v = l[i];
        if (v != v) continue;
        if (!found || v > l[best]) {
            best = i;
            found = 1;
        }
    }
    return best;
}
