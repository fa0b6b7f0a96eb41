/* Host check of the quotient the GEMM epilogues form from a per-row
 * reciprocal (i8s_inv / i8s_out_inv in ouroboros_amd/csrc/common.hpp): it
 * must equal bitnet.cpp's float division a / s bit for bit, for every
 * integer accumulator |a| <= 2^20 and activation scales
 * s = 127 / max(amax, 1e-5) with amax log-uniform over [1e-5, 3.4e38],
 * arbitrary positive floats in [127 / FLT_MAX, 1.3e7] by bit pattern, and
 * s = 0 (amax = inf).
 * Usage: i8s_quotient_check [scales] ; prints "checked N mismatches M". */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint32_t bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static uint64_t state = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return state;
}

/* The device's steps, in the same order and roundings. */
typedef struct {
    float s, inv, post;
    int zero;
} I8sInv;
static I8sInv i8s_inv(float s) {
    I8sInv r;
    const int small = s < 0x1p-76f;
    r.s = small ? s * 0x1p64f : s;
    r.inv = 1.0f / r.s;
    r.post = small ? 0x1p64f : 1.0f;
    r.zero = s == 0.0f;
    return r;
}
static float quotient(int acc, I8sInv d) {
    const float a = (float)acc;
    const float q = a * d.inv;
    const float r = fmaf(-q, d.s, a);
    return d.zero ? q : fmaf(r, d.inv, q) * d.post;
}

int main(int argc, char **argv) {
    const int ns = argc > 1 ? atoi(argv[1]) : 200;
    long long bad = 0, checked = 0;
    for (int i = 0; i <= ns; ++i) {
        float s;
        if (i == ns) {
            s = 0.0f;
        } else if (i % 4 == 0) {
            const double e = -5.0 + 43.5 * (double)(next() >> 11) / 9007199254740992.0;
            const float amax = (float)fmin(pow(10.0, e), FLT_MAX);
            s = (float)(127.0 / fmax(1e-5, (double)amax));
        } else {
            const uint32_t lo = bits(127.0f / FLT_MAX), hi = bits(1.3e7f);
            const uint32_t u = lo + (uint32_t)(next() % (hi - lo));
            memcpy(&s, &u, 4);
        }
        const I8sInv d = i8s_inv(s);
        for (int a = -(1 << 20); a <= (1 << 20); ++a) {
            const float want = (float)a / s;
            const float got = quotient(a, d);
            ++checked;
            if (bits(got) != bits(want) && !(isnan(got) && isnan(want))) {
                if (bad < 5) printf("mismatch a=%d s=%a want=%a got=%a\n", a, s, want, got);
                ++bad;
            }
        }
    }
    printf("checked %lld mismatches %lld\n", checked, bad);
    return bad != 0;
}
