// reference_kats.cpp - the reference's own unit tests for this path, restated
// in C++ against the C++ host mirror (include/ouro/infer.hpp), i.e. run on
// the GPU through the C ABI.  Each test names the reference test it follows.
// Exit status 0 when every test passes.
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <vector>

#include "../../include/ouro/infer.hpp"

using namespace ouro;
using namespace ouro::infer;

static int g_failed = 0;

#define EXPECT(cond)                                                                   \
    do {                                                                               \
        if (!(cond)) {                                                                 \
            std::printf("    expectation failed: %s (line %d)\n", #cond, __LINE__);   \
            throw std::runtime_error("expectation failed");                           \
        }                                                                              \
    } while (0)

static void run(const char *name, const std::function<void()> &fn) {
    try {
        fn();
        std::printf("PASS %s\n", name);
    } catch (const std::exception &e) {
        ++g_failed;
        std::printf("FAIL %s: %s\n", name, e.what());
    }
    std::fflush(stdout);
}

// ---- hadamard.rs tests ----------------------------------------------------

// Naive O(N^2) matrix (hadamard.rs:73-87).
static std::vector<float> naive_matrix(size_t n, size_t block) {
    const float scale = 1.0f / std::sqrt(static_cast<float>(block));
    std::vector<float> m(n * n, 0.f);
    for (size_t start = 0; start < n; start += block)
        for (size_t r = 0; r < block; ++r)
            for (size_t c = 0; c < block; ++c)
                m[(start + r) * n + start + c] = (__builtin_popcountll(r & c) & 1) ? -scale : scale;
    return m;
}

static std::vector<float> mat_vec(const std::vector<float> &m, const std::vector<float> &x) {
    const size_t n = x.size();
    std::vector<float> y(n, 0.f);
    for (size_t r = 0; r < n; ++r) {
        float s = 0.f;
        for (size_t c = 0; c < n; ++c) s += m[r * n + c] * x[c];
        y[r] = s;
    }
    return y;
}

static void test_fwd_is_h_times_diag_s() {  // hadamard.rs:96-110
    const size_t block = 16, n = block;
    std::vector<float> x(n), signs(n);
    for (size_t i = 0; i < n; ++i) {
        x[i] = static_cast<float>((i * 11) % 7) - 3.0f;
        signs[i] = i % 3 == 0 ? -1.0f : 1.0f;
    }
    std::vector<float> fast = x;
    hadamard::rotate_fwd(fast, signs, block);
    std::vector<float> sd(n);
    for (size_t i = 0; i < n; ++i) sd[i] = x[i] * signs[i];
    const auto ref = mat_vec(naive_matrix(n, block), sd);
    for (size_t i = 0; i < n; ++i) EXPECT(std::fabs(fast[i] - ref[i]) < 1e-4f);
}

static void test_inv_is_diag_s_times_h() {  // hadamard.rs:112-126
    const size_t block = 16, n = block;
    std::vector<float> x(n), signs(n);
    for (size_t i = 0; i < n; ++i) {
        x[i] = static_cast<float>((i * 5) % 9) - 4.0f;
        signs[i] = i % 4 == 0 ? -1.0f : 1.0f;
    }
    std::vector<float> fast = x;
    hadamard::rotate_inv(fast, signs, block);
    const auto hx = mat_vec(naive_matrix(n, block), x);
    for (size_t i = 0; i < n; ++i) EXPECT(std::fabs(fast[i] - hx[i] * signs[i]) < 1e-4f);
}

static std::vector<float> wave_x(size_t n) {
    std::vector<float> x(n);
    for (size_t i = 0; i < n; ++i) x[i] = static_cast<float>((i * 91) % 23) * 0.37f - 4.0f;
    return x;
}

static std::vector<float> stripe_signs(size_t n) {
    std::vector<float> s(n);
    for (size_t i = 0; i < n; ++i) s[i] = (i / 5) % 2 == 0 ? -1.0f : 1.0f;
    return s;
}

static void test_fwd_inv_roundtrip_identity() {  // hadamard.rs:128-141
    const size_t block = 64, n = block * 2;
    const auto x = wave_x(n), signs = stripe_signs(n);
    std::vector<float> y = x;
    hadamard::rotate_inv(y, signs, block);
    hadamard::rotate_fwd(y, signs, block);
    for (size_t i = 0; i < n; ++i) EXPECT(std::fabs(x[i] - y[i]) < 1e-3f);
}

static void test_rotation_preserves_l2_norm() {  // hadamard.rs:143-158
    const size_t block = 64, n = block * 3;
    const auto x = wave_x(n), signs = stripe_signs(n);
    float n0 = 0.f;
    for (float v : x) n0 += v * v;
    for (int inv = 0; inv < 2; ++inv) {
        std::vector<float> y = x;
        if (inv)
            hadamard::rotate_inv(y, signs, block);
        else
            hadamard::rotate_fwd(y, signs, block);
        float n1 = 0.f;
        for (float v : y) n1 += v * v;
        EXPECT(std::fabs(n0 - n1) / n0 < 1e-4f);
    }
}

static void test_blockwise_independence() {  // hadamard.rs:160-172
    const size_t block = 32, n = block * 2;
    std::vector<float> x(n);
    for (size_t i = 0; i < n; ++i) x[i] = static_cast<float>((i * 7) % 17) - 8.0f;
    const std::vector<float> signs(n, 1.0f);
    std::vector<float> a = x, b = x;
    hadamard::rotate_fwd(a, signs, block);
    b[3] += 5.0f;
    hadamard::rotate_fwd(b, signs, block);
    for (size_t i = block; i < n; ++i) EXPECT(a[i] == b[i]);
}

static void test_check_args_is_an_error() {  // hadamard.rs:33-37 asserts
    std::vector<float> x(24, 1.0f), signs(24, 1.0f);
    bool threw = false;
    try {
        hadamard::rotate_fwd(x, signs, 16);
    } catch (const Error &e) {
        threw = e.code == OURO_ERR_SHAPE;
    }
    EXPECT(threw);
}

// ---- qwen35.rs tests ------------------------------------------------------

static void test_delta_head_decay_only_when_beta_zero() {  // qwen35.rs:225-239
    const size_t S = qwen35::S;
    std::vector<float> state(S * S, 0.5f), q(S, 0.1f), k(S, 0.2f), v(S, 0.3f), out(S, 0.f);
    const float gate = -0.25f;
    qwen35::delta_head(state, q, k, v, {gate, 0.0f}, out);
    const float expect = 0.5f * std::exp(gate);
    for (float x : state) EXPECT(std::fabs(x - expect) < 1e-6f);
    float dot_q = 0.f;
    for (float x : q) dot_q += x;
    dot_q *= expect;
    for (float x : out) EXPECT(std::fabs(x - dot_q) < 1e-4f);
}

static void test_delta_head_single_write_read() {  // qwen35.rs:241-259
    const size_t S = qwen35::S;
    std::vector<float> state(S * S, 0.f), q(S, 0.f), k(S, 0.f), v(S, 0.f), out(S, 0.f);
    q[5] = qwen35::delta_q_scale();
    k[5] = 2.0f;
    k[9] = 1.0f;
    v[7] = 4.0f;
    qwen35::delta_head(state, q, k, v, {0.0f, 1.0f}, out);
    EXPECT(std::fabs(state[5 + 7 * S] - 8.0f) < 1e-6f);
    EXPECT(std::fabs(state[9 + 7 * S] - 4.0f) < 1e-6f);
    for (size_t j = 0; j < S; ++j) {
        if (j == 7)
            EXPECT(std::fabs(out[j] - 4.0f * qwen35::delta_q_scale() * 2.0f) < 1e-6f);
        else
            EXPECT(std::fabs(out[j]) < 1e-6f);
    }
}

static void test_delta_head_is_deterministic() {  // qwen35.rs:261-274
    const size_t S = qwen35::S;
    std::vector<float> q(S), k(S), v(S);
    for (size_t i = 0; i < S; ++i) {
        q[i] = static_cast<float>((i * 7) % 13) * 0.1f;
        k[i] = static_cast<float>((i * 5) % 11) * 0.1f;
        v[i] = static_cast<float>((i * 3) % 17) * 0.1f;
    }
    std::vector<float> s1(S * S, 0.3f), s2 = s1, o1(S, 0.f), o2(S, 0.f);
    qwen35::delta_head(s1, q, k, v, {-0.1f, 0.7f}, o1);
    qwen35::delta_head(s2, q, k, v, {-0.1f, 0.7f}, o2);
    EXPECT(s1 == s2);
    EXPECT(o1 == o2);
}

// ---- ops.rs tests (PTQ1_0 / TL1) -------------------------------------------

static float f16_to_f32(uint16_t bits) {  // dequant.rs:21-47
    const uint32_t sign = (bits >> 15) & 1u, frac = bits & 0x3ffu;
    const int32_t exp = (bits >> 10) & 0x1f;
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
            out = (sign << 31) | (static_cast<uint32_t>(127 - 15 - e) << 23) | ((f & 0x3ffu) << 13);
        }
    } else if (exp == 0x1f) {
        out = (sign << 31) | (0xffu << 23) | (frac << 13);
    } else {
        out = (sign << 31) | (static_cast<uint32_t>(exp + 127 - 15) << 23) | (frac << 13);
    }
    float f;
    std::memcpy(&f, &out, 4);
    return f;
}

// tl1_group decode (dequant.rs:146-171), restated for the test only.
static void tl1_group(const uint8_t *b, float *out) {
    static const uint8_t pow3[6] = {1, 3, 9, 27, 81, 243};
    const float d = f16_to_f32(static_cast<uint16_t>(b[26] | (b[27] << 8)));
    auto dig = [&](uint8_t byte, int n) {
        const uint8_t q = static_cast<uint8_t>(byte * pow3[n]);
        return static_cast<float>(static_cast<int>((q * 3u) >> 8) - 1) * d;
    };
    size_t o = 0;
    for (int n = 0; n < 5; ++n)
        for (int m = 0; m < 16; ++m) out[o++] = dig(b[m], n);
    for (int n = 0; n < 5; ++n)
        for (int m = 16; m < 24; ++m) out[o++] = dig(b[m], n);
    for (int n = 0; n < 4; ++n)
        for (int h = 0; h < 2; ++h) out[o++] = dig(b[24 + h], n);
}

static std::vector<uint8_t> tl1_payload(size_t out_len, size_t in_len, int shift) {
    const size_t rb = in_len / 128 * 28;
    std::vector<uint8_t> p(out_len * rb);
    for (size_t i = 0; i < p.size(); ++i)
        p[i] = static_cast<uint8_t>(static_cast<uint32_t>(i) * (0x9Bu ^ (static_cast<uint32_t>(i) >> shift)));
    for (size_t g = 0; g < p.size(); g += 28) {
        p[g + 26] = 0x10;
        p[g + 27] = 0x38;
    }
    return p;
}

static void test_matvec_tl1_fused_matches_reference() {  // ops.rs:800-838
    const size_t out_len = 37, in_len = 384, groups = in_len / 128, rb = groups * 28;
    const auto payload = tl1_payload(out_len, in_len, 7);
    std::vector<float> x(in_len);
    for (size_t i = 0; i < in_len; ++i) x[i] = (static_cast<float>(i % 7) - 3.0f) * 0.5f;
    const auto fused = ops::matvec_q(payload, QuantKind::Tl1, out_len, in_len, x);
    for (size_t row = 0; row < out_len; ++row) {
        std::vector<float> flat(in_len);
        for (size_t g = 0; g < groups; ++g) tl1_group(&payload[row * rb + g * 28], &flat[g * 128]);
        float want = 0.f;
        for (size_t i = 0; i < in_len; ++i) want += flat[i] * x[i];
        EXPECT(std::fabs(fused[row] - want) / std::fmax(std::fabs(want), 1e-9f) < 1e-5f);
    }
}

static void test_matmul_tl1_k_columns_matches_matvec() {  // ops.rs:720-750
    const size_t out_len = 97, in_len = 384, k = 4;
    const auto payload = tl1_payload(out_len, in_len, 5);
    std::vector<float> x(k * in_len);
    for (size_t i = 0; i < x.size(); ++i) x[i] = (static_cast<float>(i % 11) - 5.0f) * 0.25f;
    const auto batched = ops::matmul_q(payload, QuantKind::Tl1, out_len, in_len, x, k);
    for (size_t c = 0; c < k; ++c) {
        const std::vector<float> xc(x.begin() + c * in_len, x.begin() + (c + 1) * in_len);
        const auto want = ops::matvec_q(payload, QuantKind::Tl1, out_len, in_len, xc);
        for (size_t r = 0; r < out_len; ++r)
            EXPECT(std::fabs(batched[c * out_len + r] - want[r]) <= 1e-3f * std::fmax(std::fabs(want[r]), 1.0f));
    }
}

static void test_pool_matvec_by_name() {  // GpuPool::upload/matvec pattern (ouro-wgpu/src/lib.rs:251-356)
    const size_t out_len = 37, in_len = 384;
    const auto payload = tl1_payload(out_len, in_len, 7);
    std::vector<float> x(in_len);
    for (size_t i = 0; i < in_len; ++i) x[i] = (static_cast<float>(i % 7) - 3.0f) * 0.5f;
    HipPool pool;
    pool.upload("blk.0.ffn_up.weight", QuantKind::Tl1, payload, out_len, in_len);
    const auto a = pool.matvec("blk.0.ffn_up.weight", x);
    const auto b = ops::matvec_q(payload, QuantKind::Tl1, out_len, in_len, x);
    EXPECT(a == b);
    bool threw = false;
    try {
        pool.matvec("missing", x);
    } catch (const Error &) {
        threw = true;
    }
    EXPECT(threw);
}

static void test_pool_from_mapped_shard() {  // Stage::from_shard (mod.rs:112-135) on a BMTS file (bmts.rs:311-324)
    const size_t out_len = 37, in_len = 384;
    const auto payload = tl1_payload(out_len, in_len, 11);
    std::vector<uint8_t> data(16, 0);  // the tensor does not start the data section
    data.insert(data.end(), payload.begin(), payload.end());
    char path[] = "/tmp/ouro_kat_shard_XXXXXX";
    const int fd = mkstemp(path);
    EXPECT(fd >= 0);
    close(fd);
    bmts::Tensor t;
    t.name = "blk.2.ffn_up.weight";
    t.shape = {in_len, out_len};
    t.dtype = 143;
    t.offset = 16;
    t.length = payload.size();
    bmts::write_shard(path, 3, {t}, data);
    std::vector<float> x(in_len);
    // small multiples of 0.5: every partial sum is exact, so both decode orders agree bit for bit
    for (size_t i = 0; i < in_len; ++i) x[i] = (static_cast<float>(i % 5) - 2.0f) * 0.5f;
    std::vector<float> a;
    {
        bmts::Shard shard(path);
        EXPECT(shard.node() == 3 && shard.tensors().size() == 1);
        HipPool pool;
        pool.from_shard(shard);  // uploaded from the mapping itself
        a = pool.matvec("blk.2.ffn_up.weight", x);
    }
    std::remove(path);
    const auto b = ops::matvec_q(payload, QuantKind::Tl1, out_len, in_len, x);
    EXPECT(a == b);
}

int main() {
    try {
        init();
    } catch (const Error &e) {
        std::printf("FAIL init: %s\n", e.what());
        return 2;
    }
    run("hadamard::test_fwd_is_h_times_diag_s", test_fwd_is_h_times_diag_s);
    run("hadamard::test_inv_is_diag_s_times_h", test_inv_is_diag_s_times_h);
    run("hadamard::test_fwd_inv_roundtrip_identity", test_fwd_inv_roundtrip_identity);
    run("hadamard::test_rotation_preserves_l2_norm", test_rotation_preserves_l2_norm);
    run("hadamard::test_blockwise_independence", test_blockwise_independence);
    run("hadamard::check_args_is_an_error", test_check_args_is_an_error);
    run("qwen35::test_delta_head_decay_only_when_beta_zero", test_delta_head_decay_only_when_beta_zero);
    run("qwen35::test_delta_head_single_write_read", test_delta_head_single_write_read);
    run("qwen35::test_delta_head_is_deterministic", test_delta_head_is_deterministic);
    run("ops::test_matvec_tl1_fused_matches_reference", test_matvec_tl1_fused_matches_reference);
    run("ops::test_matmul_tl1_k_columns_matches_matvec", test_matmul_tl1_k_columns_matches_matvec);
    run("pool::matvec_by_name", test_pool_matvec_by_name);
    run("pool::from_mapped_shard", test_pool_from_mapped_shard);
    std::printf("%d failed\n", g_failed);
    return g_failed ? 1 : 0;
}
