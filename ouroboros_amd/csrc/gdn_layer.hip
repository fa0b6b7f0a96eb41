// gdn_layer.hip - the delta-net layer block of run_delta on the GPU.
//
// Between its input projections (qkv, z, beta, alpha) and its output
// projection (ssm_out), run_delta (qwen35.rs:1048-1151) does, per token:
//   beta = sigmoid(beta_raw); gate = a_log * softplus(alpha + dt_bias)
//   conv_out = silu(conv_step(ring, w, qkv)) on every channel (ring updated)
//   per v-head: l2-normed q, k of its k-head (q scaled by 1/sqrt(d)) through
//   the recurrence (delta_head_dim), giving o
//   gated = gated_norm_rms(o, norm_w, z) per head, optionally permuted to
//   the V-grouped head order.
// Here that is two launches on the caller's stream with no host round
// trip: the decode kernel computing each head's q, k, v (conv + SiLU over
// the ring, which it only reads) and its gates from the raw projections,
// then gdn_gated_norm_kernel, which also shifts the ring (every wavefront
// the channels of its v-head, and those of its k-head when it is the first
// v-head reading it).  The state update dominates the bytes (2 x 64 KiB per
// head).  gdn_decode_core (the hybrid stack's path for more than 64
// sequences) keeps the separate conv/gate kernel.
#include "common.hpp"

namespace ouro {

int gdn_decode(float *state, const void *q, const void *k, int qk_dtype, const void *v, int v_dtype,
               const float *gate, const float *beta, float gate_s, float beta_s, float *out,
               size_t B, size_t Hk, size_t Hv, size_t d, unsigned flags, float eps, void *stream,
               size_t qk_bs, size_t v_bs);
int gdn_decode_conv(float *state, const float *qkv, const float *ring, const float *conv_w, const float *beta_raw,
                    const float *alpha_raw, const float *dt_bias, const float *a_log, float *out, size_t B, size_t Hk,
                    size_t Hv, unsigned flags, float eps, void *stream);

namespace {

constexpr int kD = 128;

// conv_step + SiLU per (sequence, channel) (qwen35.rs:64-70, 1080-1088; ops.rs:34-36),
// then beta and gate per (sequence, v-head) (qwen35.rs:1066-1070, 1241-1243).
__global__ __launch_bounds__(256) void gdn_conv_gate_kernel(const float *qkv, float *ring, const float *conv_w,
                                                            const float *beta_raw, const float *alpha_raw,
                                                            const float *dt_bias, const float *a_log,
                                                            float *conv_out, float *beta, float *gate, int B,
                                                            int ch, int Hv) {
#pragma clang fp contract(off)
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i < static_cast<long long>(B) * ch) {
        const int c = static_cast<int>(i % ch);
        float *r = ring + i * 3;
        const float4 w = *reinterpret_cast<const float4 *>(conv_w + 4LL * c);
        const float x = qkv[i], r0 = r[0], r1 = r[1], r2 = r[2];
        const float y = w.x * r0 + w.y * r1 + w.z * r2 + w.w * x;
        r[0] = r1;
        r[1] = r2;
        r[2] = x;
        conv_out[i] = y / (1.0f + expf(-y));
    }
    if (i < static_cast<long long>(B) * Hv) {
        const int h = static_cast<int>(i % Hv);
        beta[i] = 1.0f / (1.0f + expf(-beta_raw[i]));
        const float x = alpha_raw[i] + dt_bias[h];
        gate[i] = a_log[h] * (x > 20.0f ? x : logf(1.0f + expf(x)));
    }
}

// The conv ring shift of conv_step (qwen35.rs:64-70) for channel c of
// sequence b: the window moves by one and the new input enters last.
__device__ __forceinline__ void ring_shift(float *ring, const float *qkv, long long b, int ch, int c) {
    const long long i = b * ch + c;
    float *r = ring + i * 3;
    const float r1 = r[1], r2 = r[2];
    r[0] = r1;
    r[1] = r2;
    r[2] = qkv[i];
}

// gated_norm_rms (qwen35.rs:82-92) per (sequence, v-head), one wavefront
// each, written at the head's V-grouped position when asked
// (qwen35.rs:1122-1138: v-head r*Hk + k goes to k*(Hv/Hk) + r).  RING: the
// wavefront also shifts the conv ring of its v-head's channels and, when
// it is the first v-head reading its k-head, of that k-head's q and k
// channels (the decode kernel before it read the ring unchanged).
template <bool RING>
__global__ __launch_bounds__(256) void gdn_gated_norm_kernel(const float *o, const float *z, const float *norm_w,
                                                             float *out, int B, int Hk, int Hv, unsigned flags,
                                                             float eps, const float *qkv, float *ring) {
#pragma clang fp contract(off)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long bh = static_cast<long long>(blockIdx.x) * 4 + wave;
    if (bh >= static_cast<long long>(B) * Hv) return;  // whole wavefront
    const long long b = bh / Hv;
    const int h = static_cast<int>(bh % Hv);
    const float2 x = *reinterpret_cast<const float2 *>(o + bh * kD + 2 * lane);
    float ss = x.x * x.x + x.y * x.y;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += xor_shfl(ss, off);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(kD) + eps);
    const float2 zz = *reinterpret_cast<const float2 *>(z + bh * kD + 2 * lane);
    const float2 w = *reinterpret_cast<const float2 *>(norm_w + 2 * lane);
    const float g0 = zz.x / (1.0f + expf(-zz.x)), g1 = zz.y / (1.0f + expf(-zz.y));
    const int dst = (flags & OURO_GDN_V_GROUPED) ? (h % Hk) * (Hv / Hk) + h / Hk : h;
    *reinterpret_cast<float2 *>(out + (b * Hv + dst) * kD + 2 * lane) =
        make_float2(x.x * inv * w.x * g0, x.y * inv * w.y * g1);
    if constexpr (RING) {
        const int ch = (2 * Hk + Hv) * kD, g = Hv / Hk;
        ring_shift(ring, qkv, b, ch, (2 * Hk + h) * kD + lane);
        ring_shift(ring, qkv, b, ch, (2 * Hk + h) * kD + 64 + lane);
        const bool div = (flags & OURO_GDN_KHEAD_DIV) != 0;
        if (div ? h % g == 0 : h < Hk) {
            const int kh = div ? h / g : h;
#pragma unroll
            for (int c = 0; c < 4; ++c) ring_shift(ring, qkv, b, ch, ((c >> 1) * Hk + kh) * kD + 64 * (c & 1) + lane);
        }
    }
}

constexpr size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

}  // namespace

// gated_norm_rms per (row, v-head) of rows x Hv heads of d = 128 (the
// prefill's token rows, or the decode's sequences).
int gdn_gated_norm(const float *o, const float *z, const float *norm_w, float *out, size_t rows, size_t Hk,
                   size_t Hv, unsigned flags, float eps, void *stream) {
    const long long items = static_cast<long long>(rows * Hv);
    if (!items) return OURO_OK;
    hipLaunchKernelGGL(gdn_gated_norm_kernel<false>, dim3(static_cast<unsigned>((items + 3) / 4)), dim3(256), 0,
                       as_stream(stream), o, z, norm_w, out, static_cast<int>(rows), static_cast<int>(Hk),
                       static_cast<int>(Hv), flags, eps, nullptr, nullptr);
    return check_launch("gdn_gated_norm_kernel");
}

// gdn_decode_core's workspace: conv_out, beta, gate, then o.
size_t gdn_layer_ws_bytes(size_t B, size_t Hk, size_t Hv) {
    const size_t ch = 2 * Hk * kD + Hv * kD;
    return align256(B * ch * 4) + 2 * align256(B * Hv * 4) + align256(B * Hv * kD * 4);
}
// ouro_gdn_layer_decode's workspace: the recurrence output o[B][Hv][d].
static size_t layer_o_bytes(size_t B, size_t Hv) { return align256(B * Hv * kD * 4); }

// run_delta's block up to the recurrence output: gates, conv + SiLU (ring
// updated), normed recurrence into o[B][Hv][d] (no gated norm).  The
// workspace holds conv_out, beta and gate (gdn_layer_ws_bytes).
int gdn_decode_core(const float *qkv, const float *beta_raw, const float *alpha_raw, const float *dt_bias,
                    const float *a_log, const float *conv_w, float *conv, float *state, float *o, size_t B, size_t Hk,
                    size_t Hv, unsigned flags, float eps, void *workspace, void *stream) {
    const size_t ch = 2 * Hk * kD + Hv * kD;
    unsigned char *ws = static_cast<unsigned char *>(workspace);
    float *conv_out = reinterpret_cast<float *>(ws);
    float *beta = reinterpret_cast<float *>(ws + align256(B * ch * 4));
    float *gate = reinterpret_cast<float *>(ws + align256(B * ch * 4) + align256(B * Hv * 4));
    const size_t n = B * ch > B * Hv ? B * ch : B * Hv;
    hipLaunchKernelGGL(gdn_conv_gate_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       as_stream(stream), qkv, conv, conv_w, beta_raw, alpha_raw, dt_bias, a_log, conv_out, beta, gate,
                       static_cast<int>(B), static_cast<int>(ch), static_cast<int>(Hv));
    int st = check_launch("gdn_conv_gate_kernel");
    if (st) return st;
    const size_t di = Hk * kD;
    return gdn_decode(state, conv_out, conv_out + di, OURO_DT_F32, conv_out + 2 * di, OURO_DT_F32, gate, beta, 0.f,
                      0.f, o, B, Hk, Hv, kD, OURO_GDN_L2NORM_QK | OURO_GDN_SCALE_Q | (flags & OURO_GDN_KHEAD_DIV), eps,
                      stream, ch, ch);
}

int gdn_layer_decode(const float *qkv, const float *z, const float *beta_raw, const float *alpha_raw,
                     const float *dt_bias, const float *a_log, const float *conv_w, const float *norm_w,
                     float *conv, float *state, float *out, size_t B, size_t Hk, size_t Hv, size_t d,
                     unsigned flags, float eps, void *workspace, void *stream) {
    if (!qkv || !z || !beta_raw || !alpha_raw || !dt_bias || !a_log || !conv_w || !norm_w || !conv || !state ||
        !out)
        return fail(OURO_ERR_INVALID_ARG, "gdn layer: NULL argument");
    if (d != static_cast<size_t>(kD)) return fail(OURO_ERR_SHAPE, "gdn layer: d = %zu, only 128", d);
    if (!B || !Hk || !Hv || Hv % Hk) return fail(OURO_ERR_SHAPE, "gdn layer: bad heads B=%zu Hk=%zu Hv=%zu", B, Hk, Hv);
    if (flags & ~(OURO_GDN_KHEAD_DIV | OURO_GDN_V_GROUPED))
        return fail(OURO_ERR_INVALID_ARG, "gdn layer: bad flags 0x%x", flags);
    const size_t ch = 2 * Hk * kD + Hv * kD;
    if (B * ch > 0x7fffffffULL) return fail(OURO_ERR_SHAPE, "gdn layer: too many channels");
    if ((reinterpret_cast<uintptr_t>(conv_w) | reinterpret_cast<uintptr_t>(workspace) |
         reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(conv) | reinterpret_cast<uintptr_t>(state)) % 16 ||
        (reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(norm_w) | reinterpret_cast<uintptr_t>(out)) % 8)
        return fail(OURO_ERR_ALIGN,
                    "gdn layer: qkv, conv ring, state, conv_w and workspace need 16-byte, z, norm_w, out 8-byte alignment");
    unsigned char *ws = static_cast<unsigned char *>(workspace);
    if (!ws) {
        ws = static_cast<unsigned char *>(ouro::workspace(layer_o_bytes(B, Hv), stream));
        if (!ws) return OURO_ERR_HIP;
    }
    float *o = reinterpret_cast<float *>(ws);
    int st = gdn_decode_conv(state, qkv, conv, conv_w, beta_raw, alpha_raw, dt_bias, a_log, o, B, Hk, Hv,
                             OURO_GDN_L2NORM_QK | OURO_GDN_SCALE_Q | (flags & OURO_GDN_KHEAD_DIV), eps, stream);
    if (st) return st;
    hipLaunchKernelGGL(gdn_gated_norm_kernel<true>, dim3(static_cast<unsigned>((B * Hv + 3) / 4)), dim3(256), 0,
                       as_stream(stream), o, z, norm_w, out, static_cast<int>(B), static_cast<int>(Hk),
                       static_cast<int>(Hv), flags, eps, qkv, conv);
    return check_launch("gdn_gated_norm_kernel");
}

}  // namespace ouro

using namespace ouro;

extern "C" {

size_t ouro_gdn_layer_workspace_bytes(size_t B, size_t Hk, size_t Hv, size_t d) {
    if (d != static_cast<size_t>(kD) || !Hk) return 0;
    return layer_o_bytes(B, Hv);
}

int ouro_gdn_layer_decode(const float *qkv, const float *z, const float *beta_raw, const float *alpha_raw,
                          const float *dt_bias, const float *a_log, const float *conv_w, const float *norm_w,
                          float *conv_state, float *state, float *out, size_t B, size_t Hk, size_t Hv, size_t d,
                          unsigned flags, float eps, void *workspace, void *stream) {
    OURO_REQUIRE_INIT();
    return gdn_layer_decode(qkv, z, beta_raw, alpha_raw, dt_bias, a_log, conv_w, norm_w, conv_state, state, out,
                            B, Hk, Hv, d, flags, eps, workspace, stream);
}

}  // extern "C"
