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
// Here that is one launch (gdn_layer_kernel, gdn_decode.hip): a workgroup
// per (sequence, k-head) computes the conv + SiLU of the channels it reads
// and the gates, runs the recurrence of the k-head's v-heads, their gated
// norms, and shifts the ring.  The state update dominates the bytes
// (2 x 64 KiB per head).  gdn_decode_core (the hybrid stack's path for more
// than 64 sequences) runs a separate conv/gate kernel and the decode kernel.
#include "common.hpp"

namespace ouro {

int gdn_decode(float *state, const void *q, const void *k, int qk_dtype, const void *v, int v_dtype,
               const float *gate, const float *beta, float gate_s, float beta_s, float *out,
               size_t B, size_t Hk, size_t Hv, size_t d, unsigned flags, float eps, void *stream,
               size_t qk_bs, size_t v_bs);
int gdn_layer_fused(const float *qkv, const float *z, const float *beta_raw, const float *alpha_raw,
                    const float *dt_bias, const float *a_log, const float *conv_w, const float *norm_w, float *ring,
                    float *state, float *out, size_t B, size_t Hk, size_t Hv, unsigned flags, float eps,
                    void *stream);

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

constexpr size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

}  // namespace

// gdn_decode_core's workspace: conv_out, beta, gate, then o.
size_t gdn_layer_ws_bytes(size_t B, size_t Hk, size_t Hv) {
    const size_t ch = 2 * Hk * kD + Hv * kD;
    return align256(B * ch * 4) + 2 * align256(B * Hv * 4) + align256(B * Hv * kD * 4);
}


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
    (void)workspace;  // the one-launch block needs none
    if ((reinterpret_cast<uintptr_t>(conv_w) | reinterpret_cast<uintptr_t>(state)) % 16 ||
        (reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(norm_w) | reinterpret_cast<uintptr_t>(out)) % 8 ||
        (reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(conv)) % 4)
        return fail(OURO_ERR_ALIGN, "gdn layer: state and conv_w need 16-byte, z, norm_w, out 8-byte alignment");
    return gdn_layer_fused(qkv, z, beta_raw, alpha_raw, dt_bias, a_log, conv_w, norm_w, conv, state, out, B, Hk, Hv,
                           flags, eps, stream);
}

}  // namespace ouro

using namespace ouro;

extern "C" {

size_t ouro_gdn_layer_workspace_bytes(size_t B, size_t Hk, size_t Hv, size_t d) {
    (void)B, (void)Hk, (void)Hv, (void)d;
    return 0;  // one launch, nothing kept between kernels
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
