// infer.hpp - C++ host mirror of the reference kernel-call surface
// (cluster/src/infer/{ops,hadamard,qwen35}.rs) over the C ABI of
// libouro_hip.so.  Same names and argument meaning as the Rust functions;
// host vectors in and out (the reference takes host slices), uploaded per
// call.  Failures throw ouro::Error where the reference would panic or bail.
// Header-only; link with -louro_hip.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../ouro_hip.h"
#include "bmts.hpp"

namespace ouro {

#ifndef OURO_ERROR_DEFINED
#define OURO_ERROR_DEFINED
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &what) : std::runtime_error(what), code(c) {}
};
#endif

inline void check(int st, const char *what) {
    if (st != OURO_OK) throw Error(st, std::string(what) + ": " + ouro_last_error());
}

inline void init(int device = -1) {
    static bool done = false;
    if (!done) {
        check(ouro_init(device), "ouro_init");
        done = true;
    }
}

// One device allocation holding n elements of T.
template <typename T>
class DeviceVec {
public:
    explicit DeviceVec(size_t n) : n_(n) {
        init();
        check(ouro_malloc(&p_, n ? n * sizeof(T) : 16), "ouro_malloc");
    }
    explicit DeviceVec(const std::vector<T> &h) : DeviceVec(h.size()) { upload(h); }
    ~DeviceVec() { if (p_) ouro_free(p_); }
    DeviceVec(const DeviceVec &) = delete;
    DeviceVec &operator=(const DeviceVec &) = delete;
    void upload(const std::vector<T> &h) {
        if (h.size() != n_) throw Error(OURO_ERR_SHAPE, "upload size mismatch");
        check(ouro_memcpy_htod(p_, h.data(), n_ * sizeof(T)), "ouro_memcpy_htod");
    }
    std::vector<T> download() const {
        std::vector<T> h(n_);
        check(ouro_memcpy_dtoh(h.data(), p_, n_ * sizeof(T)), "ouro_memcpy_dtoh");
        return h;
    }
    T *get() const { return static_cast<T *>(p_); }
    size_t size() const { return n_; }

private:
    void *p_ = nullptr;
    size_t n_;
};

namespace infer {

// QuantKind (dequant.rs:315-348), ggml dtype ids; I2 is this library's.
enum class QuantKind : int {
    F32 = 0, F16 = 1, Bf16 = 30, Q8_0 = 8, Q3K = 11, Q4K = 12, Q5K = 13, Q6K = 14, Tq1_0 = 34, Tl1 = 143,
    I2 = OURO_KIND_I2
};

namespace ops {

// y = W x (ops.rs:76).
inline std::vector<float> matvec_q(const std::vector<uint8_t> &payload, QuantKind kind, size_t out_len,
                                   size_t in_len, const std::vector<float> &x) {
    if (x.size() != in_len) throw Error(OURO_ERR_SHAPE, "matvec_q: x len != in_len");
    DeviceVec<uint8_t> p(payload);
    DeviceVec<float> xd(x), y(out_len);
    check(ouro_matvec_q(p.get(), static_cast<int>(kind), out_len, in_len, xd.get(), y.get(), nullptr),
          "matvec_q");
    return y.download();
}

// y = W X, x row-major [k][in_len], y column-major y[c*out_len + r] (ops.rs:219).
inline std::vector<float> matmul_q(const std::vector<uint8_t> &payload, QuantKind kind, size_t out_len,
                                   size_t in_len, const std::vector<float> &x, size_t k) {
    if (x.size() != k * in_len) throw Error(OURO_ERR_SHAPE, "matmul_q: x must be [k, in_len]");
    DeviceVec<uint8_t> p(payload);
    DeviceVec<float> xd(x), y(k * out_len);
    check(ouro_matmul_q(p.get(), static_cast<int>(kind), out_len, in_len, xd.get(), k, y.get(), nullptr),
          "matmul_q");
    return y.download();
}

}  // namespace ops

namespace hadamard {

inline void rotate(std::vector<float> &x, const std::vector<float> &signs, size_t block, bool inv) {
    if (x.size() != signs.size()) throw Error(OURO_ERR_SHAPE, "sign vector must match activation");
    DeviceVec<float> xd(x), sd(signs);
    check(inv ? ouro_rotate_inv(xd.get(), sd.get(), x.size(), block, nullptr)
              : ouro_rotate_fwd(xd.get(), sd.get(), x.size(), block, nullptr),
          inv ? "rotate_inv" : "rotate_fwd");
    x = xd.download();
}

// x' = H (s o x) (hadamard.rs:41).
inline void rotate_fwd(std::vector<float> &x, const std::vector<float> &signs, size_t block_size) {
    rotate(x, signs, block_size, false);
}
// h = s o (H z) (hadamard.rs:57).
inline void rotate_inv(std::vector<float> &x, const std::vector<float> &signs, size_t block_size) {
    rotate(x, signs, block_size, true);
}

}  // namespace hadamard

namespace qwen35 {

constexpr size_t S = 128;  // qwen35.rs:8

struct DeltaStep {  // qwen35.rs:12-15
    float gate;
    float beta;
};

inline float delta_q_scale() { return 1.0f / __builtin_sqrtf(static_cast<float>(S)); }

// One recurrence step for one head, in place (qwen35.rs:27).
inline void delta_head_dim(std::vector<float> &state, size_t sdim, const std::vector<float> &q,
                           const std::vector<float> &k, const std::vector<float> &v, DeltaStep step,
                           std::vector<float> &out) {
    if (state.size() != sdim * sdim || q.size() != sdim || k.size() != sdim || v.size() != sdim ||
        out.size() != sdim)
        throw Error(OURO_ERR_SHAPE, "delta_head_dim: sizes");
    DeviceVec<float> sd(state), qd(q), kd(k), vd(v), od(sdim);
    check(ouro_delta_head_dim(sd.get(), sdim, qd.get(), kd.get(), vd.get(), step.gate, step.beta, od.get(),
                              nullptr),
          "delta_head_dim");
    state = sd.download();
    out = od.download();
}

inline void delta_head(std::vector<float> &state, const std::vector<float> &q, const std::vector<float> &k,
                       const std::vector<float> &v, DeltaStep step, std::vector<float> &out) {
    delta_head_dim(state, S, q, k, v, step, out);
}

}  // namespace qwen35
}  // namespace infer

// Resident weights by name (GpuPool, ouro-wgpu/src/lib.rs:153-356).
class HipPool {
public:
    HipPool() { init(); }
    ~HipPool() {
        for (auto &kv : w_) ouro_weight_free(kv.second.h);
    }
    HipPool(const HipPool &) = delete;
    HipPool &operator=(const HipPool &) = delete;

    void upload(const std::string &name, infer::QuantKind kind, const std::vector<uint8_t> &payload,
                size_t out_len, size_t in_len, float w_scale = 1.0f, size_t max_cols = 8) {
        ouro_weight_t h = nullptr;
        check(ouro_weight_upload(static_cast<int>(kind), payload.data(), payload.size(), out_len, in_len,
                                 w_scale, max_cols, &h),
              "ouro_weight_upload");
        auto it = w_.find(name);
        if (it != w_.end()) ouro_weight_free(it->second.h);
        w_[name] = Entry{h, out_len, in_len};
    }

    // Upload straight from a view (e.g. a tensor of a mapped shard), no host copy.
    void upload_view(const std::string &name, infer::QuantKind kind, const uint8_t *bytes, size_t n, size_t out_len,
                     size_t in_len, float w_scale = 1.0f, size_t max_cols = 8) {
        ouro_weight_t h = nullptr;
        check(ouro_weight_upload(static_cast<int>(kind), bytes, n, out_len, in_len, w_scale, max_cols, &h),
              "ouro_weight_upload");
        auto it = w_.find(name);
        if (it != w_.end()) ouro_weight_free(it->second.h);
        w_[name] = Entry{h, out_len, in_len};
    }

    // Stage::from_shard (mod.rs:112-135): every tensor of the shard, its
    // ggml dtype as the kind (the kinds this path decodes; others refused).
    void from_shard(const bmts::Shard &shard, size_t max_cols = 8) {
        for (const bmts::Tensor &t : shard.tensors()) {
            const int d = static_cast<int>(t.dtype);
            if (d != OURO_KIND_F32 && d != OURO_KIND_F16 && d != OURO_KIND_BF16 && d != OURO_KIND_TQ1_0 &&
                d != OURO_KIND_TL1 && d != OURO_KIND_Q8_0 && d != OURO_KIND_Q3K && d != OURO_KIND_Q4K &&
                d != OURO_KIND_Q5K && d != OURO_KIND_Q6K)
                throw Error(OURO_ERR_KIND, "unsupported dtype " + std::to_string(t.dtype) + " on " + t.name);
            size_t out_len = 0, in_len = 0;
            shard.weight_shape(t.name, &out_len, &in_len);
            const auto v = shard.tensor_bytes(t.name);
            upload_view(t.name, static_cast<infer::QuantKind>(d), v.first, v.second, out_len, in_len, 1.0f, max_cols);
        }
    }

    std::vector<float> matvec(const std::string &name, const std::vector<float> &x) const {
        const Entry &e = get(name);
        if (x.size() != e.in_len) throw Error(OURO_ERR_SHAPE, "tensor " + name + ": in_len != x len");
        DeviceVec<float> xd(x), y(e.out_len);
        check(ouro_weight_matvec(e.h, xd.get(), y.get(), nullptr), "ouro_weight_matvec");
        return y.download();
    }

private:
    struct Entry {
        ouro_weight_t h;
        size_t out_len, in_len;
    };
    const Entry &get(const std::string &name) const {
        auto it = w_.find(name);
        if (it == w_.end()) throw Error(OURO_ERR_INVALID_ARG, "missing tensor " + name);
        return it->second;
    }
    std::map<std::string, Entry> w_;
};

}  // namespace ouro
