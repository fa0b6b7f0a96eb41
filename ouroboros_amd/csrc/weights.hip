// weights.hip - resident weight handles, the device analogue of the
// reference's GpuPool (ouro-wgpu/src/lib.rs:251-356): a tensor is uploaded
// once (and repacked on upload, as upload_q6k repacks 210 -> 212 B blocks),
// then applied by handle.  I2 codes are tiled for the int8 GEMV (and, for
// handles that expect many columns, also for the int8 MFMA GEMM); TL1
// payloads are repacked for the table-lookup GEMV.  Every handle owns the
// scratch its calls need (activation quantisation for up to max_cols columns,
// TL1 / TQ1_0 partial sums, a logits vector and the argmax keys), one set per
// stream it is used on: the null stream's set is made at upload, another
// stream's on the handle's first call on that stream; after that the calls
// allocate nothing, and calls on different streams share nothing.
#include "common.hpp"

#include <cstring>
#include <mutex>
#include <new>
#include <deque>

namespace ouro {
int matmul_q(const void *payload, int kind, size_t out_len, size_t in_len, const float *x, size_t k,
             float *y, int8_t *xq_scratch, float *act_scale_scratch, void *stream, bool use_workspace,
             float *lut_partial, size_t lut_partial_bytes);
int i2_tile(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *tiled,
            const float *w_scale, void *stream, int src_i2s);
size_t i2_tiled_bytes(size_t out_len, size_t in_len);
size_t i2_mfma_bytes(size_t out_len, size_t in_len);
int i2_tile_mfma(const uint8_t *canonical, size_t out_len, size_t in_len, uint8_t *dst, const float *w_scale,
                 void *stream, int src_i2s);
int i2_gemm_mfma(const uint8_t *w_mfma, size_t out_len, size_t in_len, const float *w_scale, const int8_t *xq,
                 const float *act_scale, size_t ncols, float *y, int32_t *acc, void *stream, int x_tiled, int swiglu = 0,
                 const GemmEpilogue *epi = nullptr);
int act_quant(const void *x, int x_dtype, size_t rows, size_t n, int8_t *xq, float *act_scale, void *stream);
size_t tl1_lut_bytes(size_t out_len, size_t in_len);
size_t tl1_lut_partial_floats(size_t out_len, size_t in_len);
int tl1_repack(const uint8_t *raw, size_t out_len, size_t in_len, void *dst, void *stream);
size_t tq1_lut_partial_floats(size_t out_len, size_t in_len);
bool tq1_lut_fits(const void *payload, size_t in_len);
int tq1_lut_matvec(const void *payload, size_t out_len, size_t in_len, const float *x, float *y, float *partial,
                   void *amax_scratch, int32_t *idx, void *stream);
int tl1_lut_matvec(const void *packed, size_t out_len, size_t in_len, const float *x, float *y, float *partial,
                   void *amax_scratch, int32_t *idx, void *stream, int raw);
int argmax_f32(const float *y, size_t n, void *scratch, int32_t *idx, void *stream);
size_t tl1_mfma_code_bytes(size_t M, size_t K);
size_t tl1_mfma_scale_bytes(size_t M, size_t K);
size_t tl1_xprep_bytes(size_t K, size_t ncols);
int tl1_tile_mfma(const uint8_t *raw, size_t M, size_t K, uint8_t *codes, uint16_t *scales, void *stream);
int tq1_tile_mfma(const uint8_t *raw, size_t M, size_t K, uint8_t *codes, uint16_t *scales, void *stream);
int tl1_mfma_matmul(const uint8_t *codes, const uint16_t *scales, size_t M, size_t K, const float *x, size_t ncols,
                    float *y, void *scratch, void *stream);
}  // namespace ouro

// The per-stream scratch of a handle: one allocation holding the I2
// activation codes and scales, the lookup kernels' partial sums, a y vector
// and the argmax key slots (each part only where the handle's kind uses it).
struct WeightScratch {
    void *stream = nullptr;
    void *block = nullptr;
    int8_t *xq = nullptr;
    float *act_scale = nullptr;
    float *partial = nullptr;
    float *y = nullptr;
    void *amax = nullptr;
    void *xprep = nullptr;  // TL1 with the MFMA layout: x digit planes of up to 16 columns
};

struct ouro_weight {
    int kind = 0;
    size_t out_len = 0, in_len = 0, max_cols = 0;
    void *payload = nullptr;  // device layout of the kind (TL1: the lookup layout)
    void *mfma = nullptr;     // I2 with max_cols >= kMfmaCols: the MFMA layout of the codes;
                              // TL1 / TQ1_0 with max_cols >= 2: the trits in that layout, then the
                              // scales of every 128-group
    size_t partial_floats = 0;  // TL1, large TQ1_0: per-block partial sums of the lookup kernels
    std::mutex mu;
    std::deque<WeightScratch> scratch;  // stable addresses as sets are added
};

using namespace ouro;

namespace {

// Columns from which an I2 matmul runs on the int8 MFMA GEMM instead of the
// multi-column GEMV (measured crossover on the 6912x2560 layer).
constexpr size_t kMfmaCols = 8;
// Rows from which a TQ1_0 handle runs the table-lookup kernel (as matvec_q).
constexpr size_t kTq1LutRows = 8192;

size_t ref_row_bytes(int kind, size_t k) {  // QuantKind::row_bytes (dequant.rs:376-387)
    switch (kind) {
    case OURO_KIND_F32: return k * 4;
    case OURO_KIND_F16:
    case OURO_KIND_BF16: return k * 2;
    case OURO_KIND_TL1: return k / 128 * 28;
    case OURO_KIND_TQ1_0: return k / 256 * 54;
    case OURO_KIND_Q8_0: return k / 32 * 34;
    case OURO_KIND_Q3K: return k / 256 * 110;
    case OURO_KIND_Q4K: return k / 256 * 144;
    case OURO_KIND_Q5K: return k / 256 * 176;
    case OURO_KIND_Q6K: return k / 256 * 210;
    case OURO_KIND_I2:
    case OURO_KIND_I2_S: return k / 4;
    default: return 0;
    }
}

// Bytes of a bitnet.cpp I2_S tensor: the codes, the fp32 scale, and up to
// 28 bytes of alignment padding (quantize_i2_s writes n/4 + 32).
bool i2s_size_ok(size_t bytes, size_t codes) { return bytes >= codes + 4 && bytes <= codes + 32; }

void release(ouro_weight *w) {
    if (!w) return;
    if (w->payload) (void)hipFree(w->payload);
    if (w->mfma) (void)hipFree(w->mfma);
    for (WeightScratch &sc : w->scratch) (void)hipFree(sc.block);
    delete w;
}

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// The handle's scratch set for `stream`, made on its first use there.
WeightScratch *scratch_for(ouro_weight *w, void *stream) {
    std::lock_guard<std::mutex> lock(w->mu);
    for (WeightScratch &sc : w->scratch)
        if (sc.stream == stream) return &sc;
    const bool i2 = w->kind == OURO_KIND_I2;
    const size_t xb = i2 ? align256(w->max_cols * w->in_len) : 0;
    const size_t sb = i2 ? align256(w->max_cols * sizeof(float)) : 0;
    const size_t pb = align256(w->partial_floats * sizeof(float));
    const size_t yb = align256(w->out_len * sizeof(float));
    const size_t mb = ((w->kind == OURO_KIND_TL1 || w->kind == OURO_KIND_TQ1_0) && w->mfma)
                          ? align256(tl1_xprep_bytes(w->in_len, 16)) : 0;
    WeightScratch sc;
    sc.stream = stream;
    if (hipMalloc(&sc.block, xb + sb + pb + yb + mb + kArgmaxBlocks * 8) != hipSuccess) {
        fail(OURO_ERR_HIP, "weight handle: scratch allocation failed");
        return nullptr;
    }
    uint8_t *p = static_cast<uint8_t *>(sc.block);
    if (i2) {
        sc.xq = reinterpret_cast<int8_t *>(p);
        sc.act_scale = reinterpret_cast<float *>(p + xb);
    }
    if (w->partial_floats) sc.partial = reinterpret_cast<float *>(p + xb + sb);
    sc.y = reinterpret_cast<float *>(p + xb + sb + pb);
    if (mb) sc.xprep = p + xb + sb + pb + yb;
    sc.amax = p + xb + sb + pb + yb + mb;
    w->scratch.push_back(sc);
    return &w->scratch.back();
}

}  // namespace

extern "C" {

int ouro_weight_upload(int kind, const void *host, size_t bytes, size_t out_len, size_t in_len,
                       float w_scale, size_t max_cols, ouro_weight_t *out) {
    OURO_REQUIRE_INIT();
    if (!host || !out) return fail(OURO_ERR_INVALID_ARG, "ouro_weight_upload: NULL argument");
    *out = nullptr;
    const size_t rb = ref_row_bytes(kind, in_len);
    if (!rb) return fail(OURO_ERR_KIND, "ouro_weight_upload: kind %d / in_len %zu unsupported", kind, in_len);
    const size_t be = kind == OURO_KIND_TL1 ? 128 : kind == OURO_KIND_Q8_0 ? 32
                      : (kind == OURO_KIND_TQ1_0 || kind == OURO_KIND_Q3K || kind == OURO_KIND_Q4K ||
                         kind == OURO_KIND_Q5K || kind == OURO_KIND_Q6K) ? 256 : 1;
    if (in_len % be)  // rows of whole blocks (QuantKind::row_bytes, dequant.rs:376-387)
        return fail(OURO_ERR_SHAPE, "ouro_weight_upload: in_len %zu not a multiple of the %zu-element block", in_len, be);
    if (!out_len || (kind == OURO_KIND_I2_S ? !i2s_size_ok(bytes, rb * out_len) : bytes != rb * out_len))
        return fail(OURO_ERR_SHAPE, "ouro_weight_upload: %zu bytes, expected %zu%s", bytes, rb * out_len,
                    kind == OURO_KIND_I2_S ? " + 4..32 (scale and padding)" : "");
    ouro_weight *w = new (std::nothrow) ouro_weight;
    if (!w) return fail(OURO_ERR_INVALID_ARG, "ouro_weight_upload: out of host memory");
    w->kind = kind;
    w->out_len = out_len;
    w->in_len = in_len;
    w->max_cols = max_cols ? max_cols : 1;
    if (kind == OURO_KIND_I2 || kind == OURO_KIND_I2_S) {
        // both are held as the tiled I2 payload (and the MFMA layout)
        const int src_i2s = kind == OURO_KIND_I2_S;
        w->kind = OURO_KIND_I2;
        const size_t tb = i2_tiled_bytes(out_len, in_len);
        if (!tb) {
            release(w);
            return fail(OURO_ERR_SHAPE, "ouro_weight_upload: I2 in_len %zu not a multiple of 256", in_len);
        }
        void *canon = nullptr;
        if (hipMalloc(&w->payload, tb + 16) != hipSuccess || hipMalloc(&canon, bytes) != hipSuccess) {
            if (canon) (void)hipFree(canon);
            release(w);
            return fail(OURO_ERR_HIP, "ouro_weight_upload: device allocation failed");
        }
        int st = OURO_OK;
        // I2_S carries its own scale right after the codes (quantize_i2_s)
        float scale = w_scale;
        if (src_i2s) memcpy(&scale, static_cast<const uint8_t *>(host) + rb * out_len, 4);
        if (hipMemcpy(canon, host, bytes, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(static_cast<uint8_t *>(w->payload) + tb, &scale, 4, hipMemcpyHostToDevice) != hipSuccess)
            st = fail(OURO_ERR_HIP, "ouro_weight_upload: copy failed");
        if (!st) st = i2_tile(static_cast<const uint8_t *>(canon), out_len, in_len,
                              static_cast<uint8_t *>(w->payload), nullptr, nullptr, src_i2s);
        if (!st && w->max_cols >= kMfmaCols) {  // second layout for many-column matmuls
            if (hipMalloc(&w->mfma, i2_mfma_bytes(out_len, in_len)) != hipSuccess)
                st = fail(OURO_ERR_HIP, "ouro_weight_upload: device allocation failed");
            else
                st = i2_tile_mfma(static_cast<const uint8_t *>(canon), out_len, in_len,
                                  static_cast<uint8_t *>(w->mfma), nullptr, nullptr, src_i2s);
        }
        if (!st && hipDeviceSynchronize() != hipSuccess) st = fail(OURO_ERR_HIP, "ouro_weight_upload: sync failed");
        (void)hipFree(canon);
        if (st) {
            release(w);
            return st;
        }
    } else if (kind == OURO_KIND_TL1) {
        // repack for the lookup kernel; the raw payload lives only during the upload
        void *raw = nullptr;
        w->partial_floats = tl1_lut_partial_floats(out_len, in_len);
        if (hipMalloc(&w->payload, tl1_lut_bytes(out_len, in_len)) != hipSuccess ||
            hipMalloc(&raw, bytes) != hipSuccess) {
            if (raw) (void)hipFree(raw);
            release(w);
            return fail(OURO_ERR_HIP, "ouro_weight_upload: device allocation failed");
        }
        int st = OURO_OK;
        if (hipMemcpy(raw, host, bytes, hipMemcpyHostToDevice) != hipSuccess)
            st = fail(OURO_ERR_HIP, "ouro_weight_upload: copy failed");
        if (!st) st = tl1_repack(static_cast<const uint8_t *>(raw), out_len, in_len, w->payload, nullptr);
        if (!st && w->max_cols >= 2) {  // matmuls of several columns: the trits on int8 MFMA
            const size_t cb = tl1_mfma_code_bytes(out_len, in_len);
            if (hipMalloc(&w->mfma, cb + tl1_mfma_scale_bytes(out_len, in_len)) != hipSuccess)
                st = fail(OURO_ERR_HIP, "ouro_weight_upload: device allocation failed");
            else
                st = tl1_tile_mfma(static_cast<const uint8_t *>(raw), out_len, in_len, static_cast<uint8_t *>(w->mfma),
                                   reinterpret_cast<uint16_t *>(static_cast<uint8_t *>(w->mfma) + cb), nullptr);
        }
        if (!st && hipDeviceSynchronize() != hipSuccess) st = fail(OURO_ERR_HIP, "ouro_weight_upload: sync failed");
        (void)hipFree(raw);
        if (st) {
            release(w);
            return st;
        }
    } else {
        if (hipMalloc(&w->payload, bytes) != hipSuccess) {
            release(w);
            return fail(OURO_ERR_HIP, "ouro_weight_upload: device allocation failed");
        }
        if (hipMemcpy(w->payload, host, bytes, hipMemcpyHostToDevice) != hipSuccess) {
            release(w);
            return fail(OURO_ERR_HIP, "ouro_weight_upload: copy failed");
        }
        // a large TQ1_0 matrix runs the lookup kernel: its block partials live with the handle
        if (kind == OURO_KIND_TQ1_0 && out_len >= kTq1LutRows && tq1_lut_fits(w->payload, in_len))
            w->partial_floats = tq1_lut_partial_floats(out_len, in_len);
        if (kind == OURO_KIND_TQ1_0 && w->max_cols >= 2) {  // matmuls of several columns: the trits on int8 MFMA
            const size_t cb = tl1_mfma_code_bytes(out_len, in_len);
            int st = OURO_OK;
            if (hipMalloc(&w->mfma, cb + tl1_mfma_scale_bytes(out_len, in_len)) != hipSuccess)
                st = fail(OURO_ERR_HIP, "ouro_weight_upload: device allocation failed");
            else
                st = tq1_tile_mfma(static_cast<const uint8_t *>(w->payload), out_len, in_len,
                                   static_cast<uint8_t *>(w->mfma),
                                   reinterpret_cast<uint16_t *>(static_cast<uint8_t *>(w->mfma) + cb), nullptr);
            if (!st && hipDeviceSynchronize() != hipSuccess) st = fail(OURO_ERR_HIP, "ouro_weight_upload: sync failed");
            if (st) {
                release(w);
                return st;
            }
        }
    }
    // the null stream's scratch set
    if (!scratch_for(w, nullptr)) {
        release(w);
        return OURO_ERR_HIP;
    }
    *out = w;
    return OURO_OK;
}

int ouro_weight_free(ouro_weight_t w) {
    OURO_REQUIRE_INIT();
    if (w) {
        (void)hipDeviceSynchronize();
        release(w);
    }
    return OURO_OK;
}

const void *ouro_weight_payload(ouro_weight_t w) {
    return (w && w->kind != OURO_KIND_TL1) ? w->payload : nullptr;
}

int ouro_weight_matmul(ouro_weight_t w, const float *x, size_t k, float *y, void *stream) {
    OURO_REQUIRE_INIT();
    if (!w) return fail(OURO_ERR_INVALID_ARG, "ouro_weight_matmul: NULL handle");
    if (!x || !y || !k) return fail(OURO_ERR_INVALID_ARG, "ouro_weight_matmul: NULL argument or k = 0");
    if (w->kind == OURO_KIND_I2 && k > w->max_cols)
        return fail(OURO_ERR_SHAPE, "ouro_weight_matmul: k %zu > max_cols %zu of the handle", k, w->max_cols);
    WeightScratch *sc = scratch_for(w, stream);
    if (!sc) return OURO_ERR_HIP;
    if ((w->kind == OURO_KIND_TL1 || w->kind == OURO_KIND_TQ1_0) && w->mfma && k >= 2) {
        // one pass over the trits for all k columns
        const size_t cb = tl1_mfma_code_bytes(w->out_len, w->in_len);
        return tl1_mfma_matmul(static_cast<const uint8_t *>(w->mfma),
                               reinterpret_cast<const uint16_t *>(static_cast<const uint8_t *>(w->mfma) + cb),
                               w->out_len, w->in_len, x, k, y, sc->xprep, stream);
    }
    if (w->kind == OURO_KIND_TL1) {  // one lookup pass per column, y column-major as matmul_q
        for (size_t c = 0; c < k; ++c) {
            const int st = tl1_lut_matvec(w->payload, w->out_len, w->in_len, x + c * w->in_len, y + c * w->out_len,
                                          sc->partial, nullptr, nullptr, stream, 0);
            if (st) return st;
        }
        return OURO_OK;
    }
    if (w->kind == OURO_KIND_TQ1_0 && sc->partial) {  // one lookup pass per column
        for (size_t c = 0; c < k; ++c) {
            const int st = tq1_lut_matvec(w->payload, w->out_len, w->in_len, x + c * w->in_len, y + c * w->out_len,
                                          sc->partial, nullptr, nullptr, stream);
            if (st) return st;
        }
        return OURO_OK;
    }
    if (w->kind == OURO_KIND_I2 && w->mfma && k >= kMfmaCols) {
        int st = act_quant(x, OURO_DT_F32, k, w->in_len, sc->xq, sc->act_scale, stream);
        if (st) return st;
        const float *w_scale =
            reinterpret_cast<const float *>(static_cast<const uint8_t *>(w->payload) + i2_tiled_bytes(w->out_len, w->in_len));
        return i2_gemm_mfma(static_cast<const uint8_t *>(w->mfma), w->out_len, w->in_len, w_scale, sc->xq,
                            sc->act_scale, k, y, nullptr, stream, 0);
    }
    return matmul_q(w->payload, w->kind, w->out_len, w->in_len, x, k, y, sc->xq, sc->act_scale, stream, false,
                    nullptr, 0);
}

int ouro_weight_matvec_argmax(ouro_weight_t w, const float *x, float *y, int32_t *idx, void *stream) {
    OURO_REQUIRE_INIT();
    if (!w || !x || !idx) return fail(OURO_ERR_INVALID_ARG, "ouro_weight_matvec_argmax: NULL argument");
    WeightScratch *sc = scratch_for(w, stream);
    if (!sc) return OURO_ERR_HIP;
    float *yy = y ? y : sc->y;
    if (w->kind == OURO_KIND_TL1)  // the argmax rides on the partial-sum kernel
        return tl1_lut_matvec(w->payload, w->out_len, w->in_len, x, yy, sc->partial, sc->amax, idx, stream, 0);
    if (w->kind == OURO_KIND_TQ1_0 && sc->partial)
        return tq1_lut_matvec(w->payload, w->out_len, w->in_len, x, yy, sc->partial, sc->amax, idx, stream);
    const int st = ouro_weight_matmul(w, x, 1, yy, stream);
    if (st) return st;
    return argmax_f32(yy, w->out_len, sc->amax, idx, stream);
}

int ouro_weight_matvec(ouro_weight_t w, const float *x, float *y, void *stream) {
    return ouro_weight_matmul(w, x, 1, y, stream);
}

}  // extern "C"
