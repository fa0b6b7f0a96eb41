// argmax.hip - finite_argmax (infer/mod.rs:70-83) over a device vector.
//
// The reference keeps the first index of the largest non-NaN value (strict
// `v > l[best]`) and returns 0 when every value is NaN.  Each (value, index)
// becomes one 64-bit key (argmax_key); workgroups write their largest key
// to a slot of their own and one workgroup reduces the slots -- no atomics,
// and the scratch needs no initial value.
#include "common.hpp"

#include <algorithm>
#include <mutex>

namespace ouro {
namespace {

constexpr int kThreads = 256;

// Stage 1: one key per workgroup into keys[blockIdx.x].
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float *y, int n, unsigned long long *keys) {
    unsigned long long k = 0;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads)
        k = argmax_key_max(k, argmax_key(y[i], static_cast<unsigned>(i)));
    k = argmax_block_key(k);
    if (threadIdx.x == 0) keys[blockIdx.x] = k;
}

}  // namespace

// Stage 2: one workgroup reduces the per-workgroup keys and writes the index.
__global__ __launch_bounds__(1024) void argmax_final_kernel(const unsigned long long *keys, int nk, int32_t *idx) {
    unsigned long long k = 0;
    for (int i = threadIdx.x; i < nk; i += 1024) k = argmax_key_max(k, keys[i]);
    k = argmax_block_key(k);
    if (threadIdx.x == 0) *idx = argmax_index(k);
}

// scratch: kArgmaxBlocks 64-bit keys of device memory (no initial value).
int argmax_f32(const float *y, size_t n, void *scratch, int32_t *idx, void *stream) {
    if (!y || !scratch || !idx) return fail(OURO_ERR_INVALID_ARG, "argmax: NULL argument");
    if (!n || n > 0x7fffffffULL) return fail(OURO_ERR_SHAPE, "argmax: n = %zu", n);
    const size_t blocks = std::min<size_t>((n + kThreads - 1) / kThreads, kArgmaxBlocks);
    auto *keys = static_cast<unsigned long long *>(scratch);
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(argmax_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, y,
                       static_cast<int>(n), keys);
    int st = check_launch("argmax_kernel");
    if (st) return st;
    return argmax_final(keys, static_cast<int>(blocks), idx, stream);
}

int argmax_final(const unsigned long long *keys, int nk, int32_t *idx, void *stream) {
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, as_stream(stream), keys, nk, idx);
    return check_launch("argmax_final_kernel");
}


// Called by ouro_init with the device current: the null stream's key slots
// are allocated there, so ouro_finite_argmax on the null stream allocates
// nothing; any other stream gets its own slots on its first call.
int argmax_scratch_init(int) {
    if (!stream_scratch(SCRATCH_ARGMAX, kArgmaxBlocks * 8, nullptr, kArgmaxBlocks * 8))
        return fail(OURO_ERR_HIP, "argmax: scratch allocation failed");
    return OURO_OK;
}

}  // namespace ouro

using namespace ouro;

extern "C" {

int ouro_finite_argmax(const float *y, size_t n, int32_t *idx, void *stream) {
    OURO_REQUIRE_INIT();
    void *scratch = stream_scratch(SCRATCH_ARGMAX, kArgmaxBlocks * 8, stream, kArgmaxBlocks * 8);
    if (!scratch) return OURO_ERR_HIP;
    return argmax_f32(y, n, scratch, idx, stream);
}

}  // extern "C"
