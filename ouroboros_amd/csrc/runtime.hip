// runtime.hip - device selection, error reporting, memory/stream plumbing and
// the per-device library workspace of libouro_hip.
#include "common.hpp"

#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

namespace ouro {

int argmax_scratch_init(int dev);

namespace {
thread_local char g_err[512] = "";
int g_device = -1;
std::mutex g_ws_mu;
// Library scratch blocks, one per (device, stream, purpose): calls issued on
// different streams never share one.
struct Scratch {
    int dev;
    void *stream;
    int kind;
    void *ptr;
    size_t bytes;
};
std::vector<Scratch> g_scratch;
}  // namespace

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = '\0'; }
bool initialised() { return g_device >= 0; }
int current_device() { return g_device; }

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(OURO_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return OURO_OK;
}

void *stream_scratch(int kind, size_t bytes, void *stream, size_t min_bytes) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    const int dev = g_device;
    if (dev < 0) {
        fail(OURO_ERR_NOT_INIT, "ouro_init() not called");
        return nullptr;
    }
    Scratch *w = nullptr;
    for (Scratch &e : g_scratch)
        if (e.dev == dev && e.stream == stream && e.kind == kind) w = &e;
    if (w && w->bytes >= bytes) return w->ptr;
    if (w) {  // growing: work already queued on this stream may still read the old block
        if (hipStreamSynchronize(as_stream(stream)) != hipSuccess) {
            fail(OURO_ERR_HIP, "scratch: synchronize before growth failed");
            return nullptr;
        }
        (void)hipFree(w->ptr);
        w->ptr = nullptr;
        w->bytes = 0;
    } else {
        g_scratch.push_back(Scratch{dev, stream, kind, nullptr, 0});
        w = &g_scratch.back();
    }
    const size_t want = bytes < min_bytes ? min_bytes : bytes;
    if (hipMalloc(&w->ptr, want) != hipSuccess) {
        w->ptr = nullptr;
        fail(OURO_ERR_HIP, "scratch: hipMalloc(%zu) failed", want);
        return nullptr;
    }
    w->bytes = want;
    return w->ptr;
}

void *workspace(size_t bytes, void *stream) { return stream_scratch(SCRATCH_WORKSPACE, bytes, stream, 1u << 20); }

// Frees the scratch blocks of one stream (after its work has finished).
void release_stream_scratch(void *stream) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    for (size_t i = 0; i < g_scratch.size();) {
        if (g_scratch[i].stream == stream && g_scratch[i].dev == g_device) {
            (void)hipFree(g_scratch[i].ptr);
            g_scratch.erase(g_scratch.begin() + static_cast<long>(i));
        } else {
            ++i;
        }
    }
}

}  // namespace ouro

using namespace ouro;

extern "C" {

int ouro_abi_version(void) { return OURO_ABI_VERSION; }

const char *ouro_last_error(void) { return g_err; }

int ouro_device_count(int *count) {
    if (!count) return fail(OURO_ERR_INVALID_ARG, "count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        return fail(OURO_ERR_NO_DEVICE, "hipGetDeviceCount: %s", hipGetErrorString(e));
    }
    *count = n;
    return OURO_OK;
}

int ouro_init(int device) {
    clear_error();
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return fail(OURO_ERR_NO_DEVICE, "no HIP device (%s)",
                    e == hipSuccess ? "count 0" : hipGetErrorString(e));
    if (device < 0) {
        const char *env = getenv("OURO_GPU_INDEX");
        device = (env && *env) ? atoi(env) : 0;
    }
    if (device < 0 || device >= n)
        return fail(OURO_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, n);
    e = hipSetDevice(device);
    if (e != hipSuccess)
        return fail(OURO_ERR_NO_DEVICE, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess)
        return fail(OURO_ERR_NO_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(OURO_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950",
                    device, prop.gcnArchName);
    const int prev = g_device;
    g_device = device;
    const int st = argmax_scratch_init(device);
    if (st) {
        g_device = prev;
        return st;
    }
    return OURO_OK;
}

int ouro_shutdown(void) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    for (Scratch &e : g_scratch) {
        (void)hipSetDevice(e.dev);
        (void)hipDeviceSynchronize();
        (void)hipFree(e.ptr);
    }
    g_scratch.clear();
    if (g_device >= 0) (void)hipSetDevice(g_device);
    return OURO_OK;
}

int ouro_device_arch(char *buf, size_t len) {
    OURO_REQUIRE_INIT();
    if (!buf || !len) return fail(OURO_ERR_INVALID_ARG, "buf is NULL");
    hipDeviceProp_t prop;
    OURO_HIP_TRY(hipGetDeviceProperties(&prop, g_device));
    snprintf(buf, len, "%s", prop.gcnArchName);
    return OURO_OK;
}

int ouro_malloc(void **ptr, size_t bytes) {
    OURO_REQUIRE_INIT();
    if (!ptr || !bytes) return fail(OURO_ERR_INVALID_ARG, "ouro_malloc: bad args");
    OURO_HIP_TRY(hipMalloc(ptr, bytes));
    return OURO_OK;
}

int ouro_free(void *ptr) {
    OURO_REQUIRE_INIT();
    if (ptr) OURO_HIP_TRY(hipFree(ptr));
    return OURO_OK;
}

int ouro_memcpy_htod(void *dst, const void *src, size_t bytes) {
    OURO_REQUIRE_INIT();
    if (!bytes) return OURO_OK;
    if (!dst || !src) return fail(OURO_ERR_INVALID_ARG, "memcpy: NULL");
    OURO_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return OURO_OK;
}

int ouro_memcpy_dtoh(void *dst, const void *src, size_t bytes) {
    OURO_REQUIRE_INIT();
    if (!bytes) return OURO_OK;
    if (!dst || !src) return fail(OURO_ERR_INVALID_ARG, "memcpy: NULL");
    OURO_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return OURO_OK;
}

int ouro_memcpy_dtod(void *dst, const void *src, size_t bytes, void *stream) {
    OURO_REQUIRE_INIT();
    if (!bytes) return OURO_OK;
    if (!dst || !src) return fail(OURO_ERR_INVALID_ARG, "memcpy: NULL");
    OURO_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
    return OURO_OK;
}

int ouro_memset(void *dst, int value, size_t bytes, void *stream) {
    OURO_REQUIRE_INIT();
    if (!bytes) return OURO_OK;
    if (!dst) return fail(OURO_ERR_INVALID_ARG, "memset: NULL");
    OURO_HIP_TRY(hipMemsetAsync(dst, value, bytes, as_stream(stream)));
    return OURO_OK;
}

int ouro_stream_create(void **stream) {
    OURO_REQUIRE_INIT();
    if (!stream) return fail(OURO_ERR_INVALID_ARG, "stream is NULL");
    hipStream_t s;
    OURO_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return OURO_OK;
}

int ouro_stream_destroy(void *stream) {
    OURO_REQUIRE_INIT();
    if (stream) {
        OURO_HIP_TRY(hipStreamSynchronize(as_stream(stream)));
        release_stream_scratch(stream);
        OURO_HIP_TRY(hipStreamDestroy(as_stream(stream)));
    }
    return OURO_OK;
}

int ouro_stream_synchronize(void *stream) {
    OURO_REQUIRE_INIT();
    OURO_HIP_TRY(hipStreamSynchronize(as_stream(stream)));
    return OURO_OK;
}

int ouro_device_synchronize(void) {
    OURO_REQUIRE_INIT();
    OURO_HIP_TRY(hipDeviceSynchronize());
    return OURO_OK;
}

int ouro_event_create(void **event) {
    OURO_REQUIRE_INIT();
    if (!event) return fail(OURO_ERR_INVALID_ARG, "event is NULL");
    hipEvent_t e;
    OURO_HIP_TRY(hipEventCreate(&e));
    *event = e;
    return OURO_OK;
}

int ouro_event_destroy(void *event) {
    OURO_REQUIRE_INIT();
    if (event) OURO_HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    return OURO_OK;
}

int ouro_event_record(void *event, void *stream) {
    OURO_REQUIRE_INIT();
    if (!event) return fail(OURO_ERR_INVALID_ARG, "event is NULL");
    OURO_HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
    return OURO_OK;
}

int ouro_event_elapsed_ms(float *ms, void *start, void *stop) {
    OURO_REQUIRE_INIT();
    if (!ms || !start || !stop) return fail(OURO_ERR_INVALID_ARG, "event args NULL");
    OURO_HIP_TRY(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
    OURO_HIP_TRY(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                     reinterpret_cast<hipEvent_t>(stop)));
    return OURO_OK;
}

}  // extern "C"
