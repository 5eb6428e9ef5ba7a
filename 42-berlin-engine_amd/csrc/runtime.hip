// runtime.hip -- error reporting, device workspace and memory plumbing.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "be42_common.h"

namespace be42 {

static thread_local char t_err[512] = "";

void set_error(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof t_err, fmt, ap);
    va_end(ap);
}

int hip_fail(hipError_t e, const char *what, const char *file, int line)
{
    set_error("%s failed: %s (%s:%d)", what, hipGetErrorString(e), file, line);
    return e == hipErrorOutOfMemory ? BE42_ENOMEM : BE42_EHIP;
}

int upload_fp8_thresholds(int device);
int gemv_scratch_init(int device);

// Grow-only workspace per device.  Growth synchronises the stream first so
// that no queued kernel still reads the old buffer when it is freed.
struct Workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
};
static Workspace g_ws[64];
static std::mutex g_ws_mu;

void *workspace(size_t bytes, hipStream_t s)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return nullptr;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace &w = g_ws[dev];
    if (w.bytes >= bytes && w.ptr)
        return w.ptr;
    if (w.ptr) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(w.ptr);
        w.ptr = nullptr;
        w.bytes = 0;
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes + bytes / 4;
    if (hipMalloc(&w.ptr, want) != hipSuccess) {
        w.ptr = nullptr;
        set_error("workspace: hipMalloc(%zu) failed", want);
        return nullptr;
    }
    w.bytes = want;
    return w.ptr;
}

}  // namespace be42

using namespace be42;

extern "C" const char *be42_last_error(void) { return t_err; }

extern "C" int be42_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess)
        return 0;
    return n;
}

extern "C" int be42_init(int device)
{
    int n = be42_device_count();
    if (n <= 0) {
        set_error("be42_init: no HIP device");
        return BE42_ENODEV;
    }
    BE42_CHECK(device >= 0 && device < n, "be42_init: device %d out of range (%d devices)", device, n);
    BE42_HIP(hipSetDevice(device));
    const int rc = gemv_scratch_init(device);
    if (rc)
        return rc;
    return upload_fp8_thresholds(device);
}

extern "C" int be42_sync(void *stream)
{
    BE42_HIP(hipStreamSynchronize(as_stream(stream)));
    return BE42_OK;
}

extern "C" void *be42_malloc(size_t bytes)
{
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
        set_error("be42_malloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

extern "C" int be42_free(void *ptr)
{
    if (ptr)
        BE42_HIP(hipFree(ptr));
    return BE42_OK;
}

extern "C" int be42_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream)
{
    if (!bytes)
        return BE42_OK;
    BE42_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
    return BE42_OK;
}

extern "C" int be42_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream)
{
    if (!bytes)
        return BE42_OK;
    BE42_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
    BE42_HIP(hipStreamSynchronize(as_stream(stream)));
    return BE42_OK;
}

extern "C" int be42_memset(void *dst, int value, size_t bytes, void *stream)
{
    if (!bytes)
        return BE42_OK;
    BE42_HIP(hipMemsetAsync(dst, value, bytes, as_stream(stream)));
    return BE42_OK;
}
