// xs_runtime.hip -- error plumbing and the device-memory shim of the C ABI
// (replaces xstar_cpp/src/cuda/cuda_allocator.cu:7-45 and the CHECK_CUDA
// message convention of xstar_cpp/include/cuda/cuda_check.h:23-31).
#include <stdarg.h>
#include <stdio.h>

#include "xs_device.hpp"

namespace xs {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

}  // namespace xs

extern "C" {

const char *xs_last_error(void) { return xs::g_last_error; }

int xs_device_count(int *count)
{
    XS_REQUIRE(count != nullptr, "count is null");
    XS_HIP(hipGetDeviceCount(count));
    return XS_OK;
}

int xs_malloc(void **ptr, size_t bytes)
{
    XS_REQUIRE(ptr != nullptr, "ptr is null");
    *ptr = nullptr;
    if (bytes == 0) bytes = 256;
    XS_HIP(hipMalloc(ptr, bytes));
    return XS_OK;
}

int xs_free(void *ptr)
{
    if (ptr) XS_HIP(hipFree(ptr));
    return XS_OK;
}

int xs_memcpy_h2d(void *dst, const void *src, size_t bytes)
{
    if (bytes) XS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return XS_OK;
}

int xs_memcpy_d2h(void *dst, const void *src, size_t bytes)
{
    if (bytes) XS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return XS_OK;
}

int xs_memcpy_d2d(void *dst, const void *src, size_t bytes)
{
    if (bytes) XS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return XS_OK;
}

int xs_free_bytes(size_t *free_bytes)
{
    size_t total = 0;
    XS_REQUIRE(free_bytes != nullptr, "free_bytes is null");
    XS_HIP(hipMemGetInfo(free_bytes, &total));
    return XS_OK;
}

int xs_stream_synchronize(void *stream)
{
    XS_HIP(hipStreamSynchronize((hipStream_t)stream));
    return XS_OK;
}

}  // extern "C"
