// libh3mi: error plumbing, version and the device-primitive entry points.
#include <atomic>
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace h3mi {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_last_error[0] = '\0';
    return H3MI_OK;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(H3MI_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

int cu_count() {
    static std::atomic<int> cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);  // racing threads store the same value
    return n;
}

__global__ void rsqrt_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t n, int mode) {
    int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = rsqrt_mode(in[i], mode);
}

__global__ void bf16_kernel(const float* __restrict__ in, uint16_t* __restrict__ out, int64_t n) {
    int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = bf16_bits(in[i]);
}

}  // namespace h3mi

using namespace h3mi;

extern "C" int h3mi_abi_version(void) { return H3MI_ABI_VERSION; }

extern "C" const char* h3mi_last_error(void) { return g_last_error; }

extern "C" int h3mi_debug_rsqrt_f32(const float* in, float* out, int64_t n, int mode, void* stream) {
    if (n < 0 || (n > 0 && (!in || !out))) return fail(H3MI_EINVAL, "debug_rsqrt: bad arguments");
    if (mode != H3MI_RSQRT_HW && mode != H3MI_RSQRT_RN) return fail(H3MI_EINVAL, "debug_rsqrt: mode %d", mode);
    if (n == 0) return ok();
    int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7FFFFFFF) return fail(H3MI_EINVAL, "debug_rsqrt: n too large");
    hipLaunchKernelGGL(rsqrt_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream), in, out, n, mode);
    return check_launch("debug_rsqrt");
}

extern "C" int h3mi_debug_bf16_rne(const float* in, uint16_t* out, int64_t n, void* stream) {
    if (n < 0 || (n > 0 && (!in || !out))) return fail(H3MI_EINVAL, "debug_bf16: bad arguments");
    if (n == 0) return ok();
    int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7FFFFFFF) return fail(H3MI_EINVAL, "debug_bf16: n too large");
    hipLaunchKernelGGL(bf16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream), in, out, n);
    return check_launch("debug_bf16");
}
