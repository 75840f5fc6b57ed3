// Shared helpers of libh3mi: argument checking, error plumbing and the device
// arithmetic primitives (bf16 rounding, rsqrt modes) every kernel uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/h3mi.h"

namespace h3mi {

// Records the message for h3mi_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);
// Clears the thread's last error and returns H3MI_OK.
int ok();
// Checks hipGetLastError() after a launch.
int check_launch(const char* what);
// Compute units of the current device (cached per device; 256 if unknown).
int cu_count();

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// [a, a+na) and [b, b+nb) (bytes) overlap.
inline bool overlap(const void* a, size_t na, const void* b, size_t nb) {
    uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + nb && y < x + na;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------------ device arithmetic

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t bf16_bits(float v) {
    __bf16 b = static_cast<__bf16>(v);
    return __builtin_bit_cast(uint16_t, b);
}

// Two fp32 -> packed bf16 pair (lo in bits 0..15), round to nearest even.
__device__ __forceinline__ uint32_t bf16x2_bits(float lo, float hi) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 r = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float bf16_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

// Round an fp32 to bf16 precision and keep it as fp32 (the reference's _rbf16).
__device__ __forceinline__ float rb(float v) { return bf16_f32(bf16_bits(v)); }

// Correctly rounded fp32 1/sqrt(v) for finite v > 0: estimate, then pick the
// neighbour whose midpoints bracket 1/sqrt(v), decided by the exact sign of
// m*m*v - 1 (m has 25 significant bits, so m*m is exact in fp64 and one fp64
// fma gives the sign exactly).
__device__ __forceinline__ float rsqrt_rn(float v) {
    if (!(v > 0.0f) || __builtin_isinf(v)) return rsqrtf(v);
    float y = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(v)));
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        // y is a positive normal float here, so its neighbours are +-1 ulp in bits
        float up = __uint_as_float(__float_as_uint(y) + 1u);
        float dn = __uint_as_float(__float_as_uint(y) - 1u);
        double mhi = 0.5 * (static_cast<double>(y) + static_cast<double>(up));
        double mlo = 0.5 * (static_cast<double>(y) + static_cast<double>(dn));
        if (__builtin_fma(mhi * mhi, static_cast<double>(v), -1.0) < 0.0) { y = up; continue; }
        if (__builtin_fma(mlo * mlo, static_cast<double>(v), -1.0) > 0.0) { y = dn; continue; }
        break;
    }
    return y;
}

__device__ __forceinline__ float rsqrt_mode(float v, int mode) {
    return mode == H3MI_RSQRT_RN ? rsqrt_rn(v) : rsqrtf(v);
}

}  // namespace h3mi
