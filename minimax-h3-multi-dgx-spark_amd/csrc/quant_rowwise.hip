// Per-token symmetric int8 quantizer for gfx950.
//
// Replaces the activation quantizer the reference calls before its GEMM
// (comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95), without the
// rotation, with the per-row semantics of the W8A8 workload:
//   s[m] = max_k |x[m,k]| / 127             (fp32, IEEE divide)
//   q[m,k] = clamp(rne(x[m,k] / s[m]), -127, 127)   (IEEE divide, half to even)
//   an all-zero row gives s = 0, q = 0.
//
// Design: one wave per row (rows up to 16384 elements; longer rows use a
// 256-lane workgroup).  Each load instruction covers 1 KiB of the row
// contiguously and the chunks stay in registers, so x is read from HBM once;
// the max is order-independent, so a wave max by lane exchange needs no LDS
// and no barrier.  HBM traffic per row: 2K bytes in, K + 4 bytes out.
//
// The quotient: an IEEE divide per element costs about ten VALU instructions,
// as much time as the row's memory traffic.  Instead t = x * r with
// r = 1/s (one IEEE divide per row): |t - fl(x/s)| < 2^-15 for |t| < 128, so
// rint(t) == rint(fl(x/s)) unless t lies within that distance of a
// half-integer.  A chunk with any element within 2^-12 of one, or a row whose
// s is not a normal number, takes the exact divide.
#include <array>
#include <utility>

#include "common.h"

namespace h3mi {
namespace {

constexpr int QT = 256;  // lanes per row
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));

// One wave per row, IT chunks of 8 elements per lane (lane l holds chunks
// it*64 + l), four rows per 256-thread workgroup.
template <int IT>
__global__ __launch_bounds__(256) void quant_wave_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ q,
                                                         float* __restrict__ s, int M, int K, int64_t ldx) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= M) return;  // whole wave
    const int nch = K / 8;
    const uint16_t* xr = x + row * ldx;
    uint4 v[IT];
    float amax = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int c = it * 64 + lane;
        v[it] = make_uint4(0, 0, 0, 0);
        if (c < nch) {
            const v4u32 t4 = __builtin_nontemporal_load(reinterpret_cast<const v4u32*>(xr + c * 8));
            v[it] = make_uint4(t4[0], t4[1], t4[2], t4[3]);
        }
        const uint32_t w4[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(w4[j])), fabsf(bf16_hi(w4[j]))));
    }
#pragma unroll
    for (int d = 32; d >= 1; d /= 2) amax = fmaxf(amax, __shfl_xor(amax, d, 64));
    const float sc = amax / 127.0f;
    if (lane == 0) s[row] = sc;
    const float r = 1.0f / sc;
    const bool fast = quot_fast(sc, r);
    int8_t* qr = q + row * static_cast<int64_t>(K);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int c = it * 64 + lane;
        if (c < nch) {
            const uint32_t w4[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
            const uint2 p = sc != 0.0f ? quant8(w4, sc, r, fast) : make_uint2(0u, 0u);
            __builtin_nontemporal_store(v2u32{p.x, p.y}, reinterpret_cast<v2u32*>(qr + c * 8));
        }
    }
}

typedef void (*wave_fn)(const uint16_t*, int8_t*, float*, int, int, int64_t);
template <int... I>
constexpr auto make_wave_table(std::integer_sequence<int, I...>) {
    return std::array<wave_fn, sizeof...(I)>{quant_wave_kernel<I + 1>...};
}
constexpr int kWaveMaxIt = 32;  // rows up to 32 * 512 = 16384 elements

template <int MAXIT>
__global__ __launch_bounds__(QT) void quant_rowwise_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ q,
                                                            float* __restrict__ s, int K, int64_t ldx) {
    __shared__ float red[QT / 64];
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x;
    const int nch = K / 8;
    const uint16_t* xr = x + row * ldx;
    uint4 v[MAXIT];
    float amax = 0.0f;
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
        const int c = it * QT + t;
        v[it] = make_uint4(0, 0, 0, 0);
        if (c < nch) {
            v[it] = *reinterpret_cast<const uint4*>(xr + c * 8);
            const uint32_t w4[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                amax = fmaxf(amax, fabsf(bf16_lo(w4[j])));
                amax = fmaxf(amax, fabsf(bf16_hi(w4[j])));
            }
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d /= 2) amax = fmaxf(amax, __shfl_xor(amax, d, 64));
    if ((t & 63) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = amax / 127.0f;
    if (t == 0) s[row] = sc;
    const float r = 1.0f / sc;
    const bool fast = quot_fast(sc, r);
    int8_t* qr = q + row * static_cast<int64_t>(K);
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
        const int c = it * QT + t;
        if (c < nch) {
            const uint32_t w4[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
            *reinterpret_cast<uint2*>(qr + c * 8) = sc != 0.0f ? quant8(w4, sc, r, fast) : make_uint2(0u, 0u);
        }
    }
}

}  // namespace
}  // namespace h3mi

using namespace h3mi;

extern "C" int h3mi_quant_rowwise_i8(const uint16_t* x, int8_t* q, float* s, int64_t M, int64_t K, int64_t ldx,
                                     void* stream) {
    if (M < 0 || K <= 0) return fail(H3MI_EINVAL, "quant: bad sizes M=%lld K=%lld", (long long)M, (long long)K);
    if (K % 8) return fail(H3MI_EINVAL, "quant: K=%lld must be a multiple of 8", (long long)K);
    if (K > 32768) return fail(H3MI_EINVAL, "quant: K=%lld exceeds 32768", (long long)K);
    if (ldx < K || ldx % 8) return fail(H3MI_EALIGN, "quant: ldx=%lld must be >= K and a multiple of 8", (long long)ldx);
    if (M > 0x7FFFFFFF) return fail(H3MI_EINVAL, "quant: M too large");
    if (M == 0) return ok();
    if (!x || !q || !s) return fail(H3MI_EINVAL, "quant: null pointer");
    if (!aligned(x, 16) || !aligned(q, 8) || !aligned(s, 4)) return fail(H3MI_EALIGN, "quant: x must be 16-byte and q 8-byte aligned");
    hipStream_t st = as_stream(stream);
    const int wit = static_cast<int>((K / 8 + 63) / 64);
    if (wit <= kWaveMaxIt) {
        static constexpr auto table = make_wave_table(std::make_integer_sequence<int, kWaveMaxIt>{});
        hipLaunchKernelGGL(table[wit - 1], dim3(static_cast<unsigned>((M + 3) / 4)), dim3(256), 0, st, x, q, s, (int)M,
                           (int)K, ldx);
        return check_launch("quant_rowwise");
    }
    const int iters = static_cast<int>((K / 8 + QT - 1) / QT);
    dim3 grid(static_cast<unsigned>(M)), block(QT);
    if (iters <= 1) hipLaunchKernelGGL(quant_rowwise_kernel<1>, grid, block, 0, st, x, q, s, (int)K, ldx);
    else if (iters <= 2) hipLaunchKernelGGL(quant_rowwise_kernel<2>, grid, block, 0, st, x, q, s, (int)K, ldx);
    else if (iters <= 4) hipLaunchKernelGGL(quant_rowwise_kernel<4>, grid, block, 0, st, x, q, s, (int)K, ldx);
    else if (iters <= 8) hipLaunchKernelGGL(quant_rowwise_kernel<8>, grid, block, 0, st, x, q, s, (int)K, ldx);
    else hipLaunchKernelGGL(quant_rowwise_kernel<16>, grid, block, 0, st, x, q, s, (int)K, ldx);
    return check_launch("quant_rowwise");
}
