// Per-token symmetric int8 quantizer for gfx950.
//
// Replaces the activation quantizer the reference calls before its GEMM
// (comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95), without the
// rotation, with the per-row semantics of the W8A8 workload:
//   s[m] = max_k |x[m,k]| / 127             (fp32, IEEE divide)
//   q[m,k] = clamp(rne(x[m,k] / s[m]), -127, 127)   (IEEE divide, half to even)
//   an all-zero row gives s = 0, q = 0.
//
// Design: one workgroup of 256 lanes per row; each lane loads 16-byte chunks
// (8 bf16) and keeps them in registers, so x is read from HBM once.  The max is
// order-independent, so a wave max (DPP/permute) plus an LDS step suffices.
// HBM traffic per row: 2K bytes in, K + 4 bytes out.
#include "common.h"

namespace h3mi {
namespace {

constexpr int QT = 256;  // lanes per row

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
    int8_t* qr = q + row * static_cast<int64_t>(K);
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
        const int c = it * QT + t;
        if (c < nch) {
            const uint32_t w4[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
            uint32_t packed[2] = {0u, 0u};
            if (sc != 0.0f) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float e = (j & 1) ? bf16_hi(w4[j >> 1]) : bf16_lo(w4[j >> 1]);
                    float r = rintf(e / sc);
                    r = fminf(fmaxf(r, -127.0f), 127.0f);
                    const uint32_t b = static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xFFu;
                    packed[j >> 2] |= b << ((j & 3) * 8);
                }
            }
            *reinterpret_cast<uint2*>(qr + c * 8) = make_uint2(packed[0], packed[1]);
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
    const int iters = static_cast<int>((K / 8 + QT - 1) / QT);
    dim3 grid(static_cast<unsigned>(M)), block(QT);
    hipStream_t st = as_stream(stream);
    if (iters <= 1) hipLaunchKernelGGL(quant_rowwise_kernel<1>, grid, block, 0, st, x, q, s, (int)K, ldx);
    else if (iters <= 2) hipLaunchKernelGGL(quant_rowwise_kernel<2>, grid, block, 0, st, x, q, s, (int)K, ldx);
    else if (iters <= 4) hipLaunchKernelGGL(quant_rowwise_kernel<4>, grid, block, 0, st, x, q, s, (int)K, ldx);
    else if (iters <= 8) hipLaunchKernelGGL(quant_rowwise_kernel<8>, grid, block, 0, st, x, q, s, (int)K, ldx);
    else hipLaunchKernelGGL(quant_rowwise_kernel<16>, grid, block, 0, st, x, q, s, (int)K, ldx);
    return check_launch("quant_rowwise");
}
