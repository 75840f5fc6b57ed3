// Per-token symmetric int8 quantizer for gfx950.
//
// Replaces the activation quantizer the reference calls before its GEMM
// (comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95), without the
// rotation, with the per-row semantics of the W8A8 workload:
//   s[m] = max_k |x[m,k]| / 127             (fp32, IEEE divide)
//   q[m,k] = clamp(rne(x[m,k] / s[m]), -127, 127)   (IEEE divide, half to even)
//   an all-zero row gives s = 0, q = 0.
//
// Design: 1, 2, 4 or 8 waves per row, the fewest that keep each wave at 8
// chunks of 512 elements or less (measured: one wave holding a
// 14336-element row ran at half the rate of four waves sharing it).  Each
// load instruction covers 1 KiB of the row contiguously and the chunks stay
// in registers, so x is read from HBM once; the max is order-independent (a
// wave max by lane exchange, then across the row's waves through LDS).  HBM
// traffic per row: 2K bytes in, K + 4 bytes out.
//
// The quotient: an IEEE divide per element costs about ten VALU instructions,
// as much time as the row's memory traffic.  Instead r = 1/s (one IEEE
// divide per row) and quant8 (common.h) forms the correctly rounded quotient
// from x * r with one fma correction, exact for bf16 x (checked exhaustively);
// a row whose s is below 2^-100 or not finite takes the exact divide.
#include <array>
#include <utility>

#include "common.h"

namespace h3mi {
namespace {

typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));

// Rows of any width up to 32768: WPR waves per row, IT chunks of 512
// elements per wave (lane l of wave w holds chunk elements
// ((it * WPR + w) * 64 + l) * 8 .. +7), rows_per_block(WPR) rows per
// workgroup.  Loads and stores are range-checked buffer operations, so no
// branch surrounds them and every load of the row is in flight at once; the
// row max crosses waves through LDS.  quant8's result does not depend on the
// lane layout, so this is bit-identical to the one-wave kernel.
template <int IT, int WPR>
__global__ __launch_bounds__(64 * WPR * rows_per_block(WPR)) void quant_multi_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ s, int M, int K, int64_t ldx) {
    constexpr int RPB = rows_per_block(WPR);
    __shared__ float red[WPR * RPB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wr = wave % WPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + wave / WPR;
    const bool in = row < M;
    const __amdgpu_buffer_rsrc_t rx = span_bytes(x + (in ? row : 0) * ldx, in ? K * 2 : 0);
    const __amdgpu_buffer_rsrc_t rq = span_bytes(q + (in ? row : 0) * static_cast<int64_t>(K), in ? K : 0);
    v4u32 v[IT];
    float amax = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int c = (it * WPR + wr) * 64 + lane;
        v[it] = __builtin_bit_cast(v4u32, __builtin_amdgcn_raw_buffer_load_b128(rx, c * 16, 0, 2));
    }
#pragma unroll
    for (int it = 0; it < IT; ++it)
#pragma unroll
        for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(v[it][j])), fabsf(bf16_hi(v[it][j]))));
    amax = wave_max(amax);
    if constexpr (WPR > 1) {
        if (lane == 0) red[wave] = amax;
        __syncthreads();
        const int w0 = wave - wr;
#pragma unroll
        for (int i = 0; i < WPR; ++i) amax = fmaxf(amax, red[w0 + i]);
    }
    amax = wave_uniform(amax);
    const float sc = amax / 127.0f;
    if (in && wr == 0 && lane == 0) s[row] = sc;
    const float r = 1.0f / sc;
    const bool exact = quot_exact(sc, r);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int c = (it * WPR + wr) * 64 + lane;
        const uint32_t w4[4] = {v[it][0], v[it][1], v[it][2], v[it][3]};
        const uint2 p = sc != 0.0f ? quant8(w4, sc, r, exact) : make_uint2(0u, 0u);
        // a cached store: the GEMM reads q next
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32, p), rq, c * 8, 0, 0);
    }
}

typedef void (*multi_fn)(const uint16_t*, int8_t*, float*, int, int, int64_t);

template <int WPR, int... I>
constexpr std::array<multi_fn, sizeof...(I)> multi_row(std::integer_sequence<int, I...>) {
    return {quant_multi_kernel<I + 1, WPR>...};
}

constexpr int kMultiMaxIt = 8;

multi_fn pick_multi(int it, int wpr) {
    static constexpr std::array<std::array<multi_fn, kMultiMaxIt>, 4> table = {
        multi_row<1>(std::make_integer_sequence<int, kMultiMaxIt>{}), multi_row<2>(std::make_integer_sequence<int, kMultiMaxIt>{}),
        multi_row<4>(std::make_integer_sequence<int, kMultiMaxIt>{}), multi_row<8>(std::make_integer_sequence<int, kMultiMaxIt>{})};
    const int wi = wpr == 1 ? 0 : wpr == 2 ? 1 : wpr == 4 ? 2 : wpr == 8 ? 3 : -1;
    if (wi < 0 || it < 1 || it > kMultiMaxIt) return nullptr;
    return table[wi][it - 1];
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
    // waves per row: the fewest of 1, 2, 4, 8 with at most kMultiMaxIt chunks of 512 elements per wave
    const int n64 = static_cast<int>((K / 8 + 63) / 64);
    int wpr = 1;
    while (wpr < 8 && (n64 + wpr - 1) / wpr > kMultiMaxIt) wpr *= 2;
    const multi_fn fn = pick_multi((n64 + wpr - 1) / wpr, wpr);
    if (!fn) return fail(H3MI_EINVAL, "quant: no kernel for K=%lld", (long long)K);
    const int rpb = rows_per_block(wpr);
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>((M + rpb - 1) / rpb)), dim3(64 * wpr * rpb), 0, as_stream(stream), x,
                       q, s, static_cast<int>(M), static_cast<int>(K), ldx);
    return check_launch("quant_rowwise");
}
