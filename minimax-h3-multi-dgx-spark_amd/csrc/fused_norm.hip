// Fused RMSNorm + adaLN modulation (+ gate/residual) kernels for gfx950.
//
// Reference: comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py
//   norm_mod        :88-114, wrapper :174-178
//   gate_norm_mod_  :117-155, wrapper :181-185
//   gate_           :158-167, wrapper :188-192
//
// Design (MI355X): one workgroup per row; the row stays in registers between
// the sum-of-squares reduction and the output pass, so HBM sees exactly one
// read of x (and o) and one write of h (and x): the reference reads x twice.
// The reduction order is a template parameter <NUMX, WARP>: logical thread t
// (one per hardware lane) sums x^2 over its 4-element chunks t, t+NUMX, ...
// in sequence, then a shuffle-down tree of width WARP (32 = half a wave64,
// 64 = a full wave), then the halving tree across warps.  Chunk loads are
// 8 bytes per lane, so a wave reads 512 contiguous bytes per instruction.
#include "common.h"

namespace h3mi {
namespace {

constexpr int VEC = 4;

struct Chunk {  // 4 bf16 values as two packed pairs
    uint32_t lo, hi;
};

__device__ __forceinline__ Chunk load_chunk(const uint16_t* p) {
    uint2 v = *reinterpret_cast<const uint2*>(p);
    return {v.x, v.y};
}

__device__ __forceinline__ void store_chunk(uint16_t* p, uint32_t lo, uint32_t hi) {
    *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}

// Halving tree over the per-lane partial sums, in the reference order:
// in-warp shuffle-down offsets WARP/2 .. 1, then warp totals combined by the
// same halving tree.  Returns the row total on every lane.
template <int NUMX, int WARP>
__device__ __forceinline__ float row_total(float acc, float* red) {
    constexpr int NW = NUMX / WARP;
#pragma unroll
    for (int d = WARP / 2; d >= 1; d /= 2) acc += __shfl_down(acc, d, WARP);
    const int t = threadIdx.x;
    if constexpr (NW > 1) {
        if ((t % WARP) == 0) red[t / WARP] = acc;
        __syncthreads();
        if (t == 0) {
            float w[NW];
#pragma unroll
            for (int i = 0; i < NW; ++i) w[i] = red[i];
#pragma unroll
            for (int d = NW / 2; d >= 1; d /= 2)
#pragma unroll
                for (int i = 0; i < d; ++i) w[i] = w[i] + w[i + d];
            red[NW] = w[0];
        }
        __syncthreads();
        return red[NW];
    } else {
        return __shfl(acc, 0, WARP);
    }
}

// One row per workgroup of NUMX threads; MAXIT = register-resident chunks per
// thread (N <= NUMX * 4 * MAXIT).  GATE selects gate_norm_mod_.
template <int NUMX, int WARP, int MAXIT, bool GATE>
__global__ __launch_bounds__(NUMX) void norm_mod_kernel(
    uint16_t* __restrict__ x, const uint16_t* __restrict__ o, const uint16_t* __restrict__ g,
    const uint16_t* __restrict__ w, const int32_t* __restrict__ ridx,
    const uint16_t* __restrict__ s1, const uint16_t* __restrict__ sh, uint16_t* __restrict__ h,
    int N, int R, float eps, int rsq_mode, float* __restrict__ row_var, float* __restrict__ row_rstd) {
    __shared__ float red[NUMX / WARP + 1];
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x;
    const int r = ridx[row];
    if (r < 0 || r >= R) return;  // uniform across the workgroup
    const int nch = N / VEC;
    uint16_t* xr = x + row * N;
    const int64_t tab = static_cast<int64_t>(r) * N;

    Chunk v[MAXIT];
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
        const int c = it * NUMX + t;
        v[it] = {0u, 0u};
        if (c < nch) {
            Chunk xc = load_chunk(xr + c * VEC);
            if constexpr (GATE) {
                // xn = rb(x + o*g): o*g of two bf16 is exact in fp32
                Chunk oc = load_chunk(o + row * N + c * VEC);
                Chunk gc = load_chunk(g + tab + c * VEC);
                float a0 = bf16_lo(xc.lo) + bf16_lo(oc.lo) * bf16_lo(gc.lo);
                float a1 = bf16_hi(xc.lo) + bf16_hi(oc.lo) * bf16_hi(gc.lo);
                float a2 = bf16_lo(xc.hi) + bf16_lo(oc.hi) * bf16_lo(gc.hi);
                float a3 = bf16_hi(xc.hi) + bf16_hi(oc.hi) * bf16_hi(gc.hi);
                xc = {bf16x2_bits(a0, a1), bf16x2_bits(a2, a3)};
            }
            v[it] = xc;
            const float e0 = bf16_lo(xc.lo), e1 = bf16_hi(xc.lo), e2 = bf16_lo(xc.hi), e3 = bf16_hi(xc.hi);
            acc += e0 * e0;
            acc += e1 * e1;
            acc += e2 * e2;
            acc += e3 * e3;
        }
    }
    const float tot = row_total<NUMX, WARP>(acc, red);
    const float var = tot / static_cast<float>(N) + eps;
    const float rstd = rsqrt_mode(var, rsq_mode);
    if (t == 0) {
        if (row_var) row_var[row] = var;
        if (row_rstd) row_rstd[row] = rstd;
    }
    uint16_t* hr = h + row * N;
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
        const int c = it * NUMX + t;
        if (c < nch) {
            const Chunk xc = v[it];
            if constexpr (GATE) store_chunk(xr + c * VEC, xc.lo, xc.hi);
            const Chunk wc = load_chunk(w + c * VEC);
            const Chunk sc = load_chunk(s1 + tab + c * VEC);
            const Chunk hc = load_chunk(sh + tab + c * VEC);
            float o4[4];
            const float xe[4] = {bf16_lo(xc.lo), bf16_hi(xc.lo), bf16_lo(xc.hi), bf16_hi(xc.hi)};
            const float we[4] = {bf16_lo(wc.lo), bf16_hi(wc.lo), bf16_lo(wc.hi), bf16_hi(wc.hi)};
            const float se[4] = {bf16_lo(sc.lo), bf16_hi(sc.lo), bf16_lo(sc.hi), bf16_hi(sc.hi)};
            const float he[4] = {bf16_lo(hc.lo), bf16_hi(hc.lo), bf16_lo(hc.hi), bf16_hi(hc.hi)};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float y = rb(we[e] * (rstd * xe[e]));
                y = rb(y * se[e]);
                o4[e] = y + he[e];
            }
            store_chunk(hr + c * VEC, bf16x2_bits(o4[0], o4[1]), bf16x2_bits(o4[2], o4[3]));
        }
    }
}

// gate_: x <- bf16(x + o*g[ridx[row]]).  Grid (rows, column blocks); each
// lane handles one 4-element chunk.
__global__ __launch_bounds__(256) void gate_kernel(uint16_t* __restrict__ x, const uint16_t* __restrict__ o,
                                                   const uint16_t* __restrict__ g, const int32_t* __restrict__ ridx,
                                                   int N, int R) {
    const int64_t row = blockIdx.x;
    const int c = blockIdx.y * 256 + threadIdx.x;
    if (c * VEC >= N) return;
    const int r = ridx[row];
    if (r < 0 || r >= R) return;
    uint16_t* xp = x + row * N + c * VEC;
    const Chunk xc = load_chunk(xp);
    const Chunk oc = load_chunk(o + row * N + c * VEC);
    const Chunk gc = load_chunk(g + static_cast<int64_t>(r) * N + c * VEC);
    float a0 = bf16_lo(xc.lo) + bf16_lo(oc.lo) * bf16_lo(gc.lo);
    float a1 = bf16_hi(xc.lo) + bf16_hi(oc.lo) * bf16_hi(gc.lo);
    float a2 = bf16_lo(xc.hi) + bf16_lo(oc.hi) * bf16_lo(gc.hi);
    float a3 = bf16_hi(xc.hi) + bf16_hi(oc.hi) * bf16_hi(gc.hi);
    store_chunk(xp, bf16x2_bits(a0, a1), bf16x2_bits(a2, a3));
}

struct OrderDesc {
    int numx, warp;
};

constexpr OrderDesc kOrders[H3MI_ORDER_COUNT] = {
    {256, 64},  // DEFAULT: eager PyTorch rms_norm on ROCm (wave64, 4 warps)
    {128, 32},  // REF
    {256, 64},  // W64
};

template <int NUMX, int WARP, bool GATE>
int launch_order(uint16_t* x, const uint16_t* o, const uint16_t* g, const uint16_t* w, const int32_t* ridx,
                 const uint16_t* s1, const uint16_t* sh, uint16_t* h, int64_t S, int N, int R, float eps,
                 int rsq, float* var, float* rstd, hipStream_t st) {
    const int iters = (N / VEC + NUMX - 1) / NUMX;
    dim3 grid(static_cast<unsigned>(S)), block(NUMX);
#define H3MI_NORM_LAUNCH(MI)                                                                                  \
    hipLaunchKernelGGL((norm_mod_kernel<NUMX, WARP, MI, GATE>), grid, block, 0, st, x, o, g, w, ridx, s1, sh, h, \
                       N, R, eps, rsq, var, rstd)
    if (iters <= 2) H3MI_NORM_LAUNCH(2);
    else if (iters <= 4) H3MI_NORM_LAUNCH(4);
    else if (iters <= 6) H3MI_NORM_LAUNCH(6);
    else if (iters <= 8) H3MI_NORM_LAUNCH(8);
    else if (iters <= 12) H3MI_NORM_LAUNCH(12);
    else if (iters <= 16) H3MI_NORM_LAUNCH(16);
    else if (iters <= 24) H3MI_NORM_LAUNCH(24);
    else if (iters <= 32) H3MI_NORM_LAUNCH(32);
    else if (iters <= 64) H3MI_NORM_LAUNCH(64);
    else return fail(H3MI_EINVAL, "norm: N=%d exceeds the register-resident limit %d", N, NUMX * VEC * 64);
#undef H3MI_NORM_LAUNCH
    return check_launch(GATE ? "gate_norm_mod" : "norm_mod");
}

template <bool GATE>
int norm_entry(uint16_t* x, const uint16_t* o, const uint16_t* g, const uint16_t* w, const int32_t* ridx,
               const uint16_t* s1, const uint16_t* sh, uint16_t* h, int64_t S, int64_t N, int64_t R, float eps,
               int order, int rsq, float* var, float* rstd, void* stream) {
    const char* name = GATE ? "gate_norm_mod" : "norm_mod";
    if (S < 0 || N <= 0 || R <= 0) return fail(H3MI_EINVAL, "%s: bad sizes S=%lld N=%lld R=%lld", name, (long long)S, (long long)N, (long long)R);
    if (N % VEC) return fail(H3MI_EINVAL, "%s: N=%lld must be a multiple of 4", name, (long long)N);
    if (N > (1 << 24)) return fail(H3MI_EINVAL, "%s: N too large", name);
    if (S > 0x7FFFFFFF) return fail(H3MI_EINVAL, "%s: S too large", name);
    if (order < 0 || order >= H3MI_ORDER_COUNT) return fail(H3MI_EINVAL, "%s: unknown order %d", name, order);
    if (rsq != H3MI_RSQRT_HW && rsq != H3MI_RSQRT_RN) return fail(H3MI_EINVAL, "%s: unknown rsqrt mode %d", name, rsq);
    if (S == 0) return ok();
    if (!x || !w || !ridx || !s1 || !sh || !h || (GATE && (!o || !g))) return fail(H3MI_EINVAL, "%s: null pointer", name);
    const void* ptrs[] = {x, w, s1, sh, h, o, g};
    for (const void* p : ptrs)
        if (p && !aligned(p, 8)) return fail(H3MI_EALIGN, "%s: tensors must be 8-byte aligned", name);
    const size_t xb = static_cast<size_t>(S) * N * 2;
    if (overlap(h, xb, x, xb)) return fail(H3MI_EALIAS, "%s: h overlaps x", name);
    if (GATE) {
        if (overlap(o, xb, x, xb)) return fail(H3MI_EALIAS, "%s: o overlaps x", name);
        if (overlap(g, static_cast<size_t>(R) * N * 2, x, xb)) return fail(H3MI_EALIAS, "%s: g overlaps x", name);
    }
    const OrderDesc od = kOrders[order];
    hipStream_t st = as_stream(stream);
    if (od.numx == 128 && od.warp == 32)
        return launch_order<128, 32, GATE>(x, o, g, w, ridx, s1, sh, h, S, (int)N, (int)R, eps, rsq, var, rstd, st);
    return launch_order<256, 64, GATE>(x, o, g, w, ridx, s1, sh, h, S, (int)N, (int)R, eps, rsq, var, rstd, st);
}

}  // namespace
}  // namespace h3mi

using namespace h3mi;

extern "C" int h3mi_norm_order_info(int order, int* numx, int* vec, int* warp) {
    if (order < 0 || order >= H3MI_ORDER_COUNT) return fail(H3MI_EINVAL, "unknown order %d", order);
    if (numx) *numx = kOrders[order].numx;
    if (vec) *vec = VEC;
    if (warp) *warp = kOrders[order].warp;
    return ok();
}

extern "C" int h3mi_norm_mod_bf16_ex(const uint16_t* x, const uint16_t* w, const int32_t* ridx, const uint16_t* s1,
                                     const uint16_t* sh, uint16_t* h, int64_t S, int64_t N, int64_t R, float eps,
                                     int order, int rsq, float* row_var, float* row_rstd, void* stream) {
    return norm_entry<false>(const_cast<uint16_t*>(x), nullptr, nullptr, w, ridx, s1, sh, h, S, N, R, eps, order, rsq,
                             row_var, row_rstd, stream);
}

extern "C" int h3mi_norm_mod_bf16(const uint16_t* x, const uint16_t* w, const int32_t* ridx, const uint16_t* s1,
                                  const uint16_t* sh, uint16_t* h, int64_t S, int64_t N, int64_t R, float eps,
                                  void* stream) {
    return h3mi_norm_mod_bf16_ex(x, w, ridx, s1, sh, h, S, N, R, eps, H3MI_ORDER_DEFAULT, H3MI_RSQRT_HW, nullptr,
                                 nullptr, stream);
}

extern "C" int h3mi_gate_norm_mod_bf16_ex(uint16_t* x, const uint16_t* o, const uint16_t* g, const uint16_t* w,
                                          const int32_t* ridx, const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                                          int64_t S, int64_t N, int64_t R, float eps, int order, int rsq,
                                          float* row_var, float* row_rstd, void* stream) {
    return norm_entry<true>(x, o, g, w, ridx, s1, sh, h, S, N, R, eps, order, rsq, row_var, row_rstd, stream);
}

extern "C" int h3mi_gate_norm_mod_bf16(uint16_t* x, const uint16_t* o, const uint16_t* g, const uint16_t* w,
                                       const int32_t* ridx, const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                                       int64_t S, int64_t N, int64_t R, float eps, void* stream) {
    return h3mi_gate_norm_mod_bf16_ex(x, o, g, w, ridx, s1, sh, h, S, N, R, eps, H3MI_ORDER_DEFAULT, H3MI_RSQRT_HW,
                                      nullptr, nullptr, stream);
}

extern "C" int h3mi_gate_bf16(uint16_t* x, const uint16_t* o, const uint16_t* g, const int32_t* ridx, int64_t S,
                              int64_t N, int64_t R, void* stream) {
    if (S < 0 || N <= 0 || R <= 0) return fail(H3MI_EINVAL, "gate: bad sizes");
    if (N % VEC) return fail(H3MI_EINVAL, "gate: N=%lld must be a multiple of 4", (long long)N);
    if (S > 0x7FFFFFFF || N > (1 << 24)) return fail(H3MI_EINVAL, "gate: sizes too large");
    if (S == 0) return ok();
    if (!x || !o || !g || !ridx) return fail(H3MI_EINVAL, "gate: null pointer");
    if (!aligned(x, 8) || !aligned(o, 8) || !aligned(g, 8)) return fail(H3MI_EALIGN, "gate: tensors must be 8-byte aligned");
    const size_t xb = static_cast<size_t>(S) * N * 2;
    if (overlap(o, xb, x, xb)) return fail(H3MI_EALIAS, "gate: o overlaps x");
    if (overlap(g, static_cast<size_t>(R) * N * 2, x, xb)) return fail(H3MI_EALIAS, "gate: g overlaps x");
    const int nch = static_cast<int>(N / VEC);
    dim3 grid(static_cast<unsigned>(S), (nch + 255) / 256);
    hipLaunchKernelGGL(gate_kernel, grid, dim3(256), 0, as_stream(stream), x, o, g, ridx, (int)N, (int)R);
    return check_launch("gate");
}
