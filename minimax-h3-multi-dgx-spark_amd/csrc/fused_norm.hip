// Fused RMSNorm + adaLN modulation (+ gate/residual) kernels for gfx950.
//
// Reference: comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py
//   norm_mod        :88-114, wrapper :174-178
//   gate_norm_mod_  :117-155, wrapper :181-185
//   gate_           :158-167, wrapper :188-192
//
// Design (MI355X): each row stays in registers between the sum-of-squares
// reduction and the output pass, so HBM sees exactly one read of x (and o)
// and one write of h (and x); the reference reads x twice.  For rows of up to
// 8192 elements (N % 8 == 0) persistent row-stream kernels run one wave per
// row with one row of lookahead; wider rows use one wave per row without
// lookahead, or one workgroup per row.  The reduction order is a template
// parameter <NUMX, WARP>: logical thread t sums x^2 over its 4-element chunks
// t, t+NUMX, ... in sequence, then a shuffle-down tree of width WARP (32 =
// half a wave64, 64 = a full wave), then the halving tree across warps.
#include <type_traits>
#include <utility>

#include "common.h"

namespace h3mi {
namespace {

// f(std::integral_constant<int, i>{}) for i = 0..N-1 (compile-time indices).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

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

// ------------------------------------------------------------------ one wave per row
//
// The main kernels.  One 64-lane wave computes a whole row.  An iteration of
// the reduction order covers NUMX*4 elements (NUMX logical threads x 4); the
// wave reads it with H = NUMX/128 load instructions of 16 bytes per lane, each
// covering 1 KiB contiguously, so lane q's h-th load holds the chunks of
// logical threads h*128 + 2q and h*128 + 2q + 1.  Every logical thread keeps
// its own accumulator and the order is kept exactly:
//   * in-warp shuffle-down levels with logical offset >= 2 are lane shuffles
//     of width WARP/2 at half the offset; offset 1 adds the lane's pair;
//   * the halving tree over the NUMX/WARP warp totals pairs warps held by the
//     same lane (other half) with in-lane adds and the rest with shuffles.
// No LDS and no barrier.  x/o are read and h/x written with non-temporal
// hints (streamed once); w and the adaLN tables stay cacheable.

typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));
typedef int32_t v4i_t __attribute__((ext_vector_type(4)));
typedef int32_t v2i_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v4u_t ld16(const uint16_t* ptr, bool stream) {
    const v4u_t* a = reinterpret_cast<const v4u_t*>(ptr);
    return stream ? __builtin_nontemporal_load(a) : *a;
}

__device__ __forceinline__ void st16(uint16_t* ptr, v4u_t v) {
    __builtin_nontemporal_store(v, reinterpret_cast<v4u_t*>(ptr));
}

// xn = rb(x + o*g) on 8 packed elements (o*g of two bf16 is exact in fp32)
__device__ __forceinline__ v4u_t gate8(v4u_t x, v4u_t o, v4u_t g) {
    v4u_t r;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        r[q] = bf16x2_bits(bf16_lo(x[q]) + bf16_lo(o[q]) * bf16_lo(g[q]),
                           bf16_hi(x[q]) + bf16_hi(o[q]) * bf16_hi(g[q]));
    return r;
}

// h = bf16(rb(rb(w*(rstd*x)) * s1) + sh) on 8 packed elements
__device__ __forceinline__ v4u_t mod8(v4u_t x, v4u_t w, v4u_t s, v4u_t t, float rstd) {
    v4u_t r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float y0 = bf16_lo(w[q]) * (rstd * bf16_lo(x[q]));
        float y1 = bf16_hi(w[q]) * (rstd * bf16_hi(x[q]));
        rb2(y0, y1);
        y0 *= bf16_lo(s[q]);
        y1 *= bf16_hi(s[q]);
        rb2(y0, y1);
        r[q] = bf16x2_bits(y0 + bf16_lo(t[q]), y1 + bf16_hi(t[q]));
    }
    return r;
}

// Table source for the modulation pass: global memory (the row's own table
// row) or a copy staged in LDS for a block of rows that share one.
struct GlobalTabs {
    const uint16_t *w, *s1, *sh, *g;  // s1/sh/g already offset to the table row
    __device__ __forceinline__ v4u_t W(int e) const { return ld16(w + e, false); }
    __device__ __forceinline__ v4u_t S1(int e) const { return ld16(s1 + e, false); }
    __device__ __forceinline__ v4u_t SH(int e) const { return ld16(sh + e, false); }
    __device__ __forceinline__ v4u_t G(int e) const { return ld16(g + e, false); }
    __device__ __forceinline__ Chunk cW(int e) const { return load_chunk(w + e); }
    __device__ __forceinline__ Chunk cS1(int e) const { return load_chunk(s1 + e); }
    __device__ __forceinline__ Chunk cSH(int e) const { return load_chunk(sh + e); }
    __device__ __forceinline__ Chunk cG(int e) const { return load_chunk(g + e); }
};

struct LdsTabs {
    const uint16_t* t;  // [w | s1 | sh | g], N elements each
    int n;
    __device__ __forceinline__ v4u_t at(int k, int e) const { return *reinterpret_cast<const v4u_t*>(t + k * n + e); }
    __device__ __forceinline__ Chunk cat(int k, int e) const {
        const uint2 v = *reinterpret_cast<const uint2*>(t + k * n + e);
        return {v.x, v.y};
    }
    __device__ __forceinline__ v4u_t W(int e) const { return at(0, e); }
    __device__ __forceinline__ v4u_t S1(int e) const { return at(1, e); }
    __device__ __forceinline__ v4u_t SH(int e) const { return at(2, e); }
    __device__ __forceinline__ v4u_t G(int e) const { return at(3, e); }
    __device__ __forceinline__ Chunk cW(int e) const { return cat(0, e); }
    __device__ __forceinline__ Chunk cS1(int e) const { return cat(1, e); }
    __device__ __forceinline__ Chunk cSH(int e) const { return cat(2, e); }
    __device__ __forceinline__ Chunk cG(int e) const { return cat(3, e); }
};

// One row on one wave (lane q = threadIdx.x & 63), split in two phases so a
// wave can issue the next row's loads before storing the current one:
//   load_row_phase: x (and o, g) into registers, sum of squares in the
//                   reduction order, rstd;
//   mod_row_phase:  x written back (gate), h = modulated norm.
template <int NUMX, int MAXIT>
struct RowRegs {
    v4u_t v[MAXIT][NUMX / 128];
};

template <int NUMX, int WARP, int MAXIT, bool GATE, class TB>
__device__ __forceinline__ void load_row_phase(RowRegs<NUMX, MAXIT>& rr, float (&acc)[NUMX / 128][2],
                                               const uint16_t* __restrict__ x, const uint16_t* __restrict__ o,
                                               const TB& tb, int64_t row, int N) {
    constexpr int H = NUMX / 128;
#pragma unroll
    for (int hh = 0; hh < H; ++hh) acc[hh][0] = acc[hh][1] = 0.0f;
    const int q = threadIdx.x & 63;
    const uint16_t* xr = x + row * N;
    const bool full_rows = (N % (NUMX * 4)) == 0;
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
#pragma unroll
        for (int hh = 0; hh < H; ++hh) {
            const int e = it * NUMX * 4 + hh * 512 + q * 8;   // first of this lane's 8 elements
            v4u_t xv = {0u, 0u, 0u, 0u};
            if (e + 8 <= N) {
                xv = ld16(xr + e, true);
                if constexpr (GATE) xv = gate8(xv, ld16(o + row * N + e, true), tb.G(e));
            } else if (!full_rows && e < N) {                  // N % 4 == 0: one 4-element chunk left
                Chunk c = load_chunk(xr + e);
                if constexpr (GATE) {
                    const Chunk oc = load_chunk(o + row * N + e), gc = tb.cG(e);
                    c = {bf16x2_bits(bf16_lo(c.lo) + bf16_lo(oc.lo) * bf16_lo(gc.lo),
                                     bf16_hi(c.lo) + bf16_hi(oc.lo) * bf16_hi(gc.lo)),
                         bf16x2_bits(bf16_lo(c.hi) + bf16_lo(oc.hi) * bf16_lo(gc.hi),
                                     bf16_hi(c.hi) + bf16_hi(oc.hi) * bf16_hi(gc.hi))};
                }
                xv[0] = c.lo;
                xv[1] = c.hi;
            }
            rr.v[it][hh] = xv;
            // logical thread hh*128 + 2q sums elements 0..3 of its chunk, thread
            // +1 elements 4..7, in iteration order; elements past N are zero
            const float e0 = bf16_lo(xv[0]), e1 = bf16_hi(xv[0]), e2 = bf16_lo(xv[1]), e3 = bf16_hi(xv[1]);
            const float e4 = bf16_lo(xv[2]), e5 = bf16_hi(xv[2]), e6 = bf16_lo(xv[3]), e7 = bf16_hi(xv[3]);
            acc[hh][0] += e0 * e0;
            acc[hh][0] += e1 * e1;
            acc[hh][0] += e2 * e2;
            acc[hh][0] += e3 * e3;
            acc[hh][1] += e4 * e4;
            acc[hh][1] += e5 * e5;
            acc[hh][1] += e6 * e6;
            acc[hh][1] += e7 * e7;
        }
    }
}

template <int NUMX, int WARP>
__device__ __forceinline__ float reduce_rstd(float (&acc)[NUMX / 128][2], int64_t row, int N, float eps,
                                            int rsq_mode, float* __restrict__ row_var, float* __restrict__ row_rstd) {
    constexpr int H = NUMX / 128;        // 1 KiB loads per iteration
    constexpr int PW = WARP / 2;         // lanes per logical warp
    constexpr int WPH = 64 / PW;         // logical warps per half
    constexpr int NW = NUMX / WARP;      // logical warps
    static_assert(NUMX % 128 == 0 && WARP >= 4 && WARP <= 128 && 64 % PW == 0, "order must map onto one wave");
    const int q = threadIdx.x & 63;
    // in-warp tree: logical offsets WARP/2 .. 2 as lane shuffles, then 1
    static_for<ilog2(WARP) - 1>([&](auto i_c) {
        constexpr int d = (WARP / 2) >> decltype(i_c)::value;
#pragma unroll
        for (int hh = 0; hh < H; ++hh) {
            acc[hh][0] += __shfl_down(acc[hh][0], d / 2, PW);
            acc[hh][1] += __shfl_down(acc[hh][1], d / 2, PW);
        }
    });
    float t[H];
#pragma unroll
    for (int hh = 0; hh < H; ++hh) t[hh] = acc[hh][0] + acc[hh][1];
    // halving tree over warps k = hh*WPH + lane/PW
    static_for<ilog2(NW)>([&](auto i_c) {
        constexpr int d = (NW / 2) >> decltype(i_c)::value;
        if constexpr (d >= WPH) {
            static_for<H>([&](auto h_c) {
                constexpr int hh = decltype(h_c)::value;
                if constexpr (hh + d / WPH < H) t[hh] = t[hh] + t[hh + d / WPH];
            });
        } else {
#pragma unroll
            for (int hh = 0; hh < H; ++hh) t[hh] = t[hh] + __shfl_down(t[hh], d * PW, 64);
        }
    });
    const float tot = __shfl(t[0], 0, 64);
    const float var = tot / static_cast<float>(N) + eps;
    const float rstd = rsqrt_mode(var, rsq_mode);
    if (q == 0) {
        if (row_var) row_var[row] = var;
        if (row_rstd) row_rstd[row] = rstd;
    }
    return rstd;
}

template <int NUMX, int MAXIT, bool GATE, class TB>
__device__ __forceinline__ void mod_row_phase(const RowRegs<NUMX, MAXIT>& rr, uint16_t* __restrict__ x,
                                              const TB& tb, uint16_t* __restrict__ h, int64_t row, int N, float rstd) {
    constexpr int H = NUMX / 128;
    const int q = threadIdx.x & 63;
    uint16_t* xr = x + row * N;
    uint16_t* hr = h + row * N;
    const bool full_rows = (N % (NUMX * 4)) == 0;
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
#pragma unroll
        for (int hh = 0; hh < H; ++hh) {
            const int e = it * NUMX * 4 + hh * 512 + q * 8;
            if (e + 8 <= N) {
                if constexpr (GATE) st16(xr + e, rr.v[it][hh]);
                st16(hr + e, mod8(rr.v[it][hh], tb.W(e), tb.S1(e), tb.SH(e), rstd));
            } else if (!full_rows && e < N) {
                if constexpr (GATE) store_chunk(xr + e, rr.v[it][hh][0], rr.v[it][hh][1]);
                const Chunk wc = tb.cW(e), sc = tb.cS1(e), tc = tb.cSH(e);
                const v4u_t o4 = mod8(v4u_t{rr.v[it][hh][0], rr.v[it][hh][1], 0u, 0u}, v4u_t{wc.lo, wc.hi, 0u, 0u},
                                      v4u_t{sc.lo, sc.hi, 0u, 0u}, v4u_t{tc.lo, tc.hi, 0u, 0u}, rstd);
                store_chunk(hr + e, o4[0], o4[1]);
            }
        }
    }
}

// A workgroup of 4 waves owns `rpb` consecutive rows (wave k does rows
// k, k+4, ...).  With STAGE, when those rows all use one table row, w / s1 /
// sh (/ g) are staged once in LDS (dynamic shared memory, 3 or 4 x N bf16)
// instead of being re-read from L2 for every row.  Measured at x[32768,5120]:
// norm_mod is fastest with one row per wave and no staging (more rows in
// flight), gate_norm_mod_ with staging over 32-row blocks (four table streams
// per row otherwise).
template <int NUMX, int WARP, int MAXIT, bool GATE, bool STAGE>
__global__ __launch_bounds__(256) void norm_mod_block_kernel(
    uint16_t* __restrict__ x, const uint16_t* __restrict__ o, const uint16_t* __restrict__ g,
    const uint16_t* __restrict__ w, const int32_t* __restrict__ ridx,
    const uint16_t* __restrict__ s1, const uint16_t* __restrict__ sh, uint16_t* __restrict__ h,
    int64_t S, int N, int R, float eps, int rsq_mode, float* __restrict__ row_var, float* __restrict__ row_rstd,
    int rpb) {
    extern __shared__ __attribute__((aligned(16))) uint16_t tabs[];
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * rpb;
    const int64_t row_end = (row0 + rpb < S) ? row0 + rpb : S;
    bool staged = false;
    if constexpr (STAGE) {
        const int r0 = ridx[row0];
        int same = 1;
        for (int64_t rr = row0 + threadIdx.x; rr < row_end; rr += 256) same &= (ridx[rr] == r0);
        staged = __syncthreads_and(same) && r0 >= 0 && r0 < R;
    }
    if (staged) {
        const int r0 = ridx[row0];
        constexpr int NT = GATE ? 4 : 3;
        const int64_t tab = static_cast<int64_t>(r0) * N;
        const uint16_t* src[4] = {w, s1 + tab, sh + tab, GATE ? g + tab : w};
        for (int k = 0; k < NT; ++k)
            for (int e = threadIdx.x * 4; e < N; e += 256 * 4)  // N % 4 == 0
                *reinterpret_cast<uint2*>(tabs + k * N + e) = *reinterpret_cast<const uint2*>(src[k] + e);
        __syncthreads();
    }
    const int wave = threadIdx.x >> 6;
    if constexpr (!STAGE) {  // one row per wave, tables from global memory
        const int64_t row = row0 + wave;
        if (row >= row_end) return;
        const int r = ridx[row];
        if (r < 0 || r >= R) return;  // out-of-range table row: leave the row unwritten
        const int64_t tab = static_cast<int64_t>(r) * N;
        const GlobalTabs tb{w, s1 + tab, sh + tab, GATE ? g + tab : nullptr};
        RowRegs<NUMX, MAXIT> rr;
        float acc[NUMX / 128][2];
        load_row_phase<NUMX, WARP, MAXIT, GATE>(rr, acc, x, o, tb, row, N);
        const float rstd = reduce_rstd<NUMX, WARP>(acc, row, N, eps, rsq_mode, row_var, row_rstd);
        mod_row_phase<NUMX, MAXIT, GATE>(rr, x, tb, h, row, N, rstd);
        return;
    }
    for (int64_t row = row0 + wave; row < row_end; row += 4) {
        RowRegs<NUMX, MAXIT> rr;
        float acc[NUMX / 128][2];
        if (staged) {
            const LdsTabs tb{tabs, N};
            load_row_phase<NUMX, WARP, MAXIT, GATE>(rr, acc, x, o, tb, row, N);
            const float rstd = reduce_rstd<NUMX, WARP>(acc, row, N, eps, rsq_mode, row_var, row_rstd);
            mod_row_phase<NUMX, MAXIT, GATE>(rr, x, tb, h, row, N, rstd);
        } else {
            const int r = ridx[row];
            if (r < 0 || r >= R) continue;  // out-of-range table row: leave the row unwritten
            const int64_t tab = static_cast<int64_t>(r) * N;
            const GlobalTabs tb{w, s1 + tab, sh + tab, GATE ? g + tab : nullptr};
            load_row_phase<NUMX, WARP, MAXIT, GATE>(rr, acc, x, o, tb, row, N);
            const float rstd = reduce_rstd<NUMX, WARP>(acc, row, N, eps, rsq_mode, row_var, row_rstd);
            mod_row_phase<NUMX, MAXIT, GATE>(rr, x, tb, h, row, N, rstd);
        }
    }
}

// gate_ (streaming): one wave per row; 16 bytes per lane per instruction, so
// each instruction covers 1 KiB of the row.  Rows whose length is not a
// multiple of 8 elements finish with one 4-element chunk.
__global__ __launch_bounds__(256) void gate_wave_kernel(uint16_t* __restrict__ x, const uint16_t* __restrict__ o,
                                                        const uint16_t* __restrict__ g,
                                                        const int32_t* __restrict__ ridx, int64_t S, int N, int R) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int q = threadIdx.x & 63;
    if (row >= S) return;
    const int r = ridx[row];
    if (r < 0 || r >= R) return;
    uint16_t* xr = x + row * N;
    const uint16_t* orow = o + row * N;
    const uint16_t* gr = g + static_cast<int64_t>(r) * N;
    constexpr int U = 4;  // 1 KiB spans in flight per wave
    for (int base = 0; base < N; base += 512 * U) {
        v4u_t xv[U], ov[U], gv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = base + u * 512 + q * 8;
            if (e + 8 <= N) {
                xv[u] = ld16(xr + e, true);
                ov[u] = ld16(orow + e, true);
                gv[u] = ld16(gr + e, false);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = base + u * 512 + q * 8;
            if (e + 8 <= N) {
                st16(xr + e, gate8(xv[u], ov[u], gv[u]));
            } else if (e < N) {
                const Chunk xc = load_chunk(xr + e), oc = load_chunk(orow + e), gc = load_chunk(gr + e);
                store_chunk(xr + e, bf16x2_bits(bf16_lo(xc.lo) + bf16_lo(oc.lo) * bf16_lo(gc.lo),
                                                bf16_hi(xc.lo) + bf16_hi(oc.lo) * bf16_hi(gc.lo)),
                            bf16x2_bits(bf16_lo(xc.hi) + bf16_lo(oc.hi) * bf16_lo(gc.hi),
                                        bf16_hi(xc.hi) + bf16_hi(oc.hi) * bf16_hi(gc.hi)));
            }
        }
    }
}

// ------------------------------------------------------------------ persistent row streams
//
// The kernels for rows of up to 16 chunks of 16 bytes per lane (N <= 8192).
// One workgroup of wpw waves per CU (blockDim.x = 64 * wpw: 4 for the norm
// kernels, 1 for gate_); wave k of workgroup b handles rows b*wpw + k,
// b*wpw + k + nw, ... (nw = wpw * gridDim.x), so the rows in flight at
// any moment form one contiguous block of the tensor.  Each wave keeps one
// row of lookahead: the next row's loads are issued before the current row
// is reduced and written, so every wave always has a row in flight and the
// chip holds about one row per wave outstanding.  Measured at
// x[32768, 5120]: more outstanding data (more waves per CU or a deeper
// lookahead) lowers the HBM rate, and so does issuing each row's loads only
// once the previous row is written.
// Loads are buffer loads against a per-row resource: the lookahead past the
// last row has no records, so it reads zeros without touching memory.
// When every row a workgroup handles uses the same adaLN table row (one
// modulation vector per sample), the tables are copied to LDS once;
// otherwise each row reads its own table row from global memory (L2).
// Lane q holds elements c*512 + 8q .. +7 of chunk c, the layout of the
// one-wave-per-row kernels above, so both reduction orders apply unchanged
// (chunk c belongs to half c % H of the order's iteration c / H).

template <int CH>
struct RowV {
    v4u_t v[CH];
};

// The eight elements of a 16-byte bf16 chunk as fp32.  The stream kernels
// unpack each operand once (a bf16 -> fp32 unpack is one VALU instruction per
// element) and keep the staged tables in LDS as fp32, so the modulation costs
// about 6.5 VALU instructions per element (each bf16 rounding one
// instruction).  The plain norms run at the HBM rate of a device copy either
// way; the variant with the fused quantizer (about 15 per element with its
// set-up) is the VALU-heaviest: its VALU instructions fill about two thirds of
// its cycles, and memory latency at its occupancy takes the rest.
struct F8 {
    float f[8];
};

__device__ __forceinline__ F8 unpack8(v4u_t v) {
    F8 r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        r.f[2 * k] = bf16_lo(v[k]);
        r.f[2 * k + 1] = bf16_hi(v[k]);
    }
    return r;
}

// mod8's h = bf16(rb(rb(w*(rstd*x)) * s1) + sh) on fp32 operands; the
// fp32 value of h is left in hf (for the fused quantizer).  PAIR rounds the
// intermediate pairs with one conversion and two unpacks instead of two
// single-value conversions: one instruction more per pair, yet measured
// faster for norm_mod's row stream (114.7 against 115.4 us at [32768, 5120],
// 142.2 against 144.5 at [38400, 5376]); the other callers are faster with
// single-value conversions.
template <bool PAIR = false>
__device__ __forceinline__ v4u_t mod8f(const F8& x, const F8& w, const F8& s, const F8& t, float rstd, F8& hf) {
    v4u_t r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float y0 = w.f[2 * k] * (rstd * x.f[2 * k]);
        float y1 = w.f[2 * k + 1] * (rstd * x.f[2 * k + 1]);
        if constexpr (PAIR) rb2_pair(y0, y1); else rb2(y0, y1);
        y0 *= s.f[2 * k];
        y1 *= s.f[2 * k + 1];
        if constexpr (PAIR) rb2_pair(y0, y1); else rb2(y0, y1);
        r[k] = bf16x2_kept(y0 + t.f[2 * k], y1 + t.f[2 * k + 1]);
        hf.f[2 * k] = bf16_lo(r[k]);
        hf.f[2 * k + 1] = bf16_hi(r[k]);
    }
    return r;
}

// mod8f's h as fp32 only (h is quantized and not written): every rounding is
// one instruction.
__device__ __forceinline__ void mod8h(const F8& x, const F8& w, const F8& s, const F8& t, float rstd, F8& hf) {
#pragma unroll
    for (int j = 0; j < 8; ++j) hf.f[j] = rb_hi(rb_hi(rb_hi(w.f[j] * (rstd * x.f[j])) * s.f[j]) + t.f[j]);
}

// gate8's xn = rb(x + o*g) with g in fp32 (o*g of two bf16 is exact in fp32).
__device__ __forceinline__ v4u_t gate8f(v4u_t x, v4u_t o, const F8& g) {
    v4u_t r;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        r[k] = bf16x2_bits(bf16_lo(x[k]) + bf16_lo(o[k]) * g.f[2 * k], bf16_hi(x[k]) + bf16_hi(o[k]) * g.f[2 * k + 1]);
    return r;
}

// Buffer resource over `bytes` bytes at p (0 = no records: every access is
// out of range, loads read zero, stores are dropped).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const uint16_t* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p), static_cast<short>(0), bytes, 0x00020000);
}

// Row `row` of a [S, N] bf16 tensor; rows past S have no records.  `row`
// is wave-uniform, so the resource lives in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const uint16_t* base, int64_t row, int64_t S, int N) {
    const bool in = row < S;
    return span_rsrc(base + (in ? row : 0) * N, in ? N * 2 : 0);
}

// Loads of one row (non-temporal).  N % 8 == 0, so a 16-byte chunk lies
// wholly inside or wholly past the row, and the range check zeroes the
// chunks past N: no branches, so the compiler's wait counts stay exact and
// the lookahead row stays in flight.
template <int CH>
__device__ __forceinline__ void issue_row(RowV<CH>& r, const uint16_t* base, int64_t row, int64_t S, int N) {
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(base, row, S, N);
    const int q = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < CH; ++c)
        r.v[c] = __builtin_bit_cast(v4u_t, __builtin_amdgcn_raw_buffer_load_b128(rs, (c * 512 + q * 8) * 2, 0, 2));
}

// Non-temporal 16-byte store of chunk element e of a row; chunks past N are
// out of range and dropped.
__device__ __forceinline__ void store_row16(__amdgpu_buffer_rsrc_t rs, int e, v4u_t v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i_t, v), rs, e * 2, 0, 2);
}

// Sum of squares of a register row in the order <NUMX, WARP>, then rstd.
template <int NUMX, int WARP, int CH>
__device__ __forceinline__ float stream_rstd(const F8 (&xf)[CH], int64_t row, int N, float eps, int rsq_mode,
                                             float* __restrict__ row_var, float* __restrict__ row_rstd) {
    constexpr int H = NUMX / 128;
    float acc[H][2];
#pragma unroll
    for (int hh = 0; hh < H; ++hh) acc[hh][0] = acc[hh][1] = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int hh = c % H;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[hh][j >> 2] += xf[c].f[j] * xf[c].f[j];
    }
    return reduce_rstd<NUMX, WARP>(acc, row, N, eps, rsq_mode, row_var, row_rstd);
}

// As stream_rstd, from the packed bf16 row: each chunk is unpacked where it
// is squared, so the unpacked row (8 registers per chunk) is never held whole.
template <int NUMX, int WARP, int CH>
__device__ __forceinline__ float stream_rstd_packed(const v4u_t (&v)[CH], int64_t row, int N, float eps, int rsq_mode,
                                                    float* __restrict__ row_var, float* __restrict__ row_rstd) {
    constexpr int H = NUMX / 128;
    float acc[H][2];
#pragma unroll
    for (int hh = 0; hh < H; ++hh) acc[hh][0] = acc[hh][1] = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int hh = c % H;
        const F8 t = unpack8(v[c]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[hh][j >> 2] += t.f[j] * t.f[j];
    }
    return reduce_rstd<NUMX, WARP>(acc, row, N, eps, rsq_mode, row_var, row_rstd);
}

// Table rows for one row, as fp32: the LDS copies or global memory through
// range-checked buffer loads.  get(k, e) = elements e .. e+7 of table k,
// e = c*512 + 8*lane.  In LDS table k starts at k * P (P = CH * 512 floats,
// zero past N), and chunk c is stored as its 64 lanes' first four elements
// followed by their last four (tab_slot), so each of the two 16-byte reads of
// a lane is one contiguous wave-wide access.
__device__ __forceinline__ int tab_slot(int e) { return (e & ~511) + ((e & 511) >> 1); }

struct StreamLds {
    const float* t;
    int p;
    __device__ __forceinline__ F8 get(int k, int e) const {
        const float* s = t + k * p + tab_slot(e);
        const float4 a = *reinterpret_cast<const float4*>(s);
        const float4 b = *reinterpret_cast<const float4*>(s + 256);
        return F8{{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}};
    }
};
struct StreamGlobal {
    __amdgpu_buffer_rsrc_t rs[4];  // w, s1 row, sh row, g row
    __device__ __forceinline__ F8 get(int k, int e) const {
        return unpack8(__builtin_bit_cast(v4u_t, __builtin_amdgcn_raw_buffer_load_b128(rs[k], e * 2, 0, 0)));
    }
};

// Table row to stage in LDS for this workgroup's rows (rows b*wpw + k + i*nw):
// of the table rows of its first and last row, the in-range one more rows
// use (-1: neither is in range).  *all_same: every row uses one table row.
__device__ __forceinline__ int stream_pick(const int32_t* __restrict__ ridx, int64_t S, int R, bool* all_same) {
    const int wpw = blockDim.x >> 6;  // waves per workgroup
    const int64_t nw = static_cast<int64_t>(gridDim.x) * wpw;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * wpw;
    const int64_t per = (S - first + nw - 1) / nw;  // rows of wave 0 (>= those of the other waves)
    int64_t last = first + (per - 1) * nw + wpw - 1;  // a late row of this workgroup
    while (last >= S) last -= nw;
    if (last < first) last = first;
    const int ra = ridx[first], rb = ridx[last];
    // Rows i = base + thread of the workgroup's row list, one per thread per
    // step (__syncthreads_count counts threads, not sums); the row of i grows
    // with i, and base is a multiple of wpw, so the loop bound is uniform.
    int ca = 0, cb = 0;
    for (int64_t base = 0; first + (base / wpw) * nw < S; base += blockDim.x) {
        const int64_t i = base + threadIdx.x;
        const int64_t row = first + (i % wpw) + (i / wpw) * nw;
        const bool in = row < S;
        const int r = in ? ridx[row] : 0;
        ca += __syncthreads_count(in && r == ra);
        cb += __syncthreads_count(in && r == rb);
    }
    int64_t rows = 0;  // rows of this workgroup
    for (int k = 0; k < wpw; ++k)
        if (first + k < S) rows += (S - first - k + nw - 1) / nw;
    *all_same = (cb > ca ? cb : ca) == rows;
    if (ra < 0 || ra >= R) ca = -1;  // only an in-range table row can be staged
    if (rb < 0 || rb >= R) cb = -1;
    if (ca < 0 && cb < 0) return -1;
    return cb > ca ? rb : ra;
}

// Copies nt table rows into LDS as fp32 in StreamLds's layout, each padded
// with zeros to P elements (N % 8 == 0, P % 512 == 0).
__device__ __forceinline__ void stage_rows(float* tabs, const uint16_t* const* src, int nt, int N, int P) {
    for (int k = 0; k < nt; ++k)
        for (int e = threadIdx.x * 8; e < P; e += blockDim.x * 8) {
            const F8 v = e < N ? unpack8(*reinterpret_cast<const v4u_t*>(src[k] + e)) : F8{};
            float* d = tabs + k * P + tab_slot(e);
            *reinterpret_cast<float4*>(d) = make_float4(v.f[0], v.f[1], v.f[2], v.f[3]);
            *reinterpret_cast<float4*>(d + 256) = make_float4(v.f[4], v.f[5], v.f[6], v.f[7]);
        }
    __syncthreads();
}

// Calls f(tables of table row r): the LDS copy when r is the staged row rs,
// global memory otherwise; nothing when r is out of range (the row is left
// unwritten).  rs = -1: nothing staged.  With MIXED false every row uses the
// staged row.
template <bool MIXED, int NT, class F>
__device__ __forceinline__ void with_tabs(int r, int rs, const float* tabs, int P, int N, int R,
                                          const uint16_t* w, const uint16_t* s1, const uint16_t* sh,
                                          const uint16_t* g, F&& f) {
    if (!MIXED || (rs >= 0 && r == rs)) {
        f(StreamLds{tabs, P});
    } else if (r >= 0 && r < R) {
        const int64_t tab = static_cast<int64_t>(r) * N;
        if constexpr (NT == 1) {
            const __amdgpu_buffer_rsrc_t gr = span_rsrc(g + tab, N * 2);
            f(StreamGlobal{{gr, gr, gr, gr}});
        } else {
            const __amdgpu_buffer_rsrc_t wr = span_rsrc(w, N * 2);
            f(StreamGlobal{{wr, span_rsrc(s1 + tab, N * 2), span_rsrc(sh + tab, N * 2),
                            NT == 4 ? span_rsrc(g + tab, N * 2) : wr}});
        }
    }
}

// norm_mod (GATE = false): double-buffered rows, next row issued before the
// current one is reduced.  gate_norm_mod_ (GATE = true; without the
// quantizer and with N a multiple of 1024, gate_norm_split_kernel runs
// instead): x and o of a row
// are folded into xn = rb(x + o*g) as soon as they arrive, and the next row's
// x and o are loaded into the same registers before xn is reduced and
// written (three row buffers instead of four; measured faster than double
// buffering both x and o).  The table row of the next row is read with its
// loads, so it is in a register when the row is processed.
// QUANT 1: h is quantized per token while it is in registers (q = the
// per-token quantizer applied to h, bit for bit, and its scale qs) and not
// written; QUANT 2: h is written too; QUANT 0: h only.
// With EARLY, A (and AO with GATE) hold the loads of the wave's first row's
// x (and o), which the kernel issued before it staged the tables; otherwise
// they are issued here.
template <int NUMX, int WARP, int CH, bool GATE, bool MIXED, int QUANT, bool EARLY>
__device__ __forceinline__ void norm_stream_rows(uint16_t* __restrict__ x, const uint16_t* __restrict__ o,
                                                 const uint16_t* __restrict__ g, const uint16_t* __restrict__ w,
                                                 const int32_t* __restrict__ ridx, const uint16_t* __restrict__ s1,
                                                 const uint16_t* __restrict__ sh, uint16_t* __restrict__ h, int64_t S,
                                                 int N, int R, float eps, int rsq_mode, float* __restrict__ row_var,
                                                 float* __restrict__ row_rstd, const float* tabs, int rs,
                                                 int8_t* __restrict__ q, float* __restrict__ qs, RowV<CH>& A,
                                                 RowV<CH>& AO) {
    constexpr int P = CH * 512;
    const int wpw = blockDim.x >> 6;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * wpw;
    const int lane = threadIdx.x & 63;
    int64_t row = static_cast<int64_t>(blockIdx.x) * wpw + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    auto next_r = [&](int64_t rw) { return (MIXED && rw < S) ? ridx[rw] : rs; };
    auto finish = [&](const RowV<CH>& xv, int64_t rw, const auto& tb) {
        const __amdgpu_buffer_rsrc_t hr = row_rsrc(h, rw, S, N);
        if constexpr (QUANT == 0 && GATE) {
            // The row is unpacked twice, for the sum of squares and chunk by
            // chunk for the modulation, rather than held unpacked in between:
            // 8 more VALU per chunk, 80-88 fewer live registers at 10-11
            // chunks, beside the next row's x and o in flight (at [19200, 5376]:
            // 151 against 161 us, the registers no longer parked in AGPRs).
            // norm_mod holds one row buffer fewer and measured no faster so.
            const float rstd = stream_rstd_packed<NUMX, WARP, CH>(xv.v, rw, N, eps, rsq_mode, row_var, row_rstd);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int e = c * 512 + lane * 8;
                v4u_t pv = xv.v[c];
                asm volatile("" : "+v"(pv));  // opaque: the compiler may not reuse the first unpack
                F8 hf;  // xn was stored when the next row's loads went out
                store_row16(hr, e, mod8f(unpack8(pv), tb.get(0, e), tb.get(1, e), tb.get(2, e), rstd, hf));
                // one chunk at a time: left alone, the scheduler hoists every
                // table read of the row and runs out of registers
                __builtin_amdgcn_sched_barrier(0);
            }
        } else if constexpr (QUANT == 0) {
            F8 xf[CH];
#pragma unroll
            for (int c = 0; c < CH; ++c) xf[c] = unpack8(xv.v[c]);
            const float rstd = stream_rstd<NUMX, WARP, CH>(xf, rw, N, eps, rsq_mode, row_var, row_rstd);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int e = c * 512 + lane * 8;
                F8 hf;
                store_row16(hr, e, mod8f<true>(xf[c], tb.get(0, e), tb.get(1, e), tb.get(2, e), rstd, hf));
                // one chunk at a time: left alone, the scheduler hoists every
                // table read of the row and runs out of registers
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            F8 xf[CH];
#pragma unroll
            for (int c = 0; c < CH; ++c) xf[c] = unpack8(xv.v[c]);
            const float rstd = stream_rstd<NUMX, WARP, CH>(xf, rw, N, eps, rsq_mode, row_var, row_rstd);
            const __amdgpu_buffer_rsrc_t xr = row_rsrc(x, rw, S, N);
            F8 hf[CH];
            float amax = 0.0f;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int e = c * 512 + lane * 8;
                if constexpr (GATE) store_row16(xr, e, xv.v[c]);
                if constexpr (QUANT == 2)
                    store_row16(hr, e, mod8f(xf[c], tb.get(0, e), tb.get(1, e), tb.get(2, e), rstd, hf[c]));
                else
                    mod8h(xf[c], tb.get(0, e), tb.get(1, e), tb.get(2, e), rstd, hf[c]);
#pragma unroll
                for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(hf[c].f[j]));
                __builtin_amdgcn_sched_barrier(0);
            }
            // chunks past N hold h = 0 (zero x, zero-padded tables), so the
            // max is the row's; the max is order-independent
            amax = wave_max(amax);
            const float sc = amax / 127.0f;
            if (lane == 0) qs[rw] = sc;
            const float r = 1.0f / sc;
            const bool exact = quot_exact(sc, r);  // h is bf16, so quant8b applies
            const bool in = rw < S;
            const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
                q + (in ? rw : 0) * static_cast<int64_t>(N), static_cast<short>(0), in ? N : 0, 0x00020000);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int e = c * 512 + lane * 8;
                const uint2 p = sc != 0.0f ? quant8b(hf[c].f, sc, r, exact) : make_uint2(0u, 0u);
                // a cached store: the GEMM reads q next
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2i_t, make_int2(p.x, p.y)), qr, e, 0, 0);
            }
        }
    };
    int r = next_r(row);
    if constexpr (!EARLY) {
        issue_row<CH>(A, x, row, S, N);
        if constexpr (GATE) issue_row<CH>(AO, o, row, S, N);
    }
    if constexpr (!GATE) {
        RowV<CH> B;
        for (;;) {
            issue_row<CH>(B, x, row + nw, S, N);
            int rn = next_r(row + nw);
            with_tabs<MIXED, 3>(r, rs, tabs, P, N, R, w, s1, sh, g, [&](const auto& tb) { finish(A, row, tb); });
            row += nw;
            r = rn;
            if (row >= S) break;
            issue_row<CH>(A, x, row + nw, S, N);
            rn = next_r(row + nw);
            with_tabs<MIXED, 3>(r, rs, tabs, P, N, R, w, s1, sh, g, [&](const auto& tb) { finish(B, row, tb); });
            row += nw;
            r = rn;
            if (row >= S) break;
        }
    } else {
        RowV<CH>& AX = A;
        RowV<CH> XN;
        for (;;) {
            with_tabs<MIXED, 4>(r, rs, tabs, P, N, R, w, s1, sh, g, [&](const auto& tb) {
#pragma unroll
                for (int c = 0; c < CH; ++c) XN.v[c] = gate8f(AX.v[c], AO.v[c], tb.get(3, c * 512 + lane * 8));
            });
            issue_row<CH>(AX, x, row + nw, S, N);
            issue_row<CH>(AO, o, row + nw, S, N);
            // Without the quantizer, xn goes back to x right behind the next
            // row's loads rather than chunk by chunk after the reduction
            // (measured 0.6% faster; stored before those loads, 1.5% slower).
            // A row with an out-of-range table index is left unwritten.
            if constexpr (QUANT == 0) {
                if (!MIXED || (r >= 0 && r < R)) {
                    const __amdgpu_buffer_rsrc_t xr = row_rsrc(x, row, S, N);
#pragma unroll
                    for (int c = 0; c < CH; ++c) store_row16(xr, c * 512 + lane * 8, XN.v[c]);
                }
            }
            const int rn = next_r(row + nw);
            with_tabs<MIXED, 4>(r, rs, tabs, P, N, R, w, s1, sh, g, [&](const auto& tb) { finish(XN, row, tb); });
            row += nw;
            r = rn;
            if (row >= S) break;
        }
    }
}

template <int NUMX, int WARP, int CH, bool GATE, int QUANT = 0>
__global__ __launch_bounds__(256) void norm_stream_kernel(
    uint16_t* __restrict__ x, const uint16_t* __restrict__ o, const uint16_t* __restrict__ g,
    const uint16_t* __restrict__ w, const int32_t* __restrict__ ridx, const uint16_t* __restrict__ s1,
    const uint16_t* __restrict__ sh, uint16_t* __restrict__ h, int64_t S, int N, int R, float eps, int rsq_mode,
    float* __restrict__ row_var, float* __restrict__ row_rstd, int8_t* __restrict__ q, float* __restrict__ qs) {
    extern __shared__ __attribute__((aligned(16))) float ftabs[];
    constexpr int NT = GATE ? 4 : 3;
    // Without the quantizer the first row's loads go out before the table
    // set-up, so their latency overlaps it (a row past S has an empty range
    // and reads nothing): measured 2-4% faster for norm_mod, 1% for
    // gate_norm_mod_.  The quantizing variants run two workgroups per CU, and
    // the registers held across the set-up would cost them that occupancy;
    // with 16 chunks per row they would spill.
    constexpr bool EARLY = QUANT == 0 && CH <= 12;
    const int64_t row0 =
        static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    RowV<CH> A, AO;
    if constexpr (EARLY) {
        issue_row<CH>(A, x, row0, S, N);
        if constexpr (GATE) issue_row<CH>(AO, o, row0, S, N);
    }
    bool all_same;
    const int rs = stream_pick(ridx, S, R, &all_same);
    if (rs >= 0) {
        const int64_t tab = static_cast<int64_t>(rs) * N;
        const uint16_t* src[4] = {w, s1 + tab, sh + tab, GATE ? g + tab : w};
        stage_rows(ftabs, src, NT, N, CH * 512);
    }
    if (row0 >= S) return;
    // norm_mod over 64 Ki rows or more runs the per-row table-index variant
    // even when every row shares one table row: measured 446.6 against 480.6
    // us at [131072, 5120] and 221.5 against 228.8 at [65536, 5120], where it
    // is 2% slower at [32768, 5120].  The other stream kernels were faster
    // with the shared-row variant at both sizes.
    const bool per_row = !GATE && QUANT == 0 && S >= 65536;
    if (all_same && rs >= 0 && !per_row)
        norm_stream_rows<NUMX, WARP, CH, GATE, false, QUANT, EARLY>(x, o, g, w, ridx, s1, sh, h, S, N, R, eps, rsq_mode,
                                                             row_var, row_rstd, ftabs, rs, q, qs, A, AO);
    else
        norm_stream_rows<NUMX, WARP, CH, GATE, true, QUANT, EARLY>(x, o, g, w, ridx, s1, sh, h, S, N, R, eps, rsq_mode,
                                                            row_var, row_rstd, ftabs, rs, q, qs, A, AO);
}

// gate_: x <- rb(x + o*g), the same persistent row stream with x and o
// double-buffered.  With EARLY, AX and AO hold the loads of the wave's first
// row, issued by the kernel before the table set-up.
template <int CH, bool MIXED, bool EARLY>
__device__ __forceinline__ void gate_stream_rows(uint16_t* __restrict__ x, const uint16_t* __restrict__ o,
                                                 const uint16_t* __restrict__ g, const int32_t* __restrict__ ridx,
                                                 int64_t S, int N, int R, const float* tabs, int rs, RowV<CH>& AX,
                                                 RowV<CH>& AO) {
    constexpr int P = CH * 512;
    const int wpw = blockDim.x >> 6;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * wpw;
    const int q = threadIdx.x & 63;
    int64_t row = static_cast<int64_t>(blockIdx.x) * wpw + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    auto next_r = [&](int64_t rw) { return (MIXED && rw < S) ? ridx[rw] : rs; };
    auto gate_row = [&](const RowV<CH>& X, const RowV<CH>& O, int64_t rw, int r) {
        with_tabs<MIXED, 1>(r, rs, tabs, P, N, R, nullptr, nullptr, nullptr, g, [&](const auto& tb) {
            const __amdgpu_buffer_rsrc_t xr = row_rsrc(x, rw, S, N);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int e = c * 512 + q * 8;
                store_row16(xr, e, gate8f(X.v[c], O.v[c], tb.get(0, e)));
            }
        });
    };
    int r = next_r(row);
    RowV<CH> BX, BO;
    if constexpr (!EARLY) {
        issue_row<CH>(AX, x, row, S, N);
        issue_row<CH>(AO, o, row, S, N);
    }
    for (;;) {
        issue_row<CH>(BX, x, row + nw, S, N);
        issue_row<CH>(BO, o, row + nw, S, N);
        int rn = next_r(row + nw);
        gate_row(AX, AO, row, r);
        row += nw;
        r = rn;
        if (row >= S) break;
        issue_row<CH>(AX, x, row + nw, S, N);
        issue_row<CH>(AO, o, row + nw, S, N);
        rn = next_r(row + nw);
        gate_row(BX, BO, row, r);
        row += nw;
        r = rn;
        if (row >= S) break;
    }
}

template <int CH>
__global__ __launch_bounds__(256) void gate_stream_kernel(uint16_t* __restrict__ x, const uint16_t* __restrict__ o,
                                                          const uint16_t* __restrict__ g,
                                                          const int32_t* __restrict__ ridx, int64_t S, int N, int R) {
    extern __shared__ __attribute__((aligned(16))) float ftabs[];
    // the first row's loads overlap the table set-up, as in norm_stream_kernel
    constexpr bool EARLY = CH <= 12;
    const int64_t row0 =
        static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    RowV<CH> AX, AO;
    if constexpr (EARLY) {
        issue_row<CH>(AX, x, row0, S, N);
        issue_row<CH>(AO, o, row0, S, N);
    }
    bool all_same;
    const int rs = stream_pick(ridx, S, R, &all_same);
    if (rs >= 0) {
        const uint16_t* src[1] = {g + static_cast<int64_t>(rs) * N};
        stage_rows(ftabs, src, 1, N, CH * 512);
    }
    if (row0 >= S) return;
    if (all_same && rs >= 0) gate_stream_rows<CH, false, EARLY>(x, o, g, ridx, S, N, R, ftabs, rs, AX, AO);
    else gate_stream_rows<CH, true, EARLY>(x, o, g, ridx, S, N, R, ftabs, rs, AX, AO);
}

// Chunk counts the stream kernels are instantiated for; a row of N elements
// uses the smallest one >= ceil(N / 512) (extra chunks read zero and are not
// stored).
#define H3MI_STREAM_CH(X) X(2) X(4) X(6) X(8) X(10) X(11) X(12) X(16)

inline int stream_ch(int N) {
    if (N % 8) return 0;  // the 4-element tail chunk takes the kernels below
    const int need = (N + 511) / 512;
    const int opts[] = {2, 4, 6, 8, 10, 11, 12, 16};
    for (int c : opts)
        if (c >= need) return c;
    return 0;
}

// per_cu workgroups per CU (wpw waves each), at most one per wpw rows.
inline unsigned stream_grid(int64_t S, int per_cu = 1, int wpw = 4) {
    const int64_t wgs = (S + wpw - 1) / wpw;
    const int64_t cap = static_cast<int64_t>(cu_count()) * per_cu;
    return static_cast<unsigned>(wgs < cap ? wgs : cap);
}

// rows per workgroup of the block kernel (4 waves, so 8 rows per wave)
constexpr int kRowsPerBlock = 32;

struct OrderDesc {
    int numx, warp;
};

constexpr OrderDesc kOrders[H3MI_ORDER_COUNT] = {
    {256, 64},  // DEFAULT: eager PyTorch rms_norm on ROCm (wave64, 4 warps)
    {128, 32},  // REF
    {256, 64},  // W64
};

// ------------------------------------------------------------------ gate_norm_mod_: one row per workgroup

// gate_norm_mod_ moves four row streams (x and o read, x and h written).  A
// wave per row puts 20 KiB of loads in flight per wave, 80 KiB per CU, where
// a flat stream of this mix runs fastest with about 16 KiB per CU (76% of
// 8 TB/s against 70%).  So here a workgroup of 4 waves holds one row: the
// default order's 256 threads (4 elements each per 1024-element iteration)
// are its 4 waves x 64 lanes, the in-warp tree is the wave's own shuffle
// tree, and the four warp totals meet in LDS behind one barrier.  One
// workgroup per CU handles rows b, b + G, b + 2G, ... with the next row's x
// and o in flight (20 KiB per CU): 229 against 240 us at [32768, 5120],
// bit-identical.  norm_mod, which reads one stream, measured slower so (one
// workgroup per CU: 10 KiB in flight) or no faster (two).
//
// Rows of N = 1024 IT + 256 (hidden 5376): in the reduction order the last
// 256 elements are one more iteration of threads 0..63, but a wave executes
// an iteration's instructions whoever holds data, so all four waves would
// run IT + 1 iterations of loads, gating, modulation and stores for IT + 1/4
// of data.  There (TAIL) that iteration keeps the reduction layout only for
// the sum of squares (loads, gating and squares, as the order requires);
// its elementwise work -- the x store, the modulation and the h store --
// runs one element per thread (element 1024 IT + t), about a quarter of an
// iteration's instructions per wave, from its own 2-byte loads of x and o
// (the same bytes, served by L2).

typedef uint32_t v2u_t __attribute__((ext_vector_type(2)));

struct F4 {
    float f[4];
};

__device__ __forceinline__ F4 unpack4(v2u_t v) {
    return F4{{bf16_lo(v[0]), bf16_hi(v[0]), bf16_lo(v[1]), bf16_hi(v[1])}};
}

// mod8f's arithmetic on 4 elements
__device__ __forceinline__ v2u_t mod4f(const F4& x, const F4& w, const F4& s, const F4& t, float rstd) {
    v2u_t r;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        float y0 = w.f[2 * k] * (rstd * x.f[2 * k]);
        float y1 = w.f[2 * k + 1] * (rstd * x.f[2 * k + 1]);
        rb2(y0, y1);
        y0 *= s.f[2 * k];
        y1 *= s.f[2 * k + 1];
        rb2(y0, y1);
        r[k] = bf16x2_kept(y0 + t.f[2 * k], y1 + t.f[2 * k + 1]);
    }
    return r;
}

// gate8f's arithmetic on 4 elements
__device__ __forceinline__ v2u_t gate4f(v2u_t x, v2u_t o, const F4& g) {
    v2u_t r;
#pragma unroll
    for (int k = 0; k < 2; ++k)
        r[k] = bf16x2_bits(bf16_lo(x[k]) + bf16_lo(o[k]) * g.f[2 * k], bf16_hi(x[k]) + bf16_hi(o[k]) * g.f[2 * k + 1]);
    return r;
}

// gate4f / mod4f's arithmetic on one element (x, o: bf16 bits)
__device__ __forceinline__ uint32_t gate1f(uint32_t x, uint32_t o, float g) {
    return bf16_bits(bf16_f32(x) + bf16_f32(o) * g);
}
__device__ __forceinline__ uint32_t mod1f(float x, float w, float s, float t, float rstd) {
    float y = w * (rstd * x);
    y = rb(y);
    y *= s;
    y = rb(y);
    return bf16_bits(y + t);
}

struct SplitLds {
    const float* t;
    int p;
    __device__ __forceinline__ F4 get(int k, int e) const {
        const float4 a = *reinterpret_cast<const float4*>(t + k * p + e);
        return F4{{a.x, a.y, a.z, a.w}};
    }
    __device__ __forceinline__ float get1(int k, int e) const { return t[k * p + e]; }
};
struct SplitGlobal {
    __amdgpu_buffer_rsrc_t rs[4];  // w, s1 row, sh row, g row
    __device__ __forceinline__ F4 get(int k, int e) const {
        return unpack4(__builtin_bit_cast(v2u_t, __builtin_amdgcn_raw_buffer_load_b64(rs[k], e * 2, 0, 0)));
    }
    __device__ __forceinline__ float get1(int k, int e) const {
        return bf16_f32(__builtin_amdgcn_raw_buffer_load_b16(rs[k], e * 2, 0, 0));
    }
};

// IT full 1024-element iterations per thread, and with TAIL a last
// 256-element iteration (N = 1024 IT + 256; the tail above).
template <int IT, int TAIL>
__global__ __launch_bounds__(256) void gate_norm_split_kernel(
    uint16_t* __restrict__ x, const uint16_t* __restrict__ o, const uint16_t* __restrict__ g,
    const uint16_t* __restrict__ w, const int32_t* __restrict__ ridx, const uint16_t* __restrict__ s1,
    const uint16_t* __restrict__ sh, uint16_t* __restrict__ h, int64_t S, int N, int R, float eps, int rsq_mode,
    float* __restrict__ row_var, float* __restrict__ row_rstd) {
    static_assert(TAIL == 0 || TAIL == 1, "tail: one 256-element iteration");
    constexpr int NT = 4;
    constexpr int NI = IT + TAIL;  // iterations of the reduction order
    constexpr int P = NI * 1024;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* const tabs = smem;
    float* const red = smem + NT * P;  // two sets of the 4 warp totals
    const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int64_t G = gridDim.x;
    int64_t row = blockIdx.x;
    const int e1 = IT * 1024 + t;  // TAIL: this thread's element of the tail's elementwise layout
    auto issue = [&](v2u_t (&d)[NI], uint32_t& d1, const uint16_t* base, int64_t rw) {
        const __amdgpu_buffer_rsrc_t rs = row_rsrc(base, rw, S, N);
#pragma unroll
        for (int it = 0; it < NI; ++it)
            d[it] = __builtin_bit_cast(v2u_t, __builtin_amdgcn_raw_buffer_load_b64(rs, (it * 1024 + 4 * t) * 2, 0, 2));
        if constexpr (TAIL) d1 = __builtin_amdgcn_raw_buffer_load_b16(rs, e1 * 2, 0, 2);
    };
    auto store = [&](__amdgpu_buffer_rsrc_t rs, int it, v2u_t v) {
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2i_t, v), rs, (it * 1024 + 4 * t) * 2, 0, 2);
    };
    auto store1 = [&](__amdgpu_buffer_rsrc_t rs, uint32_t v) {
        __builtin_amdgcn_raw_buffer_store_b16(static_cast<unsigned short>(v), rs, e1 * 2, 0, 2);
    };
    v2u_t A[NI], B[NI];  // x and o of the row
    uint32_t A1 = 0, B1 = 0;  // TAIL: x and o of element e1
    issue(A, A1, x, row);
    issue(B, B1, o, row);

    // The table row to stage: of the table rows of the first and last rows
    // of this workgroup, the in-range one more of its rows use.
    const int64_t cnt = (S - row + G - 1) / G;
    const int ra = ridx[row], rb = ridx[row + (cnt - 1) * G];
    int ca = 0, cb = 0;
    for (int64_t base = 0; base < cnt; base += 256) {
        const int64_t i = base + t;
        const int r = i < cnt ? ridx[row + i * G] : 0;
        ca += __syncthreads_count(i < cnt && r == ra);
        cb += __syncthreads_count(i < cnt && r == rb);
    }
    const bool all_same = (ca > cb ? ca : cb) == cnt;
    if (ra < 0 || ra >= R) ca = -1;
    if (rb < 0 || rb >= R) cb = -1;
    const int rs = (ca < 0 && cb < 0) ? -1 : (cb > ca ? rb : ra);
    if (rs >= 0) {
        const int64_t tab = static_cast<int64_t>(rs) * N;
        const uint16_t* src[4] = {w, s1 + tab, sh + tab, g + tab};
#pragma unroll
        for (int k = 0; k < NT; ++k)
#pragma unroll
            for (int it = 0; it < NI; ++it) {
                const int e = it * 1024 + 4 * t;
                const F4 v = e < N ? unpack4(*reinterpret_cast<const v2u_t*>(src[k] + e)) : F4{};
                *reinterpret_cast<float4*>(tabs + k * P + e) = make_float4(v.f[0], v.f[1], v.f[2], v.f[3]);
            }
    }
    __syncthreads();

    auto run = [&](auto mixed_c) {
        constexpr bool MIXED = decltype(mixed_c)::value;
        auto with_tabs = [&](int r, auto&& f) {
            if (!MIXED || (rs >= 0 && r == rs)) {
                f(SplitLds{tabs, P});
            } else if (r >= 0 && r < R) {
                const int64_t tab = static_cast<int64_t>(r) * N;
                const __amdgpu_buffer_rsrc_t wr = span_rsrc(w, N * 2);
                f(SplitGlobal{{wr, span_rsrc(s1 + tab, N * 2), span_rsrc(sh + tab, N * 2), span_rsrc(g + tab, N * 2)}});
            }
        };
        auto next_r = [&](int64_t rw) { return (MIXED && rw < S) ? ridx[rw] : rs; };
        int buf = 0;
        // Sum of squares in the order: per thread over its elements, the
        // in-warp tree, then (w0 + w2) + (w1 + w3) over the 4 warps.  xn1 is
        // the tail's element e1 (TAIL).
        auto finish = [&](const v2u_t (&v)[NI], uint32_t xn1, int64_t rw, const auto& tb) {
            float acc = 0.0f;
#pragma unroll
            for (int it = 0; it < NI; ++it) {
                const F4 f = unpack4(v[it]);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc += f.f[j] * f.f[j];
            }
#pragma unroll
            for (int d = 32; d >= 1; d /= 2) acc += __shfl_down(acc, d, 64);
            if (lane == 0) red[buf * 4 + wv] = acc;
            wait_lgkm0();
            wg_barrier();
            const float tot = (red[buf * 4 + 0] + red[buf * 4 + 2]) + (red[buf * 4 + 1] + red[buf * 4 + 3]);
            buf ^= 1;
            const float var = tot / static_cast<float>(N) + eps;
            const float rstd = rsqrt_mode(var, rsq_mode);
            if (t == 0) {
                if (row_var) row_var[rw] = var;
                if (row_rstd) row_rstd[rw] = rstd;
            }
            const __amdgpu_buffer_rsrc_t hr = row_rsrc(h, rw, S, N);
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int e = it * 1024 + 4 * t;
                store(hr, it, mod4f(unpack4(v[it]), tb.get(0, e), tb.get(1, e), tb.get(2, e), rstd));
            }
            if constexpr (TAIL)
                store1(hr, mod1f(bf16_f32(xn1), tb.get1(0, e1), tb.get1(1, e1), tb.get1(2, e1), rstd));
        };
        int r = next_r(row);
        for (;;) {
            v2u_t XN[NI];
            uint32_t XN1 = 0;
            bool done = false;  // uniform: the row's table index is in range
            with_tabs(r, [&](const auto& tb) {
#pragma unroll
                for (int it = 0; it < NI; ++it) XN[it] = gate4f(A[it], B[it], tb.get(3, it * 1024 + 4 * t));
                if constexpr (TAIL) XN1 = gate1f(A1, B1, tb.get1(3, e1));
                done = true;
            });
            issue(A, A1, x, row + G);
            issue(B, B1, o, row + G);
            const int rn = next_r(row + G);
            if (done) {
                const __amdgpu_buffer_rsrc_t xr = row_rsrc(x, row, S, N);
                // the tail's xn goes back from its elementwise layout only
#pragma unroll
                for (int it = 0; it < IT; ++it) store(xr, it, XN[it]);
                if constexpr (TAIL) store1(xr, XN1);
                with_tabs(r, [&](const auto& tb) { finish(XN, XN1, row, tb); });
            }
            row += G;
            r = rn;
            if (row >= S) break;
        }
    };
    if (all_same && rs >= 0) run(std::false_type{});
    else run(std::true_type{});
}

template <int NUMX, int WARP, bool GATE>
int launch_order(uint16_t* x, const uint16_t* o, const uint16_t* g, const uint16_t* w, const int32_t* ridx,
                 const uint16_t* s1, const uint16_t* sh, uint16_t* h, int64_t S, int N, int R, float eps,
                 int rsq, float* var, float* rstd, hipStream_t st) {
    // Persistent row stream for N <= 8192 in the product order; the reference
    // order (a parity mode) keeps the kernels below.
    const int ch = (NUMX == 256 && WARP == 64) ? stream_ch(N) : 0;
    if (GATE && ch > 0 && N >= 1024 && (N % 1024 == 0 || N % 1024 == 256)) {
        const int it = N / 1024, tail = N % 1024 ? 1 : 0;
        const size_t slds = static_cast<size_t>(4 * (it + tail) * 1024 + 8) * sizeof(float);
        const int64_t cus = cu_count();
        const dim3 grid(static_cast<unsigned>(S < cus ? S : cus)), block(256);
#define H3MI_SPLIT_LAUNCH(I, T)                                                                                  \
    if (it == I && tail == T)                                                                                    \
        hipLaunchKernelGGL((gate_norm_split_kernel<I, T>), grid, block, slds, st, x, o, g, w, ridx, s1, sh, h, S, N, \
                           R, eps, rsq, var, rstd);
        H3MI_SPLIT_LAUNCH(1, 0) H3MI_SPLIT_LAUNCH(2, 0) H3MI_SPLIT_LAUNCH(3, 0) H3MI_SPLIT_LAUNCH(4, 0)
        H3MI_SPLIT_LAUNCH(5, 0) H3MI_SPLIT_LAUNCH(6, 0) H3MI_SPLIT_LAUNCH(7, 0) H3MI_SPLIT_LAUNCH(8, 0)
        H3MI_SPLIT_LAUNCH(1, 1) H3MI_SPLIT_LAUNCH(2, 1) H3MI_SPLIT_LAUNCH(3, 1) H3MI_SPLIT_LAUNCH(4, 1)
        H3MI_SPLIT_LAUNCH(5, 1) H3MI_SPLIT_LAUNCH(6, 1) H3MI_SPLIT_LAUNCH(7, 1)
#undef H3MI_SPLIT_LAUNCH
        return check_launch("gate_norm_mod");
    }
    if (ch > 0) {
        const size_t slds = static_cast<size_t>(GATE ? 4 : 3) * ch * 512 * sizeof(float);
        const dim3 grid(stream_grid(S)), block(256);
#define H3MI_STREAM_LAUNCH(C)                                                                                    \
    if (ch == C)                                                                                                 \
        hipLaunchKernelGGL((norm_stream_kernel<256, 64, C, GATE>), grid, block, slds, st, x, o, g, w, ridx, s1, sh, h, \
                           S, N, R, eps, rsq, var, rstd, nullptr, nullptr);
        H3MI_STREAM_CH(H3MI_STREAM_LAUNCH)
#undef H3MI_STREAM_LAUNCH
        return check_launch(GATE ? "gate_norm_mod" : "norm_mod");
    }
    const int iters = (N / VEC + NUMX - 1) / NUMX;
    const size_t lds = GATE ? static_cast<size_t>(4) * N * sizeof(uint16_t) : 0;
    if (iters <= 16 && lds <= 65536) {  // one wave per row
        const int rpb = GATE ? kRowsPerBlock : 4;
        dim3 grid(static_cast<unsigned>((S + rpb - 1) / rpb)), block(256);
#define H3MI_BLOCK_LAUNCH(MI)                                                                                    \
    hipLaunchKernelGGL((norm_mod_block_kernel<NUMX, WARP, MI, GATE, GATE>), grid, block, lds, st, x, o, g, w, ridx, s1, \
                       sh, h, S, N, R, eps, rsq, var, rstd, rpb)
        if (iters <= 2) H3MI_BLOCK_LAUNCH(2);
        else if (iters <= 3) H3MI_BLOCK_LAUNCH(3);
        else if (iters <= 4) H3MI_BLOCK_LAUNCH(4);
        else if (iters <= 5) H3MI_BLOCK_LAUNCH(5);
        else if (iters <= 6) H3MI_BLOCK_LAUNCH(6);
        else if (iters <= 8) H3MI_BLOCK_LAUNCH(8);
        else if (iters <= 12) H3MI_BLOCK_LAUNCH(12);
        else H3MI_BLOCK_LAUNCH(16);
#undef H3MI_BLOCK_LAUNCH
        return check_launch(GATE ? "gate_norm_mod" : "norm_mod");
    }
    dim3 grid(static_cast<unsigned>(S)), block(NUMX);
#define H3MI_NORM_LAUNCH(MI)                                                                                  \
    hipLaunchKernelGGL((norm_mod_kernel<NUMX, WARP, MI, GATE>), grid, block, 0, st, x, o, g, w, ridx, s1, sh, h, \
                       N, R, eps, rsq, var, rstd)
    if (iters <= 24) H3MI_NORM_LAUNCH(24);
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
    // The widest kernel keeps 64 chunks of VEC elements per thread in
    // registers; wider rows are refused here, before pointers are looked at.
    const int64_t nmax = static_cast<int64_t>(kOrders[order].numx) * VEC * 64;
    if (N > nmax) return fail(H3MI_EINVAL, "%s: N=%lld exceeds the register-resident limit %lld", name, (long long)N, (long long)nmax);
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

// norm_mod / gate_norm_mod_ with the per-token quantizer of h fused in (the
// stream kernels only: N % 8 == 0, N <= 8192, the product order).
template <bool GATE>
int norm_quant_entry(uint16_t* x, const uint16_t* o, const uint16_t* g, const uint16_t* w, const int32_t* ridx,
                     const uint16_t* s1, const uint16_t* sh, uint16_t* h, int8_t* q, float* qs, int64_t S, int64_t N,
                     int64_t R, float eps, void* stream) {
    const char* name = GATE ? "gate_norm_mod_quant" : "norm_mod_quant";
    if (S < 0 || N <= 0 || R <= 0) return fail(H3MI_EINVAL, "%s: bad sizes S=%lld N=%lld R=%lld", name, (long long)S, (long long)N, (long long)R);
    const int ch = N <= 8192 ? stream_ch(static_cast<int>(N)) : 0;
    if (ch == 0) return fail(H3MI_EINVAL, "%s: N=%lld must be a multiple of 8 and at most 8192", name, (long long)N);
    if (S > 0x7FFFFFFF) return fail(H3MI_EINVAL, "%s: S too large", name);
    if (S == 0) return ok();
    if (!x || !w || !ridx || !s1 || !sh || !q || !qs || (GATE && (!o || !g))) return fail(H3MI_EINVAL, "%s: null pointer", name);
    const void* ptrs[] = {x, w, s1, sh, h, o, g, q};
    for (const void* p : ptrs)
        if (p && !aligned(p, 8)) return fail(H3MI_EALIGN, "%s: tensors must be 8-byte aligned", name);
    if (!aligned(qs, 4)) return fail(H3MI_EALIGN, "%s: qs must be 4-byte aligned", name);
    const size_t xb = static_cast<size_t>(S) * N * 2, qb = static_cast<size_t>(S) * N, sb = static_cast<size_t>(S) * 4;
    if (h && overlap(h, xb, x, xb)) return fail(H3MI_EALIAS, "%s: h overlaps x", name);
    if (overlap(q, qb, x, xb) || (h && overlap(q, qb, h, xb))) return fail(H3MI_EALIAS, "%s: q overlaps x or h", name);
    if (overlap(qs, sb, x, xb) || overlap(qs, sb, q, qb) || (h && overlap(qs, sb, h, xb)))
        return fail(H3MI_EALIAS, "%s: qs overlaps x, h or q", name);
    if (GATE) {
        if (overlap(o, xb, x, xb)) return fail(H3MI_EALIAS, "%s: o overlaps x", name);
        if (overlap(g, static_cast<size_t>(R) * N * 2, x, xb)) return fail(H3MI_EALIAS, "%s: g overlaps x", name);
    }
    const size_t slds = static_cast<size_t>(GATE ? 4 : 3) * ch * 512 * sizeof(float);
    // norm_mod with the quantizer is VALU/latency-bound at one wave per SIMD
    // (its rows move 3 bytes per element against ~14 VALU instructions); two
    // workgroups per CU measured 175 us against 208 us at x[32768, 5120], and
    // more waves (one workgroup of 8 or 12, h held packed for the 12) slower.
    // With the gate (7 bytes per element) one workgroup per CU stays best.
    const dim3 grid(stream_grid(S, GATE ? 1 : 2)), block(256);
    hipStream_t st = as_stream(stream);
#define H3MI_QUANT_LAUNCH(C)                                                                                          \
    if (ch == C) {                                                                                                    \
        if (h)                                                                                                        \
            hipLaunchKernelGGL((norm_stream_kernel<256, 64, C, GATE, 2>), grid, block, slds, st, x, o, g, w, ridx, s1, sh, \
                               h, S, (int)N, (int)R, eps, (int)H3MI_RSQRT_HW, nullptr, nullptr, q, qs);           \
        else                                                                                                          \
            hipLaunchKernelGGL((norm_stream_kernel<256, 64, C, GATE, 1>), grid, block, slds, st, x, o, g, w, ridx, s1, sh, \
                               h, S, (int)N, (int)R, eps, (int)H3MI_RSQRT_HW, nullptr, nullptr, q, qs);           \
    }
    H3MI_STREAM_CH(H3MI_QUANT_LAUNCH)
#undef H3MI_QUANT_LAUNCH
    return check_launch(name);
}

}  // namespace
}  // namespace h3mi

using namespace h3mi;

extern "C" int h3mi_norm_mod_quant_i8(const uint16_t* x, const uint16_t* w, const int32_t* ridx, const uint16_t* s1,
                                      const uint16_t* sh, uint16_t* h, int8_t* q, float* qs, int64_t S, int64_t N,
                                      int64_t R, float eps, void* stream) {
    return norm_quant_entry<false>(const_cast<uint16_t*>(x), nullptr, nullptr, w, ridx, s1, sh, h, q, qs, S, N, R, eps,
                                   stream);
}

extern "C" int h3mi_gate_norm_mod_quant_i8(uint16_t* x, const uint16_t* o, const uint16_t* g, const uint16_t* w,
                                           const int32_t* ridx, const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                                           int8_t* q, float* qs, int64_t S, int64_t N, int64_t R, float eps,
                                           void* stream) {
    return norm_quant_entry<true>(x, o, g, w, ridx, s1, sh, h, q, qs, S, N, R, eps, stream);
}

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
    const int ch = stream_ch(static_cast<int>(N));
    if (ch > 0) {  // persistent row stream, N <= 8192
        // One wave per workgroup and per CU: it has 20 KiB of x and o in
        // flight, and fewer bytes in flight stream faster here.  Measured at
        // x[32768, 5120]: 164 us (76.6% of 8 TB/s) against 170 us with four
        // waves and 167 us with two; the norm kernels, which reduce each row
        // before writing it, need their four waves.
        const dim3 grid(stream_grid(S, 1, 1)), block(64);
        const size_t slds = static_cast<size_t>(ch) * 512 * sizeof(float);
#define H3MI_GATE_LAUNCH(C)                                                                                   \
    if (ch == C)                                                                                              \
        hipLaunchKernelGGL((gate_stream_kernel<C>), grid, block, slds, as_stream(stream), x, o, g, ridx, S, (int)N, \
                           (int)R);
        H3MI_STREAM_CH(H3MI_GATE_LAUNCH)
#undef H3MI_GATE_LAUNCH
        return check_launch("gate");
    }
    dim3 grid(static_cast<unsigned>((S + 3) / 4)), block(256);
    hipLaunchKernelGGL(gate_wave_kernel, grid, block, 0, as_stream(stream), x, o, g, ridx, S, (int)N, (int)R);
    return check_launch("gate");
}
