/*
 * h3_oracle.c -- CPU restatement of the reference's W8A8 linear and fused
 * DiT-norm arithmetic.  TEST INFRASTRUCTURE ONLY: this file is the checker
 * that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg compare
 * the HIP kernels against.  Nothing in the product library links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root; LF = comfyui_nodes/h3-linear-fast,
 * FG = comfyui_nodes/h3-fuse-graph).  Arithmetic is plain IEEE fp32 in the
 * exact order the reference kernels use; the build flags in oracle/Makefile
 * forbid contraction and fast-math so the C compiler does not reassociate.
 *
 * Pinning of each function (what fixes it other than this restatement) is in
 * tests/test_oracle_pins.py.  Every function below is pinned, with one
 * exception: the ConvRot quantizer (h3o_exp_neg, h3o_silu, h3o_fwht256,
 * h3o_convrot_quant) restates arithmetic that lives in comfy-kitchen, which the
 * reference does not vendor -- PARITY UNPINNED against the reference; it is
 * pinned only to the mathematics it is defined by.  The same holds for the
 * q/k RMSNorm + RoPE (h3o_rms_rope_split_half), whose definition is pinned to
 * eager PyTorch instead.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#include "h3_oracle.h"

/* ---------------------------------------------------------------------------
 * bf16 helpers
 * ------------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* FG/h3_fuse_kernels.py:78-85 (_rbf16): round-to-nearest-even of an fp32 to
 * bf16 precision, result kept as fp32.  Integer form u + 0x7FFF + lsb, then
 * the low 16 bits cleared. */
float h3o_rbf16(float v)
{
    uint32_t u = f2u(v);
    u = u + 0x7FFFu + ((u >> 16) & 1u);
    u = (u >> 16) << 16;
    return u2f(u);
}

/* fp32 -> bf16 bits, round to nearest even (the `.to(tl.bfloat16)` stores at
 * FG/h3_fuse_kernels.py:114,149,155,167 and LF/int8_gemm_triton.py:66).
 * NaN is kept a quiet NaN (the reference never produces one on finite data). */
uint16_t h3o_bf16_bits(float v)
{
    uint32_t u = f2u(v);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu))
        return (uint16_t)((u >> 16) | 0x0040u);
    u = u + 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float h3o_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* Correctly rounded fp32 1/sqrt(v) for finite v > 0.
 * The reference uses the approximate hardware rsqrt (FG/h3_fuse_kernels.py:104
 * tl.math.rsqrt); that instruction cannot be restated on a CPU, so the oracle
 * offers (a) this correctly rounded value, which the HIP kernels also compute
 * in their "IEEE rsqrt" mode, and (b) a mode that takes the per-row rstd the
 * GPU produced and checks everything downstream of it bit-exactly.
 * Method: start from the double-precision estimate, then decide between the
 * neighbouring floats by the exact sign of m*m*v - 1 at each midpoint m
 * (m has 25 significant bits, so m*m is exact in double and fma(m*m, v, -1)
 * has the exact sign).  No midpoint can equal 1/sqrt(v) exactly. */
float h3o_rsqrt_rn(float v)
{
    if (!(v > 0.0f) || isinf(v)) {
        if (v == 0.0f) return INFINITY;
        if (isinf(v) && v > 0) return 0.0f;
        return NAN;
    }
    float y = (float)(1.0 / sqrt((double)v));
    for (int iter = 0; iter < 2; ++iter) {
        float up = nextafterf(y, INFINITY);
        float dn = nextafterf(y, 0.0f);
        double mhi = 0.5 * ((double)y + (double)up);
        double mlo = 0.5 * ((double)y + (double)dn);
        /* 1/sqrt(v) > mhi  <=>  mhi^2 * v < 1 */
        if (fma(mhi * mhi, (double)v, -1.0) < 0.0) { y = up; continue; }
        if (fma(mlo * mlo, (double)v, -1.0) > 0.0) { y = dn; continue; }
        break;
    }
    return y;
}

/* ---------------------------------------------------------------------------
 * W8A8 linear
 * ------------------------------------------------------------------------- */

/* Per-token symmetric int8 quantizer.  The reference calls comfy-kitchen's
 * quantizer here (LF/h3_linear_fast_patch.py:90-95); this build's quantizer has
 * the per-row semantics of the W8A8 workload definition:
 *   s[m] = max_k |x[m,k]| / 127 (fp32, IEEE divide)
 *   q[m,k] = clamp(round_half_even(x[m,k] / s[m]), -127, 127)   (IEEE divide)
 * A row whose absmax is 0 gets s = 0 and q = 0 (x/s would be 0/0).
 * Non-finite inputs are outside the contract. */
void h3o_quant_rowwise(const uint16_t* x, int64_t M, int64_t K, int64_t ldx,
                       int8_t* q, float* s)
{
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * ldx;
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(h3o_bf16_to_f32(xr[k]));
            if (a > amax) amax = a;
        }
        float sc = amax / 127.0f;
        s[m] = sc;
        for (int64_t k = 0; k < K; ++k) {
            if (sc == 0.0f) { q[m * K + k] = 0; continue; }
            float t = h3o_bf16_to_f32(xr[k]) / sc;
            float r = rintf(t);               /* FE_TONEAREST: half to even */
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q[m * K + k] = (int8_t)r;
        }
    }
}

/* int32 accumulator of the "NT" GEMM, LF/int8_gemm_triton.py:47-60:
 * acc[m,n] = sum_k xq[m,k] * w[n,k], both operands K-contiguous.  Exact in
 * int32 for |acc| <= K*127*127 < 2^31 (K < 133,152). */
void h3o_gemm_i32(const int8_t* xq, const int8_t* w, int64_t M, int64_t N, int64_t K,
                  int64_t ldx, int64_t ldw, int32_t* acc, int64_t ldc)
{
    for (int64_t m = 0; m < M; ++m) {
        const int8_t* a = xq + m * ldx;
        for (int64_t n = 0; n < N; ++n) {
            const int8_t* b = w + n * ldw;
            int32_t sum = 0;
            for (int64_t k = 0; k < K; ++k)
                sum += (int32_t)a[k] * (int32_t)b[k];
            acc[m * ldc + n] = sum;
        }
    }
}

/* Dequant epilogue, LF/int8_gemm_triton.py:2,61-66:
 *   out = bf16( (f32(acc) * xs[m]) * ws[n] )
 * f32(acc) is the round-to-nearest int32->fp32 conversion; both products are
 * fp32 round-to-nearest; the store rounds to bf16 nearest-even.
 * Optional bias (the reference never fuses one: LF/h3_linear_fast_patch.py:64
 * sends bias calls to the original path) is defined by this build as
 *   out = bf16( ((f32(acc) * xs[m]) * ws[n]) + f32(bias[n]) )
 * with the add a separate fp32 rounding (no fused multiply-add). */
void h3o_epilogue_bf16(const int32_t* acc, int64_t ldc, const float* xs, const float* ws,
                       const uint16_t* bias, int64_t M, int64_t N,
                       uint16_t* out, int64_t ldo)
{
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            volatile float c = (float)acc[m * ldc + n];
            c = c * xs[m];
            c = c * ws[n];
            if (bias) c = c + h3o_bf16_to_f32(bias[n]);
            out[m * ldo + n] = h3o_bf16_bits(c);
        }
    }
}

/* ---------------------------------------------------------------------------
 * Fused RMSNorm / adaLN / gate
 * ------------------------------------------------------------------------- */

/* Sum of squares of one row in the reduction order of the reference
 * (FG/h3_fuse_kernels.py:96-103 with _cols4/_sumsq4/_tree128 at :46-75, which
 * copy PyTorch's vectorized_layer_norm_kernel), generalised over the order
 * parameters the reference's own order search sweeps
 * (tests/test_rmsnorm_exact.py:82-105, 127-129):
 *   numx  logical threads; thread t accumulates, sequentially, the vec-wide
 *         chunks t, t+numx, t+2*numx, ... element by element (acc += x*x);
 *   ws    sub-group ("warp") width; within a warp a shuffle-down tree with
 *         offsets ws/2, ..., 1 (lane i += lane i+d);
 *   then across the numx/ws warps the same halving tree (warp i += warp i+d).
 * The reference is numx=128, vec=4, ws=32 (FG/h3_fuse_kernels.py:42-43).
 * x*x of a bf16 value is exact in fp32, so a fused multiply-add in the
 * accumulation gives the same sums as the separate multiply and add here. */
float h3o_row_sumsq(const float* xr, int64_t N, int numx, int vec, int ws)
{
    float* acc = (float*)calloc((size_t)numx, sizeof(float));
    int64_t chunks = (N + vec - 1) / vec;
    int64_t iters = (chunks + numx - 1) / numx;
    for (int64_t it = 0; it < iters; ++it) {
        for (int t = 0; t < numx; ++t) {
            for (int v = 0; v < vec; ++v) {
                int64_t idx = (it * numx + t) * (int64_t)vec + v;
                if (idx < N) {
                    volatile float sq = xr[idx] * xr[idx];
                    acc[t] = acc[t] + sq;
                }
            }
        }
    }
    int nw = numx / ws;
    /* in-warp tree */
    for (int w = 0; w < nw; ++w) {
        float* a = acc + (size_t)w * ws;
        for (int d = ws / 2; d >= 1; d /= 2)
            for (int i = 0; i < d; ++i)
                a[i] = a[i] + a[i + d];
    }
    /* cross-warp tree on the warp totals */
    for (int d = nw / 2; d >= 1; d /= 2)
        for (int i = 0; i < d; ++i)
            acc[(size_t)i * ws] = acc[(size_t)i * ws] + acc[(size_t)(i + d) * ws];
    float tot = acc[0];
    free(acc);
    return tot;
}

/* rstd of one row: FG/h3_fuse_kernels.py:104, rstd = rsqrt(div_rn(tot, N) + eps).
 * Writes var = tot/N + eps (the rsqrt argument) and returns the correctly
 * rounded rstd (see h3o_rsqrt_rn). */
static float row_rstd(float tot, int64_t N, float eps, float* var_out)
{
    volatile float var = tot / (float)N;
    var = var + eps;
    if (var_out) *var_out = var;
    return h3o_rsqrt_rn(var);
}

/* Second pass of _norm_mod_kernel, FG/h3_fuse_kernels.py:105-114, for one
 * element: y = rb(w*(rstd*x)); y = rb(y*s1); h = bf16(y + sh). */
static inline uint16_t mod_elem(float x, float w, float rstd, float s1, float sh)
{
    volatile float t = rstd * x;
    t = w * t;
    float y = h3o_rbf16(t);
    volatile float p = y * s1;
    y = h3o_rbf16(p);
    volatile float r = y + sh;
    return h3o_bf16_bits(r);
}

/* norm_mod, FG/h3_fuse_kernels.py:88-114 and wrapper :174-178.
 * x [S,N] bf16, w [N], ridx [S] (row -> table row), s1/sh [R,N] bf16, h [S,N].
 * rstd_in: if non-NULL, the per-row rstd to use (taken from the GPU's
 * hardware rsqrt); else the correctly rounded rsqrt.  var_out/rstd_out
 * (nullable) receive the rsqrt argument and the rstd used. */
void h3o_norm_mod(const uint16_t* x, const uint16_t* w, const int32_t* ridx,
                  const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                  int64_t S, int64_t N, float eps, int numx, int vec, int ws,
                  const float* rstd_in, float* var_out, float* rstd_out)
{
    float* xr = (float*)malloc((size_t)N * sizeof(float));
    for (int64_t r = 0; r < S; ++r) {
        for (int64_t i = 0; i < N; ++i) xr[i] = h3o_bf16_to_f32(x[r * N + i]);
        float tot = h3o_row_sumsq(xr, N, numx, vec, ws);
        float var;
        float rstd = row_rstd(tot, N, eps, &var);
        if (rstd_in) rstd = rstd_in[r];
        if (var_out) var_out[r] = var;
        if (rstd_out) rstd_out[r] = rstd;
        int64_t tr = ridx[r];
        for (int64_t i = 0; i < N; ++i)
            h[r * N + i] = mod_elem(xr[i], h3o_bf16_to_f32(w[i]), rstd,
                                    h3o_bf16_to_f32(s1[tr * N + i]),
                                    h3o_bf16_to_f32(sh[tr * N + i]));
    }
    free(xr);
}

/* gate_norm_mod_, FG/h3_fuse_kernels.py:117-155 and wrapper :181-185.
 * First xn = rb(x + o*g[ridx]) (:137,148), stored back into x (:149), then
 * norm_mod on xn.  o*g of two bf16 values is exact in fp32, so a fused
 * multiply-add gives the same xn as the separate operations here. */
void h3o_gate_norm_mod(uint16_t* x, const uint16_t* o, const uint16_t* g,
                       const uint16_t* w, const int32_t* ridx,
                       const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                       int64_t S, int64_t N, float eps, int numx, int vec, int ws,
                       const float* rstd_in, float* var_out, float* rstd_out)
{
    float* xr = (float*)malloc((size_t)N * sizeof(float));
    for (int64_t r = 0; r < S; ++r) {
        int64_t tr = ridx[r];
        for (int64_t i = 0; i < N; ++i) {
            volatile float p = h3o_bf16_to_f32(o[r * N + i]) * h3o_bf16_to_f32(g[tr * N + i]);
            volatile float a = h3o_bf16_to_f32(x[r * N + i]) + p;
            xr[i] = h3o_rbf16(a);
        }
        float tot = h3o_row_sumsq(xr, N, numx, vec, ws);
        float var;
        float rstd = row_rstd(tot, N, eps, &var);
        if (rstd_in) rstd = rstd_in[r];
        if (var_out) var_out[r] = var;
        if (rstd_out) rstd_out[r] = rstd;
        for (int64_t i = 0; i < N; ++i) {
            x[r * N + i] = h3o_bf16_bits(xr[i]);
            h[r * N + i] = mod_elem(xr[i], h3o_bf16_to_f32(w[i]), rstd,
                                    h3o_bf16_to_f32(s1[tr * N + i]),
                                    h3o_bf16_to_f32(sh[tr * N + i]));
        }
    }
    free(xr);
}

/* gate_, FG/h3_fuse_kernels.py:158-167 and wrapper :188-192:
 * x <- bf16(x + o*g[ridx]) in place. */
void h3o_gate(uint16_t* x, const uint16_t* o, const uint16_t* g, const int32_t* ridx,
              int64_t S, int64_t N)
{
    for (int64_t r = 0; r < S; ++r) {
        int64_t tr = ridx[r];
        for (int64_t i = 0; i < N; ++i) {
            volatile float p = h3o_bf16_to_f32(o[r * N + i]) * h3o_bf16_to_f32(g[tr * N + i]);
            volatile float a = h3o_bf16_to_f32(x[r * N + i]) + p;
            x[r * N + i] = h3o_bf16_bits(a);
        }
    }
}

/* ---------------------------------------------------------------------------
 * ConvRot quantizer: 256-group Hadamard rotation + per-row int8, with the
 * SwiGLU-fused input variant.
 *
 * The reference runs comfy-kitchen's _C.quantize_int8_rowwise_convrot64 here
 * (LF/h3_linear_fast_patch.py:4,90-95; tests/bench_linear.py:33-40): x [m,k]
 * bf16 (or [m,2k] with input_act="swiglu") -> x_q [m,k] int8, x_s [m,1] fp32,
 * group size 256, k % 256 == 0.  comfy-kitchen is not vendored, so its exact
 * arithmetic is not available: PARITY UNPINNED against the reference.  This
 * restatement fixes one definition, pinned to textbook mathematics in
 * tests/test_oracle_pins.py (Sylvester Hadamard matrix from scipy, float64
 * exp / silu), and the HIP kernel matches it bit for bit:
 *   u = x                               (input_act none)
 *   u = silu(a) * b,  a = x[:, :k], b = x[:, k:]   (input_act swiglu, fp32)
 *   y[g*256 + i] = (1/16) * sum_j H[i][j] u[g*256 + j],  H[i][j] = (-1)^popcount(i & j)
 *     evaluated as the in-place fast Walsh-Hadamard transform, stage h = 1, 2,
 *     ..., 128: (v[j], v[j+h]) <- (v[j] + v[j+h], v[j] - v[j+h]), then * 1/16
 *   s[m] = max|y[m,:]| / 127;  q = clamp(rne(y / s), -127, 127); s = q = 0 for
 *     an all-zero row (the per-token quantizer's rule on y).
 * ------------------------------------------------------------------------- */

/* e^x for x <= 0 in fp32, by a stated method: the argument is clamped to
 * [-86, 0] (e^-86 ~ 4.5e-38 keeps 2^k normal), k = rne(x * log2(e)),
 * Cody-Waite reduction r = x - k*ln2 in two fma steps (ln2 split into
 * 0x1.62e4p-1 + 0x1.7f7d1cp-20), degree-7 Taylor polynomial of e^r by Horner
 * with fma, times 2^k built in the exponent field. */
float h3o_exp_neg(float x)
{
    x = fmaxf(x, -86.0f);
    const float k = rintf(x * 0x1.715476p+0f);      /* log2(e) */
    float r = fmaf(k, -0x1.62e4p-1f, x);             /* ln2, high part */
    r = fmaf(k, -0x1.7f7d1cp-20f, r);                /* ln2, low part */
    float p = 0x1.a01a02p-13f;                       /* 1/7! */
    p = fmaf(p, r, 0x1.6c16c2p-10f);                 /* 1/6! */
    p = fmaf(p, r, 0x1.111112p-7f);                  /* 1/5! */
    p = fmaf(p, r, 0x1.555556p-5f);                  /* 1/4! */
    p = fmaf(p, r, 0x1.555556p-3f);                  /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const uint32_t e = (uint32_t)((int32_t)k + 127) << 23;
    return p * u2f(e);
}

/* 1/d for 1 <= d <= 2: seed 24/17 - 8/17 d (relative error <= 1/17), then
 * three Newton steps e = 1 - d y, y = y + y e, each an fma. */
float h3o_rcp12(float d)
{
    float y = fmaf(d, -0x1.e1e1e2p-2f, 0x1.69696ap+0f);
    for (int i = 0; i < 3; ++i) {
        const float e = fmaf(-d, y, 1.0f);
        y = fmaf(y, e, y);
    }
    return y;
}

/* silu(a) = a / (1 + e^-a), evaluated without overflow as
 * max(a, a * t) * rcp12(1 + t) with t = e^-|a| (the max picks a for a >= 0
 * and a * t for a < 0). */
float h3o_silu(float a)
{
    const float t = h3o_exp_neg(-fabsf(a));
    volatile float at = a * t;
    volatile float den = 1.0f + t;
    volatile float num = fmaxf(a, at);
    return num * h3o_rcp12(den);
}

/* In-place 256-point fast Walsh-Hadamard transform (unnormalised), stages in
 * the order h = 1, 2, 4, ..., 128. */
void h3o_fwht256(float* v)
{
    for (int h = 1; h < 256; h <<= 1)
        for (int i = 0; i < 256; i += 2 * h)
            for (int j = i; j < i + h; ++j) {
                volatile float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

/* ConvRot quantizer (definition above).  act: 0 none, 1 swiglu.  x bf16
 * [M, ldx] with K (act none) or 2K (swiglu) columns used; q int8 [M, K]
 * contiguous; s fp32 [M].  Requires K % 256 == 0. */
void h3o_convrot_quant(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int act,
                       int8_t* q, float* s)
{
    float* y = (float*)malloc((size_t)K * sizeof(float));
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * ldx;
        for (int64_t k = 0; k < K; ++k) {
            if (act == 1) {
                volatile float u = h3o_silu(h3o_bf16_to_f32(xr[k])) * h3o_bf16_to_f32(xr[K + k]);
                y[k] = u;
            } else {
                y[k] = h3o_bf16_to_f32(xr[k]);
            }
        }
        for (int64_t g = 0; g < K; g += 256) h3o_fwht256(y + g);
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            y[k] = y[k] * 0.0625f;
            float a = fabsf(y[k]);
            if (a > amax) amax = a;
        }
        float sc = amax / 127.0f;
        s[m] = sc;
        for (int64_t k = 0; k < K; ++k) {
            if (sc == 0.0f) { q[m * K + k] = 0; continue; }
            float r = rintf(y[k] / sc);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q[m * K + k] = (int8_t)r;
        }
    }
    free(y);
}

/* ---------------------------------------------------------------------------
 * q/k RMSNorm + split-half RoPE, in place.
 *
 * The reference calls comfy-kitchen's ck.rms_rope_split_half_(q, k, rope_freqs,
 * qw, kw, epsilon=attn.q_norm.eps, rot_dim=rope_freqs.shape[-3] * 2) on the
 * [1, s, heads, dim] views of the qkv projection
 * (comfyui_nodes/minimax-h3-sp/minimax_sp/sp_forward.py:279-296); the table
 * is rope_rotation_table(freqs, dtype) (:548), rows sliced per token.
 * comfy-kitchen is not vendored: PARITY UNPINNED against the reference.  The
 * definition restated here is the eager sequence the fused call stands for,
 * and tests/test_gpu_rms_rope.py checks it bit-exactly against eager
 * PyTorch on the GPU:
 *   y = bf16(w * (rstd * x)) per (token, head) row of D elements, the
 *       F.rms_norm of the row (sum of squares in the given order, rstd =
 *       rsqrt(tot / D + eps));
 *   for i < rot/2, with R = tab[token][i] (2 x 2, bf16):
 *       out[i]         = bf16(R00 * y[i] + R01 * y[i + rot/2])
 *       out[i + rot/2] = bf16(R10 * y[i] + R11 * y[i + rot/2])
 *     (each product and the sum rounded separately in fp32);
 *   out[j] = y[j] for rot <= j < D.
 * x [S, H, D] with token stride ldx; tab [S, rot/2, 2, 2]; w [D].
 * rstd_in (nullable): per-row rstd to use, rows in (token, head) order;
 * rstd_out (nullable) receives the rstd used. */
void h3o_rms_rope_split_half(uint16_t* x, const uint16_t* tab, const uint16_t* w,
                             int64_t S, int64_t H, int64_t D, int64_t ldx, int64_t rot, float eps,
                             int numx, int vec, int ws, const float* rstd_in, float* rstd_out)
{
    float* xr = (float*)malloc((size_t)D * sizeof(float));
    float* y = (float*)malloc((size_t)D * sizeof(float));
    const int64_t hr = rot / 2;
    for (int64_t s = 0; s < S; ++s) {
        for (int64_t h = 0; h < H; ++h) {
            uint16_t* row = x + s * ldx + h * D;
            const int64_t r = s * H + h;
            for (int64_t i = 0; i < D; ++i) xr[i] = h3o_bf16_to_f32(row[i]);
            float tot = h3o_row_sumsq(xr, D, numx, vec, ws);
            float rstd = row_rstd(tot, D, eps, NULL);
            if (rstd_in) rstd = rstd_in[r];
            if (rstd_out) rstd_out[r] = rstd;
            for (int64_t i = 0; i < D; ++i) {
                volatile float t = rstd * xr[i];
                t = h3o_bf16_to_f32(w[i]) * t;
                y[i] = h3o_rbf16(t);
            }
            for (int64_t i = 0; i < D; ++i) {
                float o = y[i];
                if (i < rot) {
                    const int64_t p = i < hr ? i : i - hr;     /* the pair (p, p + rot/2) */
                    const uint16_t* R = tab + (s * hr + p) * 4;
                    const int rr = i < hr ? 0 : 1;
                    volatile float a = h3o_bf16_to_f32(R[rr * 2 + 0]) * y[p];
                    volatile float b = h3o_bf16_to_f32(R[rr * 2 + 1]) * y[p + hr];
                    o = a + b;
                }
                row[i] = h3o_bf16_bits(o);
            }
        }
    }
    free(xr);
    free(y);
}
