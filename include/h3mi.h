/*
 * h3mi.h -- C ABI of the MI355X (gfx950) W8A8 INT8 linear and fused DiT-norm
 * kernels (libh3mi.so).
 *
 * Conventions
 *   - Every tensor pointer is a device pointer; the caller owns all memory.
 *     bf16 tensors are passed as uint16_t bit patterns.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Work is
 *     enqueued on it; no entry point synchronises with the host, except the
 *     first SwiGLU h3mi_quant_convrot_i8 call on a device (see there).
 *   - Return value: H3MI_OK (0) or a nonzero H3MI_E* code; the message for the
 *     last failure on the calling thread is h3mi_last_error().
 *   - Row-major layouts with explicit leading dimensions (in elements).
 *
 * Reference paths below are relative to the reference repository root.
 */
#ifndef H3MI_H
#define H3MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define H3MI_ABI_VERSION 1

enum h3mi_status {
    H3MI_OK = 0,
    H3MI_EINVAL = 1,   /* bad shape / stride / value */
    H3MI_EALIGN = 2,   /* pointer or leading dimension not aligned as required */
    H3MI_EALIAS = 3,   /* an output overlaps an input it must not alias */
    H3MI_ELAUNCH = 4,  /* the HIP runtime refused the launch */
    H3MI_EDEVICE = 5   /* current device is not a gfx950 part */
};

/* Reduction orders of the fused norms (logical threads, chunk width, warp
 * width of the shuffle tree).  H3MI_ORDER_DEFAULT is the order of PyTorch's
 * eager rms_norm on this platform; H3MI_ORDER_REF is the order of the
 * reference's CUDA kernels (comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:42-43,
 * 96-104). */
enum h3mi_norm_order {
    H3MI_ORDER_DEFAULT = 0,
    H3MI_ORDER_REF = 1,      /* 128 threads x 4, 32-lane tree   */
    H3MI_ORDER_W64 = 2,      /* 256 threads x 4, 64-lane tree   */
    H3MI_ORDER_COUNT = 3
};

/* rsqrt used for rstd = rsqrt(sumsq/N + eps). */
enum h3mi_rsqrt_mode {
    H3MI_RSQRT_HW = 0,       /* v_rsq_f32, the instruction eager PyTorch uses */
    H3MI_RSQRT_RN = 1        /* correctly rounded 1/sqrt                       */
};

int h3mi_abi_version(void);
const char* h3mi_last_error(void);

/* ------------------------------------------------------------------ W8A8 linear */

/* supported(K) -- comfyui_nodes/h3-linear-fast/int8_gemm_triton.py:86-87.
 * Returns 1 when the GEMM accepts this K (K > 0 and K % 128 == 0). */
int h3mi_w8a8_supported(int64_t K);

/* int8_mm_scaled(xq, w, xs, ws, out) --
 * comfyui_nodes/h3-linear-fast/int8_gemm_triton.py:74-83 (kernel :32-66).
 *   out[m,n] = bf16( (f32(sum_k xq[m,k]*w[n,k]) * xs[m]) * ws[n] )
 * and with bias != NULL (no counterpart in the reference, which never fuses
 * bias): out[m,n] = bf16( ((f32(acc)*xs[m])*ws[n]) + f32(bias[n]) ).
 * xq int8 [M, ldx], w int8 [N, ldw], xs f32 [M], ws f32 [N], bias bf16 [N],
 * out bf16 [M, ldo].  Requires K % 128 == 0, N % 4 == 0, 16-byte aligned
 * xq/w rows (ldx, ldw % 16 == 0), ldo % 4 == 0 and 8-byte aligned out. */
int h3mi_w8a8_gemm_bf16(const int8_t* xq, const int8_t* w, const float* xs, const float* ws,
                        const uint16_t* bias, uint16_t* out,
                        int64_t M, int64_t N, int64_t K,
                        int64_t ldx, int64_t ldw, int64_t ldo, void* stream);

/* The int32 accumulators of the same GEMM (the `acc` of
 * comfyui_nodes/h3-linear-fast/int8_gemm_triton.py:54-60), for parity checks.
 * acc int32 [M, ldc]; ldc % 4 == 0. */
int h3mi_w8a8_gemm_i32(const int8_t* xq, const int8_t* w, int32_t* acc,
                       int64_t M, int64_t N, int64_t K,
                       int64_t ldx, int64_t ldw, int64_t ldc, void* stream);

/* Tile configuration the GEMM uses for (M, N, K): the counterpart of the
 * autotuner's best_config (comfyui_nodes/h3-linear-fast/int8_gemm_triton.py:32,
 * read at tests/test_triton_gemm.py:24).  Writes a NUL-terminated name. */
int h3mi_w8a8_config(int64_t M, int64_t N, int64_t K, char* buf, int64_t buflen);

/* Name of the index-th tile configuration (0-based); H3MI_EINVAL past the
 * last one.  Lets callers enumerate what h3mi_w8a8_set_config accepts. */
int h3mi_w8a8_config_name(int index, char* buf, int64_t buflen);

/* Force one tile configuration by name ("auto" restores the heuristic): the
 * counterpart of H3_LINEAR_FAST_CFG (int8_gemm_triton.py:24-27). */
int h3mi_w8a8_set_config(const char* name);

/* Per-token int8 quantizer.  Replaces the activation quantizer the reference
 * calls at comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95 (without
 * the rotation): s[m] = max_k|x[m,k]|/127, q = clamp(rne(x/s), -127, 127),
 * s = 0 and q = 0 for an all-zero row.  x bf16 [M, ldx], q int8 [M, K]
 * (contiguous), s f32 [M].  Requires K % 8 == 0, ldx % 8 == 0, K <= 32768. */
int h3mi_quant_rowwise_i8(const uint16_t* x, int8_t* q, float* s,
                          int64_t M, int64_t K, int64_t ldx, void* stream);

/* Input activations of the ConvRot quantizer (the reference's input_act,
 * comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:65,91-95). */
enum h3mi_act {
    H3MI_ACT_NONE = 0,
    H3MI_ACT_SWIGLU = 1   /* u = silu(x[:, :K]) * x[:, K:] */
};

/* ConvRot quantizer: 256-group Hadamard rotation + per-row int8.  Replaces
 * comfy-kitchen's _C.quantize_int8_rowwise_convrot64 as the reference calls it
 * at comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95 (group size
 * 256, input_act none or swiglu; tests/bench_linear.py:33-40).  Definition:
 *   u = x (act NONE) or silu(x[:, :K]) * x[:, K:] (act SWIGLU), fp32;
 *   y = H u / 16 per 256-element group, H the Sylvester Hadamard matrix
 *   (fast Walsh-Hadamard transform, stages 1, 2, ..., 128);
 *   s[m] = max|y[m,:]| / 127, q = clamp(rne(y/s), -127, 127); s = q = 0 for
 *   an all-zero row.
 * x bf16 [M, ldx] with K (NONE) or 2K (SWIGLU) columns used; q int8 [M, K]
 * contiguous; s f32 [M].  Requires group_size == 256, K % 256 == 0,
 * K <= 32768, ldx % 8 == 0, x and q 16-byte aligned, no overlaps.  SWIGLU
 * reads a 32 KiB silu table (one static device array per GPU): the first
 * SWIGLU call on a device fills it on `stream` and waits for that fill (the
 * one host synchronisation in this library, once per device and process);
 * a first call under graph capture records the fill in the graph instead. */
int h3mi_quant_convrot_i8(const uint16_t* x, int8_t* q, float* s, int64_t M, int64_t K,
                          int64_t ldx, int group_size, int act, void* stream);

/* ------------------------------------------------------------------ fused DiT norms */

/* norm_mod(x, w, eps, ridx, s1, sh) --
 * comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:174-178 (kernel :88-114).
 *   h = bf16( rb( rb(w*(rstd*x)) * s1[ridx[row]] ) + sh[ridx[row]] )
 * x, h bf16 [S, N] contiguous; w bf16 [N]; ridx int32 [S] with values in
 * [0, R); s1, sh bf16 [R, N].  N % 4 == 0, 8-byte aligned rows.  A row whose
 * ridx is outside [0, R) is left unwritten. */
int h3mi_norm_mod_bf16(const uint16_t* x, const uint16_t* w, const int32_t* ridx,
                       const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                       int64_t S, int64_t N, int64_t R, float eps, void* stream);

/* gate_norm_mod_(x, o, g, w, eps, ridx, s1, sh) --
 * comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:181-185 (kernel :117-155).
 *   x <- rb(x + o*g[ridx[row]])  (in place), then h as norm_mod on the new x.
 * o, h bf16 [S, N]; g [R, N].  o, g and h must not overlap x. */
int h3mi_gate_norm_mod_bf16(uint16_t* x, const uint16_t* o, const uint16_t* g,
                            const uint16_t* w, const int32_t* ridx,
                            const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                            int64_t S, int64_t N, int64_t R, float eps, void* stream);

/* gate_(x, o, g, ridx) --
 * comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:188-192 (kernel :158-167).
 *   x <- bf16(x + o*g[ridx[row]]) in place.  o and g must not overlap x. */
int h3mi_gate_bf16(uint16_t* x, const uint16_t* o, const uint16_t* g, const int32_t* ridx,
                   int64_t S, int64_t N, int64_t R, void* stream);

/* Parity variants of the two norm kernels: explicit reduction order
 * (enum h3mi_norm_order), rsqrt mode (enum h3mi_rsqrt_mode) and optional
 * per-row outputs row_var = sumsq/N + eps and row_rstd (f32 [S], nullable).
 * The reference's own order search (tests/test_rmsnorm_exact.py:82-105)
 * varies the same parameters. */
int h3mi_norm_mod_bf16_ex(const uint16_t* x, const uint16_t* w, const int32_t* ridx,
                          const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                          int64_t S, int64_t N, int64_t R, float eps,
                          int order, int rsqrt_mode, float* row_var, float* row_rstd,
                          void* stream);
int h3mi_gate_norm_mod_bf16_ex(uint16_t* x, const uint16_t* o, const uint16_t* g,
                               const uint16_t* w, const int32_t* ridx,
                               const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                               int64_t S, int64_t N, int64_t R, float eps,
                               int order, int rsqrt_mode, float* row_var, float* row_rstd,
                               void* stream);

/* norm_mod / gate_norm_mod_ with the per-token quantizer of h fused in --
 * no counterpart in the reference: it fuses the norm above
 * (comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:88-114, :117-155) with the
 * quantizer the next linear runs on h (h3mi_quant_rowwise_i8, standing in for
 * comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95), so h need not
 * make an HBM round trip.  q int8 [S, N] and qs f32 [S] are bit-identical to
 * h3mi_norm_mod_bf16 (or h3mi_gate_norm_mod_bf16) followed by
 * h3mi_quant_rowwise_i8 on h; h (bf16 [S, N]) is written as well unless it is
 * NULL.  Default order and hardware rsqrt.  Requires N % 8 == 0 and N <= 8192
 * (H3MI_EINVAL otherwise); q, qs, h must not overlap x or each other. */
int h3mi_norm_mod_quant_i8(const uint16_t* x, const uint16_t* w, const int32_t* ridx,
                           const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                           int8_t* q, float* qs, int64_t S, int64_t N, int64_t R, float eps,
                           void* stream);
int h3mi_gate_norm_mod_quant_i8(uint16_t* x, const uint16_t* o, const uint16_t* g,
                                const uint16_t* w, const int32_t* ridx,
                                const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                                int8_t* q, float* qs, int64_t S, int64_t N, int64_t R, float eps,
                                void* stream);

/* q/k RMSNorm + split-half rotary embedding, in place --
 * comfy-kitchen's ck.rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon,
 * rot_dim) as called at comfyui_nodes/minimax-h3-sp/minimax_sp/
 * sp_forward.py:279-296 (table from rope_rotation_table, :548).  Per (token,
 * head) row of D elements:
 *   y = bf16(w * (rstd * x)), rstd = rsqrt(sum(x^2) / D + eps) with PyTorch's
 *   rms_norm summation order (the eager F.rms_norm of the row);
 *   for i < rot/2, R = tab[token][i]:  out[i] = bf16(R00 y[i] + R01 y[i+rot/2]),
 *   out[i+rot/2] = bf16(R10 y[i] + R11 y[i+rot/2]) (separately rounded fp32
 *   products and sum); out[j] = y[j] for j >= rot.
 * q, k bf16 [S, H, D] with token strides ldq / ldk (elements; heads contiguous;
 * q and k may be views into one qkv buffer); qw, kw bf16 [D]; tab bf16
 * [S, rot/2, 2, 2] (unused when rot == 0).  D in {64, 128, 256}, rot % 16 == 0,
 * rot <= D.  rsqrt_mode: enum h3mi_rsqrt_mode (HW = eager PyTorch's).
 * rstd_out (nullable) f32 [S, 2H]: per token, the q heads' rstd then the k
 * heads'. */
int h3mi_rms_rope_split_half_bf16(uint16_t* q, uint16_t* k, const uint16_t* tab,
                                  const uint16_t* qw, const uint16_t* kw,
                                  int64_t S, int64_t H, int64_t D, int64_t ldq, int64_t ldk,
                                  int64_t rot, float eps, int rsqrt_mode, float* rstd_out,
                                  void* stream);

/* (numx, vec, warp) of an order; returns H3MI_EINVAL for an unknown order. */
int h3mi_norm_order_info(int order, int* numx, int* vec, int* warp);

/* ------------------------------------------------------------------ device primitives
 * No counterpart in the reference: these expose two device operations the
 * kernels above are built from, so tests can pin them in isolation. */

/* out[i] = rsqrt(in[i]) in the given h3mi_rsqrt_mode. */
int h3mi_debug_rsqrt_f32(const float* in, float* out, int64_t n, int rsqrt_mode, void* stream);

/* out[i] = the bf16 (round to nearest even) of in[i], as the kernels store it. */
int h3mi_debug_bf16_rne(const float* in, uint16_t* out, int64_t n, void* stream);

/* One wave of 16-byte LDS-DMA loads in the form the GEMM's operand loads use
 * (buffer_load_dwordx4 ... lds: per-lane voffset, wave-uniform soffset,
 * instruction offset), over a raw buffer of `records` bytes at buf: lane l
 * loads the bytes at voff[l] + soffset + ioffset into an LDS area first filled
 * with 0xAB, and out[16l .. 16l+15] receives the 16 LDS bytes it landed in.
 * Pins which offsets the buffer range check covers (a load past `records`
 * must not return memory).  voff int32 [64] and out [1024 bytes] are device
 * memory; ioffset is 0, 1024, 2048 or 3072.  The caller owns buf up to the
 * largest voff + soffset + ioffset + 16, so every address is in its
 * allocation whatever the check does. */
int h3mi_debug_buffer_lds_load(const uint8_t* buf, int64_t records, const int32_t* voff, int32_t soffset,
                               int32_t ioffset, uint8_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* H3MI_H */
