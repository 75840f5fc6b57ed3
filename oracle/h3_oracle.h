/* h3_oracle.h -- CPU restatement of the reference arithmetic (test
 * infrastructure only; see h3_oracle.c). */
#ifndef H3_ORACLE_H
#define H3_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
float    h3o_rbf16(float v);
uint16_t h3o_bf16_bits(float v);
float    h3o_bf16_to_f32(uint16_t b);
float    h3o_rsqrt_rn(float v);
void h3o_quant_rowwise(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s);
void h3o_gemm_i32(const int8_t* xq, const int8_t* w, int64_t M, int64_t N, int64_t K,
                  int64_t ldx, int64_t ldw, int32_t* acc, int64_t ldc);
void h3o_epilogue_bf16(const int32_t* acc, int64_t ldc, const float* xs, const float* ws,
                       const uint16_t* bias, int64_t M, int64_t N, uint16_t* out, int64_t ldo);
float h3o_row_sumsq(const float* xr, int64_t N, int numx, int vec, int ws);
void h3o_norm_mod(const uint16_t* x, const uint16_t* w, const int32_t* ridx,
                  const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                  int64_t S, int64_t N, float eps, int numx, int vec, int ws,
                  const float* rstd_in, float* var_out, float* rstd_out);
void h3o_gate_norm_mod(uint16_t* x, const uint16_t* o, const uint16_t* g,
                       const uint16_t* w, const int32_t* ridx,
                       const uint16_t* s1, const uint16_t* sh, uint16_t* h,
                       int64_t S, int64_t N, float eps, int numx, int vec, int ws,
                       const float* rstd_in, float* var_out, float* rstd_out);
void h3o_gate(uint16_t* x, const uint16_t* o, const uint16_t* g, const int32_t* ridx,
              int64_t S, int64_t N);
float h3o_exp_neg(float x);
float h3o_rcp12(float d);
float h3o_silu(float a);
void h3o_fwht256(float* v);
void h3o_rms_rope_split_half(uint16_t* x, const uint16_t* tab, const uint16_t* w,
                             int64_t S, int64_t H, int64_t D, int64_t ldx, int64_t rot, float eps,
                             int numx, int vec, int ws, const float* rstd_in, float* rstd_out);
void h3o_convrot_quant(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int act,
                       int8_t* q, float* s);
#ifdef __cplusplus
}
#endif
#endif
