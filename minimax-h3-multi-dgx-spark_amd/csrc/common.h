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

// ------------------------------------------------------------------ waits and LDS pointers

// s_waitcnt with vmcnt <= N (the other counters left alone).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt lgkmcnt(0): this wave's LDS operations (and scalar loads) are done.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4)); }

// Workgroup barrier the compiler cannot move memory operations across.
__device__ __forceinline__ void wg_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// LDS address operand of the LDS-DMA load builtins.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

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

// bf16x2_bits whose result the compiler treats as opaque.  Without the empty
// asm, bf16_hi / bf16_lo of the pair are folded back into one single-value
// conversion per half plus a mask: five instructions for two values instead
// of three.
__device__ __forceinline__ uint32_t bf16x2_kept(float lo, float hi) {
    uint32_t p = bf16x2_bits(lo, hi);
    asm("" : "+v"(p));
    return p;
}

// rb(v) in one instruction: the pair conversion with +0 as the low value puts
// bf16(v) in the high half over a zero low half, which is rb(v) as fp32 (a
// pair conversion plus two unpacks takes three instructions for two values).
__device__ __forceinline__ float rb_hi(float v) {
    float r;
    asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(v));
    return r;
}

// a, b <- rb(a), rb(b)
__device__ __forceinline__ void rb2(float& a, float& b) {
    a = rb_hi(a);
    b = rb_hi(b);
}

// rb2 with one pair conversion and two unpacks.
__device__ __forceinline__ void rb2_pair(float& a, float& b) {
    const uint32_t p = bf16x2_kept(a, b);
    a = bf16_lo(p);
    b = bf16_hi(p);
}

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

// rne(t) + kQuantMagic holds rne(t) in its low mantissa bits for |t| < 2^22;
// the low byte is then rne(t) as an int8 (two's complement).
constexpr float kQuantMagic = 0x1.8p+23f;

// Byte B of w <- low byte of fl(a + b), the other bytes kept (B = 0: cleared).
// One SDWA add replaces the add plus a share of the byte packing.
template <int B>
__device__ __forceinline__ void add_low_byte(uint32_t& w, float a, float b) {
    static_assert(B >= 0 && B < 4, "byte index");
    if constexpr (B == 0)
        asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
            : "=v"(w) : "v"(a), "v"(b));
    else if constexpr (B == 1)
        asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
            : "+v"(w) : "v"(a), "v"(b));
    else if constexpr (B == 2)
        asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
            : "+v"(w) : "v"(a), "v"(b));
    else
        asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
            : "+v"(w) : "v"(a), "v"(b));
}

// A quotient whose residual |t - rne(t)| exceeds this takes the IEEE divide
// (the ConvRot quantizer).  The product t = w r' lies within 2^-17 of the
// quotient and the rounded quotient within 2^-18 of it (|quotient| < 128), and
// the computed residual is off by at most 2^-25: 2^-17 + 2^-18 + 2^-25 < 2^-16,
// so a residual within 0.5 - 2^-16 leaves the rounded quotient on the same
// side of the half-integer (tests/quant_edge_check.c; 0.5 - 2^-17 fails it).
constexpr float kQuantEdge = 0.5f - 0x1p-16f;

// Low bytes of four fp32 words into one word (v_perm_b32: selector 4 = first
// operand's byte 0, 0 = second operand's byte 0, 0x0c = zero).
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    return __builtin_amdgcn_perm(b1, b0, 0x0C0C0400u) | __builtin_amdgcn_perm(b3, b2, 0x04000C0Cu);
}

// A row scale whose quotients the ConvRot quantizer may form from e * r (sc
// and r normal).
__device__ __forceinline__ bool quot_fast(float sc, float r) {
    return sc >= 0x1p-126f && sc <= 0x1p+126f && r <= 0x1p+126f;
}

// Per-token int8 quantization of 8 elements whose values are bf16 numbers, as
// the per-token quantizer and the norm -> quantizer fusion have them (|e| <=
// amax, amax a bf16 value, sc = fl(amax / 127), r = fl(1 / sc)):
// clamp(rne(fl(e / sc)), -127, 127), with no residual test and no branch per
// chunk.  When quot_exact(sc, r), q0 = fl(e r), the remainder
// fl(e - q0 sc) is exact by fma, and one correction step with the correctly
// rounded reciprocal, q1 = fl(q0 + rem r), is the correctly rounded quotient
// fl(e / sc) (Markstein's division correction); rne(q1) by the magic add.
// An exhaustive check over every positive bf16 amax with 2^-100 <= sc <= 2^126
// and every bf16 e in [0, amax] (523,237,695 pairs; the result is odd in e)
// finds no difference from clamp(rne(fl(e / sc))) computed with the IEEE
// divide (tests/quant_exact_check.c).  With sc below 2^-100 the remainder can
// lose bits in the subnormal range, so those rows take the IEEE divide.  Four
// VALU per element, the byte packing included.  The residual test the ConvRot
// quantizer uses for its fp32 values (rne(e r) unless some element of the
// wave's chunk lies within 2^-14 of a half-integer, then the divide) would
// send about half of a bf16 row's chunks to the divide: quotients of bf16
// values land exactly on half-integers for about 0.26% of elements.
__device__ __forceinline__ bool quot_exact(float sc, float r) {
    return sc >= 0x1p-100f && sc <= 0x1p+126f && r <= 0x1p+126f;
}

__device__ __forceinline__ uint2 quant8b(const float (&e)[8], float sc, float r, bool exact) {
#pragma clang fp contract(off)
    float n[8];
    if (exact) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float q0 = e[j] * r;
            const float rem = __builtin_fmaf(-q0, sc, e[j]);
            n[j] = __builtin_fmaf(rem, r, q0);
        }
        // the magic add writes its low byte straight into place
        const float mg = kQuantMagic;
        uint32_t lo, hi;
        add_low_byte<0>(lo, n[0], mg);
        add_low_byte<1>(lo, n[1], mg);
        add_low_byte<2>(lo, n[2], mg);
        add_low_byte<3>(lo, n[3], mg);
        add_low_byte<0>(hi, n[4], mg);
        add_low_byte<1>(hi, n[5], mg);
        add_low_byte<2>(hi, n[6], mg);
        add_low_byte<3>(hi, n[7], mg);
        return make_uint2(lo, hi);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) n[j] = fminf(fmaxf(rintf(e[j] / sc), -127.0f), 127.0f) + kQuantMagic;
    }
    return make_uint2(pack_low_bytes(__float_as_uint(n[0]), __float_as_uint(n[1]), __float_as_uint(n[2]), __float_as_uint(n[3])),
                      pack_low_bytes(__float_as_uint(n[4]), __float_as_uint(n[5]), __float_as_uint(n[6]), __float_as_uint(n[7])));
}

// quant8b of 8 packed bf16 values (2 per word).
__device__ __forceinline__ uint2 quant8(const uint32_t (&w4)[4], float sc, float r, bool exact) {
    float e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = (j & 1) ? bf16_hi(w4[j >> 1]) : bf16_lo(w4[j >> 1]);
    return quant8b(e, sc, r, exact);
}

// A row's max, made wave-uniform (every lane holds the same value after a
// full butterfly), so that branches on the row's scale are scalar.
__device__ __forceinline__ float wave_uniform(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// Max of v over the wave's 64 lanes (all active), returned wave-uniform.  Six
// v_max_f32 with a DPP source: lane ^ 1 and lane ^ 2 (quad_perm), the mirror
// within 8 lanes and the rotation by 8 within 16 leave every lane of a 16-lane
// row with the row's max; row_bcast:15 then folds row 0 into row 1 and row 2
// into row 3, row_bcast:31 rows 0-1 into rows 2-3, and lane 63 holds the
// wave's max.  The inputs are canonical (results of arithmetic or of fmaxf),
// so a quiet NaN loses to a number as it does in fmaxf.  Each DPP source is
// the VGPR the instruction before wrote, which needs two wait states (s_nop 1;
// one more before the lane read).  Against __shfl_xor's butterfly (a
// ds_bpermute, its address arithmetic and a canonicalizing max per step) this
// is 6 VALU per wave.
__device__ __forceinline__ float wave_max(float v) {
    asm volatile(
        "s_nop 1\n"
        "v_max_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n"
        "s_nop 1\n"
        "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n"
        "s_nop 1\n"
        "v_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n"
        "s_nop 1\n"
        "v_max_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf\n"
        "s_nop 1\n"
        "v_max_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n"
        "s_nop 1\n"
        "v_max_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n"
        "s_nop 1\n"
        : "+v"(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Buffer resource over `bytes` bytes at p: loads past the end return 0 and
// stores past it are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_bytes(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0), bytes, 0x00020000);
}

// Rows per workgroup of a row kernel with wpr waves per row: workgroups of 4
// waves when wpr divides 4, else one row per workgroup.
constexpr int rows_per_block(int wpr) { return wpr == 1 ? 4 : wpr == 2 ? 2 : 1; }

}  // namespace h3mi
