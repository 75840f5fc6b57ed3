// ConvRot activation quantizer for gfx950: 256-group Hadamard rotation of
// each row, then per-row symmetric int8, optionally with the SwiGLU input
// activation fused in front.
//
// Replaces comfy-kitchen's _C.quantize_int8_rowwise_convrot64 as the
// reference calls it (comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:4,
// 90-95; tests/bench_linear.py:33-40): x bf16 [M, K] (or [M, 2K] for SwiGLU)
// -> q int8 [M, K], s fp32 [M], group size 256, K % 256 == 0.  comfy-kitchen's
// own arithmetic is not published with the reference, so this kernel
// implements one stated definition, bit for bit:
//   u = x,  or  u = silu(a) * b  with a = x[:, :K], b = x[:, K:]   (fp32)
//   silu(a) = max(a, a * t) * rcp12(1 + t),  t = exp_neg(-|a|)
//   y = H u / 16 per 256-group, H the Sylvester Hadamard matrix
//       (H[i][j] = (-1)^popcount(i & j)), evaluated as the fast Walsh-Hadamard
//       transform with stages h = 1, 2, ..., 128, each (a, b) -> (a + b, a - b)
//   s = max|y| / 127,  q = clamp(rne(y / s), -127, 127);  s = q = 0 if max|y| = 0
// exp_neg (e^x for x <= 0 by Cody-Waite reduction and a degree-7 Taylor
// polynomial) and rcp12 (1/d on [1, 2] by three Newton steps from a linear
// seed) are spelled out below in fma, so the same operations give the same
// bits on any IEEE machine.  With SwiGLU, silu of the 8192 bf16 values with
// |a| in [2^-25, 2^7) comes from a table that this same silu fills once per
// device (copied into LDS per workgroup); other values are evaluated.
//
// Layout: 1, 2, 4 or 8 waves per row (shape_for below).  A 16-lane team (one
// DPP row) owns one 256-group, 16 contiguous elements (one 16-element block)
// per lane, so each pass of a wave covers 4 groups = 1024 elements with two
// 16-byte loads per lane and one 16-byte int8 store.  Stages h = 1..8
// (element bits 0-3) run inside a lane.  Stages h = 16..128 (bits 0-3 of the
// block index e) pair lanes whose blocks differ in one bit; lane i of the
// team holds block e = i ^ (3 * bit 2 of i), so the four stages pair lanes
// i ^ 1, i ^ 2, i ^ 7 and i ^ 8, which are the DPP patterns quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror and row_ror:8.  Each such
// stage is one v_fmac_f32 per element with the partner's value as its DPP
// source: own + sgn * partner, sgn = -1 in the lane whose block has the
// stage's bit set.  That gives a + b in the lower lane and b - a = -(a - b) in
// the upper one, each with a single rounding as the transform does (negation
// is exact and round-to-nearest-even is symmetric), and the pair's inputs
// carry the same sign, so after the four stages lane i holds
// (-1)^popcount(e) times the transform; that sign is folded into the
// quotient's multiplier (q and s do not depend on the sign of a zero).  The
// 1/16 is folded into the quotient (y/s == w/(16 s) and w*(r/16) ==
// (w/16)*r exactly unless w/16 is subnormal; rows with max|w| < 2^-100 scale
// w first).
// Rows are read once, from HBM, with buffer loads whose range check returns 0
// past the row; q is written with buffer stores that drop what lies past it.
//
// The quotient: q = rne(fl(y / s)).  Per element the kernel forms
// n = rne(w * r') with one fma against 1.5 * 2^23 (the integer lands in the
// low mantissa bits, which are also the int8 two's-complement byte) and
// d = fl(w * r' - n), r' = fl(1/s)/16.  |w r' - y/s| < 2^-17,
// |fl(y/s) - y/s| <= 2^-18 for |y/s| < 128 and d is within 2^-25 of
// w r' - n, so n == rne(fl(y/s)) whenever |d| <= 0.5 - 2^-16 (an edge of
// 2^-14 sent four times as many passes to the divide: 4-5% of the kernel's
// time).  A pass in which any lane has an element past that edge, or a row
// whose s is not a normal number, takes the IEEE divide.
#include <array>
#include <utility>

#include <mutex>
#include <vector>

#include "common.h"

namespace h3mi {
namespace {

typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));
typedef int32_t v4i_t __attribute__((ext_vector_type(4)));

constexpr float kMagic = kQuantMagic;      // rne(t) + kMagic keeps rne(t) in the low mantissa bits
constexpr float kEdge = kQuantEdge;        // |d| beyond this takes the IEEE divide
constexpr float kTiny = 0x1p-100f;          // rows below this max|w| scale by 1/16 before quantizing

__device__ __forceinline__ __amdgpu_buffer_rsrc_t span(const void* p, int bytes) { return span_bytes(p, bytes); }

// e^x for x <= 0: the argument clamped to [-86, 0] (2^k stays normal),
// k = rne(x log2 e), r = x - k ln2 (two fma steps, ln2 split into
// 0x1.62e4p-1 + 0x1.7f7d1cp-20), Taylor polynomial of degree 7 by Horner,
// times 2^k in the exponent field.
__device__ __forceinline__ float exp_neg(float x) {
#pragma clang fp contract(off)
    x = fmaxf(x, -86.0f);
    const float k = rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(k, -0x1.62e4p-1f, x);
    r = __builtin_fmaf(k, -0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return p * __uint_as_float(static_cast<uint32_t>(static_cast<int32_t>(k) + 127) << 23);
}

// 1/d for 1 <= d <= 2: seed 24/17 - 8/17 d (relative error <= 1/17), three
// Newton steps e = 1 - d y, y = y + y e (within 0.51 ulp of 1/d).
__device__ __forceinline__ float rcp12(float d) {
    float y = __builtin_fmaf(d, -0x1.e1e1e2p-2f, 0x1.69696ap+0f);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const float e = __builtin_fmaf(-d, y, 1.0f);
        y = __builtin_fmaf(y, e, y);
    }
    return y;
}

// silu(a) = a / (1 + e^-a) as max(a, a t) * rcp12(1 + t), t = e^-|a|: the max
// is a for a >= 0 and a t for a < 0, so nothing overflows.
__device__ __forceinline__ float silu(float a) {
#pragma clang fp contract(off)
    const float t = exp_neg(-fabsf(a));
    const float num = fmaxf(a, a * t);
    return num * rcp12(1.0f + t);
}

// silu of every bf16 value whose exponent field lies in [102, 133] (|a| in
// [2^-25, 2^7)): entry (sign << 12) | ((bits & 0x7FFF) - 102 * 128).  Written
// once per device by silu_table_kernel (ensure_silu_table), with the silu
// above, so a lookup returns exactly what silu(a) computes.  Outside the range
// the quantizer evaluates silu(a) itself (a wave pass with any such element
// takes that path).
constexpr int kSiluLo = 102 * 128;   // bf16 bits (sign cleared) of the first entry
constexpr int kSiluEntries = 8192;
__device__ float g_silu_table[kSiluEntries];

__global__ __launch_bounds__(256) void silu_table_kernel() {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t bits = (static_cast<uint32_t>(i >> 12) << 15) | static_cast<uint32_t>((i & 4095) + kSiluLo);
    g_silu_table[i] = silu(bf16_f32(bits));
}

// Byte offset in the table of the bf16 value whose bits minus kSiluLo are t
// (mod 2^16, in bits 0-15), and whether the value has a table entry.
__device__ __forceinline__ uint32_t silu_slot(uint32_t t) { return ((t & 0xFFFu) << 2) | ((t >> 1) & 0x4000u); }
__device__ __forceinline__ bool silu_in_table(uint32_t t) { return (t & 0x7000u) == 0; }

// Block of the team's 256-group that lane i (0..15) of the team holds: with
// DPP on all four cross-lane stages, i ^ (3 * bit 2 of i), so the stages pair
// lanes i ^ 1, i ^ 2, i ^ 7, i ^ 8; with DPP on the first two only, i.
template <int NDPP>
__device__ __forceinline__ int team_block(int i) { return NDPP == 4 ? i ^ (((i >> 2) & 1) * 3) : i; }

// Value of lane (lane ^ MASK) within each 32-lane half, over the LDS crossbar
// (ds_swizzle bitmask mode: and 0x1f, or 0, xor MASK).
template <int MASK>
__device__ __forceinline__ float xor_lane(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (MASK << 10)));
}

// A cross-lane stage over ds_swizzle: v <- sg * v + partner, sg = -1 in the
// upper lane: a + b in the lower lane and a - b in the upper one, one
// rounding each.  Both lanes' inputs carry the same sign, which the outputs
// keep.
template <int MASK>
__device__ __forceinline__ void swizzle_stage(float (&v)[16], float sg) {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = __builtin_fmaf(sg, v[j], xor_lane<MASK>(v[j]));
}

// One cross-lane stage: v[j] += sgn * (v[j] of the DPP partner lane), one
// v_fmac_f32 with a DPP source per element.  The s_nop gives the two wait
// states a DPP read needs after a VALU write of its source; within the block
// no instruction reads a register another one writes.
#define H3MI_FMAC_DPP(J, CTRL) "v_fmac_f32_dpp %" #J ", %" #J ", %16 " CTRL " row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
#define H3MI_DPP_STAGE(v, sgn, CTRL)                                                                                \
    asm volatile("s_nop 1\n" H3MI_FMAC_DPP(0, CTRL) H3MI_FMAC_DPP(1, CTRL) H3MI_FMAC_DPP(2, CTRL)                   \
                     H3MI_FMAC_DPP(3, CTRL) H3MI_FMAC_DPP(4, CTRL) H3MI_FMAC_DPP(5, CTRL) H3MI_FMAC_DPP(6, CTRL)     \
                         H3MI_FMAC_DPP(7, CTRL) H3MI_FMAC_DPP(8, CTRL) H3MI_FMAC_DPP(9, CTRL)                       \
                             H3MI_FMAC_DPP(10, CTRL) H3MI_FMAC_DPP(11, CTRL) H3MI_FMAC_DPP(12, CTRL)                \
                                 H3MI_FMAC_DPP(13, CTRL) H3MI_FMAC_DPP(14, CTRL) H3MI_FMAC_DPP(15, CTRL)            \
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]), \
                   "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]), "+v"(v[12]), "+v"(v[13]), "+v"(v[14]),        \
                   "+v"(v[15])                                                                                       \
                 : "v"(sgn))

// Per-lane constants of the cross-lane stages: the sign of each stage (-1 in
// the lane whose block has that stage's bit set) and the sign the lane's
// values carry after them: each DPP stage flips the upper lane's, so
// (-1)^popcount of the block's bits of the NDPP DPP stages.
struct CrossSigns {
    float s[4];
    float out;
};

template <int NDPP>
__device__ __forceinline__ CrossSigns cross_signs(int lane) {
    const int e = team_block<NDPP>(lane & 15);
    CrossSigns c;
#pragma unroll
    for (int k = 0; k < 4; ++k) c.s[k] = ((e >> k) & 1) ? -1.0f : 1.0f;
    c.out = (__builtin_popcount(e & ((1 << NDPP) - 1)) & 1) ? -1.0f : 1.0f;
    return c;
}

// The 256-point transform of the team's group, up to the sign cs.out: lane i
// of the team holds elements 16 * team_block(i) + j.  The first NDPP (0, 2 or
// 4) cross-lane stages run as DPP fmacs (VALU), the others over ds_swizzle
// (the LDS crossbar): the kernel whose LDS is busy with its silu table
// lookups takes all four on DPP, the plain one none (measured).
template <int NDPP>
__device__ __forceinline__ void fwht256(float (&v)[16], const CrossSigns& cs) {
#pragma clang fp contract(off)
#pragma unroll
    for (int h = 1; h < 16; h <<= 1) {
#pragma unroll
        for (int i = 0; i < 16; i += 2 * h) {
#pragma unroll
            for (int j = i; j < i + h; ++j) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
        }
    }
    static_assert(NDPP == 0 || NDPP == 2 || NDPP == 4, "DPP stages");
    if constexpr (NDPP >= 2) {
        H3MI_DPP_STAGE(v, cs.s[0], "quad_perm:[1,0,3,2]");  // h = 16: lane i ^ 1
        H3MI_DPP_STAGE(v, cs.s[1], "quad_perm:[2,3,0,1]");  // h = 32: lane i ^ 2
    } else {
        swizzle_stage<1>(v, cs.s[0]);
        swizzle_stage<2>(v, cs.s[1]);
    }
    if constexpr (NDPP == 4) {
        H3MI_DPP_STAGE(v, cs.s[2], "row_half_mirror");      // h = 64: lane i ^ 7
        H3MI_DPP_STAGE(v, cs.s[3], "row_ror:8");            // h = 128: lane i ^ 8
    } else {
        swizzle_stage<4>(v, cs.s[2]);
        swizzle_stage<8>(v, cs.s[3]);
    }
}

__device__ __forceinline__ void unpack16(const v4u_t (&r)[2], float (&v)[16]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[h * 8 + 2 * i] = bf16_lo(r[h][i]);
            v[h * 8 + 2 * i + 1] = bf16_hi(r[h][i]);
        }
    }
}

__device__ __forceinline__ uint32_t pack4(const float* n) {
    return pack_low_bytes(__float_as_uint(n[0]), __float_as_uint(n[1]), __float_as_uint(n[2]), __float_as_uint(n[3]));
}

// P passes of 1024 elements per wave, WPR waves per row, rows_per_block(WPR)
// rows per workgroup.  Rows at or past M have empty buffer ranges.
template <int P, int WPR, bool SWIGLU>
__global__ __launch_bounds__(64 * WPR * rows_per_block(WPR)) void convrot_quant_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ s, int M, int K, int64_t ldx) {
#pragma clang fp contract(off)
    constexpr int RPB = rows_per_block(WPR);
    __shared__ float red[WPR * RPB];
    __shared__ __attribute__((aligned(16))) float tab[SWIGLU ? kSiluEntries : 1];
    const int lane = threadIdx.x & 63;
    // uniform per wave: keeps the buffer resources in SGPRs (no waterfall loops)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wr = wave % WPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + wave / WPR;
    const bool in = row < M;
    const uint16_t* xr = x + (in ? row : 0) * ldx;
    const int bytes = in ? K * 2 : 0;
    const __amdgpu_buffer_rsrc_t ra = span(xr, bytes);
    const __amdgpu_buffer_rsrc_t rb = span(xr + (SWIGLU ? K : 0), SWIGLU ? bytes : 0);
    const __amdgpu_buffer_rsrc_t rq = span(q + (in ? row : 0) * static_cast<int64_t>(K), in ? K : 0);
    constexpr int NDPP = SWIGLU ? 4 : 0;
    const CrossSigns cs = cross_signs<NDPP>(lane);
    const int blk = (lane & 48) + team_block<NDPP>(lane & 15);  // the 16-element block this lane holds in its pass

    float v[P][16];
    {
        v4u_t la[P][2];
        v4u_t lb[SWIGLU ? P : 1][2];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int off = (p * WPR + wr) * 2048 + blk * 32;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                la[p][h] = __builtin_bit_cast(v4u_t, __builtin_amdgcn_raw_buffer_load_b128(ra, off + 16 * h, 0, 2));
                if constexpr (SWIGLU)
                    lb[p][h] = __builtin_bit_cast(v4u_t, __builtin_amdgcn_raw_buffer_load_b128(rb, off + 16 * h, 0, 2));
            }
        }
        if constexpr (SWIGLU) {
            // The silu table, 32 KiB, into LDS by LDS-DMA behind the row loads:
            // each wave copies its share in 1 KiB pieces (16 bytes per lane).
            constexpr int NW = WPR * RPB, PIECES = kSiluEntries * 4 / 1024;
            static_assert(PIECES % NW == 0, "table pieces split over the waves");
            const __amdgpu_buffer_rsrc_t rt = span_bytes(g_silu_table, kSiluEntries * 4);
#pragma unroll
            for (int i = 0; i < PIECES / NW; ++i) {
                const int piece = wave * (PIECES / NW) + i;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_ptr_t)(tab + piece * 256), 16, lane * 16, piece * 1024, 0,
                                                         0);
            }
            wait_vm<0>();  // this wave's rows and table pieces have landed
            __syncthreads();
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if constexpr (SWIGLU) {
                float g[16], sl[16];
                unpack16(lb[p], g);
                bool outside = false;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t w = la[p][i >> 2][i & 3];
                    const uint32_t t0 = w - kSiluLo, t1 = (w >> 16) - kSiluLo;
                    outside |= !silu_in_table(t0) || !silu_in_table(t1);
                    sl[2 * i] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(tab) + silu_slot(t0));
                    sl[2 * i + 1] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(tab) + silu_slot(t1));
                }
                if (__builtin_amdgcn_ballot_w64(outside) != 0) {
                    float a[16];
                    unpack16(la[p], a);
#pragma unroll
                    for (int j = 0; j < 16; ++j) sl[j] = silu(a[j]);
                }
#pragma unroll
                for (int j = 0; j < 16; ++j) v[p][j] = sl[j] * g[j];
            } else {
                unpack16(la[p], v[p]);
            }
        }
    }

    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        fwht256<NDPP>(v[p], cs);
#pragma unroll
        for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(v[p][j]));
    }
    amax = wave_max(amax);
    if constexpr (WPR > 1) {
        if (lane == 0) red[wave] = amax;
        __syncthreads();
        const int w0 = wave - wr;
#pragma unroll
        for (int i = 0; i < WPR; ++i) amax = fmaxf(amax, red[w0 + i]);
        amax = wave_uniform(amax);
    }

    // w = 16 y; rows this small scale w to y first so no quotient underflows
    const bool tiny = amax < kTiny;
    if (tiny) {
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int j = 0; j < 16; ++j) v[p][j] = v[p][j] * 0.0625f;
    }
    const float sc = (amax * 0.0625f) / 127.0f;
    if (in && wr == 0 && lane == 0) s[row] = sc;
    const float r = 1.0f / sc;
    const bool zero = sc == 0.0f;
    // The sign the transform left in this lane's values is folded into the
    // multiplier (exact): n and d below are those of the true values.  An
    // all-zero row multiplies by 0: every n is the magic constant (q = 0)
    // and every residual 0, with no select per element.
    const float rr = zero ? 0.0f : (tiny ? r : r * 0.0625f) * cs.out;
    const bool fast = quot_fast(sc, r);

#pragma unroll
    for (int p = 0; p < P; ++p) {
        float n[16];
        bool near = false;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            n[j] = __builtin_fmaf(v[p][j], rr, kMagic);
            const float d = __builtin_fmaf(v[p][j], rr, -(n[j] - kMagic));
            near |= fabsf(d) > kEdge;
        }
        if (!zero && (!fast || __builtin_amdgcn_ballot_w64(near) != 0)) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float y = (tiny ? v[p][j] : v[p][j] * 0.0625f) * cs.out;
                n[j] = fminf(fmaxf(rintf(y / sc), -127.0f), 127.0f) + kMagic;
            }
        }
        const v4u_t o = {pack4(n), pack4(n + 4), pack4(n + 8), pack4(n + 12)};
        // a cached store: the GEMM reads q next
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i_t, o), rq, (p * WPR + wr) * 1024 + blk * 16, 0, 0);
    }
}

typedef void (*convrot_fn)(const uint16_t*, int8_t*, float*, int, int, int64_t);

template <bool SW, int WPR, int... P>
constexpr std::array<convrot_fn, sizeof...(P)> row_of(std::integer_sequence<int, P...>) {
    return {convrot_quant_kernel<P + 1, WPR, SW>...};
}

constexpr int kMaxP = 8;
constexpr int kWprs[] = {1, 2, 4, 8};

template <bool SW>
convrot_fn pick(int P, int WPR) {
    static constexpr std::array<std::array<convrot_fn, kMaxP>, 4> table = {
        row_of<SW, 1>(std::make_integer_sequence<int, kMaxP>{}), row_of<SW, 2>(std::make_integer_sequence<int, kMaxP>{}),
        row_of<SW, 4>(std::make_integer_sequence<int, kMaxP>{}), row_of<SW, 8>(std::make_integer_sequence<int, kMaxP>{})};
    if (P < 1 || P > kMaxP) return nullptr;
    for (int i = 0; i < 4; ++i)
        if (kWprs[i] == WPR) return table[i][P - 1];
    return nullptr;
}

// Per device: the silu table has been filled and the fill has completed.
std::mutex g_silu_mu;
std::vector<char> g_silu_ready;

// Fills the current device's silu table on `stream` the first time a SwiGLU
// call reaches that device, and waits for the fill (under the lock, so a
// concurrent first call on another thread waits too); later calls launch
// nothing, so no quantizer ever reads the table while it is being written.
// A first call under graph capture records the fill in the graph instead (the
// stream cannot be waited on), and the table counts as filled only once an
// uncaptured call has filled it: replays rewrite it with the same values.
int ensure_silu_table(hipStream_t stream) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(H3MI_ELAUNCH, "convrot: hipGetDevice failed");
    std::lock_guard<std::mutex> lk(g_silu_mu);
    if (dev < static_cast<int>(g_silu_ready.size()) && g_silu_ready[dev]) return ok();
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return fail(H3MI_ELAUNCH, "convrot: stream query failed");
    hipLaunchKernelGGL(silu_table_kernel, dim3(kSiluEntries / 256), dim3(256), 0, stream);
    if (const int rc = check_launch("silu_table_kernel")) return rc;
    if (cs != hipStreamCaptureStatusNone) return ok();
    if (hipStreamSynchronize(stream) != hipSuccess) return fail(H3MI_ELAUNCH, "convrot: silu table fill failed");
    if (dev >= static_cast<int>(g_silu_ready.size())) g_silu_ready.resize(dev + 1, 0);
    g_silu_ready[dev] = 1;
    return ok();
}

// Waves per row and passes per wave for a row of `chunks` 1024-element
// chunks.  Measured at 19200 rows: the registers of more than 3 passes (4 with
// SwiGLU, whose per-element work is larger) cost more occupancy than the
// extra waves' reductions cost, and workgroups of 3, 6 or 7 waves schedule
// worse than 4 or 8 (7 waves x 1 pass at K = 7168, every lane busy: 84.6
// against 74.9 us for 4 x 2 with one pass slot in 8 empty).  So: the fewest wasted pass slots with at most that many
// passes, ties to fewer waves per row; past 8 waves, 8 waves and more passes.
void shape_for(int chunks, bool swiglu, int* wpr, int* passes) {
    const int pmax = swiglu ? 4 : 3;
    int best_w = 8, best_p = (chunks + 7) / 8, best_slots = 1 << 30;
    for (int w : kWprs) {
        const int p = (chunks + w - 1) / w;
        if (p > pmax) continue;
        if (p * w < best_slots) best_w = w, best_p = p, best_slots = p * w;
    }
    *wpr = best_w;
    *passes = best_p;
}

}  // namespace
}  // namespace h3mi

using namespace h3mi;

extern "C" int h3mi_quant_convrot_i8(const uint16_t* x, int8_t* q, float* s, int64_t M, int64_t K, int64_t ldx,
                                     int group_size, int act, void* stream) {
    if (group_size != 256) return fail(H3MI_EINVAL, "convrot: group size %d (only 256 is supported)", group_size);
    if (act != H3MI_ACT_NONE && act != H3MI_ACT_SWIGLU) return fail(H3MI_EINVAL, "convrot: unknown input activation %d", act);
    if (M < 0 || K <= 0) return fail(H3MI_EINVAL, "convrot: bad sizes M=%lld K=%lld", (long long)M, (long long)K);
    if (K % 256) return fail(H3MI_EINVAL, "convrot: K=%lld must be a multiple of 256", (long long)K);
    if (K > 32768) return fail(H3MI_EINVAL, "convrot: K=%lld exceeds 32768", (long long)K);
    const int64_t kin = act == H3MI_ACT_SWIGLU ? 2 * K : K;
    if (ldx < kin || ldx % 8)
        return fail(H3MI_EALIGN, "convrot: ldx=%lld must be >= %lld and a multiple of 8", (long long)ldx, (long long)kin);
    if (M > 0x7FFFFFFF) return fail(H3MI_EINVAL, "convrot: M too large");
    if (M == 0) return ok();
    if (!x || !q || !s) return fail(H3MI_EINVAL, "convrot: null pointer");
    if (!aligned(x, 16) || !aligned(q, 16) || !aligned(s, 4)) return fail(H3MI_EALIGN, "convrot: x and q need 16-byte alignment");
    const size_t xb = static_cast<size_t>((M - 1) * ldx + kin) * 2, qb = static_cast<size_t>(M * K), sb = static_cast<size_t>(M) * 4;
    if (overlap(q, qb, x, xb) || overlap(s, sb, x, xb) || overlap(q, qb, s, sb))
        return fail(H3MI_EALIAS, "convrot: q, s and x must not overlap");
    const int chunks = static_cast<int>(K / 1024 + (K % 1024 ? 1 : 0));
    int wpr = 1, P = 1;
    shape_for(chunks, act == H3MI_ACT_SWIGLU, &wpr, &P);
    const convrot_fn fn = act == H3MI_ACT_SWIGLU ? pick<true>(P, wpr) : pick<false>(P, wpr);
    if (!fn) return fail(H3MI_EINVAL, "convrot: no kernel for K=%lld", (long long)K);
    const int rpb = rows_per_block(wpr);
    const int64_t blocks = (M + rpb - 1) / rpb;
    if (act == H3MI_ACT_SWIGLU) {
        if (const int rc = ensure_silu_table(as_stream(stream))) return rc;
    }
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(blocks)), dim3(64 * wpr * rpb), 0, as_stream(stream), x, q, s,
                       static_cast<int>(M), static_cast<int>(K), ldx);
    return check_launch("convrot_quant_kernel");
}
