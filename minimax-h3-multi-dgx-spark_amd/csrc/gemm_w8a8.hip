// W8A8 int8 GEMM with fused dequant epilogue for gfx950 (MI355X).
//
// Reference: comfyui_nodes/h3-linear-fast/int8_gemm_triton.py
//   kernel :32-66, wrapper int8_mm_scaled :74-83, supported :86-87.
//   out[m,n] = bf16( (f32(sum_k xq[m,k]*w[n,k]) * xs[m]) * ws[n] )
//
// Design (CDNA4, not a translation of the Triton tiling):
//   * v_mfma_i32_32x32x32_i8: one instruction multiplies a 32x32 int8 block by
//     a 32x32 int8 block (64 Ki int ops).  Both operands are K-contiguous ("NT"
//     GEMM), so a lane's 16-byte fragment is 16 consecutive K bytes of one row
//     of W or of X; the MFMA A operand is W (rows n) and B is X (rows m), which
//     makes every lane own 4 consecutive n of one output row m: the epilogue
//     stores 8 bytes of bf16 per lane.
//   * Workgroup tile BM x BN (m x n), K step BK, WM x WN waves, each wave a
//     (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks; int32 accumulators stay
//     in registers (AGPRs) for the whole K loop.
//   * Global -> LDS staging through buffer loads (out-of-range rows of the
//     last tile read as zero) into a double-buffered LDS tile with an XOR
//     swizzle of 16-byte chunks, so fragment reads of 8/16 consecutive rows at
//     the same K hit distinct banks.
//   * Tile order is XCD-aware: workgroup i runs on XCD i % 8, so the linear
//     tile index is remapped to give each XCD a contiguous run of tiles, then
//     grouped GROUP_M m-tiles at a time so concurrently running tiles share
//     X and W panels in that XCD's L2.
#include <string.h>

#include <mutex>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "common.h"

namespace h3mi {
namespace {

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

constexpr int kNumXcd = 8;
constexpr int kBufDword3 = 0x00020000;  // raw buffer, gfx9 family

template <int BM_, int BN_, int BK_, int WM_, int WN_, int GROUP_M_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, GROUP_M = GROUP_M_;
    static constexpr int NW = WM * WN;
    static constexpr int NT = NW * 64;
    static constexpr int TM = BM / WM, TN = BN / WN;  // per-wave extent
    static constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 blocks per wave
    static constexpr int KC = BK / 16;                // 16-byte chunks per tile row
    static constexpr int KS = BK / 32;                // MFMA k-steps per K tile
    static constexpr int W_BYTES = BN * BK;
    static constexpr int X_BYTES = BM * BK;
    static constexpr int STAGE = W_BYTES + X_BYTES;
    // Scale slices in LDS: ws [BN] f32, xs [BM] f32, bias [BNB] bf16, bias
    // [BNB] f32, where BNB rounds BN up to whole 128-entry (256-byte) copies.
    static constexpr int BNB = (BN + 127) / 128 * 128;
    static constexpr int SC_XS = BN * 4, SC_B16 = BN * 4 + BM * 4, SC_B32 = SC_B16 + BNB * 2;
    static constexpr int SC_BYTES = SC_B32 + BNB * 4;
    static constexpr int LW = W_BYTES / 16 / NT;      // staged chunks per thread
    static constexpr int LX = X_BYTES / 16 / NT;
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be whole 32x32 blocks");
    static_assert(W_BYTES % (16 * NT) == 0 && X_BYTES % (16 * NT) == 0, "tile must split evenly over lanes");
    static_assert(KC == 4 || KC == 8, "BK must be 64 or 128");
};

// Physical 16-byte chunk of logical chunk c in tile row `row`.  A fragment
// read is one ds_read_b128 in which lanes 0..31 read 32 consecutive rows at
// the same logical chunk (lanes 32..63 the next chunk).  gfx950's LDS has 64
// banks of 4 bytes; the forms below were measured (SQ_LDS_BANK_CONFLICT) to
// give conflict-free fragment reads, where the unswizzled layouts cost 3 (for
// 64-byte rows) and 7 (for 128-byte rows) extra cycles per read.  For 128-byte
// rows, any 16 consecutive rows of a 16-row block land in distinct 16-byte
// bank groups under both forms (two rows per 256 bytes of banks); the second
// (ROW_BITS_123) depends only on row bits 1-3, so rows 32 apart share it.
template <int KC, bool ROW_BITS_123 = false>
__device__ __forceinline__ int swz(int row, int c) {
    if constexpr (KC == 8 && ROW_BITS_123) return c ^ ((row >> 1) & 7);
    else if constexpr (KC == 8) return c ^ ((row ^ (row >> 3)) & 7);
    else return c ^ ((row >> 2) & 3);
}

template <int GROUP_M>
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    const int per = (total + kNumXcd - 1) / kNumXcd;
    const int tall = (total % kNumXcd) == 0 ? kNumXcd : (total % kNumXcd);
    const int xcd = pid % kNumXcd, local = pid / kNumXcd;
    const int lin = xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
    const int group = GROUP_M * tiles_n;
    const int first_m = (lin / group) * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    const int in = lin % group;
    tm = first_m + in % gsize;
    tn = in / gsize;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    const int n = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : static_cast<int>(bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), n, kBufDword3);
}

// Epilogue.  acc[i][j] register r holds
//   n = n0 + wn*TN + i*32 + (r/4)*8 + lk*4 + r%4,  m = m0 + wm*TM + j*32 + lr,
// so each lane owns 4 consecutive n of one row m: one 8-byte bf16 store (or a
// 16-byte int32 store) per group of 4 registers.
template <class T, bool OUT_I32, int JB = 0, int JE = T::FM>
__device__ __forceinline__ void store_tile(const v16i (&acc)[T::FN][T::FM], const float* __restrict__ xs,
                                           const float* __restrict__ ws, const uint16_t* __restrict__ bias,
                                           void* __restrict__ out, int M, int N, int64_t ldo, int m0, int n0, int wm,
                                           int wn, int lr, int lk) {
#pragma clang fp contract(off)  // the products and the bias add round separately
#pragma unroll
    for (int j = JB; j < JE; ++j) {
        const int m = m0 + wm * T::TM + j * 32 + lr;
        if (m >= M) continue;
        const float sx = OUT_I32 ? 0.0f : xs[m];
#pragma unroll
        for (int i = 0; i < T::FN; ++i) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + wn * T::TN + i * 32 + g * 8 + lk * 4;
                if (n >= N) continue;
                if constexpr (OUT_I32) {
                    int32_t* o = static_cast<int32_t*>(out) + static_cast<int64_t>(m) * ldo + n;
                    *reinterpret_cast<v4i*>(o) =
                        v4i{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                } else {
                    const float4 sw = *reinterpret_cast<const float4*>(ws + n);
                    float v0 = (static_cast<float>(acc[i][j][4 * g + 0]) * sx) * sw.x;
                    float v1 = (static_cast<float>(acc[i][j][4 * g + 1]) * sx) * sw.y;
                    float v2 = (static_cast<float>(acc[i][j][4 * g + 2]) * sx) * sw.z;
                    float v3 = (static_cast<float>(acc[i][j][4 * g + 3]) * sx) * sw.w;
                    if (bias) {
                        const uint2 b = *reinterpret_cast<const uint2*>(bias + n);
                        v0 = v0 + bf16_lo(b.x);
                        v1 = v1 + bf16_hi(b.x);
                        v2 = v2 + bf16_lo(b.y);
                        v3 = v3 + bf16_hi(b.y);
                    }
                    uint16_t* o = static_cast<uint16_t*>(out) + static_cast<int64_t>(m) * ldo + n;
                    *reinterpret_cast<uint2*>(o) = make_uint2(bf16x2_bits(v0, v1), bf16x2_bits(v2, v3));
                }
            }
        }
    }
}

// ------------------------------------------------------------------ direct-to-LDS pipeline
//
// The main kernel.  Operand tiles go from global memory straight into LDS with
// buffer_load_dwordx4 ... lds (no staging registers): one wave-wide load fills
// 1 KiB of LDS, lane l writing bytes [16l, 16l+16), so each lane fetches the
// global chunk that the XOR swizzle places at its slot.  An S-stage ring of
// K tiles keeps S-1..S tiles in flight; explicit vmcnt waits (loads complete
// in order) and a bare s_barrier replace __syncthreads, whose release fence
// would drain every prefetch.  The barrier for tile kt+1 sits before the last
// k-step of tile kt, so that step's MFMAs overlap the first fragment reads of
// the next tile; fragments are double-buffered in registers across k-steps.

// The k-step order is pinned with scheduling-group barriers (one fragment read
// for the next k-step, then one MFMA, while reads remain) instead of leaving
// the interleave to the compiler's scheduler, which moved some reads next to
// their MFMAs and waited for them there.  Measured: +2-4% on the QKV/MLP-up
// shapes, +10% on the narrow H3 fc2 shape (with GROUP_M 4).
// OCC_: waves per SIMD the register budget is sized for (at least one per 4
// waves of the workgroup; 2 lets two 4-wave workgroups share a CU).
// STAGGER_: with 8 waves, waves 4-7 (the second wave of each SIMD) issue a K
// tile's loads STAGGER_ k-steps after waves 0-3, so one wave of a SIMD is
// issuing MFMAs while the other issues its loads (0: together).
// LOADERS_: waves 0..LOADERS_-1 issue every operand load (0: all waves).  With
// 8 waves and 4 loaders, the first wave of each SIMD issues the whole K tile
// right after the barrier that frees its slot, and the second wave never
// stalls on load issue or on its own loads' arrival.
// A1_: one A fragment buffer instead of two (row i's next fragment is read
// once row i's MFMAs are issued), for wave tiles whose accumulators leave no
// room for two.
// SW_: 128-byte rows swizzled by row bits 1-3 (swz ROW_BITS_123).
// SPLITK_: K-groups of WM x WN waves each (intra-workgroup split-K).  Group g
// multiplies K tiles g, g + SPLITK, ... of the workgroup's output tile; a ring
// slot ("super stage") holds SPLITK consecutive K tiles, one per group, and
// after the K loop the groups add their int32 partial sums through LDS (exact,
// so the bytes equal the unsplit product's).  For grids of about one tile
// per CU, where the workgroup tile must stay small but each wave's sub-tile
// should not.
template <int BM_, int BN_, int BK_, int WM_, int WN_, int STAGES_, int GROUP_M_, int OCC_ = 1, int STAGGER_ = 0,
          int LOADERS_ = 0, int A1_ = 0, int SW_ = 0, int SPLITK_ = 1>
struct DTile : Tile<BM_, BN_, BK_, WM_, WN_, GROUP_M_> {
    using Base = Tile<BM_, BN_, BK_, WM_, WN_, GROUP_M_>;
    static constexpr int SPLITK = SPLITK_;
    static constexpr int GW = Base::NW;                    // waves per K-group
    static constexpr int NW = GW * SPLITK_;                // waves per workgroup
    static constexpr int NT = NW * 64;
    static constexpr int SSTAGE = Base::STAGE * SPLITK_;   // one ring slot: SPLITK K tiles
    static constexpr int STAGES = STAGES_;
    static constexpr int WPE = NW / 4 > OCC_ ? NW / 4 : OCC_;
    static constexpr int STAGGER = STAGGER_;
    static constexpr bool A1 = A1_ != 0;
    static constexpr bool SW = SW_ != 0;
    static_assert(STAGGER_ == 0 || (NW == 8 && SPLITK_ == 1 && STAGGER_ < Base::KS), "stagger: 8 waves");
    static constexpr int LOADERS = LOADERS_ > 0 ? LOADERS_ : NW;
    static_assert(LOADERS == NW || (STAGGER_ == 0 && LOADERS >= 3), "loader waves: no stagger, waves 0-2 copy scales");
    static constexpr int RPI = 1024 / BK_;                 // tile rows per wave-wide load
    static constexpr int WQ = BN_ / RPI / LOADERS;         // W-tile loads per loading lane per K tile
    static constexpr int XQ = BM_ / RPI / LOADERS;         // X-tile loads per loading lane per K tile
    static constexpr int LPT = (WQ + XQ) * SPLITK_;        // ... per ring slot
    static_assert(BN_ % (RPI * LOADERS) == 0 && BM_ % (RPI * LOADERS) == 0, "tile rows must split over waves");
    static_assert(STAGES_ >= 2 && STAGES_ * SSTAGE <= 160 * 1024, "LDS ring exceeds 160 KiB");
    static_assert(LPT * (STAGES_ - 1) <= 63, "vmcnt range");
    static_assert(Base::KS % 2 == 0, "fragment double buffer needs an even number of k-steps");
    static_assert(SPLITK_ == 1 || (SPLITK_ == 2 && !A1_ && STAGGER_ == 0), "split-K: two groups, plain tilings");
    // Split-K hand-off: each wave of group 1 stores its accumulators (XB
    // bytes) for the wave of group 0 with the same sub-tile.
    static constexpr int XB = Base::FN * Base::FM * 16 * 256;
};

// Wait until at most `tiles` K tiles of loads are still in flight.
template <int LPT>
__device__ __forceinline__ void wait_tiles(int tiles) {
    if (tiles <= 0) wait_vm<0>();
    else if (tiles == 1) wait_vm<LPT>();
    else if (tiles == 2) wait_vm<(2 * LPT < 64 ? 2 * LPT : 0)>();
    else wait_vm<(3 * LPT < 64 ? 3 * LPT : 0)>();
}

// Calls f(std::integral_constant<int, i>{}) for i = 0..N-1, so loop indices
// that select registers stay compile-time constants.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS-staged epilogue for the bf16 output, one 32-row x 64-column slab
// (4 KiB of bf16) at a time through a private 4 KiB LDS buffer per wave.
//   * Scales: the workgroup's ws, bias and xs slices were copied into LDS
//     (`sc`: ws[BN] f32, xs[BM] f32, bias[BN] bf16, then bias[BN] widened
//     to f32 by the wave that copied it) during the last K tile, so the
//     epilogue reads them at LDS latency and adds the bias with no unpacking.
//   * Writes: a lane holds 4 consecutive n of one row per register group and
//     stores them as one ds_write_b64 into the slab's 128-byte row; the
//     8-byte unit index is XORed with key = (row >> 1) & 15, so the 32 rows a
//     half-wave writes (two rows per 64 banks) land in distinct banks.
//   * Reads: 8 lanes cover one slab row (8 x 16 bytes), undoing the XOR
//     (chunk c sits at c ^ (key >> 1), its 8-byte halves swapped when key is
//     odd), and each row leaves as 128 contiguous bytes with non-temporal
//     stores (the output is never re-read, so it should not displace
//     operand panels from L2).  In a full tile a store's address is a
//     wave-uniform 64-bit base (scalar registers) plus the lane's fixed
//     32-bit byte offset: one 64-bit add per store.
// One wave reads back only what it wrote, and LDS operations of one wave
// complete in order, so no barrier is needed between slabs.
template <class T, bool BIAS, bool FULL, int JB = 0, int JE = T::FM>
__device__ __forceinline__ void store_tile_lds_impl(const v16i (&acc)[T::FN][T::FM], const uint8_t* sc,
                                                    uint16_t* __restrict__ out, int M, int N, int64_t ldo, int m0, int n0,
                                                    int wm, int wn, int lane, uint8_t* wbuf) {
    // (acc*xs)*ws and the bias add round separately, as the reference does;
    // an fma would round once.
#pragma clang fp contract(off)
    static_assert(T::TN % 32 == 0, "staged epilogue works in 64-column slabs and one 32-column half slab");
    const float* s_ws = reinterpret_cast<const float*>(sc) + wn * T::TN;
    const float* s_xs = reinterpret_cast<const float*>(sc + T::SC_XS) + wm * T::TM;
    const float* s_b = reinterpret_cast<const float*>(sc + T::SC_B32) + wn * T::TN;
    // The lane's offsets are computed here from a lane id the compiler
    // cannot see through: hoisted out of a tile loop, they would be live
    // (or spilled) through the main loop.
    asm volatile("" : "+v"(lane));
    const int lr = lane & 31, lk = lane >> 5;
    const int wkey = (lr >> 1) & 15;
    const int rr = lane >> 3, c = lane & 7;  // read side: row (within 8) and 16-byte chunk
    const int mb = m0 + wm * T::TM, nb = n0 + wn * T::TN;
    // Full tiles: chunk c of slab row r is stored at the slab row group's
    // wave-uniform address plus this lane's fixed 32-bit byte offset.
    const uint32_t lane_off = static_cast<uint32_t>((rr * ldo + c * 8) * 2);
    float sx[T::FM];
#pragma unroll
    for (int j = JB; j < JE; ++j) sx[j] = s_xs[j * 32 + lr];
    // An odd number of 32-column blocks ends in a half slab: only its first
    // 32 columns are written and read back (chunks c < 4).  It goes first,
    // so that its accumulators are free before the full slabs.
    constexpr int SLABS = (T::TN + 32) / 64;
    constexpr bool ODD = T::FN & 1;
    static_for<SLABS>([&](auto k_c) {
        constexpr int k = decltype(k_c)::value;
        constexpr int sl = ODD ? (k == 0 ? SLABS - 1 : k - 1) : k;
        constexpr bool half = ODD && k == 0;
        // Column scales of this slab, shared by its FM row blocks: held in
        // registers, or read from LDS at each use: ws when more than 128
        // accumulators are still live, the bias also when the tile holds
        // more than 128.
        constexpr int live = ODD ? (k == 0 ? T::FN : T::FN - 1 - 2 * (k - 1)) : T::FN - 2 * k;
        constexpr bool LAZY = live * T::FM > 8;
        constexpr bool LAZY_B = LAZY || T::FN * T::FM > 8;
        float4 sw[2][4], bv[2][4];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if (LAZY || (half && ii == 1)) continue;
                const int ns = ii * 32 + g * 8 + lk * 4;
                sw[ii][g] = *reinterpret_cast<const float4*>(s_ws + sl * 64 + ns);
                if constexpr (BIAS && !LAZY_B) bv[ii][g] = *reinterpret_cast<const float4*>(s_b + sl * 64 + ns);
            }
#pragma unroll
        for (int j = JB; j < JE; ++j) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                if (half && ii == 1) continue;
                const int i = 2 * sl + ii;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int ns = ii * 32 + g * 8 + lk * 4;  // column within the slab
                    float4 w4, b2;
                    if constexpr (LAZY) w4 = *reinterpret_cast<const float4*>(s_ws + sl * 64 + ns);
                    else w4 = sw[ii][g];
                    if constexpr (BIAS && LAZY_B) b2 = *reinterpret_cast<const float4*>(s_b + sl * 64 + ns);
                    else if constexpr (BIAS) b2 = bv[ii][g];
                    float v0 = (static_cast<float>(acc[i][j][4 * g + 0]) * sx[j]) * w4.x;
                    float v1 = (static_cast<float>(acc[i][j][4 * g + 1]) * sx[j]) * w4.y;
                    float v2 = (static_cast<float>(acc[i][j][4 * g + 2]) * sx[j]) * w4.z;
                    float v3 = (static_cast<float>(acc[i][j][4 * g + 3]) * sx[j]) * w4.w;
                    if constexpr (BIAS) {
                        v0 = v0 + b2.x;
                        v1 = v1 + b2.y;
                        v2 = v2 + b2.z;
                        v3 = v3 + b2.w;
                    }
                    const int u8 = (ns >> 2) ^ wkey;
                    *reinterpret_cast<uint2*>(wbuf + lr * 128 + u8 * 8) = make_uint2(bf16x2_bits(v0, v1), bf16x2_bits(v2, v3));
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (half && c >= 4) continue;
                const int r = q * 8 + rr;
                const int key = (r >> 1) & 15;
                v4u v = *reinterpret_cast<const v4u*>(wbuf + r * 128 + ((c ^ (key >> 1)) * 16));
                if (key & 1) v = v4u{v[2], v[3], v[0], v[1]};
                if constexpr (FULL) {
                    uint16_t* row = out + static_cast<int64_t>(mb + j * 32 + q * 8) * ldo + nb + sl * 64;
                    __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(reinterpret_cast<char*>(row) + lane_off));
                    continue;
                }
                const int m = mb + j * 32 + r;
                const int n = nb + sl * 64 + c * 8;
                uint16_t* o = out + static_cast<int64_t>(m) * ldo + n;
                if (m < M && n < N) {
                    if (n + 8 <= N) {
                        __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(o));
                    } else {  // N % 4 == 0: the row ends half-way through this chunk
                        __builtin_nontemporal_store(v2u{v[0], v[1]}, reinterpret_cast<v2u*>(o));
                    }
                }
            }
        }
    });
}

template <class T, int JB = 0, int JE = T::FM>
__device__ __forceinline__ void store_tile_lds(const v16i (&acc)[T::FN][T::FM], const uint8_t* sc, bool has_bias,
                                               uint16_t* __restrict__ out, int M, int N, int64_t ldo, int m0, int n0,
                                               int wm, int wn, int lane, uint8_t* wbuf) {
    // Uniform branches around the whole epilogue, none inside it: bias or
    // not, and whether the workgroup tile lies wholly inside the output (and
    // eight output rows span under 2^31 bytes, so lane offsets fit 32 bits).
    const bool full = m0 + T::BM <= M && n0 + T::BN <= N && ldo < (int64_t{1} << 27);
    if (has_bias) {
        if (full) store_tile_lds_impl<T, true, true, JB, JE>(acc, sc, out, M, N, ldo, m0, n0, wm, wn, lane, wbuf);
        else store_tile_lds_impl<T, true, false, JB, JE>(acc, sc, out, M, N, ldo, m0, n0, wm, wn, lane, wbuf);
    } else {
        if (full) store_tile_lds_impl<T, false, true, JB, JE>(acc, sc, out, M, N, ldo, m0, n0, wm, wn, lane, wbuf);
        else store_tile_lds_impl<T, false, false, JB, JE>(acc, sc, out, M, N, ldo, m0, n0, wm, wn, lane, wbuf);
    }
}

// Copies the workgroup's scale slices into LDS at `sc` with LDS-DMA (no
// registers, so the loads cannot be sunk next to their uses): wave 0 copies
// ws[n0 .. n0+BN), wave 1 xs[m0 .. m0+BM), wave 2 bias[n0 .. n0+BNB) (the
// entries past BN are copied and never read).  Entries past N or M are out of
// the buffer range and read as zero.
template <class T>
__device__ __forceinline__ void issue_scales(const float* xs, const float* ws, const uint16_t* bias, int M, int N, int m0,
                                             int n0, int lane, int wid, uint8_t* sc) {
    static_assert(T::NW >= 3 && T::BN % 64 == 0 && T::BM % 64 == 0, "scale copy layout");
    if (wid == 0) {
        const __amdgpu_buffer_rsrc_t r = make_rsrc(ws + n0, static_cast<int64_t>(N - n0) * 4);
#pragma unroll
        for (int q = 0; q < T::BN / 64; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(sc + q * 256), 4, lane * 4, q * 256, 0, 0);
    } else if (wid == 1) {
        const __amdgpu_buffer_rsrc_t r = make_rsrc(xs + m0, static_cast<int64_t>(M - m0) * 4);
#pragma unroll
        for (int q = 0; q < T::BM / 64; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(sc + T::SC_XS + q * 256), 4, lane * 4, q * 256, 0, 0);
    } else if (wid == 2 && bias) {
        const __amdgpu_buffer_rsrc_t r = make_rsrc(bias + n0, static_cast<int64_t>(N - n0) * 2);
#pragma unroll
        for (int q = 0; q < T::BNB / 128; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(sc + T::SC_B16 + q * 256), 4, lane * 4, q * 256, 0,
                                                     0);
    }
}

// The copying wave widens the bias slice at sc + SC_B16 (bf16) into f32 at
// sc + SC_B32, once per tile, after its copy has landed.
template <class T>
__device__ __forceinline__ void widen_bias(uint8_t* sc, int lane) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(sc + T::SC_B16);
    float2* dst = reinterpret_cast<float2*>(sc + T::SC_B32);
#pragma unroll
    for (int q = 0; q < T::BNB / 128; ++q) {
        const uint32_t p = src[q * 64 + lane];
        dst[q * 64 + lane] = make_float2(bf16_lo(p), bf16_hi(p));
    }
}

template <class T, bool OUT_I32>
__global__ __launch_bounds__(T::NT) __attribute__((amdgpu_waves_per_eu(T::WPE, T::WPE))) void w8a8_gemm_direct_kernel(
    const int8_t* __restrict__ X, const int8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, void* __restrict__ out, int M, int N, int K,
    int ldx, int ldw, int64_t ldo, int tiles_m, int tiles_n) {
    // The body uses device builtins inside generic lambdas, which the host
    // pass cannot instantiate; the host only needs the launch stub.
#if defined(__HIP_DEVICE_COMPILE__)
    // A workgroup computes output tiles blockIdx.x, blockIdx.x + gridDim.x,
    // ... (a grid of one workgroup per tile computes one each).
    // LDS: a two-slot operand ring, each slot one K tile (W rows, then X
    // rows), then (bf16 output, when the ring leaves room) the scale slices.
    // The epilogue works in the slot the last K tile was NOT read from: its
    // 4 KiB slab per wave at the slot's start, the scale slices at its end
    // when they have no region of their own.  Meanwhile the next tile's first
    // K tile loads into the other slot.
    // With split-K (T::SPLITK > 1) a ring slot holds one K tile per K-group;
    // every wave runs the epilogue for half of its sub-tile, so every wave
    // has a slab, and the hand-off regions (one per wave) fill the slot just
    // read (XPC regions) and, past that, the free slot behind the slabs.
    static_assert(T::STAGES == 2, "the tile loop keeps two K tiles in the ring");
    constexpr int LDS_BYTES = 2 * T::SSTAGE;
    constexpr bool STAGED = !OUT_I32;  // bf16 output through the LDS-staged epilogue
    constexpr int SC_BYTES = STAGED ? T::SC_BYTES : 0;
    constexpr bool SC_IN_RING = LDS_BYTES + SC_BYTES > 160 * 1024;
    // Split-K hand-off: every wave sends half of its row blocks (XH bytes) to
    // the wave of the other group with the same sub-tile and keeps the other
    // half, and every wave runs the epilogue for the half it keeps.
    static_assert(T::SPLITK == 1 || T::FM % 2 == 0, "split-K hand-off halves the row blocks");
    constexpr int XH = T::SPLITK > 1 ? T::XB / 2 : 1;
    constexpr int XPC = T::SPLITK > 1 ? T::SSTAGE / XH : 0;                // hand-off regions in the read slot
    constexpr int XFR = T::SPLITK > 1 && T::NW > XPC ? T::NW - XPC : 0;   // ... and in the free slot
    static_assert(T::SPLITK == 1 || XPC > 0, "split-K hand-off slot");
    static_assert(T::NW * 4096 * (STAGED ? 1 : 0) + XFR * XH + (SC_IN_RING ? SC_BYTES : 0) <= T::SSTAGE,
                  "epilogue slabs, split-K hand-off and scale slices must fit in one ring slot");
    static_assert(!SC_IN_RING || (T::SSTAGE - SC_BYTES) % 256 == 0, "scale slices must be 256-byte aligned");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES + (SC_IN_RING ? 0 : SC_BYTES)];

    const int tid = threadIdx.x;
    // wid is wave-uniform; reading it through readfirstlane lets the LDS
    // destinations of the operand loads (M0) be computed in scalar registers.
    const int lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wid / T::GW, wl = wid % T::GW;  // K-group, and the wave's sub-tile within the group
    const int wm = wl % T::WM, wn = wl / T::WM;
    const int lr = lane & 31, lk = lane >> 5;
    const int tiles = tiles_m * tiles_n;

    int t = blockIdx.x;
    int m0, n0;
    {
        int tm, tn;
        tile_coords<T::GROUP_M>(t, tiles_m, tiles_n, tm, tn);
        m0 = tm * T::BM;
        n0 = tn * T::BN;
    }
    __amdgpu_buffer_rsrc_t rx = make_rsrc(X + static_cast<int64_t>(m0) * ldx, static_cast<int64_t>(M - m0) * ldx);
    __amdgpu_buffer_rsrc_t rw = make_rsrc(W + static_cast<int64_t>(n0) * ldw, static_cast<int64_t>(N - n0) * ldw);

    // Operand loads.  Load j of a wave fills the 1 KiB LDS block wid*Q + j of
    // its operand (Q = WQ or XQ loads per wave), i.e. tile rows
    // (wid*Q + j)*RPI .. +RPI-1; each lane fetches the global chunk the XOR
    // swizzle places at its LDS slot.  The LDS destination of an LDS-DMA load
    // is M0 + instruction offset + 16*lane, and changing M0 between loads
    // roughly doubles what a wave pays to issue them, so four consecutive
    // loads share one M0 and step through their blocks with the instruction
    // offset (0..3 KiB).  That offset is also added to the global address, so
    // it is taken back out of the lane's voffset here; the buffer range check
    // sees voffset + soffset + offset, the true offset of the chunk, and rows
    // past the operand still read as zero.
    // With the row-bits-1..3 swizzle and 8-row loads, load g = wid*Q + j
    // covers tile rows 8g .. 8g+7, whose swizzle is 4*(g&1) + (lane>>4): the
    // lane's share of the offset takes one of two values, by g's parity, and
    // the rest, 8g*ld - (j&3)*1024 (>= 0, as ld >= K >= 128), is wave-uniform
    // and goes into soffset.  The range check tests voffset + soffset +
    // instruction offset as one sum (a probe on gfx950: a load whose soffset
    // alone exceeds the record count reads zero), so rows past the operand
    // still read as zero.  Two registers per operand instead of one per load:
    // the room the A1 tiling's read order needs (its main loop spilled without
    // it); the other tilings keep one register per load (in SGPRs the offsets
    // spilled there and cost 0.6-1.5%).
    constexpr bool PAR = T::A1 && T::SW && T::RPI == 8 && T::KC == 8;
    int wv[PAR ? 2 : T::WQ], xv[PAR ? 2 : T::XQ];
    const int KT = K / (T::BK * T::SPLITK);  // ring slots of K
    auto load_w = [&](uint8_t* base, auto j_c, int k0) {
        constexpr int j = decltype(j_c)::value;
        if constexpr (PAR)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(base + (wid * T::WQ + (j & ~3)) * 1024), 16,
                                                     wv[j & 1], k0 + (wid * T::WQ + j) * 8 * ldw - (j & 3) * 1024,
                                                     (j & 3) * 1024, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(base + (wid * T::WQ + (j & ~3)) * 1024), 16, wv[j],
                                                     k0, (j & 3) * 1024, 0);
    };
    auto load_x = [&](uint8_t* base, auto j_c, int k0) {
        constexpr int j = decltype(j_c)::value;
        if constexpr (PAR)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(base + T::W_BYTES + (wid * T::XQ + (j & ~3)) * 1024),
                                                     16, xv[j & 1], k0 + (wid * T::XQ + j) * 8 * ldx - (j & 3) * 1024,
                                                     (j & 3) * 1024, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(base + T::W_BYTES + (wid * T::XQ + (j & ~3)) * 1024),
                                                     16, xv[j], k0, (j & 3) * 1024, 0);
    };
    auto issue = [&](int kt, int stage) {
        static_for<T::SPLITK>([&](auto s_c) {
            constexpr int sub = decltype(s_c)::value;
            uint8_t* base = lds + stage * T::SSTAGE + sub * T::STAGE;
            const int k0 = (kt * T::SPLITK + sub) * T::BK;
            static_for<T::WQ>([&](auto j_c) { load_w(base, j_c, k0); });
            static_for<T::XQ>([&](auto j_c) { load_x(base, j_c, k0); });
        });
    };
    // Fragment f of a k-step reads tile row base + 32f.  With 64-byte rows
    // (BK = 64), or 128-byte rows swizzled by row bits 1-3 (SW), the swizzle
    // does not depend on the row bits 32f changes, so one offset per k-step
    // serves every f (fewer live registers); otherwise each fragment keeps
    // its own row.
    constexpr bool K64 = T::KC == 4 || T::SW;
    const int ra = wn * T::TN + lr, rb = wm * T::TM + lr;
    int oa[T::KS], ob[T::KS];
    // The per-lane load and fragment offsets, recomputed for every tile from
    // a lane id the compiler cannot see through, so that they are not kept
    // live across the epilogue (whose accumulators fill the registers).
    auto offsets = [&]() {
        int l = lane;
        asm volatile("" : "+v"(l));
        if constexpr (PAR) {
            // parity p of j: g = wid*Q + j has parity ((wid*Q) & 1) ^ p
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int gw = ((wid * T::WQ) & 1) ^ p, gx = ((wid * T::XQ) & 1) ^ p;
                wv[p] = (l >> 3) * ldw + ((l & 7) ^ (4 * gw + (l >> 4))) * 16;
                xv[p] = (l >> 3) * ldx + ((l & 7) ^ (4 * gx + (l >> 4))) * 16;
            }
        } else {
#pragma unroll
            for (int j = 0; j < T::WQ; ++j) {
                const int row = (wid * T::WQ + j) * T::RPI + l / T::KC;
                wv[j] = row * ldw + swz<T::KC, T::SW>(row, l % T::KC) * 16 - (j & 3) * 1024;
            }
#pragma unroll
            for (int j = 0; j < T::XQ; ++j) {
                const int row = (wid * T::XQ + j) * T::RPI + l / T::KC;
                xv[j] = row * ldx + swz<T::KC, T::SW>(row, l % T::KC) * 16 - (j & 3) * 1024;
            }
        }
        if constexpr (K64) {
            const int ra_l = wn * T::TN + (l & 31), rb_l = wm * T::TM + (l & 31), lk_l = l >> 5;
#pragma unroll
            for (int ks = 0; ks < T::KS; ++ks) {
                oa[ks] = grp * T::STAGE + ra_l * T::BK + swz<T::KC, T::SW>(ra_l, 2 * ks + lk_l) * 16;
                ob[ks] = grp * T::STAGE + T::W_BYTES + rb_l * T::BK + swz<T::KC, T::SW>(rb_l, 2 * ks + lk_l) * 16;
            }
        }
    };
    v4i a[T::A1 ? 1 : 2][T::FN], b[2][T::FM];
    auto frag_a = [&](int stage, int ks, int f) {
        if constexpr (K64)
            return *reinterpret_cast<const v4i*>(lds + stage * T::SSTAGE + oa[ks] + f * 32 * T::BK);
        const int row = ra + 32 * f;
        return *reinterpret_cast<const v4i*>(lds + stage * T::SSTAGE + grp * T::STAGE + row * T::BK +
                                             swz<T::KC>(row, 2 * ks + lk) * 16);
    };
    auto frag_b = [&](int stage, int ks, int f) {
        if constexpr (K64)
            return *reinterpret_cast<const v4i*>(lds + stage * T::SSTAGE + ob[ks] + f * 32 * T::BK);
        const int row = rb + 32 * f;
        return *reinterpret_cast<const v4i*>(lds + stage * T::SSTAGE + grp * T::STAGE + T::W_BYTES + row * T::BK +
                                             swz<T::KC>(row, 2 * ks + lk) * 16);
    };
    auto load_frags = [&](int stage, int ks, int slot) {
#pragma unroll
        for (int f = 0; f < T::FN; ++f) a[T::A1 ? 0 : slot][f] = frag_a(stage, ks, f);
#pragma unroll
        for (int f = 0; f < T::FM; ++f) b[slot][f] = frag_b(stage, ks, f);
    };
    v16i acc[T::FN][T::FM];

    // One k-step: the MFMAs of fragment slot SLOT, with the reads of the next
    // step's fragments (stage ns, step nks) into slot SLOT^1 interleaved with
    // them (NEXT), in a pinned order that issues each read as long before its
    // first use as the registers allow.  With two fragment buffers, the reads
    // go in the order the next step uses them (a0, b0 .. b[FM-1], a1 ..
    // a[FN-1]), spread evenly over the MFMA rows.  With one A buffer (A1), row
    // i's next A fragment is read once row i's MFMAs are issued, B fragment i
    // before row i; the B fragments past FN-1 replace theirs in the last row,
    // which issues the MFMAs that use them first.  Against one read pair per
    // row with the leftover reads at the end, the waits for fragments read in
    // the previous step drop from lgkmcnt(0..2) to lgkmcnt(2..7).
    auto step = [&](auto slot_c, auto next_c, int ns, int nks) {
        constexpr int SLOT = decltype(slot_c)::value;
        constexpr bool NEXT = decltype(next_c)::value;
        constexpr int AS = T::A1 ? 0 : SLOT;
        constexpr int NR = T::FN + T::FM, RB = NR / T::FN, RX = NR % T::FN;  // reads per step, per row, extra rows
        auto rd = [&](auto r_c) {
            constexpr int r = decltype(r_c)::value;
            if constexpr (r == 0) a[SLOT ^ 1][0] = frag_a(ns, nks, 0);
            else if constexpr (r <= T::FM) b[SLOT ^ 1][r - 1] = frag_b(ns, nks, r - 1);
            else a[SLOT ^ 1][r - T::FM] = frag_a(ns, nks, r - T::FM);
        };
        static_for<T::FN>([&](auto i_c) {
            constexpr int i = decltype(i_c)::value;
            if constexpr (NEXT && !T::A1) {
                constexpr int cnt = RB + (i < RX ? 1 : 0), start = i * RB + (i < RX ? i : RX);
                static_for<cnt>([&](auto q_c) { rd(std::integral_constant<int, start + decltype(q_c)::value>{}); });
            }
            if constexpr (NEXT && T::A1 && i < T::FM) b[SLOT ^ 1][i] = frag_b(ns, nks, i);
            static_for<T::FM>([&](auto j_c) {
                constexpr int j0 = decltype(j_c)::value;
                constexpr int j = (T::A1 && i == T::FN - 1) ? (j0 + T::FN) % T::FM : j0;
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[AS][i], b[SLOT][j], acc[i][j], 0, 0, 0);
                if constexpr (NEXT && T::A1 && i == T::FN - 1 && j0 + 1 == T::FM - T::FN)
                    static_for<T::FM - T::FN>([&](auto f_c) {
                        constexpr int f = T::FN + decltype(f_c)::value;
                        b[SLOT ^ 1][f] = frag_b(ns, nks, f);
                    });
            });
            // single A buffer: row i's next fragment replaces its current one
            // once the row's MFMAs have been issued
            if constexpr (NEXT && T::A1) a[0][i] = frag_a(ns, nks, i);
        });
        // the pinned order: per MFMA row, its fragment reads for the next
        // k-step and its MFMAs, one of each in turn
        static_for<T::FN>([&](auto i_c) {
            constexpr int i = decltype(i_c)::value;
            if constexpr (T::A1) {
                if constexpr (NEXT && i < T::FM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // B read
                static_for<T::FM>([&](auto j_c) {
                    constexpr int j0 = decltype(j_c)::value;
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if constexpr (NEXT && i == T::FN - 1 && j0 + 1 == T::FM - T::FN)
                        __builtin_amdgcn_sched_group_barrier(0x100, T::FM - T::FN, 0);  // extra B reads
                });
                if constexpr (NEXT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // A read
            } else {
                constexpr int cnt = RB + (i < RX ? 1 : 0);
                static_for<T::FM>([&](auto j_c) {
                    constexpr int j = decltype(j_c)::value;
                    if constexpr (NEXT && j < cnt) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                               // MFMA
                });
                if constexpr (NEXT && cnt > T::FM) __builtin_amdgcn_sched_group_barrier(0x100, cnt - T::FM, 0);
            }
        });
    };
    using yes = std::true_type;
    using no = std::false_type;

    const bool loader = wid < T::LOADERS;  // wave-uniform
    // STAGGER: the second wave of each SIMD (wid >= 4, uniform per wave)
    // issues the loads of K tile kt+2 STAGGER k-steps into tile kt+1 instead
    // of right after the barrier that freed their slot; its loads in flight
    // at every wait are the same tiles as the first wave's.
    const bool late = T::STAGGER > 0 && wid >= 4;
    // The first tile's first two K tiles; a later tile's were issued around
    // the previous tile's epilogue.
    offsets();
    if (loader) {
        issue(0, 0);
        if (KT > 1) issue(1, 1);
    }
    int base = 0;  // ring slot of the current tile's K tile 0
    for (;;) {
        // This wave's loads of K tile 0 have landed (with two K tiles in
        // flight, vmcnt <= LPT; the previous epilogue's stores, issued between
        // them, complete too, whatever their order against the loads).
        wait_tiles<T::LPT>(min(1, KT - 1));
        wg_barrier();  // every wave's share of K tile 0 is in LDS
#pragma unroll
        for (int i = 0; i < T::FN; ++i)
#pragma unroll
            for (int j = 0; j < T::FM; ++j) acc[i][j] = v16i{};
        load_frags(base, 0, 0);
        // All K tiles but the last: every step has a successor.
        for (int kt = 0; kt + 1 < KT; ++kt) {
            const int cur = (kt + base) & 1;
            static_for<T::KS>([&](auto ks_c) {
                constexpr int ks = decltype(ks_c)::value;
                constexpr int slot = ks & 1;
                if constexpr (T::STAGGER > 0 && ks == T::STAGGER - 1) {
                    if (late && kt > 0 && kt + 1 < KT) issue(kt + 1, cur ^ 1);
                }
                if constexpr (ks + 1 < T::KS) {
                    step(std::integral_constant<int, slot>{}, yes{}, cur, ks + 1);
                } else {
                    wait_lgkm0();  // this wave's reads of slot `cur` have landed
                    wait_vm<0>();  // and its share of K tile kt+1
                    wg_barrier();  // every wave is done with `cur`; K tile kt+1 is in LDS
                    if (loader && !late && kt + 2 < KT) issue(kt + 2, cur);
                    step(std::integral_constant<int, slot>{}, yes{}, cur ^ 1, 0);
                }
            });
        }
        // Last K tile, in slot `cur`; slot `fr` is free (it held K tile
        // KT-2, or nothing).  Every ring wait is behind us, so the scale copy
        // can join the loads in flight without disturbing the vmcnt counts.
        const int cur = (KT - 1 + base) & 1, fr = cur ^ 1;
        uint8_t* const sc = SC_IN_RING ? lds + fr * T::SSTAGE + T::SSTAGE - SC_BYTES : lds + LDS_BYTES;
        if constexpr (STAGED) issue_scales<T>(xs, ws, bias, M, N, m0, n0, lane, wid, sc);
        static_for<T::KS>([&](auto ks_c) {
            constexpr int ks = decltype(ks_c)::value;
            constexpr int slot = ks & 1;
            if constexpr (ks + 1 < T::KS) step(std::integral_constant<int, slot>{}, yes{}, cur, ks + 1);
            else step(std::integral_constant<int, slot>{}, no{}, 0, 0);
        });
        const int tnext = t + static_cast<int>(gridDim.x);
        // uniform; a split-K workgroup computes one tile (the host launches one
        // workgroup per tile): its hand-off uses the slot the next tile's first
        // K tile would load into
        const bool more = T::SPLITK == 1 && tnext < tiles;
        if (STAGED || more || T::SPLITK > 1) {
            if constexpr (STAGED) {
                wait_vm<0>();  // this wave's scale copy has landed
                if (wid == 2 && bias) {
                    widen_bias<T>(sc, lane);
                    wait_lgkm0();  // the widened bias is in LDS before the barrier
                }
            }
            wg_barrier();  // every wave is done reading the ring; the scales are in LDS
        }
        int m0n = 0, n0n = 0;
        if (more) {
            int tm, tn;
            tile_coords<T::GROUP_M>(tnext, tiles_m, tiles_n, tm, tn);
            m0n = tm * T::BM;
            n0n = tn * T::BN;
            rx = make_rsrc(X + static_cast<int64_t>(m0n) * ldx, static_cast<int64_t>(M - m0n) * ldx);
            rw = make_rsrc(W + static_cast<int64_t>(n0n) * ldw, static_cast<int64_t>(N - n0n) * ldw);
            if (loader) issue(0, cur);
        }
        if constexpr (T::SPLITK > 1) {
            // The two groups' waves with the same sub-tile (same lane layout)
            // swap halves of their partial sums: group 0 keeps row blocks
            // [0, FM/2) and sends [FM/2, FM), group 1 the reverse, one 16-byte
            // row of 64 lanes per register quad into the sender's region; every
            // wave is past its last ring read (barrier above).  Each wave then
            // adds what it received and runs the epilogue for its half, so all
            // eight waves share the epilogue.
            constexpr int FMH = T::FM / 2;
            auto region = [&](int r) {
                return r < XPC ? lds + cur * T::SSTAGE + r * XH
                               : lds + fr * T::SSTAGE + (STAGED ? T::NW * 4096 : 0) + (r - XPC) * XH;
            };
            auto swap_halves = [&](auto g_c) {
                constexpr int G = decltype(g_c)::value;
                constexpr int SB = G == 0 ? FMH : 0, KB = G == 0 ? 0 : FMH;  // sent and kept row blocks
                uint8_t* const mine = region(G * T::GW + wl);
                const uint8_t* const theirs = region((1 - G) * T::GW + wl);
#pragma unroll
                for (int i = 0; i < T::FN; ++i)
#pragma unroll
                    for (int jj = 0; jj < FMH; ++jj)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            *reinterpret_cast<v4i*>(mine + ((i * FMH + jj) * 4 + q) * 1024 + lane * 16) =
                                v4i{acc[i][SB + jj][4 * q], acc[i][SB + jj][4 * q + 1], acc[i][SB + jj][4 * q + 2],
                                    acc[i][SB + jj][4 * q + 3]};
                wait_lgkm0();
                wg_barrier();  // both groups' halves are in LDS
#pragma unroll
                for (int i = 0; i < T::FN; ++i)
#pragma unroll
                    for (int jj = 0; jj < FMH; ++jj)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const v4i p =
                                *reinterpret_cast<const v4i*>(theirs + ((i * FMH + jj) * 4 + q) * 1024 + lane * 16);
#pragma unroll
                            for (int r = 0; r < 4; ++r) acc[i][KB + jj][4 * q + r] += p[r];
                        }
                if constexpr (STAGED) {
                    store_tile_lds<T, KB, KB + FMH>(acc, sc, bias != nullptr, static_cast<uint16_t*>(out), M, N, ldo,
                                                     m0, n0, wm, wn, lane, lds + fr * T::SSTAGE + wid * 4096);
                } else {
                    store_tile<T, OUT_I32, KB, KB + FMH>(acc, xs, ws, bias, out, M, N, ldo, m0, n0, wm, wn, lr, lk);
                }
            };
            if (grp == 0) swap_halves(std::integral_constant<int, 0>{});
            else swap_halves(std::integral_constant<int, 1>{});
        } else if constexpr (STAGED) {
            store_tile_lds<T>(acc, sc, bias != nullptr, static_cast<uint16_t*>(out), M, N, ldo, m0, n0, wm, wn, lane,
                              lds + fr * T::SSTAGE + wl * 4096);
        } else {
            store_tile<T, OUT_I32>(acc, xs, ws, bias, out, M, N, ldo, m0, n0, wm, wn, lr, lk);
        }
        if (!more) break;
        if constexpr (STAGED) {
            wait_lgkm0();  // this wave's slab and scale reads have landed
            wg_barrier();  // every wave is done with slot `fr`
        }
        offsets();
        if (loader && KT > 1) issue(1, fr);
        base = cur;
        t = tnext;
        m0 = m0n;
        n0 = n0n;
    }
#endif
}

// ------------------------------------------------------------------ configurations

// 8 waves, two per SIMD: 128x64 (w8m) or 64x128 (w8n) per wave.  While one
// wave of a SIMD issues its operand loads or waits at a barrier, the other's
// MFMAs run; the accumulators (128 per wave) fit the VGPRs of two waves.
using D256w8a = DTile<256, 256, 128, 2, 4, 2, 4>;
using D256w8b = DTile<256, 256, 128, 4, 2, 2, 4>;
using D256w8g8 = DTile<256, 256, 128, 2, 4, 2, 8>;
// ... with the second wave of each SIMD issuing its loads one k-step later (the default)
using D256w8st1 = DTile<256, 256, 128, 2, 4, 2, 4, 1, 1>;
// ... with waves 0-3 issuing every load (two 8 KiB bursts per wave per K tile)
using D256w8l4 = DTile<256, 256, 128, 2, 4, 2, 4, 1, 0, 4>;
// 128x128 tiles, 4 waves of 64x64, registers sized for two workgroups per CU
// (2 waves per SIMD; 66.8 KB of LDS each): the configuration for small grids
using D128o2 = DTile<128, 128, 128, 2, 2, 2, 4, 2>;
// 256x256 tiles as D256w8st1, with fragment offsets shared by every
// fragment of a k-step (swizzle by row bits 1-3): the default for big grids
// whose N does not split into 384-column tiles as well
using D256sw = DTile<256, 256, 128, 2, 4, 2, 4, 1, 1, 0, 0, 1>;
// 256x384 tiles, 8 waves of 128x96 (192 accumulators per wave, so one A
// fragment buffer): 7 KiB of fragment reads per 12 MFMAs instead of 6 KiB per
// 8, and 20 KiB of operand tile per K step of 32 for 96 MFMAs instead of 16 KiB
// for 64, so 21% less LDS traffic per MFMA.  The ring fills the 160 KiB LDS;
// the scale slices share the free ring slot with the epilogue slabs.  Waves
// 0-3 issue every operand load right after the K-tile barrier (loader waves):
// the MFMA pipe favours them, so they reach the barrier first, and the loads'
// issue time evens that out (0.1-0.7% faster than each wave issuing its share,
// the second wave of each SIMD one k-step late).
using D384 = DTile<256, 384, 128, 2, 4, 2, 8, 1, 0, 4, 1, 1>;
// ... in groups of 4 m-tiles: for operands (X and W together) past the 256 MB
// infinity cache (pick_config)
using D384g4 = DTile<256, 384, 128, 2, 4, 2, 4, 1, 0, 4, 1, 1>;
// 320x256 tiles, 8 waves of 160x64: for N that 384-column tiles do not split
// well and M whose 320-row tiles fill the last round of tiles better (the H3
// out / fc2 layers, N = 5376: 19200 rows make 6.15 rounds of 256x256 tiles but
// 4.92 of 320x256)
using D320 = DTile<320, 256, 128, 2, 4, 2, 4, 1, 1, 0, 0, 1>;
// 256x320 tiles, 8 waves of 64x160 (4x2 waves; 10 blocks, 160 accumulators):
// 7 KiB of fragment reads per 10 MFMAs and 72 KiB of operand tile per K step
// of 32 for 80 MFMAs, 7.5% less LDS traffic per MFMA than 256x256, for shapes
// whose 320-column tiles fill whole rounds (N = 15360 at M = 4096: 768 tiles,
// 3 rounds, against 3.75 rounds of 256x256); loader waves as D384, 0.4-1.3%
// faster than the staggered issue (on 320x256 and 256x256 they were not);
// groups of 4 m-tiles, 0.9-1.3% faster than 8 at N = 5120, K = 13824
using D320n = DTile<256, 320, 128, 4, 2, 2, 4, 1, 0, 4, 0, 1>;
// 128x192 tiles, two K-groups of 2x2 waves of 64x96 (split-K inside the
// workgroup, 96 accumulators per wave): for grids of about one tile per CU.
// C0's 2048 x 3072 output is exactly 256 such tiles.  Per k-step a wave reads
// 5 KiB of fragments for 6 MFMAs (a 4-wave 128x192 workgroup's waves would
// hold 32x96 and read 4 KiB for 3), and the ring holds two slots of two
// 40 KiB K tiles; the hand-off is 96 KiB of LDS once per tile.  K % 256 == 0.
using D192k2 = DTile<128, 192, 128, 2, 2, 2, 8, 1, 0, 0, 0, 1, 2>;

typedef void (*kernel_fn)(const int8_t*, const int8_t*, const float*, const float*, const uint16_t*, void*, int, int,
                          int, int, int, int64_t, int, int);

struct Config {
    const char* name;
    int bm, bn, kmul, threads;  // kmul: K must be a multiple of it (BK, times the K-groups)
    kernel_fn bf16_kernel;
    kernel_fn i32_kernel;
    bool resident;  // grid of resident workgroups looping over the tiles (else one workgroup per tile)
};

#define H3MI_DCFG(NAME, T)                                                                                      \
    {NAME, T::BM, T::BN, T::BK * T::SPLITK, T::NT, w8a8_gemm_direct_kernel<T, false>,                         \
     w8a8_gemm_direct_kernel<T, true>, false}
// Resident grids: one tile per workgroup at a time, so no split-K tiling.
#define H3MI_RCFG(NAME, T)                                                                                      \
    {NAME, T::BM, T::BN, T::BK + 0 * sizeof(char[T::SPLITK == 1 ? 1 : -1]), T::NT,                             \
     w8a8_gemm_direct_kernel<T, false>, w8a8_gemm_direct_kernel<T, true>, true}

const Config kConfigs[] = {
    H3MI_DCFG("d_bm256_bn256_bk128_s2_g4_w8m_st1", D256w8st1),
    H3MI_DCFG("d_bm128_bn128_bk128_s2_g4_o2", D128o2),
    H3MI_DCFG("d_bm256_bn256_bk128_s2_g4_w8m_l4", D256w8l4),
    H3MI_DCFG("d_bm256_bn256_bk128_s2_g4_w8m", D256w8a),
    H3MI_DCFG("d_bm256_bn256_bk128_s2_g8_w8m", D256w8g8),
    H3MI_DCFG("d_bm256_bn256_bk128_s2_g4_w8n", D256w8b),
    H3MI_RCFG("d_bm256_bn384_bk128_s2_g8_w8m_l4_a1_sw_res", D384),
    H3MI_RCFG("d_bm256_bn256_bk128_s2_g4_w8m_st1_sw_res", D256sw),
    H3MI_RCFG("d_bm320_bn256_bk128_s2_g4_w8m_st1_sw_res", D320),
    H3MI_RCFG("d_bm256_bn320_bk128_s2_g4_w4x2_l4_sw_res", D320n),
    H3MI_DCFG("d_bm128_bn192_bk128_s2_g8_w2x2_sw_k2", D192k2),
    H3MI_RCFG("d_bm256_bn384_bk128_s2_g4_w8m_l4_a1_sw_res", D384g4),
};
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);

std::mutex g_cfg_mu;
int g_forced = -1;  // index into kConfigs, -1 = heuristic

int config_index(const char* name) {
    for (int i = 0; i < kNumConfigs; ++i)
        if (strcmp(name, kConfigs[i].name) == 0) return i;
    return -1;
}

// Workgroups of `fn` one CU holds at once (registers, LDS, waves), cached per kernel.
int resident_per_cu(kernel_fn fn, int threads) {
    static std::mutex mu;
    static std::vector<std::pair<kernel_fn, int>> cache;
    std::lock_guard<std::mutex> lk(mu);
    for (const auto& e : cache)
        if (e.first == fn) return e.second;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(fn), threads, 0) != hipSuccess ||
        n <= 0)
        n = 1;
    cache.emplace_back(fn, n);
    return n;
}

// Big grids (at least two 256x256 tiles per CU) run one resident workgroup
// per CU over the tiles.  Of the 256x256, 256x384, 320x256 and 256x320
// tilings, the one whose busiest workgroup has the least work runs: its tile
// count rounded up to whole rounds over the CUs, times the tile area, with the
// 256x384 and 256x320 tiles' measured 3% and 2.4% higher rates per area.  Smaller grids run 128x128 tiles (two
// workgroups per CU) or one 256x256 tile per workgroup, by the model below.
int pick_config(int64_t M, int64_t N, int64_t K) {
    {
        // a forced configuration that cannot take this K (split-K tilings
        // need K % 256 == 0) leaves the call to the heuristic
        std::lock_guard<std::mutex> lk(g_cfg_mu);
        if (g_forced >= 0 && K % kConfigs[g_forced].kmul == 0) return g_forced;
    }
    static const int wide = config_index("d_bm256_bn384_bk128_s2_g8_w8m_l4_a1_sw_res");
    static const int wide4 = config_index("d_bm256_bn384_bk128_s2_g4_w8m_l4_a1_sw_res");
    static const int big = config_index("d_bm256_bn256_bk128_s2_g4_w8m_st1_sw_res");
    static const int tall = config_index("d_bm320_bn256_bk128_s2_g4_w8m_st1_sw_res");
    static const int flat = config_index("d_bm256_bn320_bk128_s2_g4_w4x2_l4_sw_res");
    static const int small = config_index("d_bm128_bn128_bk128_s2_g4_o2");
    static const int split = config_index("d_bm128_bn192_bk128_s2_g8_w2x2_sw_k2");
    const int64_t cus = cu_count();
    auto rounds = [&](int64_t bm, int64_t bn) {
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        return static_cast<double>((tiles + cus - 1) / cus);
    };
    // 256x320 tiles get through 2.4% more work per second than 256x256 ones
    // when N splits into whole 320-column tiles (same-process A/B at equal
    // work per CU: N = 15360 and 5120); with a ragged last column (N = 5376)
    // they measured 3-4% slower than 320x256, so they are offered only then.
    const bool n320 = N % 320 == 0;
    const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
    if (t256 < 2 * cus) {
        // Fewer than two 256x256 tiles per CU: 128x128 tiles (two workgroups
        // per CU), 256x256 or 256x320 ones, whichever leaves the busiest CU
        // the least work.  Measured per CU, the 8-wave 256x256 tile gets
        // through 1.4-1.7x the int8 ops per second of the 128x128 one (which
        // runs at the same rate per CU with one or two workgroups), so 256x256
        // wins once a CU would hold three or more 128x128 tiles against one
        // 256x256 (M=2048, N=5120 or M=4096, N=3072: 13-18% faster), and
        // 128x128 wins at two (M=2048, N=3072: 22% faster).  M=4096, N=5120:
        // 256 tiles of 256x320 (one per CU) against 320 of 256x256, 21%
        // faster than 128x128.
        // The split-K 128x192 tiling (K % 256 == 0) gets through 0.88 times
        // the 128x128 one's work per CU, but at C0 (2048 x 3072) one such tile
        // per CU replaces two 128x128 ones: 24.2 against 27.5 us; the block's
        // cross-attention KV projection (512 x 10240, K = 5120): 34.4 against
        // 37.2 us.  With more tiles than CUs, or half of them idle, 128x128
        // wins (M = 1536, N = K = 4096: 31.5 against 48.2 us).
        const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
        const double c128 = static_cast<double>((t128 + cus - 1) / cus) * 128.0 * 128.0;
        const double c256 = static_cast<double>((t256 + cus - 1) / cus) * 256.0 * 256.0 / 1.5;
        const double c320 = n320 ? rounds(256, 320) * 256.0 * 320.0 / (1.5 * 1.024) : 1e300;
        const double ck2 = K % 256 == 0 ? rounds(128, 192) * 128.0 * 192.0 / 0.88 : 1e300;
        if (c320 < c256 && c320 < c128 && c320 < ck2) return flat;
        if (ck2 < c256 && ck2 < c128) return split;
        return c256 < c128 ? big : small;
    }
    const double w256 = rounds(256, 256) * 256.0 * 256.0;
    const double w384 = rounds(256, 384) * 256.0 * 384.0 / 1.03;
    const double w320 = rounds(320, 256) * 320.0 * 256.0;
    const double w320n = n320 ? rounds(256, 320) * 256.0 * 320.0 / 1.024 : 1e300;
    if (w320n < w256 && w320n < w384 && w320n < w320) return flat;
    if (w384 < w256 && w384 <= w320) {
        // Operands past ~240 MiB (the 256 MB infinity cache, less what else
        // it holds) run 256x384 tiles in groups of 4 m-tiles: same-process
        // A/B, 2.5-3.1% faster at N = 28672 (19200 x 5376 and 32768 x 5120
        // rows), 1.8% at N = 43008; below it groups of 8, 0.5-0.9% faster at
        // QKV (247 MB), N = 24576 and N = 18432 with 19200 x 5376 rows.
        const double operands = static_cast<double>(M + N) * static_cast<double>(K);
        return operands > 240.0 * 1024 * 1024 ? wide4 : wide;
    }
    return w320 < w256 ? tall : big;
}

template <bool OUT_I32>
int gemm_entry(const int8_t* xq, const int8_t* w, const float* xs, const float* ws, const uint16_t* bias, void* out,
               int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldo, void* stream) {
    const char* name = OUT_I32 ? "w8a8_gemm_i32" : "w8a8_gemm_bf16";
    if (M < 0 || N < 0 || K <= 0) return fail(H3MI_EINVAL, "%s: bad sizes M=%lld N=%lld K=%lld", name, (long long)M, (long long)N, (long long)K);
    if (K % 128) return fail(H3MI_EINVAL, "%s: K=%lld must be a multiple of 128", name, (long long)K);
    if (N % 4) return fail(H3MI_EINVAL, "%s: N=%lld must be a multiple of 4", name, (long long)N);
    if (ldx < K || ldw < K || ldo < N) return fail(H3MI_EINVAL, "%s: leading dimension smaller than the row", name);
    if (ldx % 16 || ldw % 16) return fail(H3MI_EALIGN, "%s: ldx and ldw must be multiples of 16", name);
    if (ldo % 4) return fail(H3MI_EALIGN, "%s: ldo must be a multiple of 4", name);
    // The kernels form a tile row's offset as row * ld in 32 bits, rows up to
    // 383 (384-row tiles) plus a K offset below ld: ld * 512 must fit.
    if (ldx * 512 > 0x7FFFFFFFLL || ldw * 512 > 0x7FFFFFFFLL) return fail(H3MI_EINVAL, "%s: leading dimension too large", name);
    if (M > (1LL << 30) || N > (1LL << 30)) return fail(H3MI_EINVAL, "%s: M or N too large", name);
    if (M == 0 || N == 0) return ok();
    if (!xq || !w || !out || (!OUT_I32 && (!xs || !ws))) return fail(H3MI_EINVAL, "%s: null pointer", name);
    if (!aligned(xq, 16) || !aligned(w, 16)) return fail(H3MI_EALIGN, "%s: xq and w must be 16-byte aligned", name);
    if (!aligned(out, OUT_I32 ? 16 : 8)) return fail(H3MI_EALIGN, "%s: out misaligned", name);
    if (!OUT_I32 && (!aligned(ws, 16) || (bias && !aligned(bias, 8)))) return fail(H3MI_EALIGN, "%s: ws must be 16-byte and bias 8-byte aligned", name);
    const size_t ob = static_cast<size_t>(M) * ldo * (OUT_I32 ? 4 : 2);
    if (overlap(out, ob, xq, static_cast<size_t>(M) * ldx) || overlap(out, ob, w, static_cast<size_t>(N) * ldw))
        return fail(H3MI_EALIAS, "%s: out overlaps an input", name);
    const Config& c = kConfigs[pick_config(M, N, K)];
    const int tiles_m = static_cast<int>((M + c.bm - 1) / c.bm), tiles_n = static_cast<int>((N + c.bn - 1) / c.bn);
    const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
    if (tiles > 0x7FFFFFFF) return fail(H3MI_EINVAL, "%s: too many tiles", name);
    const kernel_fn fn = OUT_I32 ? c.i32_kernel : c.bf16_kernel;
    int64_t grid = tiles;
    if (c.resident) {
        const int64_t cap = static_cast<int64_t>(cu_count()) * resident_per_cu(fn, c.threads);
        if (cap < grid) grid = cap;
    }
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(c.threads), 0,
                       as_stream(stream), xq, w, xs, ws, OUT_I32 ? nullptr : bias, out, (int)M, (int)N, (int)K,
                       (int)ldx, (int)ldw, ldo, tiles_m, tiles_n);
    return check_launch(name);
}

// One wave of LDS-DMA loads in the GEMM's operand-load form (per-lane
// voffset, wave-uniform soffset, instruction offset IOFF), for pinning what
// the buffer range check covers: LDS is first filled with 0xAB, lane l loads
// 16 bytes at voff[l] + soffset + IOFF into lds + IOFF + 16 l (the
// instruction offset moves the LDS destination too), and out[16 l ..] gets
// those 16 LDS bytes.
template <int IOFF>
__global__ __launch_bounds__(64) void lds_load_probe_kernel(const uint8_t* __restrict__ buf, int records,
                                                            const int32_t* __restrict__ voff, int soffset,
                                                            uint8_t* __restrict__ out) {
#if defined(__HIP_DEVICE_COMPILE__)
    __shared__ __attribute__((aligned(1024))) uint8_t lds[4096];
    const int l = threadIdx.x;
    for (int i = l; i < 1024; i += 64) reinterpret_cast<uint32_t*>(lds)[i] = 0xABABABABu;
    const int v = voff[l];
    wait_lgkm0();
    wg_barrier();
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(buf), static_cast<short>(0), records, kBufDword3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, v, soffset, IOFF, 0);
    wait_vm<0>();
    wg_barrier();
    *reinterpret_cast<v4u*>(out + 16 * l) = *reinterpret_cast<const v4u*>(lds + IOFF + 16 * l);
#endif
}

}  // namespace
}  // namespace h3mi

using namespace h3mi;

extern "C" int h3mi_debug_buffer_lds_load(const uint8_t* buf, int64_t records, const int32_t* voff, int32_t soffset,
                                          int32_t ioffset, uint8_t* out, void* stream) {
    if (!buf || !voff || !out) return fail(H3MI_EINVAL, "debug_buffer_lds_load: null pointer");
    if (records < 0 || records > 0x7FFFFFFF || soffset < 0)
        return fail(H3MI_EINVAL, "debug_buffer_lds_load: records in [0, 2^31) and soffset >= 0");
    if (!aligned(out, 16)) return fail(H3MI_EALIGN, "debug_buffer_lds_load: out must be 16-byte aligned");
    typedef void (*probe_fn)(const uint8_t*, int, const int32_t*, int, uint8_t*);
    probe_fn fn = ioffset == 0      ? lds_load_probe_kernel<0>
                  : ioffset == 1024 ? lds_load_probe_kernel<1024>
                  : ioffset == 2048 ? lds_load_probe_kernel<2048>
                  : ioffset == 3072 ? lds_load_probe_kernel<3072>
                                    : nullptr;
    if (!fn) return fail(H3MI_EINVAL, "debug_buffer_lds_load: ioffset %d (0, 1024, 2048 or 3072)", ioffset);
    hipLaunchKernelGGL(fn, dim3(1), dim3(64), 0, as_stream(stream), buf, static_cast<int>(records), voff, soffset, out);
    return check_launch("debug_buffer_lds_load");
}

extern "C" int h3mi_w8a8_supported(int64_t K) { return K > 0 && K % 128 == 0; }

extern "C" int h3mi_w8a8_gemm_bf16(const int8_t* xq, const int8_t* w, const float* xs, const float* ws,
                                   const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, int64_t ldx,
                                   int64_t ldw, int64_t ldo, void* stream) {
    return gemm_entry<false>(xq, w, xs, ws, bias, out, M, N, K, ldx, ldw, ldo, stream);
}

extern "C" int h3mi_w8a8_gemm_i32(const int8_t* xq, const int8_t* w, int32_t* acc, int64_t M, int64_t N, int64_t K,
                                  int64_t ldx, int64_t ldw, int64_t ldc, void* stream) {
    return gemm_entry<true>(xq, w, nullptr, nullptr, nullptr, acc, M, N, K, ldx, ldw, ldc, stream);
}

extern "C" int h3mi_w8a8_config(int64_t M, int64_t N, int64_t K, char* buf, int64_t buflen) {
    if (!buf || buflen <= 0) return fail(H3MI_EINVAL, "w8a8_config: no buffer");
    const char* nm = kConfigs[pick_config(M, N, K)].name;
    strncpy(buf, nm, static_cast<size_t>(buflen - 1));
    buf[buflen - 1] = '\0';
    return ok();
}

extern "C" int h3mi_w8a8_config_name(int index, char* buf, int64_t buflen) {
    if (!buf || buflen <= 0) return fail(H3MI_EINVAL, "w8a8_config_name: no buffer");
    if (index < 0 || index >= kNumConfigs) return fail(H3MI_EINVAL, "w8a8_config_name: index %d out of range", index);
    strncpy(buf, kConfigs[index].name, static_cast<size_t>(buflen - 1));
    buf[buflen - 1] = '\0';
    return ok();
}

extern "C" int h3mi_w8a8_set_config(const char* name) {
    if (!name) return fail(H3MI_EINVAL, "w8a8_set_config: null name");
    std::lock_guard<std::mutex> lk(g_cfg_mu);
    if (strcmp(name, "auto") == 0 || name[0] == '\0') {
        g_forced = -1;
        return ok();
    }
    const int i = config_index(name);
    if (i < 0) return fail(H3MI_EINVAL, "w8a8_set_config: unknown configuration '%s'", name);
    g_forced = i;
    return ok();
}
