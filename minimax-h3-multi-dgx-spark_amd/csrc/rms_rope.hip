// q/k RMSNorm + split-half rotary embedding, in place, for gfx950.
//
// Replaces comfy-kitchen's ck.rms_rope_split_half_(q, k, rope_freqs, qw, kw,
// epsilon, rot_dim) as the reference calls it on the [1, s, heads, dim] views
// of the qkv projection (comfyui_nodes/minimax-h3-sp/minimax_sp/
// sp_forward.py:279-296; table from rope_rotation_table, :548).  comfy-kitchen's
// arithmetic is not published with the reference; this kernel implements the
// eager sequence the fused call stands for, bit for bit:
//   y = bf16(w * (rstd * x)) per (token, head) row of D elements -- F.rms_norm
//       of the row: in-thread sequential sums of squares over 4-element
//       chunks, a shuffle tree over the chunks, rstd = rsqrt(tot / D + eps);
//   for i < rot/2, R = tab[token][i] (2 x 2, bf16):
//       out[i]         = bf16(R00 y[i] + R01 y[i + rot/2])
//       out[i + rot/2] = bf16(R10 y[i] + R11 y[i + rot/2])
//     (products and sum each rounded in fp32); out[j] = y[j] for j >= rot.
//
// Layout: a row of D = 8 * LPR elements is LPR lanes x 8 contiguous elements
// (one 16-byte load and store per lane); a wave holds 64 / LPR rows at a time
// and NIT such sets; rows run (token, q heads, k heads), so a wave's rows
// mostly share one token's table.  The
// sum-of-squares order of PyTorch's rms_norm (256 logical threads, 4-element
// chunks, 64-wide shuffle-down tree, then the cross-warp tree) puts chunk t
// in thread t; only D/4 <= 64 threads hold data, so the tree reduces to: lane
// l holds chunks 2l and 2l+1, butterflies over lanes l ^ LPR/2, ..., l ^ 1 sum
// each parity class, and the total is even + odd.  Sums with the zero
// partials of the other threads are exact and are skipped.  The rotation
// partner of element i (< rot/2) sits in the same slot of lane l + rot/16.
#include <type_traits>

#include "common.h"

namespace h3mi {
namespace {

typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));

// One wave handles NIT sets of 64 / LPR rows; every load of the wave is
// issued before the first row is reduced, so a wave keeps NIT x 1 KiB of rows
// (plus their table entries) in flight.  Branches around memory operations
// make the compiler drain all loads at the join, so the bulk launch covers
// whole workgroups (GUARD = false: no row test) and a second, guarded launch
// takes the remaining rows; RSTD (the per-row rstd output) is for tests;
// ROPE: 0 no rotation (rot = 0), 2 full rotation (rot = D), 1 partial; with
// a rotation every lane loads table words (lanes outside a partial rotation
// load pair 0 and ignore it) so no branch surrounds the loads;
// RN selects the correctly rounded rsqrt (else the hardware one, as eager).
//
// VALU economy (about 20 instructions per element, so the shader clock
// shows in the kernel's time):
// each lane loads exactly the 8 table words it uses (lower lanes word 0 =
// R00 | R01 << 16 of its 8 pairs, upper lanes word 1 = R10 | R11 << 16), so no
// table words are exchanged or selected; the weights are staged once per
// workgroup in LDS as fp32, q's then k's; the cross-lane sums and the partner
// values go over the LDS crossbar.
template <int LPR, int NIT, bool GUARD, bool RSTD, int ROPE, bool RN>
__global__ __launch_bounds__(256) void rms_rope_kernel(uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                                                       const uint16_t* __restrict__ tab,
                                                       const uint16_t* __restrict__ qw,
                                                       const uint16_t* __restrict__ kw, int S, int H, int64_t ldq,
                                                       int64_t ldk, int rot, float eps, int mode,
                                                       float* __restrict__ rstd_out, int64_t row_base) {
#pragma clang fp contract(off)
    constexpr int D = LPR * 8;
    constexpr int RPW = 64 / LPR;
    static_assert(D <= 256, "one weight element per thread of the workgroup");
    __shared__ __attribute__((aligned(16))) float wsh[2 * D];
    const int lane = threadIdx.x & 63;
    const int sub = lane % LPR;
    const int64_t rows = static_cast<int64_t>(S) * 2 * H;
    const int64_t row0 =
        row_base + (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * (RPW * NIT) + lane / LPR;
    // rotation: lanes [0, rot/16) of a row hold the first halves, [rot/16,
    // rot/8) the second halves, the partner lane rot/16 away
    const int hl = rot / 16;
    const bool lower = sub < hl;
    const bool rotated = ROPE == 2 || sub < 2 * hl;
    const int src = rotated ? (lower ? lane + hl : lane - hl) : lane;
    const int pair0 = rotated ? (lower ? sub : sub - hl) * 8 : 0;
    const int word = (rotated && !lower) ? 1 : 0;
    // v_perm selectors (bytes 4-7 = first operand, 0x0c = zero): the low half
    // of a word as an fp32 is bytes {5, 4} on top, the high half bytes {7, 6}
    const uint32_t sel_lo = 0x05040C0Cu, sel_hi = 0x07060C0Cu;
    const uint32_t sel_own = lower ? sel_lo : sel_hi, sel_par = lower ? sel_hi : sel_lo;

    // the weights first (loads complete in order): thread t stages element
    // t % D of both; threads past D write the same values again
    const int wt = static_cast<int>(threadIdx.x) % D;
    const uint16_t wq1 = qw[wt], wk1 = kw[wt];

    // rows < 2^31 (checked by the caller), so 32-bit arithmetic; one division
    // for the wave's first set, then steps of RPW rows
    const uint32_t rows_per_tok = 2u * static_cast<uint32_t>(H);
    uint32_t tok = static_cast<uint32_t>(row0) / rows_per_tok;
    uint32_t jr = static_cast<uint32_t>(row0) - tok * rows_per_tok;
    int64_t row[NIT];
    bool in[NIT], isk[NIT];
    uint16_t* px[NIT];
    v4u_t xv[NIT];
    uint32_t tw[NIT][8];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        if (it > 0) {
            jr += RPW;
            while (jr >= rows_per_tok) {
                jr -= rows_per_tok;
                ++tok;
            }
        }
        row[it] = row0 + static_cast<int64_t>(it) * RPW;
        in[it] = !GUARD || row[it] < rows;
        const uint32_t t32 = in[it] ? tok : 0u;
        const int j = static_cast<int>(jr);
        isk[it] = j >= H;
        px[it] = (isk[it] ? k + static_cast<int64_t>(t32) * ldk : q + static_cast<int64_t>(t32) * ldq) +
                 static_cast<int64_t>(isk[it] ? j - H : j) * D + sub * 8;
        xv[it] = v4u_t{0u, 0u, 0u, 0u};
        if (!GUARD || in[it]) xv[it] = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(px[it]));
        if constexpr (ROPE > 0) {
            // rows past the end (GUARD) have token 0, whose table row exists;
            // pair m's words are elements 4m .. 4m+3 of the table row
            const uint32_t* pt = reinterpret_cast<const uint32_t*>(tab + (static_cast<int64_t>(t32) * (rot / 2) + pair0) * 4) + word;
#pragma unroll
            for (int i = 0; i < 8; ++i) tw[it][i] = pt[2 * i];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before any row is reduced
    wsh[wt] = bf16_f32(wq1);
    wsh[D + wt] = bf16_f32(wk1);
    wait_lgkm0();  // the writes are done
    wg_barrier();

#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = bf16_lo(xv[it][i]);
            x[2 * i + 1] = bf16_hi(xv[it][i]);
        }
        // chunks 2*sub (elements 0..3 of the lane) and 2*sub + 1 (4..7)
        float pe = x[0] * x[0], po = x[4] * x[4];
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            pe = pe + x[i] * x[i];
            po = po + x[4 + i] * x[4 + i];
        }
#pragma unroll
        for (int d = LPR / 2; d >= 1; d /= 2) {
            pe = pe + __shfl_xor(pe, d, 64);
            po = po + __shfl_xor(po, d, 64);
        }
        // D is a power of two: the product by 1/D is the IEEE quotient
        const float var = (pe + po) * (1.0f / static_cast<float>(D)) + eps;
        const float rstd = RN ? rsqrt_rn(var) : rsqrtf(var);
        if constexpr (RSTD) {
            if (in[it] && sub == 0) rstd_out[row[it]] = rstd;
        }

        const float* wr = wsh + (isk[it] ? D : 0) + sub * 8;
        const float4 w0 = *reinterpret_cast<const float4*>(wr), w1 = *reinterpret_cast<const float4*>(wr + 4);
        const float wf[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = wf[i] * (rstd * x[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) rb2(y[2 * i], y[2 * i + 1]);
        if constexpr (ROPE > 0) {
            float p[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) p[i] = __shfl(y[i], src, 64);
            if (rotated) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    // lower lane: out = R00 y + R01 p; upper lane: R10 p + R11 y,
                    // the same sum in the other order; c_own / c_par pick the
                    // halves of the lane's word by a per-lane selector
                    const float c_own = __uint_as_float(__builtin_amdgcn_perm(tw[it][i], 0u, sel_own));
                    const float c_par = __uint_as_float(__builtin_amdgcn_perm(tw[it][i], 0u, sel_par));
                    const float u = c_own * y[i];
                    const float v = c_par * p[i];
                    y[i] = u + v;
                }
            }
        }
        v4u_t ov;
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[i] = bf16x2_bits(y[2 * i], y[2 * i + 1]);
        if (!GUARD || in[it]) __builtin_nontemporal_store(ov, reinterpret_cast<v4u_t*>(px[it]));
    }
}

}  // namespace
}  // namespace h3mi

using namespace h3mi;

extern "C" int h3mi_rms_rope_split_half_bf16(uint16_t* q, uint16_t* k, const uint16_t* tab, const uint16_t* qw,
                                             const uint16_t* kw, int64_t S, int64_t H, int64_t D, int64_t ldq,
                                             int64_t ldk, int64_t rot, float eps, int rsqrt_mode_,
                                             float* rstd_out, void* stream) {
    if (S < 0 || H <= 0) return fail(H3MI_EINVAL, "rms_rope: bad sizes S=%lld H=%lld", (long long)S, (long long)H);
    if (D != 64 && D != 128 && D != 256) return fail(H3MI_EINVAL, "rms_rope: head dim %lld (64, 128 or 256)", (long long)D);
    if (rot < 0 || rot > D || rot % 16) return fail(H3MI_EINVAL, "rms_rope: rot_dim %lld must be a multiple of 16 in [0, %lld]",
                                                    (long long)rot, (long long)D);
    if (rsqrt_mode_ != H3MI_RSQRT_HW && rsqrt_mode_ != H3MI_RSQRT_RN) return fail(H3MI_EINVAL, "rms_rope: unknown rsqrt mode");
    if (ldq < H * D || ldk < H * D || ldq % 8 || ldk % 8)
        return fail(H3MI_EALIGN, "rms_rope: token strides must be >= heads*dim and multiples of 8");
    if (S * 2 * H > 0x7FFFFFFF || H > 0x3FFFFFFF) return fail(H3MI_EINVAL, "rms_rope: more than 2^31 rows");
    if (S == 0) return ok();
    if (!q || !k || !qw || !kw || (rot && !tab)) return fail(H3MI_EINVAL, "rms_rope: null pointer");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(qw, 16) || !aligned(kw, 16) || (rot && !aligned(tab, 16)) ||
        (rstd_out && !aligned(rstd_out, 4)))
        return fail(H3MI_EALIGN, "rms_rope: q, k, weights and table need 16-byte alignment");
    const size_t qb = static_cast<size_t>((S - 1) * ldq + H * D) * 2, kb = static_cast<size_t>((S - 1) * ldk + H * D) * 2;
    const size_t tb = static_cast<size_t>(S * rot / 2 * 4) * 2, wb = static_cast<size_t>(D) * 2;
    // q and k may interleave in one qkv buffer: then every token's q heads and
    // every token's k heads must be disjoint, i.e. equal strides and the k
    // offset (mod the stride) at least H*D elements from q on both sides
    if (overlap(q, qb, k, kb)) {
        const intptr_t db = reinterpret_cast<const char*>(k) - reinterpret_cast<const char*>(q);
        const int64_t hd = H * D;
        if (ldq != ldk || db % 2) return fail(H3MI_EALIAS, "rms_rope: q and k overlap");
        const int64_t dm = ((db / 2) % ldq + ldq) % ldq;
        if (dm < hd || dm > ldq - hd) return fail(H3MI_EALIAS, "rms_rope: q and k heads overlap");
    }
    if ((rot && (overlap(q, qb, tab, tb) || overlap(k, kb, tab, tb))) || overlap(q, qb, qw, wb) || overlap(q, qb, kw, wb) ||
        overlap(k, kb, qw, wb) || overlap(k, kb, kw, wb))
        return fail(H3MI_EALIAS, "rms_rope: q/k overlap the table or the weights");
    if (rstd_out) {
        const size_t rb_ = static_cast<size_t>(S * 2 * H) * 4;
        if (overlap(rstd_out, rb_, q, qb) || overlap(rstd_out, rb_, k, kb)) return fail(H3MI_EALIAS, "rms_rope: rstd_out overlaps q/k");
    }
    constexpr int NIT = 4;
    const int lpr = static_cast<int>(D / 8);
    const int64_t rows = S * 2 * H;
    const int64_t rows_per_block = 4 * (64 / lpr) * NIT;
    const int64_t full = rows / rows_per_block;  // workgroups whose rows all exist
    const int64_t tail = rows - full * rows_per_block;
    auto launch = [&](auto kern, int64_t blocks, int64_t base) {
        if (blocks <= 0) return;
        hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream), q, k, tab, qw, kw,
                           static_cast<int>(S), static_cast<int>(H), ldq, ldk, static_cast<int>(rot), eps, rsqrt_mode_,
                           rstd_out, base);
    };
    auto run3 = [&](auto lpr_c, auto rstd_c, auto rope_c, auto rn_c) {
        constexpr int L = decltype(lpr_c)::value;
        constexpr bool R = decltype(rstd_c)::value, N = decltype(rn_c)::value;
        constexpr int P = decltype(rope_c)::value;
        launch(rms_rope_kernel<L, NIT, false, R, P, N>, full, 0);
        launch(rms_rope_kernel<L, NIT, true, R, P, N>, tail ? 1 : 0, full * rows_per_block);
    };
    using T = std::true_type;
    using F = std::false_type;
    auto run2 = [&](auto lpr_c, auto rstd_c, auto rope_c) {
        if (rsqrt_mode_ == H3MI_RSQRT_RN) run3(lpr_c, rstd_c, rope_c, T{});
        else run3(lpr_c, rstd_c, rope_c, F{});
    };
    using R0 = std::integral_constant<int, 0>;
    using R1 = std::integral_constant<int, 1>;
    using R2 = std::integral_constant<int, 2>;
    auto run1 = [&](auto lpr_c, auto rstd_c) {
        if (rot == D) run2(lpr_c, rstd_c, R2{});
        else if (rot) run2(lpr_c, rstd_c, R1{});
        else run2(lpr_c, rstd_c, R0{});
    };
    auto run = [&](auto lpr_c) {
        if (rstd_out) run1(lpr_c, T{});
        else run1(lpr_c, F{});
    };
    if (lpr == 8) run(std::integral_constant<int, 8>{});
    else if (lpr == 16) run(std::integral_constant<int, 16>{});
    else run(std::integral_constant<int, 32>{});
    return check_launch("rms_rope_kernel");
}
