"""Seeded random shapes through every kernel family, against the CPU oracle:
row counts, widths and table-index patterns the hand-picked cases do not
name (ragged GEMM edges on both sides, norm widths on every kernel path from
the 8-wide row stream to the one-wave-per-row kernels, mixed table rows).
Each case prints its shape before it runs."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits, norm_inputs

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


def _gemm_cases(n, seed):
    g = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(g.integers(1, 700))
        N = int(g.integers(1, 400)) * 4
        K = int(g.integers(1, 24)) * 128
        out.append((M, N, K))
    return out


@pytest.mark.parametrize("M,N,K", _gemm_cases(12, 2026))
def test_random_gemm_matches_oracle(M, N, K):
    h = _h3mi()
    g = np.random.default_rng(M * 131 + N * 7 + K)
    x = torch.from_numpy(g.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16)
    w = g.integers(-127, 128, (N, K), dtype=np.int8)
    ws = (1e-3 + 9e-3 * g.random(N)).astype(np.float32)
    bias = O.f32_to_bf16_bits((0.02 * g.standard_normal((1, N))).astype(np.float32))[0]
    print(f"[random] gemm M={M} N={N} K={K} tile={h.config_for(M, N, K)}", flush=True)
    ref, oq, os_, acc = O.w8a8_linear(bits(x), w, ws, bias)
    q, s = h.quantize_rowwise(x.cuda())
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))
    wd = torch.from_numpy(w).cuda()
    assert np.array_equal(h.int8_mm_i32(q, wd).cpu().numpy(), acc)
    bd = torch.from_numpy(bias.view(np.int16)).view(torch.bfloat16).cuda()
    out = h.int8_mm_scaled(q, wd, s.reshape(-1, 1), torch.from_numpy(ws).cuda(), bias=bd)
    assert np.array_equal(bits(out), ref)


def _norm_cases(seed):
    """One random row count and table height per width: widths on each kernel
    path (8-wide row stream, the hidden-5376 kernel, the 4-element tail, and
    past 8192 the one-workgroup-per-row kernels)."""
    g = np.random.default_rng(seed)
    widths = [8, 24, 512, 1000, 1024, 1032, 2056, 3072, 4096, 4104, 5120, 5376, 6144, 7168, 8192, 8200, 12292]
    return [(int(g.integers(1, 3000)), N, int(g.integers(1, 4))) for N in widths]


@pytest.mark.parametrize("S,N,R", _norm_cases(7))
def test_random_norms_match_oracle(S, N, R):
    h = _h3mi()
    x, w, s1, sh, gt, o, ridx = norm_inputs(S, N, R, seed=S * 3 + N + R, stress=S % 2 == 0)
    if S > 10:  # a run of rows on one table row, as a batch of one sample has
        ridx[S // 3: 2 * S // 3] = 0
    print(f"[random] norms S={S} N={N} R={R}", flush=True)
    cu = lambda *ts: [t.cuda() for t in ts]
    order = h.order_info(0)
    eps = 1e-6
    hout, var, rstd = h.norm_mod_ex(*cu(x, w), eps, ridx.cuda(), *cu(s1, sh), rsqrt_mode=1, stats=True)
    oh, ovar, orstd = O.norm_mod(bits(x), bits(w), eps, ridx.numpy(), bits(s1), bits(sh), order=order)
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), orstd.view(np.uint32))
    assert np.array_equal(bits(hout), oh)
    xd = x.cuda()
    hg, gvar, _ = h.gate_norm_mod_ex(xd, *cu(o, gt, w), eps, ridx.cuda(), *cu(s1, sh), rsqrt_mode=1, stats=True)
    ox, ogh, ogvar, _ = O.gate_norm_mod(bits(x), bits(o), bits(gt), bits(w), eps, ridx.numpy(), bits(s1), bits(sh),
                                        order=order)
    assert np.array_equal(bits(xd), ox)
    assert np.array_equal(gvar.cpu().numpy().view(np.uint32), ogvar.view(np.uint32))
    assert np.array_equal(bits(hg), ogh)
    xg = x.cuda()
    h.gate_(xg, *cu(o, gt), ridx.cuda())
    assert np.array_equal(bits(xg), O.gate(bits(x), bits(o), bits(gt), ridx.numpy()))
    if N % 8 == 0 and N <= 8192:  # the fused quantizing kernels' domain
        xd, wd, rd, s1d, shd, od, gd = cu(x, w, ridx, s1, sh, o, gt)
        ref_q, ref_s = h.quantize_rowwise(h.norm_mod(xd, wd, eps, rd, s1d, shd))
        q, qs = h.norm_mod_q(xd, wd, eps, rd, s1d, shd)
        assert torch.equal(q, ref_q) and torch.equal(qs.view(torch.int32), ref_s.view(torch.int32))
        xa, xb = xd.clone(), xd.clone()
        ref_q, ref_s = h.quantize_rowwise(h.gate_norm_mod_(xa, od, gd, wd, eps, rd, s1d, shd))
        q, qs = h.gate_norm_mod_q_(xb, od, gd, wd, eps, rd, s1d, shd)
        assert torch.equal(xa, xb)
        assert torch.equal(q, ref_q) and torch.equal(qs.view(torch.int32), ref_s.view(torch.int32))


@pytest.mark.parametrize("M,K,act", [(int(m), int(k) * 256, a) for m, k, a in
                                     zip(np.random.default_rng(5).integers(1, 900, 6),
                                         np.random.default_rng(6).integers(1, 40, 6),
                                         [None, "swiglu"] * 3)])
def test_random_convrot_matches_oracle(M, K, act):
    h = _h3mi()
    g = np.random.default_rng(M + K)
    kin = 2 * K if act else K
    x = torch.from_numpy(g.standard_normal((M, kin)).astype(np.float32)).to(torch.bfloat16)
    print(f"[random] convrot M={M} K={K} act={act}", flush=True)
    q, s = h.quantize_rowwise_convrot(x.cuda(), act)
    oq, os_ = O.convrot_quant(bits(x), act)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), oq)
