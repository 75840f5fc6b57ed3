"""Rows of finite special values through the GPU kernels, against the CPU
oracle: bf16 subnormals of both signs, signed zeros, the smallest normal and
the largest finite value (whose square overflows, so the row's variance is
infinite and its rstd 0).  The quantizer's scale of a subnormal row is far
below 2^-100, so its quotients take the IEEE divide; a row of largest finite
values has the largest scale.  The norms run with the correctly rounded rsqrt
(bit-exact to the oracle, var and rstd included); the fused norm -> quantizer
kernels are checked against the norm followed by the quantizer."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits, from_bits, norm_inputs

pytestmark = pytest.mark.gpu

SUB = np.arange(1, 0x80, dtype=np.uint16)  # positive bf16 subnormals
MAXF, MINN, NZERO = 0x7F7F, 0x0080, 0x8000


def _h3mi():
    import h3mi
    return h3mi


def _special_rows(N, seed):
    """bf16 bit rows: [0] subnormals of both signs, [1] subnormals with one
    normal, [2] -0 and +0 only, [3] the largest finite value with random
    normals, [4] +-largest finite only, [5] the smallest normal and
    subnormals, [6] random normals with a few subnormals and zeros,
    [7] one largest finite value among zeros."""
    g = np.random.default_rng(seed)
    rnd = (g.standard_normal(N).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    rows = np.empty((8, N), np.uint16)
    rows[0] = g.choice(SUB, N) | (g.integers(0, 2, N).astype(np.uint16) << 15)
    rows[1] = g.choice(SUB, N)
    rows[1, N // 3] = 0x3F80  # 1.0
    rows[2] = np.where(g.integers(0, 2, N) == 1, NZERO, 0).astype(np.uint16)
    rows[3] = rnd
    rows[3, 5] = MAXF
    rows[4] = MAXF | (g.integers(0, 2, N).astype(np.uint16) << 15)
    rows[5] = g.choice(SUB, N)
    rows[5, ::7] = MINN
    rows[6] = rnd[::-1]
    idx = g.choice(N, 16, replace=False)
    rows[6, idx[:8]] = g.choice(SUB, 8)
    rows[6, idx[8:]] = NZERO
    rows[7] = 0
    rows[7, N - 1] = MAXF | 0x8000
    return rows


@pytest.mark.parametrize("K", [512, 5120, 14336])
def test_quant_special_rows(K):
    h = _h3mi()
    xb = _special_rows(K, seed=K)
    q, s = h.quantize_rowwise(from_bits(xb).cuda())
    oq, os_ = O.quant_rowwise(xb)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), oq)


@pytest.mark.parametrize("K", [1024, 5376])
def test_convrot_special_rows(K):
    """Rows without the largest finite value (a 256-point sum of those
    overflows): subnormals, zeros, the smallest normal, random normals."""
    h = _h3mi()
    xb = _special_rows(K, seed=K + 1)[[0, 1, 2, 5, 6]]
    q, s = h.quantize_rowwise_convrot(from_bits(xb).cuda())
    oq, os_ = O.convrot_quant(xb)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), oq)


@pytest.mark.parametrize("N", [1024, 5120, 5376])
def test_norms_special_rows(N):
    h = _h3mi()
    xb = _special_rows(N, seed=N + 2)
    S = xb.shape[0]
    _, w, s1, sh, g, o, _ = norm_inputs(S, N, 2, seed=N, stress=False)
    ridx = torch.tensor([0, 1] * (S // 2), dtype=torch.int32)
    x = from_bits(xb)
    eps = 1e-6
    cu = lambda *ts: [t.cuda() for t in ts]
    order = h.order_info(0)

    hout, var, rstd = h.norm_mod_ex(*cu(x, w), eps, ridx.cuda(), *cu(s1, sh), rsqrt_mode=1, stats=True)
    oh, ovar, orstd = O.norm_mod(xb, bits(w), eps, ridx.numpy(), bits(s1), bits(sh), order=order)
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), orstd.view(np.uint32))
    assert np.array_equal(bits(hout), oh)

    xd = x.cuda()
    hg, gvar, grstd = h.gate_norm_mod_ex(xd, *cu(o, g, w), eps, ridx.cuda(), *cu(s1, sh), rsqrt_mode=1, stats=True)
    ox, ogh, ogvar, _ = O.gate_norm_mod(xb, bits(o), bits(g), bits(w), eps, ridx.numpy(), bits(s1), bits(sh),
                                        order=order)
    assert np.array_equal(bits(xd), ox)
    assert np.array_equal(gvar.cpu().numpy().view(np.uint32), ogvar.view(np.uint32))
    assert np.array_equal(bits(hg), ogh)

    # the fused quantizing variants (product rsqrt) against the norm followed by the quantizer
    xd, wd, rd, s1d, shd, od, gd = cu(x, w, ridx, s1, sh, o, g)
    ref_q, ref_s = h.quantize_rowwise(h.norm_mod(xd, wd, eps, rd, s1d, shd))
    q, qs = h.norm_mod_q(xd, wd, eps, rd, s1d, shd)
    assert torch.equal(q, ref_q) and torch.equal(qs.view(torch.int32), ref_s.view(torch.int32))
    xa, xb2 = xd.clone(), xd.clone()
    ref_q, ref_s = h.quantize_rowwise(h.gate_norm_mod_(xa, od, gd, wd, eps, rd, s1d, shd))
    q, qs = h.gate_norm_mod_q_(xb2, od, gd, wd, eps, rd, s1d, shd)
    assert torch.equal(xa, xb2)
    assert torch.equal(q, ref_q) and torch.equal(qs.view(torch.int32), ref_s.view(torch.int32))
