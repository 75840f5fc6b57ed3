"""The fused norms with many adaLN table rows: 257 rows of s1 / shift / gate and
a random row per token, so that almost every row reads its table row through
the range-checked global loads rather than the workgroup's row staged in LDS,
at widths on the row-stream, hidden-5376 and widest stream paths."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits, norm_inputs

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


@pytest.mark.parametrize("N", [1024, 5120, 5376, 8192])
def test_norms_with_many_table_rows(N):
    h = _h3mi()
    S, R = 999, 257
    x, w, s1, sh, gt, o, _ = norm_inputs(S, N, R, seed=N + R, stress=True)
    ridx = torch.from_numpy(np.random.default_rng(N).integers(0, R, S).astype(np.int32))
    print(f"[tables] S={S} N={N} R={R}", flush=True)
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
    # the fused quantizing kernels against the norm followed by the quantizer
    xd, wd, rd, s1d, shd, od, gd = cu(x, w, ridx, s1, sh, o, gt)
    ref_q, ref_s = h.quantize_rowwise(h.norm_mod(xd, wd, eps, rd, s1d, shd))
    q, qs = h.norm_mod_q(xd, wd, eps, rd, s1d, shd)
    assert torch.equal(q, ref_q) and torch.equal(qs.view(torch.int32), ref_s.view(torch.int32))
    xa, xb = xd.clone(), xd.clone()
    ref_q, ref_s = h.quantize_rowwise(h.gate_norm_mod_(xa, od, gd, wd, eps, rd, s1d, shd))
    q, qs = h.gate_norm_mod_q_(xb, od, gd, wd, eps, rd, s1d, shd)
    assert torch.equal(xa, xb)
    assert torch.equal(q, ref_q) and torch.equal(qs.view(torch.int32), ref_s.view(torch.int32))
