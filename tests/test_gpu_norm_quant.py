"""Norm -> quantizer fusion on the GPU: norm_mod_q / gate_norm_mod_q_ return
the per-token int8 quantization of h (and its scales) computed inside the
norm kernel.  Bar: bit-identical to norm_mod / gate_norm_mod_ followed by
quantize_rowwise (the two kernels pinned against the oracle elsewhere), and,
on a small case, to the oracle chain norm_mod -> quant_rowwise fed the GPU's
rstd."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits, norm_inputs

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


def _cuda(*ts):
    return [t.cuda() for t in ts]


CASES = [("uniform", 3001, 5120, 1), ("segments", 2603, 5120, 2), ("random", 700, 5376, 3), ("widest", 300, 8192, 2),
         ("small", 37, 1032, 1), ("one row", 1, 512, 1), ("past", 64, 8200, 1)]


def _inputs(kind, S, N, R, seed):
    x, w, s1, sh, g, o, ridx = norm_inputs(S, N, R, seed=seed, stress=kind != "segments")
    if kind == "segments":
        ridx[:] = 0
        ridx[: S // 9] = 1
    if kind in ("uniform", "small", "one row", "past"):
        ridx[:] = R - 1
    if S > 3:
        x[3] = 0  # an all-zero input row (its h is the shift row)
    return x, w, s1, sh, g, o, ridx


@pytest.mark.parametrize("want_h", [False, True])
@pytest.mark.parametrize("kind,S,N,R", CASES)
def test_norm_mod_q_equals_norm_then_quant(kind, S, N, R, want_h):
    h = _h3mi()
    x, w, s1, sh, _, _, ridx = _inputs(kind, S, N, R, seed=S * 7 + N)
    xd, wd, rd, s1d, shd = _cuda(x, w, ridx, s1, sh)
    ref_h = h.norm_mod(xd, wd, 1e-6, rd, s1d, shd)
    ref_q, ref_s = h.quantize_rowwise(ref_h)
    out = h.norm_mod_q(xd, wd, 1e-6, rd, s1d, shd, want_h=want_h)
    if want_h:
        assert torch.equal(out[0], ref_h)
        out = out[1:]
    assert torch.equal(out[0], ref_q)
    assert torch.equal(out[1].view(torch.int32), ref_s.view(torch.int32))


@pytest.mark.parametrize("want_h", [False, True])
@pytest.mark.parametrize("kind,S,N,R", CASES)
def test_gate_norm_mod_q_equals_gate_norm_then_quant(kind, S, N, R, want_h):
    h = _h3mi()
    x, w, s1, sh, g, o, ridx = _inputs(kind, S, N, R, seed=S * 5 + N)
    od, gd, wd, rd, s1d, shd = _cuda(o, g, w, ridx, s1, sh)
    x_ref = x.cuda()
    ref_h = h.gate_norm_mod_(x_ref, od, gd, wd, 1e-6, rd, s1d, shd)
    ref_q, ref_s = h.quantize_rowwise(ref_h)
    xd = x.cuda()
    out = h.gate_norm_mod_q_(xd, od, gd, wd, 1e-6, rd, s1d, shd, want_h=want_h)
    assert torch.equal(xd, x_ref)
    if want_h:
        assert torch.equal(out[0], ref_h)
        out = out[1:]
    assert torch.equal(out[0], ref_q)
    assert torch.equal(out[1].view(torch.int32), ref_s.view(torch.int32))


def test_norm_mod_q_matches_oracle_chain():
    h = _h3mi()
    S, N, R = 48, 5120, 2
    x, w, s1, sh, _, _, ridx = norm_inputs(S, N, R, seed=21)
    xd, wd, rd, s1d, shd = _cuda(x, w, ridx, s1, sh)
    _, _, rstd = h.norm_mod_ex(xd, wd, 1e-6, rd, s1d, shd, stats=True)
    q, qs = h.norm_mod_q(xd, wd, 1e-6, rd, s1d, shd)
    oh, _, _ = O.norm_mod(bits(x), bits(w), 1e-6, ridx.numpy(), bits(s1), bits(sh), order=h.order_info(0),
                          rstd=rstd.cpu().numpy())
    oq, os_ = O.quant_rowwise(oh)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(qs.cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))


def test_gate_norm_mod_q_matches_oracle_chain():
    """gate_norm_mod_q_ against the oracle chain gate_norm_mod -> quant_rowwise
    fed the GPU's rstd (x updated in place as the oracle's x)."""
    h = _h3mi()
    S, N, R = 48, 5120, 2
    x, w, s1, sh, g, o, ridx = norm_inputs(S, N, R, seed=22)
    od, gd, wd, rd, s1d, shd = _cuda(o, g, w, ridx, s1, sh)
    x_stats = x.cuda()
    _, _, rstd = h.gate_norm_mod_ex(x_stats, od, gd, wd, 1e-6, rd, s1d, shd, stats=True)
    xd = x.cuda()
    q, qs = h.gate_norm_mod_q_(xd, od, gd, wd, 1e-6, rd, s1d, shd)
    ox, oh, _, _ = O.gate_norm_mod(bits(x), bits(o), bits(g), bits(w), 1e-6, ridx.numpy(), bits(s1), bits(sh),
                                   order=h.order_info(0), rstd=rstd.cpu().numpy())
    oq, os_ = O.quant_rowwise(oh)
    assert np.array_equal(bits(xd), ox)
    assert np.array_equal(q.cpu().numpy(), oq)
    assert np.array_equal(qs.cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))


def test_norm_mod_q_out_of_range_rows_untouched():
    """Rows whose table index is out of range leave q, qs (and h) unwritten."""
    h = _h3mi()
    from h3mi import _lib as L
    S, N, R = 2100, 5120, 2
    x, w, s1, sh, _, _, ridx = norm_inputs(S, N, R, seed=9, stress=False)
    ridx[:] = 1
    ridx[7::11] = -1
    ridx[900:1300] = R
    bad = ((ridx < 0) | (ridx >= R)).cuda()
    xd, wd, rd, s1d, shd = _cuda(x, w, ridx, s1, sh)
    q = torch.full((S, N), 55, dtype=torch.int8, device="cuda")
    qs = torch.full((S, 1), 3.0, device="cuda")
    hh = torch.full((S, N), 7.0, dtype=torch.bfloat16, device="cuda")
    L.check(L.lib.h3mi_norm_mod_quant_i8(L.ptr(xd), L.ptr(wd), L.ptr(rd), L.ptr(s1d), L.ptr(shd), L.ptr(hh), L.ptr(q),
                                         L.ptr(qs), S, N, R, 1e-6, L.stream_of(xd)))
    assert bool((q[bad] == 55).all()) and bool((qs[bad] == 3.0).all()) and bool((hh[bad] == 7.0).all())
    good = ~bad
    ref_h = h.norm_mod(xd, wd, 1e-6, rd, s1d, shd)
    ref_q, ref_s = h.quantize_rowwise(ref_h)
    assert torch.equal(q[good], ref_q[good]) and torch.equal(qs[good], ref_s[good]) and torch.equal(hh[good], ref_h[good])


def test_rows_the_quantizer_cannot_take_are_rejected():
    """The per-token quantizer needs N % 8 == 0; so do the fused entry points."""
    h = _h3mi()
    from h3mi._lib import H3miError
    x, w, s1, sh, g, o, ridx = norm_inputs(8, 1028, 1, seed=3, stress=False)
    xd, wd, rd, s1d, shd, od, gd = _cuda(x, w, ridx, s1, sh, o, g)
    with pytest.raises(H3miError):
        h.quantize_rowwise(h.norm_mod(xd, wd, 1e-6, rd, s1d, shd))
    with pytest.raises(H3miError):
        h.norm_mod_q(xd, wd, 1e-6, rd, s1d, shd)
    with pytest.raises(H3miError):
        h.gate_norm_mod_q_(xd, od, gd, wd, 1e-6, rd, s1d, shd)
