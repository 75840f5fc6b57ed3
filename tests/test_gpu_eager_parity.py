"""Fused norms vs the eager PyTorch sequence they replace, on the same GPU.

The reference's fused kernels are built to be bit-identical to
F.rms_norm -> mul_(1+scale) -> add_(shift) -> addcmul_(o, gate) on the GPU
they run on (comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:3-16).  On MI355X
the eager path is PyTorch-ROCm; this file measures which reduction order it
uses (the method of the reference's tests/test_rmsnorm_exact.py:116-142, run
through the CPU oracle plus the GPU's own rsqrt) and checks the default
kernels against eager.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from util import bits, norm_inputs

pytestmark = pytest.mark.gpu

CANDIDATES = [(128, 4, 32), (256, 4, 64), (128, 4, 64), (256, 4, 32), (512, 4, 64), (1024, 4, 64),
              (256, 8, 64), (512, 8, 64), (128, 8, 64), (256, 2, 64), (64, 4, 64), (1024, 8, 64)]


def _dev_rsqrt_hw(v):
    from h3mi import _lib as L
    t = torch.from_numpy(np.ascontiguousarray(v, np.float32)).cuda()
    out = torch.empty_like(t)
    L.check(L.lib.h3mi_debug_rsqrt_f32(L.ptr(t), L.ptr(out), t.numel(), 0, L.stream_of(t)))
    return out.cpu().numpy()


def _eager_rstd(x, w, eps):
    try:
        y, rstd = torch.ops.aten._fused_rms_norm(x, [x.shape[1]], w, eps)
        return y, rstd.reshape(-1)
    except Exception:  # noqa: BLE001
        return None, None


def test_order_search_against_eager_rms_norm(capsys):
    """At the reference's stress size and distribution (tests/test_rmsnorm_exact.py:117-124: seed 0, 8192 x 5376,
    logspace row scales, 7 hot columns x50, w = 1 + 0.3 randn, eps 1e-5)."""
    torch.manual_seed(0)
    S, N, eps = 8192, 5376, 1e-5
    x, w, _, _, _, _, _ = norm_inputs(S, N, 1, seed=0)
    xd, wd = x.cuda(), w.cuda()
    ref = F.rms_norm(xd, (N,), wd, eps)
    y2, trstd = _eager_rstd(xd, wd, eps)
    if y2 is not None:
        assert torch.equal(y2, ref)
    xf = O.bf16_bits_to_f32(bits(x))
    lines = []
    for cand in CANDIDATES:
        var = np.array([np.float32(np.float32(O.row_sumsq(xf[i], cand)) / np.float32(N)) + np.float32(eps)
                        for i in range(S)], np.float32)
        rstd = _dev_rsqrt_hw(var)
        ones = O.f32_to_bf16_bits(np.ones((1, N), np.float32))
        zeros = O.f32_to_bf16_bits(np.zeros((1, N), np.float32))
        y, _, _ = O.norm_mod(bits(x), bits(w), eps, np.zeros(S, np.int32), ones, zeros, order=cand, rstd=rstd)
        bad = int((y != bits(ref)).sum())
        bad_rows = int((y != bits(ref)).any(1).sum())
        rs_bad = -1 if trstd is None else int((rstd.view(np.uint32) != trstd.cpu().numpy().view(np.uint32)).sum())
        lines.append((cand, bad, bad_rows, rs_bad))
    with capsys.disabled():
        print("\n[order search] torch", torch.__version__)
        for cand, bad, bad_rows, rs_bad in lines:
            print(f"  numx={cand[0]:4d} vec={cand[1]} warp={cand[2]:2d}: differing elements {bad:8d} "
                  f"rows {bad_rows:4d}/{S}  rstd mismatches {rs_bad}")
    from h3mi import order_info
    default = order_info(0)
    got = dict(((c, b) for c, b, _, _ in lines))
    assert got[default] == 0, f"default order {default} differs from eager rms_norm"


def test_default_norm_mod_matches_eager_sequence():
    h = pytest.importorskip("h3mi")
    S, N, R, eps = 512, 5120, 1, 1e-6
    x, w, s1, sh, _, _, ridx = norm_inputs(S, N, R, seed=5, stress=False)
    xd, wd, s1d, shd = x.cuda(), w.cuda(), s1.cuda(), sh.cuda()
    ours = h.norm_mod(xd, wd, eps, torch.zeros(S, dtype=torch.int32, device="cuda"), s1d, shd)
    ref = F.rms_norm(xd, (N,), wd, eps)
    ref.mul_(s1d[0]).add_(shd[0])
    diff = int((bits(ours) != bits(ref)).sum())
    assert diff == 0, f"{diff} elements differ from eager"


def test_default_gate_norm_mod_matches_eager_sequence():
    h = pytest.importorskip("h3mi")
    S, N, R, eps = 512, 5120, 1, 1e-6
    x, w, s1, sh, g, o, _ = norm_inputs(S, N, R, seed=6, stress=False)
    xd, od, gd, wd, s1d, shd = (t.cuda() for t in (x, o, g, w, s1, sh))
    ridx = torch.zeros(S, dtype=torch.int32, device="cuda")
    x_ours = xd.clone()
    ours = h.gate_norm_mod_(x_ours, od, gd, wd, eps, ridx, s1d, shd)
    x_ref = xd.clone()
    x_ref.addcmul_(od, gd[0])
    ref = F.rms_norm(x_ref, (N,), wd, eps)
    ref.mul_(s1d[0]).add_(shd[0])
    assert torch.equal(x_ours, x_ref)
    diff = int((bits(ours) != bits(ref)).sum())
    assert diff == 0, f"{diff} elements differ from eager"
