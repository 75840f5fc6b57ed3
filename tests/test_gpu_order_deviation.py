"""The distance between this library's default norm order and the reference's.

The reference's fused norms sum squares in CUDA PyTorch's order: 128 threads
x 4 elements with a 32-lane tree (comfyui_nodes/h3-fuse-graph/
h3_fuse_kernels.py:12-16,42-43).  On MI355X the eager path they must match is
PyTorch-ROCm, whose order (256 x 4, 64-lane tree; tests/test_gpu_eager_parity.py)
is this library's default.  The two orders round the sum of squares
differently, so their outputs may differ; this file states by how much.

The reference-order side is the CPU oracle in the reference order fed the
GPU's own v_rsq_f32 of the oracle's sum, so that only the summation order
differs from the product kernel.  Bound, from the rounding points of the
formula h = bf16(rb(rb(w*(rstd*x))*s1) + sh):
  * y = rb(w*(rstd*x)), the normalised row (tables s1 = 1, sh = 0): the two
    orders' rstd differ by a few fp32 ulps, far below half a bf16 ulp, so y
    differs by at most 1 bf16 ulp;
  * h: that ulp of y passes through the two modulation roundings, so
    |dh| <= |s1| ulp(y) + 2 ulp(y s1) + 2 ulp(h) with the ulps taken at the
    reference-order values (each rounding moves by half an ulp of either
    side's value, which is at most one ulp of the reference value across a
    binade edge).  Where the shift add cancels, that is more ulps of h itself.
Both workloads are checked: C3 (x[32768, 5120] ~ N(0,1), eps 1e-6, one adaLN
row) and the reference's stress set (tests/test_rmsnorm_exact.py:117-124:
8192 x 5376, rows scaled over 1e-2..1e3, 7 hot columns x50, w = 1 + 0.3 randn,
eps 1e-5)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits, gen, norm_inputs

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


def _dev_rsqrt_hw(v):
    from h3mi import _lib as L
    t = torch.from_numpy(np.ascontiguousarray(v, np.float32)).cuda()
    out = torch.empty_like(t)
    L.check(L.lib.h3mi_debug_rsqrt_f32(L.ptr(t), L.ptr(out), t.numel(), 0, L.stream_of(t)))
    return out.cpu().numpy()


def _ordered(b):
    """bf16 bit patterns -> integers in the order of the values (ulp steps)."""
    b = b.astype(np.int32)
    mag = b & 0x7FFF
    return np.where(b & 0x8000, -mag, mag)


def _ulp(v):
    """bf16 ulp at |v| (fp32 array): 2^(floor(log2|v|) - 7), normal range."""
    a = np.maximum(np.abs(v.astype(np.float32)), np.float32(2.0 ** -126))
    return np.ldexp(np.float32(1.0), np.floor(np.log2(a)).astype(np.int32) - 7).astype(np.float32)


def _c3_inputs():
    S, N = 32768, 5120
    g = gen(3)
    x = torch.randn(S, N, generator=g).to(torch.bfloat16)
    o = torch.randn(S, N, generator=g).to(torch.bfloat16)
    shift = (0.1 * torch.randn(1, N, generator=g)).to(torch.bfloat16)
    scale = (0.1 * torch.randn(1, N, generator=g)).to(torch.bfloat16)
    gate = (0.1 * torch.randn(1, N, generator=g)).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(N, generator=g)).to(torch.bfloat16)
    return x, w, (1.0 + scale).contiguous(), shift, gate, o, torch.zeros(S, dtype=torch.int32), 1e-6


def _stress_inputs():
    x, w, s1, sh, g, o, _ = norm_inputs(8192, 5376, 1, seed=0)
    return x, w, s1, sh, g, o, torch.zeros(8192, dtype=torch.int32), 1e-5


def _ref_order(x_bits, w, s1, sh, ridx, eps):
    """Reference-order oracle outputs (h, y) with the device rsqrt of the reference-order sum."""
    S, N = x_bits.shape
    _, var, _ = O.norm_mod(x_bits, bits(w), eps, ridx, bits(s1), bits(sh), order=O.REF_ORDER)
    rstd = _dev_rsqrt_hw(var)
    h, _, _ = O.norm_mod(x_bits, bits(w), eps, ridx, bits(s1), bits(sh), order=O.REF_ORDER, rstd=rstd)
    ones = O.f32_to_bf16_bits(np.ones((1, N), np.float32))
    zeros = O.f32_to_bf16_bits(np.zeros((1, N), np.float32))
    y, _, _ = O.norm_mod(x_bits, bits(w), eps, ridx, ones, zeros, order=O.REF_ORDER, rstd=rstd)
    return h, y


def _compare(tag, h_prod, y_prod, h_ref, y_ref, s1_row, capsys):
    dy = np.abs(_ordered(y_prod) - _ordered(y_ref))
    hp = O.bf16_bits_to_f32(h_prod)
    hr = O.bf16_bits_to_f32(h_ref)
    yr = O.bf16_bits_to_f32(y_ref)
    dh = np.abs(hp - hr)
    s1v = np.abs(O.bf16_bits_to_f32(s1_row))[None, :]
    bound = s1v * _ulp(yr) + 2.0 * _ulp(yr * s1v) + 2.0 * _ulp(hr)
    ulps_h = np.abs(_ordered(h_prod) - _ordered(h_ref))
    n = h_prod.size
    with capsys.disabled():
        print(f"\n[order deviation] {tag}: {n} elements; y differs in {int((dy > 0).sum())} "
              f"(max {int(dy.max())} ulp); h differs in {int((ulps_h > 0).sum())} "
              f"({100.0 * (ulps_h > 0).sum() / n:.4f}%), {int((ulps_h == 1).sum())} of them by 1 ulp, "
              f"max {int(ulps_h.max())} ulp of h, max |dh| / bound {float((dh / bound).max()):.3f}")
    assert int(dy.max()) <= 1, "normalised rows differ by more than 1 bf16 ulp"
    assert bool((dh <= bound).all()), "h differs by more than the propagated ulp of y"
    return int((ulps_h > 0).sum())


@pytest.mark.parametrize("workload", ["c3", "stress"])
def test_default_order_vs_reference_order(workload, capsys):
    h3 = _h3mi()
    x, w, s1, sh, _, _, ridx, eps = _c3_inputs() if workload == "c3" else _stress_inputs()
    S, N = x.shape
    print(f"[order deviation] {workload} [{S}, {N}] eps {eps}", flush=True)
    xb = bits(x)
    h_ref, y_ref = _ref_order(xb, w, s1, sh, ridx.numpy(), eps)
    xd, wd, rd = x.cuda(), w.cuda(), ridx.cuda()
    h_prod = bits(h3.norm_mod(xd, wd, eps, rd, s1.cuda(), sh.cuda()))
    ones = torch.ones(1, N, dtype=torch.bfloat16, device="cuda")
    zeros = torch.zeros(1, N, dtype=torch.bfloat16, device="cuda")
    y_prod = bits(h3.norm_mod(xd, wd, eps, rd, ones, zeros))
    _compare(f"norm_mod {workload}", h_prod, y_prod, h_ref, y_ref, bits(s1)[0], capsys)


def test_default_order_vs_reference_order_gate(capsys):
    """gate_norm_mod_ at C3: xn = rb(x + o g) does not depend on the order
    (exactly equal); the norm of xn deviates as above."""
    h3 = _h3mi()
    x, w, s1, sh, g, o, ridx, eps = _c3_inputs()
    S, N = x.shape
    xn_ref = O.gate(bits(x), bits(o), bits(g), ridx.numpy())
    h_ref, y_ref = _ref_order(xn_ref, w, s1, sh, ridx.numpy(), eps)
    xd = x.cuda()
    hd = h3.gate_norm_mod_(xd, o.cuda(), g.cuda(), w.cuda(), eps, ridx.cuda(), s1.cuda(), sh.cuda())
    assert np.array_equal(bits(xd), xn_ref)
    ones = torch.ones(1, N, dtype=torch.bfloat16, device="cuda")
    zeros = torch.zeros(1, N, dtype=torch.bfloat16, device="cuda")
    y_prod = bits(h3.norm_mod(xd, w.cuda(), eps, ridx.cuda(), ones, zeros))
    _compare("gate_norm_mod_ c3", bits(hd), y_prod, h_ref, y_ref, bits(s1)[0], capsys)


def test_reference_order_mode_matches_reference_order_oracle():
    """The library's reference-order mode (norm_mod_ex order="ref") is the
    reference's order itself: bit-exact against the reference-order oracle
    given the kernel's own rstd, at the stress set."""
    h3 = _h3mi()
    x, w, s1, sh, _, _, ridx, eps = _stress_inputs()
    xd = x.cuda()
    h, var, rstd = h3.norm_mod_ex(xd, w.cuda(), eps, ridx.cuda(), s1.cuda(), sh.cuda(), order="ref", stats=True)
    oh, ovar, _ = O.norm_mod(bits(x), bits(w), eps, ridx.numpy(), bits(s1), bits(sh), order=O.REF_ORDER,
                             rstd=rstd.cpu().numpy())
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    assert np.array_equal(bits(h), oh)
