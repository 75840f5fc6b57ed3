"""q/k RMSNorm + split-half RoPE on the GPU.

h3mi.rms_rope_split_half_ (C ABI h3mi_rms_rope_split_half_bf16) stands in for
comfy-kitchen's ck.rms_rope_split_half_ as the reference calls it on the q / k
views of the qkv projection (comfyui_nodes/minimax-h3-sp/minimax_sp/
sp_forward.py:279-296).  Bars, all bit-exact:
  * eager PyTorch on the same GPU: F.rms_norm of each (token, head) row, then
    the split-half rotation in separate fp32 torch ops -- the sequence the
    fused call stands for -- at small shapes and at the full H3 size
    (19200 tokens x 56 heads x 128);
  * the oracle (h3o_rms_rope_split_half) fed the kernel's rstd (hardware
    rsqrt), and with the correctly rounded rsqrt end to end;
  * in place on q and k views of one qkv buffer: v and the gaps untouched.
The first test measures which summation order eager rms_norm uses for a
128-element row (the reference's own method, tests/test_rmsnorm_exact.py:
116-142) and checks the kernel's order is it.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from util import bits

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


def _table(S, rot, seed):
    g = torch.Generator().manual_seed(seed)
    ang = torch.rand(S, rot // 2, generator=g) * 6.3
    t = torch.stack([torch.stack([ang.cos(), -ang.sin()], -1), torch.stack([ang.sin(), ang.cos()], -1)], -2)
    return t.to(torch.bfloat16)


def _qkv(S, H, D, seed, spread=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(S, 3, H, D, generator=g)
    if spread:
        x = x * torch.logspace(-2, 2, S)[:, None, None, None]
        x[:, :, :, :3] *= 30
    return x.to(torch.bfloat16)


def _eager(x, w, tab, rot, eps):
    """F.rms_norm per row, then the rotation in separate fp32 torch ops, on the GPU."""
    S, H, D = x.shape
    y = F.rms_norm(x.reshape(S * H, D), (D,), w, eps).reshape(S, H, D).float()
    out = y.clone()
    h = rot // 2
    if rot:
        R = tab.float()[:, None]
        a, b = y[..., :h], y[..., h:rot]
        out[..., :h] = (R[..., 0, 0] * a) + (R[..., 0, 1] * b)
        out[..., h:rot] = (R[..., 1, 0] * a) + (R[..., 1, 1] * b)
    return out.to(torch.bfloat16)


def test_eager_rms_norm_order_for_head_rows(capsys):
    from test_gpu_eager_parity import CANDIDATES, _dev_rsqrt_hw
    S, D, eps = 512, 128, 1e-6
    x = _qkv(S, 1, D, seed=0)[:, 0, 0].contiguous()
    w = (1 + 0.2 * torch.randn(D, generator=torch.Generator().manual_seed(1))).to(torch.bfloat16)
    ref = F.rms_norm(x.cuda(), (D,), w.cuda(), eps)
    xf = O.bf16_bits_to_f32(bits(x))
    ones = O.f32_to_bf16_bits(np.ones((1, D), np.float32))
    zeros = O.f32_to_bf16_bits(np.zeros((1, D), np.float32))
    got = {}
    for cand in CANDIDATES:
        var = np.array([np.float32(np.float32(O.row_sumsq(xf[i], cand)) / np.float32(D)) + np.float32(eps)
                        for i in range(S)], np.float32)
        y, _, _ = O.norm_mod(bits(x), bits(w), eps, np.zeros(S, np.int32), ones, zeros, order=cand,
                             rstd=_dev_rsqrt_hw(var))
        got[cand] = int((y != bits(ref)).sum())
    with capsys.disabled():
        print("\n[order search, 128-element rows]", {c: n for c, n in got.items()})
    assert got[(256, 4, 64)] == 0


@pytest.mark.parametrize("S,H,D,rot", [(33, 3, 128, 128), (17, 2, 128, 64), (9, 4, 128, 0), (21, 5, 64, 64),
                                       (13, 2, 256, 128), (10, 1, 128, 16), (1, 56, 128, 128), (11, 2, 128, 96),
                                       (37, 1, 64, 32), (19, 3, 256, 256)])
def test_matches_eager_and_oracle(S, H, D, rot):
    print(f"[rms_rope] S={S} H={H} D={D} rot={rot}", flush=True)
    h = _h3mi()
    eps = 1e-6
    qkv = _qkv(S, H, D, seed=S * 100 + D + rot)
    g = torch.Generator().manual_seed(7)
    qw = (1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    tab = _table(S, rot, seed=S) if rot else None
    buf = qkv.reshape(S, 3 * H * D).cuda()
    q = buf[:, :H * D].view(1, S, H, D)
    k = buf[:, H * D:2 * H * D].view(1, S, H, D)
    v_before = buf[:, 2 * H * D:].clone()
    rstd = torch.empty(S * 2 * H, dtype=torch.float32, device="cuda")
    tdev = tab[None].cuda() if rot else None
    h.rms_rope_split_half_(q, k, tdev, qw.cuda(), kw.cuda(), epsilon=eps, rot_dim=rot, rstd_out=rstd)
    torch.cuda.synchronize()
    assert torch.equal(buf[:, 2 * H * D:], v_before)
    # eager GPU sequence
    for i, w in ((0, qw), (1, kw)):
        ref = _eager(qkv[:, i].cuda(), w.cuda(), tab.cuda() if rot else None, rot, eps)
        got = (q if i == 0 else k)[0]
        assert torch.equal(got, ref), f"{'qk'[i]}: {int((got != ref).sum())} elements differ from eager"
    # oracle with the kernel's rstd
    rs = rstd.cpu().numpy().reshape(S, 2, H)
    for i, w in ((0, qw), (1, kw)):
        oo, _ = O.rms_rope_split_half(bits(qkv[:, i]), bits(tab) if rot else None, bits(w), eps, rot, rstd=rs[:, i])
        assert np.array_equal(bits((q if i == 0 else k)[0]), oo)


def test_correctly_rounded_rsqrt_mode_matches_oracle():
    h = _h3mi()
    S, H, D, rot, eps = 40, 3, 128, 128, 1e-5
    qkv = _qkv(S, H, D, seed=11)
    qw = (1 + 0.2 * torch.randn(D, generator=torch.Generator().manual_seed(2))).to(torch.bfloat16)
    tab = _table(S, rot, seed=3)
    q = qkv[:, 0].contiguous().cuda()
    k = qkv[:, 1].contiguous().cuda()
    h.rms_rope_split_half_(q, k, tab.cuda(), qw.cuda(), qw.cuda(), epsilon=eps, rsqrt="rn")
    for i, t in ((0, q), (1, k)):
        oo, _ = O.rms_rope_split_half(bits(qkv[:, i]), bits(tab), bits(qw), eps, rot)
        assert np.array_equal(bits(t), oo)


def test_out_of_place_form():
    h = _h3mi()
    S, H, D = 8, 2, 128
    qkv = _qkv(S, H, D, seed=12).cuda()
    q, k = qkv[:, 0], qkv[:, 1]
    w = torch.ones(D, dtype=torch.bfloat16, device="cuda")
    tab = _table(S, D, seed=4).cuda()
    q0, k0 = q.clone(), k.clone()
    qo, ko = h.rms_rope_split_half(q, k, tab, w, w, 1e-6)
    assert torch.equal(q, q0) and torch.equal(k, k0)
    qi, ki = h.rms_rope_split_half_(q0, k0, tab, w, w, 1e-6)
    assert torch.equal(qo, qi) and torch.equal(ko, ki)


def test_h3_size_matches_eager():
    """19200 tokens x 56 heads x 128, full rotation, in place on the qkv buffer."""
    print("[rms_rope] H3 size", flush=True)
    h = _h3mi()
    S, H, D, eps = 19200, 56, 128, 1e-6
    buf = torch.randn(S, 3 * H * D, device="cuda").to(torch.bfloat16)
    qw = (1 + 0.2 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(D, device="cuda")).to(torch.bfloat16)
    ang = torch.rand(S, D // 2, device="cuda") * 6.3
    tab = torch.stack([torch.stack([ang.cos(), -ang.sin()], -1), torch.stack([ang.sin(), ang.cos()], -1)], -2)
    tab = tab.to(torch.bfloat16)
    refq = _eager(buf[:, :H * D].view(S, H, D), qw, tab, D, eps)
    refk = _eager(buf[:, H * D:2 * H * D].view(S, H, D), kw, tab, D, eps)
    v0 = buf[:, 2 * H * D:].clone()
    q = buf[:, :H * D].view(1, S, H, D)
    k = buf[:, H * D:2 * H * D].view(1, S, H, D)
    h.rms_rope_split_half_(q, k, tab[None], qw, kw, epsilon=eps)
    assert torch.equal(q[0], refq) and torch.equal(k[0], refk) and torch.equal(buf[:, 2 * H * D:], v0)
