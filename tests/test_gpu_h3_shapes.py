"""The W8A8 linear and the fused norms at the real H3 DiT shapes (hidden 5376,
56 x 128 heads; reference bench/gemm_peak.py:7-8) and token counts
(19,200 and 38,400 per GPU; tests/test_triton_gemm.py:8), where the reference
checks its Triton GEMM bit for bit against the CUTLASS path with real weights.
No checkpoint is available here, so the weights are random with the
checkpoint's dtypes; the bar is the same: bit-exact.

  * int32 accumulators == torch._int_mm (hipBLASLt, a different implementation)
  * bf16 outputs == the epilogue in separate torch GPU ops (one IEEE rounding
    each: f32(acc) * xs, then * ws, then + bias, then bf16)
  * quantizer rows == the CPU oracle (row sample)
  * fused norms == the eager PyTorch sequence on the GPU
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from h3mi import h3_weights as HW
from oracle import oracle as O
from util import bits

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


@pytest.mark.parametrize("M", HW.TOKENS)
@pytest.mark.parametrize("layer", ["qkv", "out", "fc1", "fc2"])
def test_h3_linear_shapes_bitexact(layer, M):
    h = _h3mi()
    K, N = HW.SHAPES[layer]
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
    ws = (1e-3 + 9e-3 * torch.rand(N, device="cuda", generator=g)).contiguous()
    bias = (0.02 * torch.randn(N, device="cuda", generator=g)).to(torch.bfloat16)
    xq, xs = h.quantize_rowwise(x)
    rows = torch.arange(0, M, 997)
    oq, os_ = O.quant_rowwise(bits(x[rows.cuda()]))
    assert np.array_equal(xq[rows.cuda()].cpu().numpy(), oq)
    assert np.array_equal(xs[rows.cuda()].cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))
    acc = h.int8_mm_i32(xq, w)
    ref = torch._int_mm(xq, w.t())
    assert torch.equal(acc, ref)
    del acc
    y = ref.float()
    del ref
    y = (y * xs) * ws[None, :]
    out = h.int8_mm_scaled(xq, w, xs, ws)
    assert torch.equal(out, y.to(torch.bfloat16))
    outb = h.int8_mm_scaled(xq, w, xs, ws, bias=bias)
    assert torch.equal(outb, (y + bias.float()[None, :]).to(torch.bfloat16))


@pytest.mark.parametrize("S", HW.TOKENS)
def test_h3_norms_match_eager(S):
    """norm_mod / gate_norm_mod_ / gate_ at [S, 5376] (N % 512 != 0: each row's
    last chunk is half in range) == F.rms_norm -> mul_(1 + scale) -> add_(shift)
    and addcmul_(o, gate) on the GPU."""
    h = _h3mi()
    N, eps = HW.HIDDEN, 1e-6
    g = torch.Generator(device="cuda").manual_seed(S)
    x = torch.randn(S, N, device="cuda", generator=g).to(torch.bfloat16)
    o = torch.randn(S, N, device="cuda", generator=g).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(N, device="cuda", generator=g)).to(torch.bfloat16)
    s1 = (1.0 + (0.1 * torch.randn(1, N, device="cuda", generator=g)).to(torch.bfloat16)).contiguous()
    sh = (0.1 * torch.randn(1, N, device="cuda", generator=g)).to(torch.bfloat16)
    gt = (0.1 * torch.randn(1, N, device="cuda", generator=g)).to(torch.bfloat16)
    ridx = torch.zeros(S, dtype=torch.int32, device="cuda")

    def eager_nm(t):
        return F.rms_norm(t, (N,), w, eps).mul_(s1[0]).add_(sh[0])

    assert torch.equal(h.norm_mod(x, w, eps, ridx, s1, sh), eager_nm(x))
    xg = x.clone()
    hg = h.gate_norm_mod_(xg, o, gt, w, eps, ridx, s1, sh)
    xe = x.clone().addcmul_(o, gt[0])
    assert torch.equal(xg, xe)
    assert torch.equal(hg, eager_nm(xe))
    x2 = x.clone()
    h.gate_(x2, o, gt, ridx)
    assert torch.equal(x2, xe)
