"""PyTorch-eager CPU restatement of the reference path, used as the CPU
baseline that bench.py times next to the GPU kernels.

TEST INFRASTRUCTURE ONLY (imported by tests/ and bench.py's cpu_baseline leg).
It restates the same arithmetic as oracle/h3_oracle.c with vectorised torch
CPU ops, so it is fast enough to time on real shapes:
  * W8A8 linear: per-row quantize (s = absmax/127, round half to even, clamp
    +-127) -> torch._int_mm (int32) -> bf16(((f32(acc) * xs) * ws) + bias)
    (comfyui_nodes/h3-linear-fast/int8_gemm_triton.py:2,61-66);
  * fused norms: the eager sequence the fused kernels replace,
    F.rms_norm -> mul_(s1) -> add_(sh) and addcmul_(o, g)
    (comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:3-7).
The norm sequence on the CPU sums in a different order from the GPU kernels,
so it is a timing baseline, not a bit-exact checker; the W8A8 path is exact.
"""
import torch
import torch.nn.functional as F


def quant_rowwise(x):
    xf = x.float()
    s = xf.abs().amax(dim=1, keepdim=True) / 127.0
    safe = torch.where(s == 0, torch.ones_like(s), s)
    q = torch.round(xf / safe).clamp_(-127, 127)
    q = torch.where(s == 0, torch.zeros_like(q), q).to(torch.int8)
    return q, s


def w8a8_linear(x, w, ws, bias=None):
    q, s = quant_rowwise(x)
    acc = torch._int_mm(q, w.t())
    c = (acc.float() * s) * ws[None, :]
    if bias is not None:
        c = c + bias.float()[None, :]
    return c.to(torch.bfloat16)


def norm_mod(x, w, eps, s1, sh):
    h = F.rms_norm(x, (x.shape[1],), w, eps)
    return h.mul_(s1).add_(sh)


def gate_(x, o, g):
    return x.addcmul_(o, g)


def gate_norm_mod_(x, o, g, w, eps, s1, sh):
    x.addcmul_(o, g)
    return norm_mod(x, w, eps, s1, sh)
