"""The whole W8A8 linear: per-token quantize, int8 GEMM, fused dequant epilogue."""
import torch

from .gemm import int8_mm_scaled
from .quant import quantize_rowwise


def w8a8_linear(x, weight, weight_scale, bias=None, out=None):
    """x bf16 [..., K], weight int8 [N, K], weight_scale fp32 [N] (or scalar),
    bias bf16 [N] or None -> bf16 [..., N]."""
    K = x.shape[-1]
    N = weight.shape[0]
    x2 = x if (x.dim() == 2 and x.stride(1) == 1) else x.reshape(-1, K).contiguous()
    ws = weight_scale.to(device=x.device, dtype=torch.float32).reshape(-1)
    if ws.numel() != N:
        ws = ws.expand(N)
    ws = ws.contiguous()
    xq, xs = quantize_rowwise(x2)
    o = int8_mm_scaled(xq, weight, xs, ws, out=out, bias=bias)
    return o if x.dim() == 2 else o.reshape(*x.shape[:-1], N)
