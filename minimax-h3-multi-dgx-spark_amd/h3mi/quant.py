"""Per-token symmetric int8 quantizer (HIP, gfx950).

Replaces the activation quantizer the reference runs before its GEMM
(comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95), without rotation:
s[m] = max|x[m,:]|/127, q = clamp(round_half_even(x/s), -127, 127), s = q = 0
for an all-zero row.
"""
import torch

from ._lib import check, lib, ptr, same_gpu, stream_of


def quantize_rowwise(x, xq=None, xs=None):
    """x bf16 [M,K] (row stride may exceed K) -> (xq int8 [M,K], xs fp32 [M,1])."""
    if x.dim() != 2 or x.dtype != torch.bfloat16 or not x.is_cuda:
        raise ValueError("x must be a 2-D bfloat16 GPU tensor")
    if x.stride(1) != 1:
        raise ValueError("x must have unit column stride")
    M, K = x.shape
    if xq is None:
        xq = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if xs is None:
        xs = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    if xq.shape != (M, K) or not xq.is_contiguous() or xq.dtype != torch.int8:
        raise ValueError("xq must be contiguous int8 [M, K]")
    if xs.numel() != M or not xs.is_contiguous() or xs.dtype != torch.float32:
        raise ValueError("xs must be contiguous float32 with M elements")
    same_gpu(x, xq=xq, xs=xs)
    check(lib.h3mi_quant_rowwise_i8(ptr(x), ptr(xq), ptr(xs), M, K, x.stride(0), stream_of(x)))
    return xq, xs


_ACTS = {None: 0, "none": 0, "swiglu": 1}


def quantize_rowwise_convrot(x, act=None, group_size=256, xq=None, xs=None):
    """ConvRot quantizer: 256-group Hadamard rotation then per-row int8.

    Stands in for comfy-kitchen's _C.quantize_int8_rowwise_convrot64 as the
    reference calls it (comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:
    90-95): x bf16 [M, K] (act None) or [M, 2K] (act "swiglu": silu of the
    first half times the second) -> (xq int8 [M, K], xs fp32 [M, 1]) with
    y = H u / 16 per 256-group (Sylvester Hadamard), xs = max|y|/127,
    xq = clamp(rne(y/xs), -127, 127).  K % 256 == 0, K <= 32768."""
    if act not in _ACTS:
        raise ValueError(f"unsupported input activation {act!r}")
    if x.dim() != 2 or x.dtype != torch.bfloat16 or not x.is_cuda:
        raise ValueError("x must be a 2-D bfloat16 GPU tensor")
    if x.stride(1) != 1:
        raise ValueError("x must have unit column stride")
    M, kin = x.shape
    a = _ACTS[act]
    if a == 1 and kin % 2:
        raise ValueError("swiglu input needs an even number of columns")
    K = kin // 2 if a == 1 else kin
    if xq is None:
        xq = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if xs is None:
        xs = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    if xq.shape != (M, K) or not xq.is_contiguous() or xq.dtype != torch.int8:
        raise ValueError("xq must be contiguous int8 [M, K]")
    if xs.numel() != M or not xs.is_contiguous() or xs.dtype != torch.float32:
        raise ValueError("xs must be contiguous float32 with M elements")
    same_gpu(x, xq=xq, xs=xs)
    check(lib.h3mi_quant_convrot_i8(ptr(x), ptr(xq), ptr(xs), M, K, x.stride(0), group_size, a, stream_of(x)))
    return xq, xs
