"""q/k RMSNorm + split-half rotary embedding (HIP, gfx950), in place.

Stands in for comfy-kitchen's ck.rms_rope_split_half_ / rms_rope_split_half as
the reference calls them on the attention's q and k
(comfyui_nodes/minimax-h3-sp/minimax_sp/sp_forward.py:279-296): q, k
[1, s, heads, dim] views of the qkv projection, rope_freqs from
rope_rotation_table (:548) with rot_dim = rope_freqs.shape[-3] * 2.  Each
(token, head) row becomes the eager F.rms_norm of the row followed by the
split-half rotation: the pair (y[i], y[i + rot/2]) times the token's 2 x 2
table entry i, in fp32, rounded to bf16.
"""
import torch

from ._lib import RSQRT_HW, RSQRT_RN, check, lib, ptr, same_gpu, stream_of

_MODES = {"hw": RSQRT_HW, "rn": RSQRT_RN}


def _rows(t, name):
    if t.dtype != torch.bfloat16 or not t.is_cuda:
        raise ValueError(f"{name} must be a bfloat16 GPU tensor")
    if t.dim() == 4:
        if t.shape[0] != 1:
            raise ValueError(f"{name}: batch dimension must be 1")
        t = t[0]
    if t.dim() != 3:
        raise ValueError(f"{name} must be [1, s, heads, dim] or [s, heads, dim]")
    S, H, D = t.shape
    if t.stride(2) != 1 or (H > 1 and t.stride(1) != D):
        raise ValueError(f"{name}: heads must be contiguous (strides [*, dim, 1])")
    return t, S, H, D, t.stride(0) if S > 1 else H * D


def rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon=1e-6, rot_dim=None, rsqrt="hw", rstd_out=None):
    """In place on q and k; returns (q, k).  rope_freqs: [..., s, rot/2, 2, 2]
    bf16 (leading singleton dimensions allowed), or None with rot_dim 0."""
    q3, S, H, D, ldq = _rows(q, "q")
    k3, Sk, Hk, Dk, ldk = _rows(k, "k")
    if (Sk, Hk, Dk) != (S, H, D):
        raise ValueError("q and k must have the same [s, heads, dim]")
    if rot_dim is None:
        rot_dim = 0 if rope_freqs is None else rope_freqs.shape[-3] * 2
    tab = None
    if rot_dim:
        if rope_freqs is None or rope_freqs.dtype != torch.bfloat16 or not rope_freqs.is_cuda:
            raise ValueError("rope_freqs must be a bfloat16 GPU tensor")
        if tuple(rope_freqs.shape[-4:]) != (S, rot_dim // 2, 2, 2) or any(d != 1 for d in rope_freqs.shape[:-4]):
            raise ValueError(f"rope_freqs must be [.., {S}, {rot_dim // 2}, 2, 2]")
        tab = rope_freqs.contiguous()
    for w, name in ((qw, "qw"), (kw, "kw")):
        if w.dtype != torch.bfloat16 or not w.is_cuda or w.numel() != D or not w.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bfloat16 GPU tensor of {D} elements")
    if rstd_out is not None and (rstd_out.dtype != torch.float32 or rstd_out.numel() != S * 2 * H
                                 or not rstd_out.is_contiguous()):
        raise ValueError("rstd_out must be contiguous float32 with s * 2 * heads elements")
    same_gpu(q3, k=k3, rope_freqs=tab, qw=qw, kw=kw, rstd_out=rstd_out)
    check(lib.h3mi_rms_rope_split_half_bf16(ptr(q3), ptr(k3), ptr(tab) if tab is not None else None, ptr(qw), ptr(kw),
                                            S, H, D, ldq, ldk, rot_dim, float(epsilon), _MODES[rsqrt],
                                            ptr(rstd_out) if rstd_out is not None else None, stream_of(q3)))
    return q, k


def rms_rope_split_half(q, k, rope_freqs, qw, kw, epsilon=1e-6, rot_dim=None, rsqrt="hw"):
    """Out-of-place form (the reference's in_training branch): returns new (q, k)."""
    qo = q.contiguous().clone()
    ko = k.contiguous().clone()
    return rms_rope_split_half_(qo, ko, rope_freqs, qw, kw, epsilon, rot_dim, rsqrt)
