"""Fused RMSNorm + adaLN modulation + gate/residual (HIP, gfx950).

Same API as comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:
  norm_mod(x, w, eps, ridx, s1, sh) -> h                        (:174-178)
  gate_norm_mod_(x, o, g, w, eps, ridx, s1, sh) -> h, x updated (:181-185)
  gate_(x, o, g, ridx) -> x, updated in place                   (:188-192)
x, o, h: bf16 [S, N] contiguous; w: bf16 [N]; ridx: int32 [S] row -> table row;
s1, sh, g: bf16 [R, N] tables (s1 = 1 + scale already applied).

norm_mod_q / gate_norm_mod_q_ (no counterpart in the reference) also return h
quantized per token for the next W8A8 linear -- (q int8 [S, N], qs fp32
[S, 1]), bit-identical to quantize_rowwise(h) -- computed while the row is
still in registers, so h can skip its HBM round trip.
"""
import ctypes

import torch

from ._lib import ORDER_DEFAULT, RSQRT_HW, check, lib, ptr, same_gpu, stream_of

ORDER_NAMES = {"default": 0, "ref": 1, "w64": 2}


def order_info(order):
    """(numx, vec, warp) of a reduction order (int or name)."""
    o = ORDER_NAMES.get(order, order)
    a, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(lib.h3mi_norm_order_info(int(o), ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
    return a.value, b.value, c.value


def _rows(x):
    if x.dim() != 2 or x.dtype != torch.bfloat16 or not x.is_cuda or not x.is_contiguous():
        raise ValueError("x must be a contiguous 2-D bfloat16 GPU tensor")
    return x.shape


def _table(t, n, name):
    if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.numel() % n or t.numel() == 0:
        raise ValueError(f"{name} must be a contiguous bfloat16 [R, {n}] table")
    return t.numel() // n


def _ridx(ridx, s):
    if ridx.dtype != torch.int32 or ridx.numel() != s or not ridx.is_contiguous():
        raise ValueError("ridx must be contiguous int32 with one entry per row")


def _weight(w, n):
    if w.dtype != torch.bfloat16 or w.numel() != n or not w.is_contiguous():
        raise ValueError("w must be contiguous bfloat16 [N]")


def norm_mod_ex(x, w, eps, ridx, s1, sh, order=ORDER_DEFAULT, rsqrt_mode=RSQRT_HW, stats=False, h=None):
    """norm_mod with an explicit reduction order / rsqrt mode.  With stats=True
    returns (h, var, rstd) where var = sumsq/N + eps and rstd are fp32 [S]."""
    s, n = _rows(x)
    _weight(w, n)
    _ridx(ridx, s)
    r = _table(s1, n, "s1")
    if _table(sh, n, "sh") != r:
        raise ValueError("s1 and sh must have the same number of rows")
    if h is None:
        h = torch.empty_like(x)
    var = rstd = None
    if stats:
        var = torch.empty(s, dtype=torch.float32, device=x.device)
        rstd = torch.empty(s, dtype=torch.float32, device=x.device)
    same_gpu(x, w=w, ridx=ridx, s1=s1, sh=sh, h=h, var=var, rstd=rstd)
    check(lib.h3mi_norm_mod_bf16_ex(ptr(x), ptr(w), ptr(ridx), ptr(s1), ptr(sh), ptr(h), s, n, r, float(eps),
                                    int(ORDER_NAMES.get(order, order)), int(rsqrt_mode), ptr(var), ptr(rstd),
                                    stream_of(x)))
    return (h, var, rstd) if stats else h


def gate_norm_mod_ex(x, o, g, w, eps, ridx, s1, sh, order=ORDER_DEFAULT, rsqrt_mode=RSQRT_HW, stats=False, h=None):
    s, n = _rows(x)
    if o.shape != x.shape or o.dtype != torch.bfloat16 or not o.is_contiguous():
        raise ValueError("o must be contiguous bfloat16 like x")
    _weight(w, n)
    _ridx(ridx, s)
    r = _table(s1, n, "s1")
    if _table(sh, n, "sh") != r or _table(g, n, "g") != r:
        raise ValueError("g, s1 and sh must have the same number of rows")
    if h is None:
        h = torch.empty_like(x)
    var = rstd = None
    if stats:
        var = torch.empty(s, dtype=torch.float32, device=x.device)
        rstd = torch.empty(s, dtype=torch.float32, device=x.device)
    same_gpu(x, o=o, g=g, w=w, ridx=ridx, s1=s1, sh=sh, h=h, var=var, rstd=rstd)
    check(lib.h3mi_gate_norm_mod_bf16_ex(ptr(x), ptr(o), ptr(g), ptr(w), ptr(ridx), ptr(s1), ptr(sh), ptr(h),
                                         s, n, r, float(eps), int(ORDER_NAMES.get(order, order)), int(rsqrt_mode),
                                         ptr(var), ptr(rstd), stream_of(x)))
    return (h, var, rstd) if stats else h


def norm_mod(x, w, eps, ridx, s1, sh):
    s, n = _rows(x)
    _weight(w, n)
    _ridx(ridx, s)
    r = _table(s1, n, "s1")
    if _table(sh, n, "sh") != r:
        raise ValueError("s1 and sh must have the same number of rows")
    h = torch.empty_like(x)
    same_gpu(x, w=w, ridx=ridx, s1=s1, sh=sh)
    check(lib.h3mi_norm_mod_bf16(ptr(x), ptr(w), ptr(ridx), ptr(s1), ptr(sh), ptr(h), s, n, r, float(eps),
                                 stream_of(x)))
    return h


def gate_norm_mod_(x, o, g, w, eps, ridx, s1, sh):
    s, n = _rows(x)
    if o.shape != x.shape or o.dtype != torch.bfloat16 or not o.is_contiguous():
        raise ValueError("o must be contiguous bfloat16 like x")
    _weight(w, n)
    _ridx(ridx, s)
    r = _table(s1, n, "s1")
    if _table(sh, n, "sh") != r or _table(g, n, "g") != r:
        raise ValueError("g, s1 and sh must have the same number of rows")
    h = torch.empty_like(x)
    same_gpu(x, o=o, g=g, w=w, ridx=ridx, s1=s1, sh=sh)
    check(lib.h3mi_gate_norm_mod_bf16(ptr(x), ptr(o), ptr(g), ptr(w), ptr(ridx), ptr(s1), ptr(sh), ptr(h),
                                      s, n, r, float(eps), stream_of(x)))
    return h


def gate_(x, o, g, ridx):
    s, n = _rows(x)
    if o.shape != x.shape or o.dtype != torch.bfloat16 or not o.is_contiguous():
        raise ValueError("o must be contiguous bfloat16 like x")
    _ridx(ridx, s)
    r = _table(g, n, "g")
    same_gpu(x, o=o, g=g, ridx=ridx)
    check(lib.h3mi_gate_bf16(ptr(x), ptr(o), ptr(g), ptr(ridx), s, n, r, stream_of(x)))
    return x


def _fused_ok(n):
    return n % 8 == 0 and n <= 8192


def norm_mod_q(x, w, eps, ridx, s1, sh, want_h=False):
    """norm_mod with the per-token quantizer of h fused in.  Returns (q, qs),
    or (h, q, qs) with want_h.  Rows the fused kernel does not take (N % 8 != 0
    or N > 8192) run norm_mod then quantize_rowwise."""
    s, n = _rows(x)
    _weight(w, n)
    _ridx(ridx, s)
    r = _table(s1, n, "s1")
    if _table(sh, n, "sh") != r:
        raise ValueError("s1 and sh must have the same number of rows")
    if not _fused_ok(n):
        from .quant import quantize_rowwise
        h = norm_mod(x, w, eps, ridx, s1, sh)
        q, qs = quantize_rowwise(h)
        return (h, q, qs) if want_h else (q, qs)
    h = torch.empty_like(x) if want_h else None
    q = torch.empty((s, n), dtype=torch.int8, device=x.device)
    qs = torch.empty((s, 1), dtype=torch.float32, device=x.device)
    same_gpu(x, w=w, ridx=ridx, s1=s1, sh=sh)
    check(lib.h3mi_norm_mod_quant_i8(ptr(x), ptr(w), ptr(ridx), ptr(s1), ptr(sh), ptr(h), ptr(q), ptr(qs), s, n, r,
                                     float(eps), stream_of(x)))
    return (h, q, qs) if want_h else (q, qs)


def gate_norm_mod_q_(x, o, g, w, eps, ridx, s1, sh, want_h=False):
    """gate_norm_mod_ (x updated in place) with the per-token quantizer of h
    fused in.  Returns (q, qs), or (h, q, qs) with want_h."""
    s, n = _rows(x)
    if o.shape != x.shape or o.dtype != torch.bfloat16 or not o.is_contiguous():
        raise ValueError("o must be contiguous bfloat16 like x")
    _weight(w, n)
    _ridx(ridx, s)
    r = _table(s1, n, "s1")
    if _table(sh, n, "sh") != r or _table(g, n, "g") != r:
        raise ValueError("g, s1 and sh must have the same number of rows")
    if not _fused_ok(n):
        from .quant import quantize_rowwise
        h = gate_norm_mod_(x, o, g, w, eps, ridx, s1, sh)
        q, qs = quantize_rowwise(h)
        return (h, q, qs) if want_h else (q, qs)
    h = torch.empty_like(x) if want_h else None
    q = torch.empty((s, n), dtype=torch.int8, device=x.device)
    qs = torch.empty((s, 1), dtype=torch.float32, device=x.device)
    same_gpu(x, o=o, g=g, w=w, ridx=ridx, s1=s1, sh=sh)
    check(lib.h3mi_gate_norm_mod_quant_i8(ptr(x), ptr(o), ptr(g), ptr(w), ptr(ridx), ptr(s1), ptr(sh), ptr(h), ptr(q),
                                          ptr(qs), s, n, r, float(eps), stream_of(x)))
    return (h, q, qs) if want_h else (q, qs)
