"""W8A8 GEMM with fused dequant epilogue (HIP, gfx950).

Same API as comfyui_nodes/h3-linear-fast/int8_gemm_triton.py:
  int8_mm_scaled(xq, w, xs, ws, out=None)   (:74-83)
  supported(K)                               (:86-87)
  _int8_mm_scaled_kernel.best_config         (read by tests/test_triton_gemm.py:24)

Tile configurations: a measured heuristic picks one per shape (config_for).
H3_LINEAR_FAST_CFG pins one, as the reference's _FIXED does (:24-27):
  * a configuration name of this library (list_configs()) forces it;
  * the reference's own format "BM,BN,BK,stages,warps" names a Triton tile
    that has no counterpart among the MFMA tilings here; the pin's purpose
    there is to skip autotuning, which the heuristic never runs, so such a
    value keeps the heuristic and logs one warning;
  * anything else logs one warning and keeps the heuristic.
  A pin of either kind turns H3_LINEAR_FAST_ALLCFG off, as in the reference.
  Import never fails on the value; fixed_config_note() says what happened.
H3_LINEAR_FAST_ALLCFG=1 autotunes instead, as the reference's autotune over
its wider candidate list does (:11-21, 69-71): the first call per
(N, K, ceil(M / 4096)) times every configuration on the caller's operands and
keeps the fastest.  Every configuration gives the same bytes, so tuning never
changes a result.  A forced configuration (set_config, the pin, a tuned call)
is process-wide: a GEMM another thread launches meanwhile runs under it, which
can change its speed, never its bytes (a configuration whose K multiple does not
divide the call's K is ignored for that call).
"""
import ctypes
import logging
import os
import re

import torch

from ._lib import H3miError, check, lib, ptr, same_gpu, stream_of

log = logging.getLogger("h3mi")


class _KernelInfo:
    """Stand-in for the autotuned kernel object: best_config names the tile
    configuration the last call used.  It is looked up when read, not on every
    call (a ctypes round trip per GEMM launch otherwise)."""

    def __init__(self):
        self._shape = None  # (M, N, K) of the last call that took the heuristic
        self._name = None   # the configuration an autotuned call used

    def _record(self, shape=None, name=None):
        self._shape, self._name = shape, name

    @property
    def best_config(self):
        if self._name is not None:
            return self._name
        return config_for(*self._shape) if self._shape is not None else None

    def __repr__(self):
        return f"h3mi w8a8 kernel (best_config={self.best_config!r})"


_int8_mm_scaled_kernel = _KernelInfo()


def supported(K):
    return bool(lib.h3mi_w8a8_supported(int(K)))


def config_for(M, N, K):
    buf = ctypes.create_string_buffer(64)
    check(lib.h3mi_w8a8_config(int(M), int(N), int(K), buf, 64))
    return buf.value.decode()


def list_configs():
    """Names of every tile configuration the library carries."""
    names, buf = [], ctypes.create_string_buffer(64)
    while lib.h3mi_w8a8_config_name(len(names), buf, 64) == 0:
        names.append(buf.value.decode())
    return names


def set_config(name):
    """Force a tile configuration by name; "auto" restores the heuristic."""
    check(lib.h3mi_w8a8_set_config(name.encode()))


_TRITON_TILE = re.compile(r"^\s*\d+\s*(,\s*\d+\s*){4}$")  # BM,BN,BK,stages,warps


def _apply_fixed(value):
    """Apply an H3_LINEAR_FAST_CFG value; returns None when a configuration
    was pinned (or the value is empty / "auto"), else the reason it was not."""
    if not value or value.strip() == "auto":
        return None
    if _TRITON_TILE.match(value):
        return (f"H3_LINEAR_FAST_CFG={value!r} is a Triton tile (BM,BN,BK,stages,warps) with no counterpart among "
                f"this library's MFMA tilings; the per-shape heuristic stays in use (autotuning stays off)")
    try:
        set_config(value.strip())
    except H3miError:
        return (f"H3_LINEAR_FAST_CFG={value!r} names no tile configuration of this library (known: "
                f"{', '.join(list_configs())}); the per-shape heuristic stays in use")
    return None


_FIXED = os.environ.get("H3_LINEAR_FAST_CFG")
_FIXED_NOTE = _apply_fixed(_FIXED)
if _FIXED_NOTE:
    log.warning("[h3mi] %s", _FIXED_NOTE)


def fixed_config_note():
    """Why the H3_LINEAR_FAST_CFG value seen at import pinned nothing (None when
    it pinned a configuration or was unset)."""
    return _FIXED_NOTE


_TUNED = {}  # (N, K, M bucket) -> configuration name


def _autotune():
    return os.environ.get("H3_LINEAR_FAST_ALLCFG") == "1" and not _FIXED


def _tune(key, launch, device):
    """Time launch() under every configuration (HIP events, 1 warm-up + 3 timed) and cache the fastest for key."""
    best, best_ms = None, float("inf")
    try:
        for name in list_configs():
            set_config(name)
            launch()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(3):
                launch()
            b.record()
            torch.cuda.synchronize(device)
            ms = a.elapsed_time(b)
            if ms < best_ms:
                best, best_ms = name, ms
    finally:
        set_config("auto")
    _TUNED[key] = best
    return best


def _check_operands(xq, w):
    if xq.dim() != 2 or w.dim() != 2:
        raise ValueError("xq and w must be 2-D")
    M, K = xq.shape
    N = w.shape[0]
    assert w.shape[1] == K and xq.is_contiguous() and w.is_contiguous()
    if xq.dtype != torch.int8 or w.dtype != torch.int8:
        raise TypeError("xq and w must be int8")
    if not (xq.is_cuda and w.is_cuda) or xq.device != w.device:
        raise ValueError("xq and w must be on the same GPU")
    return M, N, K


def int8_mm_scaled(xq, w, xs, ws, out=None, bias=None):
    """xq [M,K] int8, w [N,K] int8, xs [M,1] fp32, ws [N] fp32 -> [M,N] bf16.

    out[m,n] = bf16((f32(sum_k xq[m,k]*w[n,k]) * xs[m]) * ws[n])
    (+ bias[n] in fp32 before the rounding when bias, bf16 [N], is given)."""
    M, N, K = _check_operands(xq, w)
    if xs.dtype != torch.float32 or xs.numel() != M or not xs.is_contiguous():
        raise ValueError("xs must be contiguous float32 with M elements")
    if ws.dtype != torch.float32 or ws.numel() != N or not ws.is_contiguous():
        raise ValueError("ws must be contiguous float32 with N elements")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.numel() != N or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous bfloat16 with N elements")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=xq.device)
    elif out.dtype != torch.bfloat16 or out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be bfloat16 [M, N] with unit column stride")
    same_gpu(xq, xs=xs, ws=ws, bias=bias, out=out)

    def launch():
        check(lib.h3mi_w8a8_gemm_bf16(ptr(xq), ptr(w), ptr(xs), ptr(ws), ptr(bias), ptr(out),
                                      M, N, K, xq.stride(0), w.stride(0), out.stride(0), stream_of(xq)))

    if _autotune() and M > 0 and N > 0:
        key = (N, K, -(-M // 4096))
        name = _TUNED.get(key)
        if name is None and not torch.cuda.is_current_stream_capturing():
            name = _tune(key, launch, xq.device)
        if name is not None:
            set_config(name)
            try:
                _int8_mm_scaled_kernel._record(name=name)
                launch()
            finally:
                set_config("auto")
            return out
    _int8_mm_scaled_kernel._record(shape=(M, N, K))
    launch()
    return out


def int8_mm_i32(xq, w, out=None):
    """The int32 accumulators sum_k xq[m,k]*w[n,k] of the same GEMM ([M,N] int32)."""
    M, N, K = _check_operands(xq, w)
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32, device=xq.device)
    elif out.dtype != torch.int32 or out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be int32 [M, N] with unit column stride")
    same_gpu(xq, out=out)
    check(lib.h3mi_w8a8_gemm_i32(ptr(xq), ptr(w), ptr(out), M, N, K, xq.stride(0), w.stride(0),
                                 out.stride(0), stream_of(xq)))
    return out
