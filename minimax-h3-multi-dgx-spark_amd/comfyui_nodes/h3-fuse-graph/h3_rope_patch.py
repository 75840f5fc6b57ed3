"""Replace comfy-kitchen's q/k RMSNorm + split-half RoPE with the MI355X kernel.

The reference's attention calls comfy.quant_ops.ck.rms_rope_split_half_(q, k,
rope_freqs, qw, kw, epsilon=attn.q_norm.eps, rot_dim=rope_freqs.shape[-3] * 2)
on the [1, s, heads, dim] views of the qkv projection, and the out-of-place
rms_rope_split_half in its training branch
(comfyui_nodes/minimax-h3-sp/minimax_sp/sp_forward.py:279-296).  comfy-kitchen's
kernel is a CUDA extension; this patch points both names at h3mi.rope, which
computes the eager sequence the fused call stands for (F.rms_norm of each
head row, then the split-half rotation in fp32).  Calls it does not take go to
the original; a kernel error disables it for the rest of the process.
Not in the reference (which has no such patch); off by default.

Environment:
  H3_FUSE_ROPE=1     enable (also installed by h3_fuse_patch.install())
  H3_ROPE_TARGET     module whose `ck` attribute holds the functions
                     (comfy.quant_ops)
"""
import importlib
import logging
import os

import torch

log = logging.getLogger("h3-fuse-rope")
_state = {"installed": False, "fast_calls": 0, "fallback_calls": 0, "disabled": False, "ck": None, "orig": None}
TARGET = os.environ.get("H3_ROPE_TARGET", "comfy.quant_ops")


def enabled():
    return os.environ.get("H3_FUSE_ROPE", "0") == "1"


def eligible(q, k, rope_freqs, qw, kw, rot):
    """Whether the kernel takes the call: bf16 GPU [1, s, heads, dim] (or
    [s, heads, dim]) q and k of one shape with contiguous heads, 16-byte
    aligned, token strides a multiple of 8; dim 64 / 128 / 256; rot a multiple
    of 16 up to dim with a bf16 [.., s, rot/2, 2, 2] table; bf16 [dim] weights;
    no autograd."""
    bf16 = torch.bfloat16
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad):
        return False
    for t in (q, k):
        if not (t.is_cuda and t.dtype == bf16 and t.dim() in (3, 4)) or (t.dim() == 4 and t.shape[0] != 1):
            return False
    if q.shape != k.shape:
        return False
    s, h, d = q.shape[-3:]
    if d not in (64, 128, 256) or rot is None or rot % 16 or not 0 <= rot <= d:
        return False
    for t in (q, k):
        if t.stride(-1) != 1 or (h > 1 and t.stride(-2) != d) or (s > 1 and t.stride(-3) % 8) or t.data_ptr() % 16:
            return False
    for w in (qw, kw):
        if not (w.is_cuda and w.dtype == bf16 and w.numel() == d and w.is_contiguous() and w.data_ptr() % 16 == 0):
            return False
    if rot:
        if rope_freqs is None or not (rope_freqs.is_cuda and rope_freqs.dtype == bf16):
            return False
        if tuple(rope_freqs.shape[-4:]) != (s, rot // 2, 2, 2) or any(x != 1 for x in rope_freqs.shape[:-4]):
            return False
    return True


def install():
    if _state["installed"]:
        return True
    if not enabled():
        return False
    try:
        mod = importlib.import_module(TARGET)
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-fuse-rope] cannot import %s; disabled: %s", TARGET, e)
        return False
    ck = getattr(mod, "ck", None)
    if ck is None or not hasattr(ck, "rms_rope_split_half_"):
        log.warning("[h3-fuse-rope] %s.ck has no rms_rope_split_half_; disabled", TARGET)
        return False
    try:
        from h3mi import rope
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-fuse-rope] HIP library unavailable; disabled: %s", e)
        return False
    orig_ = ck.rms_rope_split_half_
    orig = getattr(ck, "rms_rope_split_half", None)

    def run(inplace, q, k, rope_freqs, qw, kw, epsilon, rot_dim, extra):
        original = orig_ if inplace else orig
        rot = rot_dim if rot_dim is not None else (rope_freqs.shape[-3] * 2 if rope_freqs is not None else 0)
        if _state["disabled"] or extra or not eligible(q, k, rope_freqs, qw, kw, rot):
            _state["fallback_calls"] += 1
            if _state["fallback_calls"] <= 5:
                log.warning("[h3-fuse-rope] original path: q=%s rot=%s", tuple(q.shape), rot)
            return original(q, k, rope_freqs, qw, kw, epsilon=epsilon, rot_dim=rot_dim, **extra)
        try:
            fn = rope.rms_rope_split_half_ if inplace else rope.rms_rope_split_half
            out = fn(q, k, rope_freqs, qw, kw, float(epsilon), rot)
        except Exception as e:  # noqa: BLE001  (argument errors are raised before anything is written)
            _state["disabled"] = True
            log.warning("[h3-fuse-rope] HIP kernel failed; original path from now on: %s", e)
            return original(q, k, rope_freqs, qw, kw, epsilon=epsilon, rot_dim=rot_dim, **extra)
        _state["fast_calls"] += 1
        return out

    def rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon=1e-6, rot_dim=None, **extra):
        return run(True, q, k, rope_freqs, qw, kw, epsilon, rot_dim, extra)

    def rms_rope_split_half(q, k, rope_freqs, qw, kw, epsilon=1e-6, rot_dim=None, **extra):
        return run(False, q, k, rope_freqs, qw, kw, epsilon, rot_dim, extra)

    ck.rms_rope_split_half_ = rms_rope_split_half_
    if orig is not None:
        ck.rms_rope_split_half = rms_rope_split_half
    _state.update(installed=True, ck=ck, orig=(orig_, orig))
    log.warning("[h3-fuse-rope] %s.ck.rms_rope_split_half_ -> MI355X HIP kernel", TARGET)
    return True


def uninstall():
    if not _state["installed"]:
        return
    ck, (orig_, orig) = _state["ck"], _state["orig"]
    ck.rms_rope_split_half_ = orig_
    if orig is not None:
        ck.rms_rope_split_half = orig
    _state["installed"] = False


def stats():
    return {k: _state[k] for k in ("installed", "fast_calls", "fallback_calls", "disabled")}
