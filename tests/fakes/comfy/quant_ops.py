"""Stand-in for comfy.quant_ops (tests only): `ck` holds eager
rms_rope_split_half_ / rms_rope_split_half with the call signature the
reference uses (comfyui_nodes/minimax-h3-sp/minimax_sp/sp_forward.py:289-293):
F.rms_norm of each (token, head) row, then the split-half rotation by the
token's 2 x 2 table entries in separate fp32 ops, rounded to bf16."""
import types

import torch
import torch.nn.functional as F

CALLS = {"rms_rope_split_half_": 0, "rms_rope_split_half": 0}


def _apply(x, w, tab, rot, eps):
    shape = x.shape
    x3 = x.reshape(shape[-3], shape[-2], shape[-1])
    s, h, d = x3.shape
    y = F.rms_norm(x3.reshape(s * h, d), (d,), w, eps).reshape(s, h, d).float()
    out = y.clone()
    if rot:
        R = tab.reshape(s, rot // 2, 2, 2).float()[:, None]
        a, b = y[..., :rot // 2], y[..., rot // 2:rot]
        out[..., :rot // 2] = (R[..., 0, 0] * a) + (R[..., 0, 1] * b)
        out[..., rot // 2:rot] = (R[..., 1, 0] * a) + (R[..., 1, 1] * b)
    return out.to(x.dtype).reshape(shape)


def rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon=1e-6, rot_dim=None):
    CALLS["rms_rope_split_half_"] += 1
    rot = rot_dim if rot_dim is not None else rope_freqs.shape[-3] * 2
    q.copy_(_apply(q, qw, rope_freqs, rot, epsilon))
    k.copy_(_apply(k, kw, rope_freqs, rot, epsilon))
    return q, k


def rms_rope_split_half(q, k, rope_freqs, qw, kw, epsilon=1e-6, rot_dim=None):
    CALLS["rms_rope_split_half"] += 1
    rot = rot_dim if rot_dim is not None else rope_freqs.shape[-3] * 2
    return _apply(q, qw, rope_freqs, rot, epsilon), _apply(k, kw, rope_freqs, rot, epsilon)


ck = types.SimpleNamespace(rms_rope_split_half_=rms_rope_split_half_, rms_rope_split_half=rms_rope_split_half)
