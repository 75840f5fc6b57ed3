"""Replace the H3 DiTBlock.forward with one that runs the fused MI355X kernels.

Counterpart of comfyui_nodes/h3-fuse-graph/h3_fuse_patch.py (enabled :22-23,
_fallback :26-29, _row_index :32-56, _norm_weight/_Plain :59-75, install :78-149,
_AfterImport/after_import :152-184).

Enabled only with H3_FUSE=1.  The replacement computes the same values in the
same order as the original block: the RMSNorm, adaLN modulation, gate and
residual steps become three HIP kernels (norm_mod, gate_norm_mod_, gate_);
attention and the MLP are called unchanged.  Calls that do not fit (not a 2-D
contiguous bf16 GPU tensor, grad enabled, segments that do not tile the rows,
non-bf16 norm weights) run the original forward.

Environment:
  H3_FUSE=1          enable
  H3_FUSE_TARGET     module that defines DiTBlock (comfy.ldm.minimax.model)
  H3_FUSE_QUANT=1    also quantize h per token inside the norm kernels and
                     offer it (h3mi.prequant) to the INT8 linear that opens the
                     attention / MLP call, which then skips its own quantizer
                     (same bytes; not in the reference; off by default)
  H3_FUSE_ROPE=1     also replace comfy-kitchen's q/k RMSNorm + RoPE
                     (h3_rope_patch.py; not in the reference; off by default)
"""
import functools
import importlib
import importlib.abc
import importlib.machinery
import logging
import os
import sys

import torch

log = logging.getLogger("h3-fuse-graph")
_HERE = os.path.dirname(os.path.abspath(__file__))
_state = {"installed": False, "fused": 0, "fallback": 0, "ridx_key": None, "ridx": None, "disabled": False}
TARGET = os.environ.get("H3_FUSE_TARGET", "comfy.ldm.minimax.model")


def enabled():
    return os.environ.get("H3_FUSE", "0") == "1"


def _quant_handoff():
    return os.environ.get("H3_FUSE_QUANT", "0") == "1"


def _fallback(reason):
    _state["fallback"] += 1
    if _state["fallback"] <= 5:
        log.warning("[h3-fuse] original forward: %s", reason)


def _row_index(mod_segments, s, device):
    """mod_segments, a sequence of (start, stop, row) where row is an int or a
    per-row LongTensor, -> int32 [s] table-row index per token row, or None when
    the segments do not tile [0, s) exactly.  The result for the last list seen
    is cached (every block of one forward passes the same list; the cache keeps
    a reference so the id cannot be reused)."""
    key = _state["ridx_key"]
    if key is not None and key[0] is mod_segments and key[1] == s and key[2] == device:
        return _state["ridx"]
    segs = sorted(((a, b, row) for a, b, row in mod_segments), key=lambda t: t[0])
    pos = 0
    for a, b, row in segs:
        if a != pos or b < a:
            return None
        if torch.is_tensor(row) and row.numel() != b - a:
            return None
        pos = b
    if pos != s:
        return None
    host = torch.empty(s, dtype=torch.int32)
    dev_parts = []
    for a, b, row in segs:
        if torch.is_tensor(row):
            if row.device.type == "cpu":
                host[a:b] = row.to(torch.int32)
            else:
                dev_parts.append((a, b, row))
        else:
            host[a:b] = int(row)
    r = host.to(device)
    for a, b, row in dev_parts:
        r[a:b] = row.to(device=device, dtype=torch.int32)
    _state["ridx_key"] = (mod_segments, s, device)
    _state["ridx"] = r
    return r


class _Plain:
    """Context manager yielding (weight, None) for an uncast norm weight."""

    def __init__(self, w):
        self.w = w

    def __enter__(self):
        return self.w, None

    def __exit__(self, *a):
        return False


def _norm_weight(norm, x):
    """The norm weight as the upstream RMSNorm.forward obtains it: through the
    cast/patch-aware context when casting or weight/bias functions apply,
    otherwise the parameter itself."""
    needs_cast = (getattr(norm, "comfy_cast_weights", False) or len(getattr(norm, "weight_function", ())) > 0
                  or len(getattr(norm, "bias_function", ())) > 0)
    if needs_cast and hasattr(norm, "cast_weight"):
        return norm.cast_weight(x)
    return _Plain(norm.weight)


def install():
    if _state["installed"] or not enabled():
        return _state["installed"]
    try:
        mm = importlib.import_module(TARGET)
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-fuse] cannot import %s; disabled: %s", TARGET, e)
        return False
    try:
        ops = importlib.import_module("comfy.ops")
    except Exception:  # noqa: BLE001
        ops = None
    if _HERE not in sys.path:
        sys.path.append(_HERE)
    try:
        import h3_fuse_kernels as fk
        from h3mi import prequant
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-fuse] HIP library unavailable; disabled: %s", e)
        return False

    orig = mm.DiTBlock.forward
    run_every_op = getattr(ops, "run_every_op", None) if ops is not None else None
    bf16 = torch.bfloat16

    @functools.wraps(orig)
    def forward(self, x, t_emb, mod_segments, rope_freqs, transformer_options={}, attention=None):  # noqa: B006
        def original(reason):
            _fallback(reason)
            return orig(self, x, t_emb, mod_segments, rope_freqs, transformer_options=transformer_options,
                        attention=attention)

        n1, n2 = self.norm1, self.norm2
        s = x.shape[0] if x.dim() == 2 else 0
        ok = (not _state["disabled"] and x.dim() == 2 and x.is_cuda and x.dtype == bf16 and x.is_contiguous()
              and x.data_ptr() % 16 == 0 and x.shape[1] % 4 == 0 and n1.eps is not None and n2.eps is not None
              and tuple(n1.normalized_shape) == (x.shape[1],) and tuple(n2.normalized_shape) == (x.shape[1],)
              and not torch.is_grad_enabled())
        if not ok:
            return original(f"x={tuple(x.shape)} {x.dtype} contiguous={x.is_contiguous()} "
                            f"grad={torch.is_grad_enabled()} disabled={_state['disabled']}")
        ridx = _row_index(mod_segments, s, x.device)
        if ridx is None:
            return original("mod_segments do not tile the rows exactly")
        handoff = _quant_handoff() and x.shape[1] % 8 == 0  # the per-token quantizer's row rule
        attn = self.attn if attention is None else attention
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = self.adaln_proj(t_emb)
        # the upstream modulation takes vecs[row].to(dtype) and 1.0 + that value
        # in bf16; build whole tables with the same operations
        s1a = (1.0 + scale_msa.to(bf16)).contiguous()
        sha = shift_msa.to(bf16).contiguous()
        ga = gate_msa.to(bf16).contiguous()
        s1m = (1.0 + scale_mlp.to(bf16)).contiguous()
        shm = shift_mlp.to(bf16).contiguous()
        gm = gate_mlp.to(bf16).contiguous()
        if run_every_op is not None:
            run_every_op()
        with _norm_weight(n1, x) as (w1, _):
            if w1 is None or w1.dtype != bf16 or not w1.is_contiguous():
                return original(f"norm1 weight {None if w1 is None else w1.dtype}")
            try:
                if handoff:
                    h, q, qs = fk.norm_mod_q(x, w1, float(n1.eps), ridx, s1a, sha, want_h=True)
                else:
                    h = fk.norm_mod(x, w1, float(n1.eps), ridx, s1a, sha)
            except Exception as e:  # noqa: BLE001  (nothing has been modified yet)
                _state["disabled"] = True
                log.warning("[h3-fuse] HIP kernel failed; original forward from now on: %s", e)
                return original("kernel error")
        if handoff:
            with prequant.offer(h, q, qs):
                o = attn(h, rope_freqs=rope_freqs, transformer_options=transformer_options)
            del q, qs
        else:
            o = attn(h, rope_freqs=rope_freqs, transformer_options=transformer_options)
        del h
        if not o.is_contiguous():
            o = o.contiguous()
        if run_every_op is not None:
            run_every_op()
        with _norm_weight(n2, x) as (w2, _):
            if handoff:
                h, q, qs = fk.gate_norm_mod_q_(x, o, ga, w2, float(n2.eps), ridx, s1m, shm, want_h=True)
            else:
                h = fk.gate_norm_mod_(x, o, ga, w2, float(n2.eps), ridx, s1m, shm)
        del o
        if handoff:
            with prequant.offer(h, q, qs):
                o = self.mlp(h)
            del q, qs
        else:
            o = self.mlp(h)
        del h
        if not o.is_contiguous():
            o = o.contiguous()
        fk.gate_(x, o, gm, ridx)
        _state["fused"] += 1
        if _state["fused"] in (1, 1000, 10000):
            log.warning("[h3-fuse] fused forward %d (original %d)", _state["fused"], _state["fallback"])
        return x

    forward._h3_fuse_orig = orig
    mm.DiTBlock.forward = forward
    _state["installed"] = True
    _state["module"] = mm
    log.warning("[h3-fuse] %s.DiTBlock.forward replaced by the fused MI355X version", TARGET)
    try:
        import h3_rope_patch
        h3_rope_patch.install()  # a no-op unless H3_FUSE_ROPE=1
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-fuse] q/k norm + RoPE patch not installed: %s", e)
    return True


def uninstall():
    """Restore the original forward (not in the reference; used by tests)."""
    if not _state["installed"]:
        return
    mm = _state["module"]
    mm.DiTBlock.forward = mm.DiTBlock.forward._h3_fuse_orig
    _state["installed"] = False


def stats():
    return {k: _state[k] for k in ("installed", "fused", "fallback", "disabled")}


class _AfterImport(importlib.abc.MetaPathFinder):
    """Calls fn(module) right after the first module whose name matches has
    been executed (used by worker launchers)."""

    def __init__(self, match, fn):
        self.match = match
        self.fn = fn

    def find_spec(self, name, path=None, target=None):
        if not self.match(name):
            return None
        sys.meta_path.remove(self)
        try:
            spec = importlib.machinery.PathFinder.find_spec(name, path)
        finally:
            sys.meta_path.insert(0, self)
        if spec is None or spec.loader is None:
            return spec
        inner = spec.loader.exec_module
        fn = self.fn
        me = self

        def exec_module(module):
            inner(module)
            if me in sys.meta_path:
                sys.meta_path.remove(me)
            fn(module)

        spec.loader.exec_module = exec_module
        return spec


def after_import(match, fn):
    sys.meta_path.insert(0, _AfterImport(match, fn))
