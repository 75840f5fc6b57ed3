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
                     (same bytes; not in the reference; off by default; rows
                     of at most 8192 elements, a multiple of 8)
  H3_FUSE_ROPE=1     also replace comfy-kitchen's q/k RMSNorm + RoPE
                     (h3_rope_patch.py; not in the reference; off by default)

Errors: a kernel call rejected for its arguments (ValueError, H3miError
EINVAL / EALIGN / EALIAS; nothing has been written then) runs the original
forward for that call, or, for the quantizing second norm, the plain fused
norm; any other failure in the first norm disables the fused block for the
process.
"""
import functools
import importlib
import logging
import os
import sys

import torch

log = logging.getLogger("h3-fuse-graph")
_HERE = os.path.dirname(os.path.abspath(__file__))
_state = {"installed": False, "fused": 0, "fallback": 0, "disabled": False}
TARGET = os.environ.get("H3_FUSE_TARGET", "comfy.ldm.minimax.model")


def enabled():
    return os.environ.get("H3_FUSE", "0") == "1"


def _quant_handoff():
    return os.environ.get("H3_FUSE_QUANT", "0") == "1"


def _argument_error(e):
    """True for a rejection of a kernel call's arguments, raised before any
    launch (that call falls back), False for a failure that disables the block."""
    from h3mi import _lib as L
    if isinstance(e, L.H3miError):
        return e.code in (L.EINVAL, L.EALIGN, L.EALIAS)
    return isinstance(e, (ValueError, TypeError))


def _fits(x, n1, n2):
    """The reference's gate for the fused forward (FG/h3_fuse_patch.py:98-101):
    a 2-D contiguous, 16-byte aligned bf16 GPU tensor whose width (a multiple
    of 4) both norms normalise, with epsilons set and no autograd."""
    return (x.dim() == 2 and x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.data_ptr() % 16 == 0
            and x.shape[1] % 4 == 0 and n1.eps is not None and n2.eps is not None
            and tuple(n1.normalized_shape) == (x.shape[1],) and tuple(n2.normalized_shape) == (x.shape[1],)
            and not torch.is_grad_enabled())


def _handoff_fits(n):
    """Rows the fused norm -> quantizer kernels take: a multiple of 8 elements,
    at most 8192 (h3mi_norm_mod_quant_i8 rejects anything else)."""
    return n % 8 == 0 and 0 < n <= 8192


def _fallback(reason):
    _state["fallback"] += 1
    if _state["fallback"] <= 5:
        log.warning("[h3-fuse] original forward: %s", reason)


def _segment_plan(mod_segments, s):
    """The (start, stop, row) triples sorted by start when they tile [0, s)
    exactly -- contiguous, non-negative lengths, a per-row tensor as long as
    its segment -- else None."""
    plan = sorted(mod_segments, key=lambda seg: seg[0])
    if not plan:
        return plan if s == 0 else None
    starts = [a for a, _, _ in plan]
    stops = [b for _, b, _ in plan]
    if starts[0] != 0 or stops[-1] != s or starts[1:] != stops[:-1]:
        return None
    for a, b, row in plan:
        if b < a or (torch.is_tensor(row) and row.numel() != b - a):
            return None
    return plan


def _segments_key(mod_segments, s, device):
    """Content key of a segment list: ints by value, per-row tensors by
    identity and version (an in-place change invalidates the entry)."""
    parts = []
    for a, b, row in mod_segments:
        parts.append((a, b, ("t", id(row), row._version) if torch.is_tensor(row) else int(row)))
    return (tuple(parts), s, str(device))


class _RowIndexCache:
    """Table-row index per token row, built once per distinct segment list.
    Every block of a forward passes the same segments, so one hit per block
    after the first; two entries cover alternating conditional / unconditional
    passes.  Entries hold the segment tensors, so their ids stay unique."""

    def __init__(self, size=2):
        self.size = size
        self.entries = []  # [(key, tensors kept alive, index)]

    def get(self, mod_segments, s, device):
        key = _segments_key(mod_segments, s, device)
        for i, (k, _, idx) in enumerate(self.entries):
            if k == key:
                self.entries.insert(0, self.entries.pop(i))
                return idx
        plan = _segment_plan(mod_segments, s)
        if plan is None:
            return None
        idx = self._build(plan, s, device)
        keep = [row for _, _, row in plan if torch.is_tensor(row)]
        self.entries.insert(0, (key, keep, idx))
        del self.entries[self.size:]
        return idx

    @staticmethod
    def _build(plan, s, device):
        # int rows: one repeat_interleave on the host, one copy to the device;
        # tensor rows are then written in place (on their own device)
        lengths = torch.tensor([b - a for a, b, _ in plan], dtype=torch.int64)
        ids = torch.tensor([0 if torch.is_tensor(r) else int(r) for _, _, r in plan], dtype=torch.int32)
        idx = torch.repeat_interleave(ids, lengths)
        for a, b, row in plan:
            if torch.is_tensor(row) and row.device.type == "cpu":
                idx[a:b] = row.to(torch.int32)
        idx = idx.to(device)
        for a, b, row in plan:
            if torch.is_tensor(row) and row.device.type != "cpu":
                idx[a:b] = row.to(device=device, dtype=torch.int32)
        return idx


_ridx_cache = _RowIndexCache()


def _row_index(mod_segments, s, device):
    """mod_segments, (start, stop, row) with row an int or a per-row
    LongTensor -> int32 [s] table-row index, or None when the segments do not
    tile the rows exactly (reference: FG/h3_fuse_patch.py:32-56)."""
    return _ridx_cache.get(mod_segments, s, device)


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
        ok = not _state["disabled"] and _fits(x, n1, n2)
        if not ok:
            return original(f"x={tuple(x.shape)} {x.dtype} contiguous={x.is_contiguous()} "
                            f"grad={torch.is_grad_enabled()} disabled={_state['disabled']}")
        ridx = _row_index(mod_segments, s, x.device)
        if ridx is None:
            return original("mod_segments do not tile the rows exactly")
        handoff = _quant_handoff() and _handoff_fits(x.shape[1])
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
                if _argument_error(e):
                    return original(f"arguments rejected: {e}")
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
                try:
                    h, q, qs = fk.gate_norm_mod_q_(x, o, ga, w2, float(n2.eps), ridx, s1m, shm, want_h=True)
                except Exception as e:  # noqa: BLE001
                    if not _argument_error(e):
                        raise
                    # rejected before any launch, so x is unchanged: the plain fused norm, no hand-off
                    log.warning("[h3-fuse] quantizing norm rejected its arguments; plain norm: %s", e)
                    handoff = False
            if not handoff:
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


def after_import(match, fn):
    """Call fn(module) right after the first module whose name satisfies
    match(name) has been imported (worker launchers; reference
    FG/h3_fuse_patch.py:183-184).  Implemented by h3_import_hooks."""
    import _h3mi_path
    _h3mi_path.ensure()
    import h3_import_hooks
    h3_import_hooks.after_import(match, fn)
