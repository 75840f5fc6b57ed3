"""Optional timing / torch.profiler hook around whole H3 forwards.

Counterpart of comfyui_nodes/h3-fuse-graph/h3_fg_profile.py (:16-83).  Active
only when H3_FG_PROFILE lists forward indices to profile (e.g. "3,7") or
H3_FG_TIMING=1 (logs the synchronised wall time of every forward).
  H3_FG_PROFILE_DIR   output folder for chrome traces and tables (./h3_fg_prof)
  H3_FG_PROFILE_TAG   file name prefix (prof)
  H3_FG_RANK          rank shown in file names (0)
  H3_FUSE_TARGET      module that defines MiniMaxH3Model (comfy.ldm.minimax.model)
"""
import functools
import importlib
import logging
import os
import time

import torch

log = logging.getLogger("h3-fuse-graph")
_state = {"calls": 0, "installed": set()}
OUTDIR = os.environ.get("H3_FG_PROFILE_DIR", "./h3_fg_prof")


def _targets():
    spec = os.environ.get("H3_FG_PROFILE", "")
    return {int(v) for v in spec.replace(" ", "").split(",") if v}


def _enabled():
    return bool(_targets()) or os.environ.get("H3_FG_TIMING", "0") == "1"


def _sync():
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def _wrap(orig, label):
    targets = _targets()

    @functools.wraps(orig)
    def wrapped(*a, **k):
        _state["calls"] += 1
        n = _state["calls"]
        _sync()
        t0 = time.perf_counter()
        if n not in targets:
            out = orig(*a, **k)
            _sync()
            log.warning("[h3-fg] %s forward %d %.3f s", label, n, time.perf_counter() - t0)
            return out
        from torch.profiler import ProfilerActivity, profile
        acts = [ProfilerActivity.CPU] + ([ProfilerActivity.CUDA] if torch.cuda.is_available() else [])
        with profile(activities=acts) as prof:
            out = orig(*a, **k)
            _sync()
        wall = time.perf_counter() - t0
        os.makedirs(OUTDIR, exist_ok=True)
        tag = os.environ.get("H3_FG_PROFILE_TAG", "prof")
        rank = os.environ.get("H3_FG_RANK", "0")
        base = os.path.join(OUTDIR, f"{tag}-r{rank}-fwd{n}")
        prof.export_chrome_trace(base + ".json")
        ka = prof.key_averages()
        with open(base + ".txt", "w") as f:
            f.write(f"wall {wall:.3f} s\n")
            for key in ("self_device_time_total", "self_cuda_time_total", "self_cpu_time_total"):
                try:
                    f.write(ka.table(sort_by=key, row_limit=120, max_name_column_width=90))
                    break
                except Exception:  # noqa: BLE001
                    continue
        log.warning("[h3-fg] %s forward %d profiled %.3f s -> %s", label, n, wall, base)
        return out

    wrapped._h3_fg_orig = orig
    return wrapped


def install():
    if not _enabled() or "single" in _state["installed"]:
        return
    try:
        mm = importlib.import_module(os.environ.get("H3_FUSE_TARGET", "comfy.ldm.minimax.model"))
        mm.MiniMaxH3Model._forward = _wrap(mm.MiniMaxH3Model._forward, "single")
        _state["installed"].add("single")
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-fg] cannot wrap the single-process forward: %s", e)


def install_sp(spf_module):
    if not _enabled() or "sp" in _state["installed"]:
        return
    spf_module.sp_forward = _wrap(spf_module.sp_forward, "sp")
    _state["installed"].add("sp")
    log.warning("[h3-fg] sp_forward wrapped")
