"""Optional measurement of whole H3 forwards: synchronised wall time per
forward, and a torch.profiler capture of chosen forwards.

Interface of comfyui_nodes/h3-fuse-graph/h3_fg_profile.py (install :67-75,
install_sp :78-83, _enabled :24-25) and its environment:
  H3_FG_PROFILE=3,7   profile the 3rd and 7th forward (1-based count over every
                      wrapped forward of the process)
  H3_FG_TIMING=1      log the synchronised wall time of every other forward
  H3_FG_PROFILE_DIR   output folder (./h3_fg_prof)
  H3_FG_PROFILE_TAG   file-name prefix (prof)
  H3_FG_RANK          rank in the file names (0)
  H3_FUSE_TARGET      module that defines MiniMaxH3Model (comfy.ldm.minimax.model)
A profiled forward n writes <dir>/<tag>-r<rank>-fwd<n>.json (chrome trace) and
.txt (its wall time, then the operator table sorted by self device time).
The single-process forward (MiniMaxH3Model._forward) and the distributed one
(sp_forward) share one forward counter.
"""
import functools
import importlib
import logging
import os
import time

import torch

log = logging.getLogger("h3-fuse-graph")


def _selected():
    """Forward numbers to profile, from H3_FG_PROFILE."""
    out = set()
    for tok in os.environ.get("H3_FG_PROFILE", "").split(","):
        tok = tok.strip()
        if tok:
            out.add(int(tok))
    return out


def _enabled():
    return bool(_selected()) or os.environ.get("H3_FG_TIMING", "0") == "1"


class ForwardMeter:
    """Counts wrapped forwards across the process and measures each one."""

    def __init__(self):
        self.count = 0
        self.wrapped = {}  # label -> wrapper

    @staticmethod
    def _drain():
        if torch.cuda.is_available():
            torch.cuda.synchronize()

    def _paths(self, n):
        folder = os.environ.get("H3_FG_PROFILE_DIR", "./h3_fg_prof")
        stem = "{}-r{}-fwd{}".format(os.environ.get("H3_FG_PROFILE_TAG", "prof"), os.environ.get("H3_FG_RANK", "0"), n)
        os.makedirs(folder, exist_ok=True)
        return os.path.join(folder, stem)

    @staticmethod
    def _table(events):
        """Operator table sorted by self device time when this torch build
        records it, else by self CPU time."""
        first = next(iter(events), None)
        for key in ("self_device_time_total", "self_cuda_time_total"):
            if first is not None and hasattr(first, key):
                return events.table(sort_by=key, row_limit=120, max_name_column_width=90)
        return events.table(sort_by="self_cpu_time_total", row_limit=120, max_name_column_width=90)

    def _profiled(self, fn, args, kwargs, label, n):
        from torch.profiler import ProfilerActivity, profile
        activities = [ProfilerActivity.CPU]
        if torch.cuda.is_available():
            activities.append(ProfilerActivity.CUDA)
        start = time.perf_counter()
        with profile(activities=activities) as session:
            result = fn(*args, **kwargs)
            self._drain()
        wall = time.perf_counter() - start
        stem = self._paths(n)
        session.export_chrome_trace(stem + ".json")
        with open(stem + ".txt", "w") as out:
            out.write("wall {:.3f} s\n".format(wall))
            out.write(self._table(session.key_averages()))
        log.warning("[h3-fg] %s forward %d profiled in %.3f s -> %s.{json,txt}", label, n, wall, stem)
        return result

    def _timed(self, fn, args, kwargs, label, n):
        self._drain()
        start = time.perf_counter()
        result = fn(*args, **kwargs)
        self._drain()
        log.warning("[h3-fg] %s forward %d %.3f s", label, n, time.perf_counter() - start)
        return result

    def wrap(self, fn, label):
        picks = _selected()

        @functools.wraps(fn)
        def measured(*args, **kwargs):
            self.count += 1
            run = self._profiled if self.count in picks else self._timed
            return run(fn, args, kwargs, label, self.count)

        measured._h3_fg_orig = fn
        self.wrapped[label] = measured
        return measured


_meter = ForwardMeter()


def install():
    """Wrap MiniMaxH3Model._forward (once) when measurement is enabled."""
    if not _enabled() or "single" in _meter.wrapped:
        return
    name = os.environ.get("H3_FUSE_TARGET", "comfy.ldm.minimax.model")
    try:
        model = importlib.import_module(name).MiniMaxH3Model
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-fg] MiniMaxH3Model._forward not wrapped: %s", e)
        return
    model._forward = _meter.wrap(model._forward, "single")


def install_sp(spf_module):
    """Wrap the distributed forward of the given sp_forward module (once)."""
    if not _enabled() or "sp" in _meter.wrapped:
        return
    spf_module.sp_forward = _meter.wrap(spf_module.sp_forward, "sp")
    log.warning("[h3-fg] sp_forward wrapped for measurement")
