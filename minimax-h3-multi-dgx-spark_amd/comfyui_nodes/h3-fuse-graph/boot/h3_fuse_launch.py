"""Launcher that gives h3-fuse-graph to worker processes that do not load
ComfyUI custom nodes.

Usage: python -s h3_fuse_launch.py <worker.py> [worker args...]
Registers an after-import hook so DiTBlock.forward is replaced (H3_FUSE=1) as
soon as the model module is imported, wraps sp_forward for measurement when
H3_FG_PROFILE / H3_FG_TIMING are set, then runs the worker script as __main__.
Compatible with the h3-linear-fast sitecustomize boot hook (PYTHONPATH).
Counterpart of comfyui_nodes/h3-fuse-graph/boot/h3_fuse_launch.py:20-32.
"""
import os
import runpy
import sys

_here = os.path.dirname(os.path.abspath(__file__))
_node = os.path.dirname(_here)
if _node not in sys.path:
    sys.path.append(_node)

import h3_fg_profile  # noqa: E402
import h3_fuse_patch  # noqa: E402


def _on_model(_module):
    h3_fuse_patch.install()
    h3_fg_profile.install()


def main(argv):
    target = os.environ.get("H3_FUSE_TARGET", "comfy.ldm.minimax.model")
    h3_fuse_patch.after_import(lambda n: n == target, _on_model)
    if h3_fg_profile._enabled():
        h3_fuse_patch.after_import(lambda n: n.endswith("minimax_sp.sp_forward"), h3_fg_profile.install_sp)
    script = os.path.abspath(argv[1])
    sys.argv = argv[1:]
    sys.path[0] = os.path.dirname(script)
    runpy.run_path(script, run_name="__main__")


if __name__ == "__main__":
    main(sys.argv)
