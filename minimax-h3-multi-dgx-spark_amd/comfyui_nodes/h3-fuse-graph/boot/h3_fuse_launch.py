"""Launcher that gives h3-fuse-graph to worker processes that do not load
ComfyUI custom nodes.

Usage: python -s h3_fuse_launch.py <worker.py> [worker args...]
Arms two import hooks and then runs the worker script as __main__:
  * when the model module (H3_FUSE_TARGET, default comfy.ldm.minimax.model)
    has been imported: replace DiTBlock.forward (H3_FUSE=1) and wrap
    MiniMaxH3Model._forward for measurement (H3_FG_PROFILE / H3_FG_TIMING);
  * with measurement on, when minimax_sp.sp_forward has been imported: wrap
    sp_forward.
Works beside the h3-linear-fast sitecustomize boot hook (PYTHONPATH).
Counterpart of comfyui_nodes/h3-fuse-graph/boot/h3_fuse_launch.py:20-32.
"""
import os
import runpy
import sys


def _import_node_modules():
    node_dir = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if node_dir not in sys.path:
        sys.path.append(node_dir)
    import h3_fg_profile
    import h3_fuse_patch
    return h3_fuse_patch, h3_fg_profile


def arm_hooks():
    patch, profile = _import_node_modules()
    model_module = os.environ.get("H3_FUSE_TARGET", "comfy.ldm.minimax.model")

    def on_model_import(_module):
        patch.install()
        profile.install()

    patch.after_import(lambda name: name == model_module, on_model_import)
    if profile._enabled():
        patch.after_import(lambda name: name.endswith("minimax_sp.sp_forward"), profile.install_sp)


def run_worker(argv):
    """Run argv[0] as __main__ with argv as its sys.argv, its folder first on
    sys.path (as `python argv[0] ...` would)."""
    script = os.path.abspath(argv[0])
    sys.argv = list(argv)
    sys.path[0] = os.path.dirname(script)
    runpy.run_path(script, run_name="__main__")


def main(argv):
    if len(argv) < 2:
        sys.exit("usage: python -s h3_fuse_launch.py <worker.py> [args...]")
    arm_hooks()
    run_worker(argv[1:])


if __name__ == "__main__":
    main(sys.argv)
