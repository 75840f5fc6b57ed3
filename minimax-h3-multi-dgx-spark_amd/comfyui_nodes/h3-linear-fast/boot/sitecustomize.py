"""Worker boot hook for h3-linear-fast: lets processes that never load ComfyUI
custom nodes (distributed workers) get the patch.

Usage: start the worker with PYTHONPATH=<this folder> and H3_LINEAR_FAST=1.
Python imports `sitecustomize` by itself at start-up.  This module first runs
the `sitecustomize` it shadows (the next one on sys.path, if any), then asks
h3_import_hooks to call h3_linear_fast_patch.install() once the target module
(H3_LINEAR_FAST_TARGET, default comfy_kitchen.backends.cuda) has been
imported.  Only the standard library is imported here, so the interpreter
starts as fast as before.
Counterpart of comfyui_nodes/h3-linear-fast/boot/sitecustomize.py:10-44.
"""
import os
import sys

_here = os.path.dirname(os.path.abspath(__file__))


def _chain_shadowed():
    """Execute the sitecustomize this file hides from the interpreter; a broken
    one must not stop the worker."""
    for entry in sys.path:
        if not entry or os.path.abspath(entry) == _here:
            continue
        path = os.path.join(entry, "sitecustomize.py")
        if not os.path.isfile(path):
            continue
        try:
            with open(path, encoding="utf-8") as f:
                source = f.read()
            exec(compile(source, path, "exec"), {"__name__": "sitecustomize_shadowed", "__file__": path})
        except Exception:  # noqa: BLE001
            pass
        return path
    return None


def _arm():
    node = os.path.dirname(_here)
    if node not in sys.path:
        sys.path.insert(0, node)
    import _h3mi_path
    _h3mi_path.ensure()
    import h3_import_hooks

    def _install(_module):
        import h3_linear_fast_patch
        h3_linear_fast_patch.install()

    target = os.environ.get("H3_LINEAR_FAST_TARGET", "comfy_kitchen.backends.cuda")
    h3_import_hooks.after_import(lambda name: name == target, _install)


_chain_shadowed()
if os.environ.get("H3_LINEAR_FAST", "0") == "1":
    _arm()
