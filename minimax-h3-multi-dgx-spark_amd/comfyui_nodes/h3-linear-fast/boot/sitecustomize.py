"""Worker boot hook for h3-linear-fast: lets processes that never load ComfyUI
custom nodes (distributed workers) get the patch.

Usage: start the worker with PYTHONPATH=<this folder> and H3_LINEAR_FAST=1.
Python imports `sitecustomize` automatically.  This module first runs the
`sitecustomize` that this folder shadows (the next one on sys.path, if any),
then installs an import hook that calls h3_linear_fast_patch.install() right
after the target module (H3_LINEAR_FAST_TARGET, default
comfy_kitchen.backends.cuda) finishes importing.
Counterpart of comfyui_nodes/h3-linear-fast/boot/sitecustomize.py:10-44.
"""
import os
import sys

_here = os.path.dirname(os.path.abspath(__file__))


def _run_shadowed_sitecustomize():
    for p in sys.path:
        if not p or os.path.abspath(p) == _here:
            continue
        cand = os.path.join(p, "sitecustomize.py")
        if os.path.exists(cand):
            try:
                with open(cand, encoding="utf-8") as f:
                    code = compile(f.read(), cand, "exec")
                exec(code, {"__name__": "sitecustomize_shadowed", "__file__": cand})
            except Exception:  # noqa: BLE001  (a broken system hook must not stop the worker)
                pass
            return cand
    return None


_run_shadowed_sitecustomize()

if os.environ.get("H3_LINEAR_FAST", "0") == "1":
    import importlib.abc
    import importlib.machinery

    _node = os.path.dirname(_here)
    if _node not in sys.path:
        sys.path.insert(0, _node)
    _target = os.environ.get("H3_LINEAR_FAST_TARGET", "comfy_kitchen.backends.cuda")

    class _InstallAfterImport(importlib.abc.MetaPathFinder):
        """Wraps the loader of the target module so install() runs once the
        module body has executed."""

        def find_spec(self, name, path=None, target=None):
            if name != _target:
                return None
            sys.meta_path.remove(self)
            spec = importlib.machinery.PathFinder.find_spec(name, path)
            if spec is None or spec.loader is None:
                return spec
            inner = spec.loader.exec_module

            def exec_module(module):
                inner(module)
                import h3_linear_fast_patch
                h3_linear_fast_patch.install()

            spec.loader.exec_module = exec_module
            return spec

    sys.meta_path.insert(0, _InstallAfterImport())
