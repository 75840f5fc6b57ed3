"""Run callbacks right after a module finishes importing (worker boot hooks).

Serves the reference's after_import(match, fn) contract
(comfyui_nodes/h3-fuse-graph/h3_fuse_patch.py:183-184, used by
boot/h3_fuse_launch.py:25,27 and __init__.py:19) and the linear patch's
sitecustomize (comfyui_nodes/h3-linear-fast/boot/sitecustomize.py:26-44):
a worker that never loads ComfyUI custom nodes must still get the patches,
and they can only be applied once the upstream module exists.

Design: one watcher finder sits at the front of sys.meta_path for all pending
hooks.  When a watched name is imported it asks the finders behind it for the
real spec and hands the import system a proxy loader that executes the module
with the real loader and then calls the hooks.  A hook fires once; a module
that is already imported when its hook is registered gets the call at once.
Imports only the standard library (it runs from sitecustomize, before torch).
"""
import importlib.abc
import sys
import threading

_lock = threading.RLock()
_pending = []  # [(match, fn)] not fired yet


class _HookedLoader(importlib.abc.Loader):
    """Delegates to the real loader; runs the hooks after exec_module."""

    def __init__(self, inner, hooks):
        self._inner = inner
        self._entries = hooks  # [(match, fn)]

    def create_module(self, spec):
        make = getattr(self._inner, "create_module", None)
        return make(spec) if make is not None else None

    def exec_module(self, module):
        try:
            self._inner.exec_module(module)
        except BaseException:
            with _lock:  # the import failed: the hooks wait for the next attempt
                _pending.extend(self._entries)
                _install_watcher()
            raise
        for _, fn in self._entries:
            fn(module)

    def __getattr__(self, name):  # get_resource_reader, is_package, get_code, ...
        return getattr(self._inner, name)


class _Watcher(importlib.abc.MetaPathFinder):
    def find_spec(self, fullname, path=None, target=None):
        with _lock:
            hit = [h for h in _pending if h[0](fullname)]
            if not hit:
                return None
            for h in hit:
                _pending.remove(h)
            if not _pending and self in sys.meta_path:
                sys.meta_path.remove(self)
        spec = None
        for finder in list(sys.meta_path):
            if finder is self or not hasattr(finder, "find_spec"):
                continue
            spec = finder.find_spec(fullname, path, target)
            if spec is not None:
                break
        if spec is None or spec.loader is None:
            with _lock:  # nothing to load (yet): keep waiting
                _pending.extend(hit)
                _install_watcher()
            return spec
        spec.loader = _HookedLoader(spec.loader, hit)
        return spec


_watcher = _Watcher()


def _install_watcher():
    if _watcher not in sys.meta_path:
        sys.meta_path.insert(0, _watcher)


def after_import(match, fn):
    """Call fn(module) once, right after the first module whose name satisfies
    match(name) has executed; at once if such a module is already imported."""
    for name, mod in list(sys.modules.items()):
        if mod is not None and match(name):
            fn(mod)
            return
    with _lock:
        _pending.append((match, fn))
        _install_watcher()


def pending():
    """Number of hooks still waiting (tests)."""
    with _lock:
        return len(_pending)
