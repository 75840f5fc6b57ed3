"""h3-linear-fast (MI355X): replaces the GEMM of the upstream int8_linear with
hand-written gfx950 HIP kernels when H3_LINEAR_FAST=1.  Adds no nodes and
edits no upstream files.  Reference counterpart:
comfyui_nodes/h3-linear-fast/__init__.py:12-17.
"""
import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

import h3_linear_fast_patch  # noqa: E402

h3_linear_fast_patch.install()

NODE_CLASS_MAPPINGS = {}
NODE_DISPLAY_NAME_MAPPINGS = {}
