"""h3-fuse-graph (MI355X): fuses the H3 DiT block's norm / adaLN modulation /
gate / residual steps into HIP kernels when H3_FUSE=1 (outputs bit-identical to
the eager path).  H3_FG_PROFILE / H3_FG_TIMING enable the measurement hook.
Adds no nodes and edits no upstream files.  Workers that do not load custom
nodes get it through boot/h3_fuse_launch.py.
Counterpart of comfyui_nodes/h3-fuse-graph/__init__.py:14-23.
"""
import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

import h3_fg_profile  # noqa: E402
import h3_fuse_patch  # noqa: E402

h3_fg_profile.install()
if h3_fg_profile._enabled():
    h3_fuse_patch.after_import(lambda n: n.endswith("minimax_sp.sp_forward"), h3_fg_profile.install_sp)
h3_fuse_patch.install()

NODE_CLASS_MAPPINGS = {}
NODE_DISPLAY_NAME_MAPPINGS = {}
