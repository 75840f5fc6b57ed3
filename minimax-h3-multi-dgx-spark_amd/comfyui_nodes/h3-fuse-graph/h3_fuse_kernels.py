"""Fused DiT-block kernels (RMSNorm + adaLN modulation + gate/residual) on
MI355X (gfx950) HIP kernels.

Module-level API of comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:
  norm_mod(x, w, eps, ridx, s1, sh) -> h                  h = (rmsnorm(x) * s1[row]) + sh[row]
  gate_norm_mod_(x, o, g, w, eps, ridx, s1, sh) -> h      x += o * g[row]; then as norm_mod
  gate_(x, o, g, ridx) -> x                               x += o * g[row]
Rounding points match the eager sequence the kernels replace (rms_norm output,
after the multiply, after the add, after the residual), and the sum of squares
follows eager PyTorch's rms_norm reduction order on this GPU (256 threads x 4
elements, 64-lane shuffle tree, then the cross-warp halving tree), so outputs
are bit-identical to F.rms_norm -> mul_ -> add_ / addcmul_.
"""
import _h3mi_path

_h3mi_path.ensure()

from h3mi.fused import gate_, gate_norm_mod_, norm_mod, order_info  # noqa: E402,F401
from h3mi.fused import gate_norm_mod_q_, norm_mod_q  # noqa: E402,F401  (h with its per-token int8 quantization)

NUMX, VEC, WARP = order_info(0)
