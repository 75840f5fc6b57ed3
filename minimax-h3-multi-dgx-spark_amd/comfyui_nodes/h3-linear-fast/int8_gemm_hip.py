"""INT8 GEMM with per-row x per-column scales written straight to bf16, on
MI355X (gfx950) HIP kernels.

Module-level API of comfyui_nodes/h3-linear-fast/int8_gemm_triton.py:
  out[m, n] = bf16( (float(sum_k xq[m,k]*w[n,k]) * xs[m]) * ws[n] )
  int8_mm_scaled(xq, w, xs, ws, out=None)
  supported(K)
  _int8_mm_scaled_kernel.best_config   (the tile configuration last used)
H3_LINEAR_FAST_CFG=<configuration name> pins one tile configuration (the
reference's "BM,BN,BK,stages,warps" form keeps the heuristic, with a warning);
H3_LINEAR_FAST_ALLCFG=1 autotunes over every configuration per
(N, K, ceil(M / 4096)) on the first call, as the reference's wider autotune.
"""
import _h3mi_path

_h3mi_path.ensure()

from h3mi.gemm import (_int8_mm_scaled_kernel, config_for, fixed_config_note, int8_mm_scaled,  # noqa: E402,F401
                       set_config, supported)
