"""h3mi: MI355X (gfx950) kernels for the H3 DiT W8A8 linear and fused norms.

Host side of libh3mi.so: PyTorch supplies device memory and the current HIP
stream; every computation runs in the hand-written HIP kernels behind the C ABI
in include/h3mi.h.  Importing this package fails if the library is not built.
"""
from . import _lib  # noqa: F401  (loads libh3mi.so; raises if missing)
from .gemm import int8_mm_scaled, int8_mm_i32, supported, config_for, set_config, list_configs  # noqa: F401
from .quant import quantize_rowwise, quantize_rowwise_convrot  # noqa: F401
from .fused import norm_mod, gate_norm_mod_, gate_, norm_mod_ex, gate_norm_mod_ex, order_info  # noqa: F401
from .fused import norm_mod_q, gate_norm_mod_q_  # noqa: F401
from .linear import w8a8_linear  # noqa: F401
from .rope import rms_rope_split_half_, rms_rope_split_half  # noqa: F401

__all__ = ["int8_mm_scaled", "int8_mm_i32", "supported", "config_for", "set_config", "list_configs", "quantize_rowwise", "quantize_rowwise_convrot",
           "norm_mod", "gate_norm_mod_", "gate_", "norm_mod_ex", "gate_norm_mod_ex", "order_info", "w8a8_linear",
           "norm_mod_q", "gate_norm_mod_q_", "rms_rope_split_half_", "rms_rope_split_half"]
