"""ctypes binding of libh3mi.so (the C ABI declared in include/h3mi.h).

The library is loaded from this package directory.  There is no fallback: if
the library is missing or does not export the ABI, importing the callers
fails loudly (build it with `make -C minimax-h3-multi-dgx-spark_amd` or
the repository's `build()` entry point).
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libh3mi.so")
ABI_VERSION = 1

# Status codes (enum h3mi_status)
OK, EINVAL, EALIGN, EALIAS, ELAUNCH, EDEVICE = range(6)
# Norm orders (enum h3mi_norm_order) and rsqrt modes (enum h3mi_rsqrt_mode)
ORDER_DEFAULT, ORDER_REF, ORDER_W64 = 0, 1, 2
RSQRT_HW, RSQRT_RN = 0, 1
# ConvRot input activations (enum h3mi_act)
ACT_NONE, ACT_SWIGLU = 0, 1

_P = ctypes.c_void_p
_I = ctypes.c_int64
_F = ctypes.c_float
_C = ctypes.c_int

# name -> argtypes (restype int unless listed in _RESTYPE)
SIGNATURES = {
    "h3mi_abi_version": [],
    "h3mi_last_error": [],
    "h3mi_w8a8_supported": [_I],
    "h3mi_w8a8_gemm_bf16": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "h3mi_w8a8_gemm_i32": [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "h3mi_w8a8_config": [_I, _I, _I, ctypes.c_char_p, _I],
    "h3mi_w8a8_set_config": [ctypes.c_char_p],
    "h3mi_w8a8_config_name": [_C, ctypes.c_char_p, _I],
    "h3mi_quant_rowwise_i8": [_P, _P, _P, _I, _I, _I, _P],
    "h3mi_quant_convrot_i8": [_P, _P, _P, _I, _I, _I, _C, _C, _P],
    "h3mi_rms_rope_split_half_bf16": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _C, _P, _P],
    "h3mi_norm_mod_bf16": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P],
    "h3mi_gate_norm_mod_bf16": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P],
    "h3mi_gate_bf16": [_P, _P, _P, _P, _I, _I, _I, _P],
    "h3mi_norm_mod_bf16_ex": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _C, _C, _P, _P, _P],
    "h3mi_gate_norm_mod_bf16_ex": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _C, _C, _P, _P, _P],
    "h3mi_norm_mod_quant_i8": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P],
    "h3mi_gate_norm_mod_quant_i8": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P],
    "h3mi_norm_order_info": [_C, ctypes.POINTER(_C), ctypes.POINTER(_C), ctypes.POINTER(_C)],
    "h3mi_debug_rsqrt_f32": [_P, _P, _I, _C, _P],
    "h3mi_debug_bf16_rne": [_P, _P, _I, _P],
    "h3mi_debug_buffer_lds_load": [_P, _I, _P, ctypes.c_int32, ctypes.c_int32, _P, _P],
}
_RESTYPE = {"h3mi_last_error": ctypes.c_char_p}


class H3miError(RuntimeError):
    """A nonzero status from libh3mi; .code is the h3mi_status value."""

    def __init__(self, code, msg):
        super().__init__(f"libh3mi error {code}: {msg}")
        self.code = code


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libh3mi.so not built at {LIB_PATH}; run `make -C {os.path.dirname(_HERE)}`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    v = lib.h3mi_abi_version()
    if v != ABI_VERSION:
        raise ImportError(f"libh3mi ABI {v} != expected {ABI_VERSION}")
    return lib


lib = _load()


def check(status):
    if status != OK:
        msg = lib.h3mi_last_error()
        raise H3miError(status, msg.decode() if msg else "")
    return status


def same_gpu(ref, **tensors):
    """Raise ValueError unless ref and every named tensor (None entries are
    skipped) live on the same GPU.  The C ABI takes bare addresses and cannot
    tell host memory from device memory, so this check stands between a CPU
    tensor and a kernel that would fault on its address."""
    if not ref.is_cuda:
        raise ValueError(f"expected GPU tensors, got one on {ref.device}")
    for name, t in tensors.items():
        if t is not None and t.device != ref.device:
            raise ValueError(f"{name} is on {t.device}, expected {ref.device}")


def ptr(t):
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    """The current torch stream on t's device, as a hipStream_t."""
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
