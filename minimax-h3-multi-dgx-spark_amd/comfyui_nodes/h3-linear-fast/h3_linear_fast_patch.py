"""Swap the upstream INT8 linear's GEMM for the MI355X HIP W8A8 kernels.

Counterpart of comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py
(install :41-116, patched int8_linear :60-110, uninstall :119-124, stats :127-128).

The patched function keeps the upstream 12-argument signature of
comfy_kitchen.backends.cuda.int8_linear.  An eligible call runs
  1. the activation quantizer: for convrot=True this library's ConvRot
     quantizer (256-group Hadamard rotation, then per-row int8; with
     input_act="swiglu" silu of the first half of x times the second half is
     rotated) -- where the reference calls comfy-kitchen's
     _C.quantize_int8_rowwise_convrot64, a CUDA extension that has no ROCm
     build; for convrot=False the per-token quantizer (s = absmax/127, round
     half to even, clamp +-127);
  2. the HIP int8 GEMM with the dequant epilogue bf16((f32(acc)*xs)*ws).
Ineligible calls go to the original function; a kernel error disables the
fast path for the rest of the process (same contract as the reference).

Environment:
  H3_LINEAR_FAST=1          enable (install() is a no-op otherwise)
  H3_LINEAR_FAST_MIN_M      smallest row count sent to the fast path (256)
  H3_LINEAR_FAST_TARGET     module whose int8_linear is replaced
                            (comfy_kitchen.backends.cuda)
  H3_LINEAR_FAST_BIAS=1     also take calls with a bias, fused in the epilogue
                            as bf16(((f32(acc)*xs)*ws) + bias) (off by default:
                            the reference sends bias calls to the original)
  H3_LINEAR_FAST_CFG        pin one GEMM tile configuration by name
  H3_LINEAR_FAST_CONVROT    "own" (default): the HIP ConvRot quantizer;
                            "upstream": comfy-kitchen's rotation kernel, where
                            its extension is present (the reference's choice)
On the per-token path, an input that the fused DiT block has offered already
quantized (h3mi.prequant, H3_FUSE_QUANT=1 in h3-fuse-graph) skips the
quantizer; the bytes are the same.
"""
import importlib
import logging
import os
import sys

import torch

log = logging.getLogger("h3-linear-fast")
_HERE = os.path.dirname(os.path.abspath(__file__))
_state = {"installed": False, "orig": None, "fast_calls": 0, "fallback_calls": 0, "disabled": False,
          "module": None, "prequant_calls": 0}
MIN_M = int(os.environ.get("H3_LINEAR_FAST_MIN_M", "256"))
TARGET = os.environ.get("H3_LINEAR_FAST_TARGET", "comfy_kitchen.backends.cuda")
MAX_K_OWN = 32768  # row limit of this library's quantizers


def _fuse_bias():
    return os.environ.get("H3_LINEAR_FAST_BIAS", "0") == "1"


def _upstream_convrot(ckc):
    """The upstream rotation+quantizer entry points, or None when absent."""
    C = getattr(ckc, "_C", None)
    need = ("_wrap_for_dlpack", "_act_weight_arg", "_input_act_code", "_convrot_fused_shared_memory_fits",
            "_CONVROT_FUSED_MAX_K")
    if C is None or not hasattr(C, "quantize_int8_rowwise_convrot64") or not all(hasattr(ckc, a) for a in need):
        return None
    return C.quantize_int8_rowwise_convrot64


def _weight_scale(ckc, weight_scale, n, device):
    f = getattr(ckc, "_int8_weight_scale_arg", None)
    ws = f(weight_scale, device) if f is not None else weight_scale
    ws = ws.to(device=device, dtype=torch.float32).reshape(-1)
    if ws.numel() != n:
        ws = ws.expand(n)
    return ws.contiguous()


def eligible(x, weight, bias, out_dtype, convrot, convrot_groupsize, input_act, residual, *, have_convrot,
             max_k_convrot, supported):
    """Whether a call can take the fast path, and its (m, k, n).

    Mirrors the reference gate (LF/h3_linear_fast_patch.py:62-73, 82): bf16 GPU
    input and output, 2-D int8 weight, no residual, an activation the quantizer
    handles, m >= MIN_M, k accepted by the GEMM, n % 8 == 0.  ConvRot calls need
    the upstream rotation quantizer (k % 256 == 0, 256 <= k <= its maximum);
    other calls use the per-token quantizer (no fused activation, k <= 32768).
    have_convrot / max_k_convrot describe the ConvRot quantizer in use (this
    library's: k <= 32768; comfy-kitchen's: its _CONVROT_FUSED_MAX_K).
    A bias is accepted only with H3_LINEAR_FAST_BIAS=1."""
    bf16 = torch.bfloat16
    out_dtype_eff = out_dtype or x.dtype
    act_w = 2 if input_act == "swiglu" else 1
    ok = (not _state["disabled"] and (bias is None or _fuse_bias()) and residual is None
          and input_act in (None, "none", "swiglu") and x.is_cuda and x.dtype == bf16
          and out_dtype_eff == bf16 and weight.dtype == torch.int8 and weight.dim() == 2 and x.dim() >= 1)
    if ok and convrot:
        ok = have_convrot and convrot_groupsize == 256
    elif ok:
        ok = input_act in (None, "none")
    if not ok:
        return False, 0, 0, 0
    kin = x.shape[-1]
    k = kin // act_w
    m = x.numel() // kin if kin else 0
    n = weight.shape[0]
    ok = (m >= MIN_M and kin % act_w == 0 and weight.shape[1] == k and supported(k) and n % 8 == 0)
    if ok and convrot:
        ok = k % 256 == 0 and 256 <= k <= max_k_convrot
    elif ok:
        ok = k <= MAX_K_OWN
    if ok and bias is not None:
        ok = bias.dtype == bf16 and bias.numel() == n and bias.is_cuda
    return ok, m, k, n


def install():
    if _state["installed"]:
        return True
    if os.environ.get("H3_LINEAR_FAST", "0") != "1":
        return False
    try:
        ckc = importlib.import_module(TARGET)
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-linear-fast] cannot import %s; disabled: %s", TARGET, e)
        return False
    if _HERE not in sys.path:
        sys.path.insert(0, _HERE)
    try:
        import int8_gemm_hip as tg
        from h3mi import prequant
        from h3mi.quant import quantize_rowwise, quantize_rowwise_convrot
    except Exception as e:  # noqa: BLE001
        log.warning("[h3-linear-fast] HIP library unavailable; disabled: %s", e)
        return False

    orig = ckc.int8_linear
    conv_q = _upstream_convrot(ckc) if os.environ.get("H3_LINEAR_FAST_CONVROT", "own") == "upstream" else None
    max_k_convrot = getattr(ckc, "_CONVROT_FUSED_MAX_K", 0) if conv_q is not None else MAX_K_OWN

    def int8_linear(x, weight, weight_scale, bias=None, out_dtype=None, convrot=False, convrot_groupsize=256,
                    input_act=None, input_act_weight=None, input_act_eps=0.0, residual=None, residual_scale=None):
        def fallback():
            return orig(x, weight, weight_scale, bias, out_dtype, convrot, convrot_groupsize, input_act,
                        input_act_weight, input_act_eps, residual, residual_scale)

        ok, m, k, n = eligible(x, weight, bias, out_dtype, convrot, convrot_groupsize, input_act, residual,
                               have_convrot=True, max_k_convrot=max_k_convrot, supported=tg.supported)
        kin = x.shape[-1] if x.dim() else 0
        use_bias = ok and bias is not None
        if not ok:
            _state["fallback_calls"] += 1
            if _state["fallback_calls"] <= 5:
                log.warning("[h3-linear-fast] original path: x=%s w=%s convrot=%s bias=%s act=%s", tuple(x.shape),
                            tuple(weight.shape), convrot, bias is not None, input_act)
            return fallback()
        x_2d = x if x.dim() == 2 and x.is_contiguous() else x.reshape(-1, kin).contiguous()
        if convrot and conv_q is not None and not ckc._convrot_fused_shared_memory_fits(x_2d, k, convrot_groupsize):
            _state["fallback_calls"] += 1
            return fallback()
        if not weight.is_contiguous():
            weight = weight.contiguous()
        try:
            if convrot and conv_q is None:
                x_q, x_s = quantize_rowwise_convrot(x_2d, "swiglu" if input_act == "swiglu" else None)
            elif convrot:
                W = ckc._wrap_for_dlpack
                stream_ptr = torch.cuda.current_stream(x.device).cuda_stream
                x_q = torch.empty((m, k), dtype=torch.int8, device=x.device)
                x_s = torch.empty((m, 1), dtype=torch.float32, device=x.device)
                act_weight_arg = ckc._act_weight_arg(input_act, input_act_weight, x.device, x_2d.dtype)
                conv_q(W(x_2d), W(x_q), W(x_s), convrot_groupsize, False, ckc._input_act_code(input_act), 0,
                       W(act_weight_arg), float(input_act_eps), stream_ptr)
            else:
                pre = prequant.take(x_2d)  # h quantized by the fused norm that produced it
                if pre is not None:
                    _state["prequant_calls"] += 1
                x_q, x_s = pre if pre is not None else quantize_rowwise(x_2d)
            ws = _weight_scale(ckc, weight_scale, n, x.device)
            out = tg.int8_mm_scaled(x_q, weight, x_s, ws, bias=bias.reshape(-1).contiguous() if use_bias else None)
        except Exception as e:  # noqa: BLE001
            _state["disabled"] = True
            log.warning("[h3-linear-fast] HIP kernel failed; original path from now on: %s", e)
            return fallback()
        _state["fast_calls"] += 1
        if _state["fast_calls"] in (1, 1000, 10000):
            log.warning("[h3-linear-fast] fast path call %d (original path %d)", _state["fast_calls"],
                        _state["fallback_calls"])
        return out if x.dim() == 2 else out.reshape(*x.shape[:-1], n)

    int8_linear._h3_linear_fast_orig = orig
    ckc.int8_linear = int8_linear
    _state["orig"] = orig
    _state["module"] = ckc
    _state["installed"] = True
    log.warning("[h3-linear-fast] enabled: %s.int8_linear GEMM -> MI355X HIP kernels (MIN_M=%d, ConvRot quantizer: %s)",
                TARGET, MIN_M, "comfy-kitchen" if conv_q is not None else "HIP")
    return True


def uninstall():
    if not _state["installed"]:
        return
    _state["module"].int8_linear = _state["orig"]
    _state["installed"] = False


def stats():
    # the reference's keys; calls that used an offered quantization are counted in _state["prequant_calls"]
    return {k: _state[k] for k in ("installed", "fast_calls", "fallback_calls", "disabled")}
