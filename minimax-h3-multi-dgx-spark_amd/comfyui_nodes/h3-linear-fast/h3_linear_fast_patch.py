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
     build; for convrot=False calls, only with H3_LINEAR_FAST_PLAIN=1, the
     per-token quantizer (s = absmax/127, round half to even, clamp +-127);
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
  H3_LINEAR_FAST_CFG        pin one GEMM tile configuration by name (a value
                            in the reference's "BM,BN,BK,stages,warps" form,
                            or an unknown name, keeps the heuristic; install()
                            logs a warning)
  H3_LINEAR_FAST_CONVROT    quantizer for convrot=True calls:
                            "auto" (default): comfy-kitchen's rotation kernel
                            when its extension is present (the reference's),
                            else this library's, with a one-time warning that
                            its parity against comfy-kitchen is unpinned;
                            "own": this library's; "upstream": comfy-kitchen's
                            only (convrot calls go to the original without it)
  H3_LINEAR_FAST_PLAIN      "0" (default): convrot=False calls go to the
                            original, as in the reference; "1" (opt-in): they
                            take the fast path with the per-token quantizer,
                            whose bytes against comfy-kitchen's own
                            convrot=False quantizer are unpinned
On the per-token path, an input that the fused DiT block has offered already
quantized (h3mi.prequant, H3_FUSE_QUANT=1 in h3-fuse-graph) skips the
quantizer; the bytes are the same.

Errors: a call the HIP entry points reject for its arguments (ValueError,
H3miError EINVAL / EALIGN / EALIAS) goes to the original for that call only;
any other failure (a launch error) disables the fast path for the rest of the
process, as the reference does for its GEMM.
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


def _plain_takeover():
    return os.environ.get("H3_LINEAR_FAST_PLAIN", "0") == "1"


def _weight_scale(ckc, weight_scale, n, device):
    """Per-output-channel fp32 scales [n] on the device: the upstream argument
    normaliser when it exists, then a per-tensor (one-element) scale expanded
    to every channel (reference LF/h3_linear_fast_patch.py:97-99)."""
    f = getattr(ckc, "_int8_weight_scale_arg", None)
    ws = f(weight_scale, device) if f is not None else weight_scale
    ws = ws.to(device=device, dtype=torch.float32).reshape(-1)
    if ws.numel() == 1 and n != 1:
        ws = ws.expand(n)
    return ws.contiguous()


def eligible(x, weight, bias, out_dtype, convrot, convrot_groupsize, input_act, residual, *, have_convrot,
             max_k_convrot, supported, input_act_weight=None, input_act_eps=0.0, own_convrot=True,
             weight_scale=None):
    """Whether a call can take the fast path, and its (m, k, n).

    Mirrors the reference gate (LF/h3_linear_fast_patch.py:62-73, 82): bf16 GPU
    input and output, 2-D int8 weight, no residual, an activation the quantizer
    handles, m >= MIN_M, k accepted by the GEMM, n % 8 == 0.  ConvRot calls need
    a ConvRot quantizer (k % 256 == 0, 256 <= k <= its maximum); other calls use
    the per-token quantizer (no fused activation, k <= 32768) only with
    H3_LINEAR_FAST_PLAIN=1.  have_convrot / max_k_convrot describe the ConvRot
    quantizer in use (this library's: k <= 32768; comfy-kitchen's: its
    _CONVROT_FUSED_MAX_K).  This library's quantizers take no activation weight
    and no epsilon, so calls with either go to the original unless comfy-kitchen's
    quantizer serves them (own_convrot False).  The weight must be 16-byte
    aligned and the weight scale hold 1 or n values.  A bias is accepted only
    with H3_LINEAR_FAST_BIAS=1."""
    bf16 = torch.bfloat16
    out_dtype_eff = out_dtype or x.dtype
    act_w = 2 if input_act == "swiglu" else 1
    ok = (not _state["disabled"] and (bias is None or _fuse_bias()) and residual is None
          and input_act in (None, "none", "swiglu") and x.is_cuda and x.dtype == bf16
          and out_dtype_eff == bf16 and weight.dtype == torch.int8 and weight.dim() == 2 and x.dim() >= 1
          and weight.is_cuda and weight.device == x.device)
    if ok and convrot:
        ok = have_convrot and convrot_groupsize == 256
        if ok and own_convrot:
            ok = input_act_weight is None and not input_act_eps
    elif ok:
        ok = _plain_takeover() and input_act in (None, "none") and input_act_weight is None and not input_act_eps
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
    if ok and weight.is_contiguous():
        ok = weight.data_ptr() % 16 == 0
    if ok and weight_scale is not None and hasattr(weight_scale, "numel"):
        ok = weight_scale.numel() in (1, n)
    if ok and bias is not None:
        ok = bias.dtype == bf16 and bias.numel() == n and bias.is_cuda and bias.device == x.device
    return ok, m, k, n


def _argument_error(e):
    """True for a rejection of the call's arguments (that call falls back), False
    for a failure that should disable the fast path."""
    from h3mi import _lib as L
    if isinstance(e, L.H3miError):
        return e.code in (L.EINVAL, L.EALIGN, L.EALIAS)
    return isinstance(e, (ValueError, TypeError))


def _pick_convrot(ckc):
    """(upstream quantizer or None, whether convrot=True calls have a quantizer)."""
    mode = os.environ.get("H3_LINEAR_FAST_CONVROT", "auto")
    up = _upstream_convrot(ckc)
    if mode == "own":
        return None, True
    if mode == "upstream":
        return up, up is not None
    return up, True  # auto


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

    note = tg.fixed_config_note()
    if note:
        log.warning("[h3-linear-fast] %s", note)
    orig = ckc.int8_linear
    conv_q, have_convrot = _pick_convrot(ckc)
    max_k_convrot = getattr(ckc, "_CONVROT_FUSED_MAX_K", 0) if conv_q is not None else MAX_K_OWN
    warned = {"own": False}

    def int8_linear(x, weight, weight_scale, bias=None, out_dtype=None, convrot=False, convrot_groupsize=256,
                    input_act=None, input_act_weight=None, input_act_eps=0.0, residual=None, residual_scale=None):
        def fallback():
            return orig(x, weight, weight_scale, bias, out_dtype, convrot, convrot_groupsize, input_act,
                        input_act_weight, input_act_eps, residual, residual_scale)

        def decline(why):
            _state["fallback_calls"] += 1
            if _state["fallback_calls"] <= 5:
                log.warning("[h3-linear-fast] original path (%s): x=%s w=%s convrot=%s bias=%s act=%s", why,
                            tuple(x.shape), tuple(weight.shape), convrot, bias is not None, input_act)
            return fallback()

        ok, m, k, n = eligible(x, weight, bias, out_dtype, convrot, convrot_groupsize, input_act, residual,
                               have_convrot=have_convrot, max_k_convrot=max_k_convrot, supported=tg.supported,
                               input_act_weight=input_act_weight, input_act_eps=input_act_eps,
                               own_convrot=conv_q is None, weight_scale=weight_scale)
        if not ok:
            return decline("not eligible")
        kin = x.shape[-1]
        x_2d = x if x.dim() == 2 and x.is_contiguous() else x.reshape(-1, kin).contiguous()
        if x_2d.data_ptr() % 16:  # an offset view: the quantizers read 16-byte chunks
            x_2d = x_2d.clone()
        if convrot and conv_q is not None and not ckc._convrot_fused_shared_memory_fits(x_2d, k, convrot_groupsize):
            return decline("ConvRot shared memory")
        w = weight if weight.is_contiguous() else weight.contiguous()
        try:
            if convrot and conv_q is None:
                if not warned["own"]:
                    warned["own"] = True
                    log.warning("[h3-linear-fast] convrot=True calls use this library's ConvRot quantizer "
                                "(comfy-kitchen's is absent); its parity against comfy-kitchen is unpinned")
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
            b = bias.reshape(-1).contiguous() if bias is not None else None
            out = tg.int8_mm_scaled(x_q, w, x_s, ws, bias=b)
        except Exception as e:  # noqa: BLE001
            if _argument_error(e):
                return decline(f"arguments rejected: {e}")
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
    log.warning("[h3-linear-fast] enabled: %s.int8_linear -> MI355X HIP kernels (MIN_M=%d; ConvRot quantizer: %s; "
                "convrot=False calls: %s)", TARGET, MIN_M,
                "comfy-kitchen" if conv_q is not None else ("HIP (parity unpinned vs comfy-kitchen)" if have_convrot
                                                            else "none, original path"),
                "HIP per-token quantizer" if _plain_takeover() else "original path")
    return True


def uninstall():
    if not _state["installed"]:
        return
    _state["module"].int8_linear = _state["orig"]
    _state["installed"] = False


def stats():
    # the reference's keys; calls that used an offered quantization are counted in _state["prequant_calls"]
    return {k: _state[k] for k in ("installed", "fast_calls", "fallback_calls", "disabled")}
