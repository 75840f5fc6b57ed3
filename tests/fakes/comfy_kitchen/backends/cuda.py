"""Stand-in for comfy_kitchen.backends.cuda: an eager int8_linear with the
upstream 12-argument signature (tests only).  convrot=False path: per-row
symmetric quantize, int32 GEMM, bf16((f32(acc)*xs)*ws) (+ bias)."""
import torch

CALLS = {"int8_linear": 0}
_CONVROT_FUSED_MAX_K = 16384


def _int8_weight_scale_arg(weight_scale, device):
    return weight_scale.to(device=device, dtype=torch.float32)


def int8_linear(x, weight, weight_scale, bias=None, out_dtype=None, convrot=False, convrot_groupsize=256,
                input_act=None, input_act_weight=None, input_act_eps=0.0, residual=None, residual_scale=None):
    CALLS["int8_linear"] += 1
    if convrot or input_act not in (None, "none") or residual is not None:
        raise NotImplementedError("stand-in covers the plain per-row path only")
    k = x.shape[-1]
    x2 = x.reshape(-1, k).float()
    amax = x2.abs().amax(dim=1, keepdim=True)
    # divide by a tensor: eager GPU PyTorch turns division by a Python scalar
    # into a multiply by its reciprocal, which is not the IEEE quotient
    s = amax / torch.full_like(amax, 127.0)
    safe = torch.where(s == 0, torch.ones_like(s), s)
    q = torch.where(s == 0, torch.zeros_like(x2), torch.round(x2 / safe).clamp_(-127, 127)).to(torch.int8)
    if q.shape[0] > 16:
        acc = torch._int_mm(q, weight.t())
    else:  # exact in fp64 for K * 127^2 < 2^53
        acc = (q.double() @ weight.double().t()).round().to(torch.int32)
    ws = weight_scale.to(torch.float32).reshape(-1)
    c = (acc.float() * s) * ws[None, :]
    if bias is not None:
        c = c + bias.float()[None, :]
    out = c.to(out_dtype or x.dtype)
    return out.reshape(*x.shape[:-1], weight.shape[0])
