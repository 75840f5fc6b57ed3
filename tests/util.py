"""Helpers shared by the tests: bf16 <-> uint16 bit views and seeded inputs."""
import numpy as np
import torch


def bits(t):
    """bf16 tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(b, device="cpu"):
    t = torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    return t.to(device)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def gemm_inputs(M, N, K, seed, outliers=0.0):
    """Workload-style W8A8 inputs on the CPU: X ~ N(0,1) bf16 (a fraction of
    elements scaled by 20), W int8 uniform in [-127, 127], ws ~ U(1e-3, 1e-2),
    bias ~ N(0, 0.02) bf16."""
    g = gen(seed)
    x = torch.randn(M, K, generator=g)
    if outliers > 0:
        n_out = max(1, int(outliers * M * K))
        idx = torch.randperm(M * K, generator=g)[:n_out]
        x.view(-1)[idx] *= 20
    x = x.to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    ws = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    bias = (0.02 * torch.randn(N, generator=g)).to(torch.bfloat16)
    return x, w, ws, bias


def norm_inputs(S, N, R, seed, stress=True):
    """Fused-norm inputs: x (optionally with per-row magnitudes spread over
    1e-2..1e3 and 7 hot columns x50, the stress pattern of the reference's
    tests/test_rmsnorm_exact.py:117-124), w = 1 + N(0, 0.02..0.3), adaLN tables
    s1 = 1 + scale (bf16), sh, g ~ N(0, 0.1), o ~ N(0, 1), ridx in [0, R)."""
    g = gen(seed)
    x = torch.randn(S, N, generator=g)
    if stress:
        x = x * torch.logspace(-2, 3, S)[:, None]
        x[:, :7] *= 50
    x = x.to(torch.bfloat16)
    w = (1 + (0.3 if stress else 0.02) * torch.randn(N, generator=g)).to(torch.bfloat16)
    scale = (0.1 * torch.randn(R, N, generator=g)).to(torch.bfloat16)
    s1 = (1.0 + scale).contiguous()
    sh = (0.1 * torch.randn(R, N, generator=g)).to(torch.bfloat16)
    gt = (0.1 * torch.randn(R, N, generator=g)).to(torch.bfloat16)
    o = torch.randn(S, N, generator=g).to(torch.bfloat16)
    ridx = torch.randint(0, R, (S,), generator=g, dtype=torch.int32)
    return x, w, s1, sh, gt, o, ridx
