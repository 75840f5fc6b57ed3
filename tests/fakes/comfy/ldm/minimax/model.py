"""Stand-in for comfy.ldm.minimax.model (tests and the block benchmark only):
an H3-like DiT block with the eager norm / adaLN / gate / residual sequence
the fused kernels replace (comfyui_nodes/h3-fuse-graph/h3_fuse_kernels.py:3-7)
and the forward signature the patch mirrors (h3_fuse_patch.py:96).

linear: optional callable(x, module) used for every projection (e.g. a W8A8
path); by default a bf16 torch linear."""
import torch
import torch.nn as nn
import torch.nn.functional as F


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6, dtype=torch.bfloat16, device=None):
        super().__init__()
        self.normalized_shape = (dim,)
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype, device=device))
        self.comfy_cast_weights = False
        self.weight_function = []
        self.bias_function = []

    def forward(self, x):
        return F.rms_norm(x, self.normalized_shape, self.weight, self.eps)


class Linear(nn.Module):
    def __init__(self, din, dout, dtype=torch.bfloat16, device=None, linear=None):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(dout, din, dtype=torch.float32, device=device).mul_(din ** -0.5).to(dtype))
        self.linear = linear

    def forward(self, x):
        if self.linear is not None:
            return self.linear(x, self)
        return F.linear(x, self.weight)


class Attention(nn.Module):
    def __init__(self, dim, heads, dtype=torch.bfloat16, device=None, linear=None):
        super().__init__()
        self.heads = heads
        self.qkv_proj = Linear(dim, 3 * dim, dtype, device, linear)
        self.out_proj = Linear(dim, dim, dtype, device, linear)

    def forward(self, h, rope_freqs=None, transformer_options={}):  # noqa: B006
        s, d = h.shape
        q, k, v = self.qkv_proj(h).view(s, 3, self.heads, d // self.heads).permute(1, 2, 0, 3)
        o = F.scaled_dot_product_attention(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0))[0]
        return self.out_proj(o.permute(1, 0, 2).reshape(s, d))


class MLP(nn.Module):
    def __init__(self, dim, hidden, dtype=torch.bfloat16, device=None, linear=None):
        super().__init__()
        self.fc1 = Linear(dim, hidden, dtype, device, linear)
        self.fc2 = Linear(hidden, dim, dtype, device, linear)

    def forward(self, h):
        return self.fc2(F.gelu(self.fc1(h), approximate="tanh"))


class AdaLN(nn.Module):
    def __init__(self, tdim, dim, device=None):
        super().__init__()
        self.proj = nn.Linear(tdim, 6 * dim, device=device, dtype=torch.float32)

    def forward(self, t_emb):
        return (0.1 * self.proj(t_emb)).chunk(6, dim=-1)


class DiTBlock(nn.Module):
    def __init__(self, dim, heads, mlp_hidden, tdim=256, eps=1e-6, dtype=torch.bfloat16, device=None, linear=None):
        super().__init__()
        self.norm1 = RMSNorm(dim, eps, dtype, device)
        self.norm2 = RMSNorm(dim, eps, dtype, device)
        self.attn = Attention(dim, heads, dtype, device, linear)
        self.mlp = MLP(dim, mlp_hidden, dtype, device, linear)
        self.adaln_proj = AdaLN(tdim, dim, device)

    def forward(self, x, t_emb, mod_segments, rope_freqs, transformer_options={}, attention=None):  # noqa: B006
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = self.adaln_proj(t_emb)
        dt = x.dtype
        h = self.norm1(x)
        for a, b, row in mod_segments:
            h[a:b].mul_(1.0 + scale_msa[row].to(dt)).add_(shift_msa[row].to(dt))
        attention = self.attn if attention is None else attention
        o = attention(h, rope_freqs=rope_freqs, transformer_options=transformer_options)
        for a, b, row in mod_segments:
            x[a:b].addcmul_(o[a:b], gate_msa[row].to(dt))
        h = self.norm2(x)
        for a, b, row in mod_segments:
            h[a:b].mul_(1.0 + scale_mlp[row].to(dt)).add_(shift_mlp[row].to(dt))
        o = self.mlp(h)
        for a, b, row in mod_segments:
            x[a:b].addcmul_(o[a:b], gate_mlp[row].to(dt))
        return x


class MiniMaxH3Model(nn.Module):
    def __init__(self, blocks):
        super().__init__()
        self.blocks = nn.ModuleList(blocks)

    def _forward(self, x, t_emb, mod_segments, rope_freqs=None):
        for blk in self.blocks:
            x = blk(x, t_emb, mod_segments, rope_freqs)
        return x
