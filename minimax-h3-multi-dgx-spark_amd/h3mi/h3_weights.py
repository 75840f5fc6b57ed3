"""H3 DiT INT8 linear layers: the real model's shapes and its checkpoint format.

Shapes (reference bench/gemm_peak.py:7-8): hidden 5376, 56 heads x 128,
  qkv 5376 -> 21504, out 7168 -> 5376, fc1 5376 -> 28672, fc2 14336 -> 5376,
at 19,200 or 38,400 tokens per GPU (tests/test_triton_gemm.py:8).
Checkpoint keys (tests/bench_linear.py:12,25-29): blocks.<i>.<module>.weight
(int8 [N, K]) and blocks.<i>.<module>.weight_scale (per-output-channel scale,
any shape with N elements, or one element for a per-tensor scale), read with
safetensors (no code executes from the file).
"""
import torch

HIDDEN = 5376
HEADS, HEAD_DIM = 56, 128
LAYERS = {"qkv": "attn.qkv_proj", "out": "attn.out_proj", "fc1": "mlp.fc1", "fc2": "mlp.fc2"}
SHAPES = {"qkv": (5376, 21504), "out": (7168, 5376), "fc1": (5376, 28672), "fc2": (14336, 5376)}  # (K, N)
TOKENS = (19200, 38400)


def keys(layer, block=0):
    """(weight key, weight_scale key) of one linear layer in an H3 checkpoint."""
    if layer not in LAYERS:
        raise KeyError(f"unknown H3 linear '{layer}' (one of {sorted(LAYERS)})")
    base = f"blocks.{int(block)}.{LAYERS[layer]}"
    return base + ".weight", base + ".weight_scale"


def weight_scale_vector(scale, n):
    """A checkpoint's weight_scale as the fp32 [N] vector the GEMM takes (a
    per-tensor scale is repeated), as the reference test builds it
    (tests/test_triton_gemm.py:13: s.reshape(-1).float())."""
    s = scale.reshape(-1).float()
    if s.numel() == 1:
        s = s.expand(n)
    if s.numel() != n:
        raise ValueError(f"weight_scale has {s.numel()} elements for {n} output channels")
    return s.contiguous()


def load_linear(path, layer, block=0, device="cpu"):
    """(w int8 [N, K], ws fp32 [N]) of one linear layer from an H3 INT8
    safetensors checkpoint, on `device`."""
    from safetensors import safe_open
    kw, ks = keys(layer, block)
    with safe_open(path, "pt", device="cpu") as f:
        present = set(f.keys())
        for k in (kw, ks):
            if k not in present:
                raise KeyError(f"{path}: no tensor '{k}'")
        w = f.get_tensor(kw)
        s = f.get_tensor(ks)
    if w.dtype != torch.int8 or w.dim() != 2:
        raise ValueError(f"{kw}: expected a 2-D int8 weight, got {tuple(w.shape)} {w.dtype}")
    if layer in SHAPES and tuple(w.shape) != (SHAPES[layer][1], SHAPES[layer][0]):
        raise ValueError(f"{kw}: shape {tuple(w.shape)} is not H3's {(SHAPES[layer][1], SHAPES[layer][0])}")
    return w.contiguous().to(device), weight_scale_vector(s, w.shape[0]).to(device)
