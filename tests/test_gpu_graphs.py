"""The HIP kernels under HIP-graph capture (torch.cuda.CUDAGraph).

Every entry point launches on the caller's stream, allocates nothing and
never synchronises, so a chain of them can be captured once and replayed.
The test captures quantize -> GEMM (a small grid and a resident one), norm_mod -> gate_norm_mod_ -> gate_, the
norm -> quantizer fusion, the ConvRot quantizer (SwiGLU) and the q/k
RMSNorm + RoPE, then replays the graph several times with new inputs copied
in between (and eager work and synchronisations between the replays) and
checks every replay against the same calls run eagerly.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


def _inputs(g, dev):
    M, N, K, S, Nn, H, D = 512, 768, 1024, 300, 1280, 4, 128
    return {
        "x": torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev),
        "w": torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev),
        "ws": (1e-3 + 9e-3 * torch.rand(N, generator=g)).to(dev),
        "bias": (0.02 * torch.randn(N, generator=g)).to(torch.bfloat16).to(dev),
        "xn": torch.randn(S, Nn, generator=g).to(torch.bfloat16).to(dev),
        "o": torch.randn(S, Nn, generator=g).to(torch.bfloat16).to(dev),
        "wn": (1 + 0.02 * torch.randn(Nn, generator=g)).to(torch.bfloat16).to(dev),
        "s1": (1.0 + (0.1 * torch.randn(2, Nn, generator=g)).to(torch.bfloat16)).to(dev),
        "sh": (0.1 * torch.randn(2, Nn, generator=g)).to(torch.bfloat16).to(dev),
        "gt": (0.1 * torch.randn(2, Nn, generator=g)).to(torch.bfloat16).to(dev),
        "ridx": torch.randint(0, 2, (S,), generator=g, dtype=torch.int32).to(dev),
        "xc": torch.randn(S, 2 * 1024, generator=g).to(torch.bfloat16).to(dev),
        "qkv": torch.randn(S, 3 * H * D, generator=g).to(torch.bfloat16).to(dev),
        "qw": (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev),
        "tab": torch.randn(1, S, D // 2, 2, 2, generator=g).to(torch.bfloat16).to(dev),
        # a grid of 512 256x256 tiles: the resident configuration, two tiles per workgroup
        "xb": torch.randn(4096, 512, generator=g).to(torch.bfloat16).to(dev),
        "wb": torch.randint(-127, 128, (8192, 512), generator=g, dtype=torch.int8).to(dev),
        "wsb": (1e-3 + 9e-3 * torch.rand(8192, generator=g)).to(dev),
    }


def _chain(h, t):
    """The captured work; returns the tensors to compare.  Mutates xn and qkv in place."""
    H, D = 4, 128
    S = t["xn"].shape[0]
    xq, xs = h.quantize_rowwise(t["x"])
    y = h.int8_mm_scaled(xq, t["w"], xs, t["ws"], bias=t["bias"])
    hn = h.norm_mod(t["xn"], t["wn"], 1e-6, t["ridx"], t["s1"], t["sh"])
    h2 = h.gate_norm_mod_(t["xn"], t["o"], t["gt"], t["wn"], 1e-6, t["ridx"], t["s1"], t["sh"])
    hq, q8, qs = h.norm_mod_q(t["xn"], t["wn"], 1e-6, t["ridx"], t["s1"], t["sh"], want_h=True)
    h.gate_(t["xn"], t["o"], t["gt"], t["ridx"])
    cq, cs = h.quantize_rowwise_convrot(t["xc"], "swiglu")
    q = t["qkv"][:, :H * D].view(1, S, H, D)
    k = t["qkv"][:, H * D:2 * H * D].view(1, S, H, D)
    h.rms_rope_split_half_(q, k, t["tab"], t["qw"], t["qw"], epsilon=1e-6)
    xqb, xsb = h.quantize_rowwise(t["xb"])
    yb = h.int8_mm_scaled(xqb, t["wb"], xsb, t["wsb"])
    return [xq, xs, y, hn, h2, hq, q8, qs, cq, cs, yb]


def test_capture_and_replay_matches_eager():
    h = _h3mi()
    dev = torch.device("cuda", 0)
    static = _inputs(torch.Generator().manual_seed(0), dev)
    # warm up on a side stream (first calls cache per-device state), as torch requires before capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work = {k: v.clone() for k, v in static.items()}
        _chain(h, work)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _chain(h, static)
    for rep in range(4):
        fresh = _inputs(torch.Generator().manual_seed(100 + rep), dev)
        for k in static:
            static[k].copy_(fresh[k])
        graph.replay()
        torch.cuda.synchronize()
        eager_in = {k: v.clone() for k, v in fresh.items()}
        want = _chain(h, eager_in)                  # eager work between replays
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, want)):
            assert torch.equal(a, b), f"replay {rep}: output {i} differs from eager"
        assert torch.equal(static["xn"], eager_in["xn"]) and torch.equal(static["qkv"], eager_in["qkv"])
