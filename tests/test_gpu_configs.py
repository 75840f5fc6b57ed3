"""The workload configurations at their own sizes on the GPU.

C1 (the fused QKV projection): 32768 x 5120 -> 15360 on bf16 N(0,1)
activations with exactly 0.1% of the elements scaled by 20 before the
per-token quantizer.
C2 (the MLP pair): up projection 32768 x 5120 -> 13824 and down projection
32768 x 13824 -> 5120 whose input is GELU-tanh of N(0,1), re-quantized per
token -- the shapes the reference checks bit for bit at full token counts
(tests/test_triton_gemm.py:9-26).
C4 (one H3-like DiT block at world_size=1): the block with this library's
fused norms against the same block with the eager sequence the fused kernels
replace (F.rms_norm -> mul_ -> add_, addcmul_), compared with torch.equal.

At these sizes the CPU oracle is too slow for whole tensors, so: the quantizer
is compared with the oracle on a sample of rows, the int32 accumulators with
torch._int_mm (hipBLASLt, an independent implementation), and the bf16 output
with the epilogue computed by separate torch GPU ops (each op one IEEE
rounding, which is the formula bf16(((f32(acc)*xs)*ws) + bias)).
Inputs come from bench.py's own generators, so these are the bench's data."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


def _bench():
    import bench
    return bench


def _linear_case(name):
    B = _bench()
    M, N, K, outl, kind, seed, _ = B.WORKLOADS[name]
    x, w, ws, bias = B.make_linear_inputs(torch, M, N, K, outl, seed=seed, kind=kind)
    return M, N, K, x, w, ws, bias


@pytest.mark.parametrize("name", ["qkv", "up", "down"])
def test_c1_c2_linear_full_size(name):
    """Quantize + GEMM + bias at the C1 (qkv, with its outliers) and C2 shapes:
    quantizer rows vs the oracle, int32 vs hipBLASLt, bf16 vs the torch
    epilogue, with and without bias (the counterpart of the reference's
    full-token-count check, tests/test_triton_gemm.py:9-26)."""
    h = _h3mi()
    M, N, K, x_cpu, w_cpu, ws_cpu, b_cpu = _linear_case(name)
    print(f"[c1/c2] {name}: M={M} N={N} K={K}", flush=True)
    x, w, ws, bias = (t.cuda() for t in (x_cpu, w_cpu, ws_cpu, b_cpu))
    xq, xs = h.quantize_rowwise(x)
    rows = np.unique(np.concatenate([np.arange(8), np.linspace(0, M - 1, 248).astype(np.int64)]))
    oq, os_ = O.quant_rowwise(bits(x_cpu[torch.from_numpy(rows)]))
    assert np.array_equal(xq[torch.from_numpy(rows).cuda()].cpu().numpy(), oq)
    assert np.array_equal(xs[torch.from_numpy(rows).cuda()].cpu().numpy().reshape(-1).view(np.uint32),
                          os_.view(np.uint32))
    del x
    acc = h.int8_mm_i32(xq, w)
    ref_acc = torch._int_mm(xq, w.t())
    assert torch.equal(acc, ref_acc)
    del acc
    out = h.int8_mm_scaled(xq, w, xs, ws)
    assert torch.equal(out, ((ref_acc.float() * xs) * ws[None, :]).to(torch.bfloat16))
    outb = h.int8_mm_scaled(xq, w, xs, ws, out=out, bias=bias)
    refb = (((ref_acc.float() * xs) * ws[None, :]) + bias.float()[None, :]).to(torch.bfloat16)
    assert torch.equal(outb, refb)


def test_c1_input_has_its_outliers():
    """The QKV workload's activations carry exactly 0.1% of their elements
    scaled by 20 (the C1 workload): most rows then hold a few elements far outside
    N(0,1), which sets their per-token scale."""
    M, N, K, x, _, _, _ = _linear_case("qkv")
    assert (M, N, K) == (32768, 15360, 5120)
    big = (x[:512].float().abs() > 6.0).sum()
    n_expect = 0.001 * 512 * K
    assert 0.5 * n_expect < float(big) < 1.2 * n_expect


def test_c2_down_input_is_gelu_of_normal():
    """The down projection's input is GELU-tanh of N(0,1) (the C2 workload): its
    rows are bounded below by min gelu = -0.17 and the per-token scales are
    those of such rows."""
    M, N, K, x, _, _, _ = _linear_case("down")
    assert (M, N, K) == (32768, 5120, 13824)
    xs = x[:64].float()
    assert float(xs.min()) > -0.171 and float(xs.max()) > 2.0


def test_c4_block_fused_equals_eager():
    """One H3-like DiT block (32768 video + 512 text tokens, hidden 5120,
    40 x 128 heads, W8A8 self-QKV/out, cross-Q/KV/out, MLP 5120 -> 13824 ->
    5120): the fused norms, gates and residuals give exactly the bytes of the
    eager sequence they replace."""
    h = _h3mi()
    B = _bench()
    fused = B.DiTBlockC4(torch, h, norms="fused")
    eager = B.DiTBlockC4(torch, h, norms="eager")
    assert torch.equal(fused.x0, eager.x0)
    print("[c4] fused block", flush=True)
    xf = fused.forward(fused.x0.clone())
    torch.cuda.synchronize()
    print("[c4] eager block", flush=True)
    xe = eager.forward(eager.x0.clone())
    torch.cuda.synchronize()
    diff = int((xf != xe).sum())
    assert diff == 0, f"{diff} elements differ between the fused and the eager block"
    assert not torch.equal(xf, fused.x0)
    del fused, eager
    torch.cuda.empty_cache()


def test_c4_block_fused_quant_handoff_equals_eager():
    """The same block with the norms that feed a linear quantizing h for it
    (norm_mod_q / gate_norm_mod_q_): the int8 rows are the quantizer's bytes,
    so the block output is unchanged."""
    h = _h3mi()
    B = _bench()
    fq = B.DiTBlockC4(torch, h, norms="fused", fuse_quant=True)
    xq = fq.forward(fq.x0.clone())
    torch.cuda.synchronize()
    del fq
    eager = B.DiTBlockC4(torch, h, norms="eager")
    xe = eager.forward(eager.x0.clone())
    torch.cuda.synchronize()
    assert torch.equal(xq, xe)
    del eager
    torch.cuda.empty_cache()
