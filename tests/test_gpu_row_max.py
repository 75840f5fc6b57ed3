"""The quantizers' row max (a DPP reduction across the wave, then across the
waves of a row) with the row's unique largest magnitude placed in every lane,
wave and pass of the kernels' layouts, against the CPU oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits, from_bits, norm_inputs

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


@pytest.mark.parametrize("K", [1024, 5120, 14336])
def test_quant_max_in_every_chunk(K):
    """Row r holds small values and one spike in 8-element chunk r (a lane
    owns one chunk per pass), so every (pass, wave, lane) holds a row's max."""
    h = _h3mi()
    chunks = K // 8
    g = np.random.default_rng(K)
    x = (g.random((chunks, K), dtype=np.float32) * 2 - 1).astype(np.float32)
    r = np.arange(chunks)
    x[r, 8 * r + r % 8] = np.where(r % 2 == 0, 1.0, -1.0) * (3.0 + r / chunks)
    xb = O.f32_to_bf16_bits(x)
    print(f"[row max] quant K={K} rows={chunks}", flush=True)
    q, s = h.quantize_rowwise(from_bits(xb).cuda())
    oq, os_ = O.quant_rowwise(xb)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), oq)


@pytest.mark.parametrize("N", [1024, 5120, 5376])
def test_norm_quant_max_in_every_lane(N):
    """norm_mod_q and gate_norm_mod_q_ with each row's spike in another
    (512-element chunk, lane) slot, against the norm followed by the quantizer."""
    h = _h3mi()
    ch = (N + 511) // 512
    rows = ch * 64
    _, w, s1, sh, gt, o, _ = norm_inputs(rows, N, 1, seed=N, stress=False)
    g = np.random.default_rng(N + 1)
    x = (g.random((rows, N), dtype=np.float32) - 0.5).astype(np.float32)
    r = np.arange(rows)
    e = np.minimum((r % ch) * 512 + (r // ch) * 8 + r % 8, N - 1)
    x[r, e] = np.where(r % 3 == 0, -1.0, 1.0) * 40.0
    xd = from_bits(O.f32_to_bf16_bits(x)).cuda()
    ridx = torch.zeros(rows, dtype=torch.int32, device="cuda")
    wd, s1d, shd, od, gd = (t.cuda() for t in (w, s1, sh, o, gt))
    print(f"[row max] norm_mod_q N={N} rows={rows}", flush=True)
    ref_q, ref_s = h.quantize_rowwise(h.norm_mod(xd, wd, 1e-6, ridx, s1d, shd))
    q, qs = h.norm_mod_q(xd, wd, 1e-6, ridx, s1d, shd)
    assert torch.equal(q, ref_q) and torch.equal(qs.view(torch.int32), ref_s.view(torch.int32))
    xa, xb = xd.clone(), xd.clone()
    ref_q, ref_s = h.quantize_rowwise(h.gate_norm_mod_(xa, od, gd, wd, 1e-6, ridx, s1d, shd))
    q, qs = h.gate_norm_mod_q_(xb, od, gd, wd, 1e-6, ridx, s1d, shd)
    assert torch.equal(xa, xb)
    assert torch.equal(q, ref_q) and torch.equal(qs.view(torch.int32), ref_s.view(torch.int32))


def _hadamard_column(p):
    """Column p of the 256-point Sylvester Hadamard matrix (entries +-1)."""
    i = np.arange(256)
    pc = np.array([bin(v & p).count("1") for v in i])
    return np.where(pc % 2 == 0, 1.0, -1.0).astype(np.float32)


@pytest.mark.parametrize("K,act", [(1024, None), (5376, None), (3072, "swiglu")])
def test_convrot_max_at_every_position(K, act):
    """Row r's group r // 256 holds c * H e_p (p = r % 256), whose rotation
    H (c H e_p) / 16 = 16 c e_p is one spike: every position of the row holds
    its max in turn (SwiGLU: a = 4 everywhere, so c = silu(4))."""
    h = _h3mi()
    rows = K
    u = np.zeros((rows, K), np.float32)
    for r in range(rows):
        g0 = (r // 256) * 256
        u[r, g0:g0 + 256] = _hadamard_column(r % 256) * (1.0 if r % 2 == 0 else -1.0)
    if act == "swiglu":
        x = np.concatenate([np.full((rows, K), 4.0, np.float32), u], axis=1)
    else:
        x = u
    xb = O.f32_to_bf16_bits(x)
    print(f"[row max] convrot K={K} act={act} rows={rows}", flush=True)
    q, s = h.quantize_rowwise_convrot(from_bits(xb).cuda(), act)
    oq, os_ = O.convrot_quant(xb, act)
    assert np.array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), oq)
    # the spike is where the construction puts it
    assert np.array_equal(np.argmax(np.abs(oq.astype(np.int32)), axis=1), np.arange(rows))
