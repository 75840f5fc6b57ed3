"""Fused norm kernels on the GPU, through the C ABI, against the CPU oracle
and against PyTorch eager on the same GPU.

Bar: with the correctly rounded rsqrt mode everything is bit-exact to the
oracle (sum-of-squares order included, checked through the exported per-row
var).  With the hardware rsqrt (the product default), var is bit-exact, rstd is
within 1 ulp of the correctly rounded value, and every output is bit-exact to
the oracle fed the GPU's rstd."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits, norm_inputs

pytestmark = pytest.mark.gpu

ORDERS = {1: (128, 4, 32), 2: (256, 4, 64)}


def _h3mi():
    import h3mi
    return h3mi


def _cuda(*ts):
    return [t.cuda() for t in ts]


CASES = [(64, 5120, 1), (33, 5376, 3), (16, 4, 1), (8, 1028, 2), (5, 12288, 2), (4, 32768, 1)]


@pytest.mark.parametrize("order", [1, 2])
@pytest.mark.parametrize("S,N,R", CASES)
def test_norm_mod_rn_bitexact(order, S, N, R):
    h = _h3mi()
    x, w, s1, sh, _, _, ridx = norm_inputs(S, N, R, seed=S + N)
    eps = 1e-6
    hout, var, rstd = h.norm_mod_ex(*_cuda(x, w), eps, ridx.cuda(), *_cuda(s1, sh), order=order,
                                    rsqrt_mode=1, stats=True)
    oh, ovar, orstd = O.norm_mod(bits(x), bits(w), eps, ridx.numpy(), bits(s1), bits(sh), order=ORDERS[order])
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), orstd.view(np.uint32))
    assert np.array_equal(bits(hout), oh)


@pytest.mark.parametrize("order", [0, 1, 2])
@pytest.mark.parametrize("S,N,R", CASES[:4])
def test_norm_mod_hw_rsqrt_downstream_bitexact(order, S, N, R):
    h = _h3mi()
    x, w, s1, sh, _, _, ridx = norm_inputs(S, N, R, seed=7 * S + N)
    eps = 1e-5
    hout, var, rstd = h.norm_mod_ex(*_cuda(x, w), eps, ridx.cuda(), *_cuda(s1, sh), order=order,
                                    rsqrt_mode=0, stats=True)
    o = ORDERS[order] if order else h.order_info(0)
    oh, ovar, orn = O.norm_mod(bits(x), bits(w), eps, ridx.numpy(), bits(s1), bits(sh), order=o)
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    d = np.abs(rstd.cpu().numpy().view(np.int32).astype(np.int64) - orn.view(np.int32).astype(np.int64))
    assert d.max() <= 1
    oh2, _, _ = O.norm_mod(bits(x), bits(w), eps, ridx.numpy(), bits(s1), bits(sh), order=o,
                           rstd=rstd.cpu().numpy())
    assert np.array_equal(bits(hout), oh2)
    # the plain entry point is the default order with the hardware rsqrt
    if order == 0:
        assert torch.equal(h.norm_mod(*_cuda(x, w), eps, ridx.cuda(), *_cuda(s1, sh)), hout)


@pytest.mark.parametrize("order", [1, 2])
@pytest.mark.parametrize("S,N,R", CASES)
def test_gate_norm_mod_rn_bitexact(order, S, N, R):
    h = _h3mi()
    x, w, s1, sh, g, o, ridx = norm_inputs(S, N, R, seed=3 * S + N, stress=False)
    eps = 1e-6
    xd = x.cuda()
    hout, var, rstd = h.gate_norm_mod_ex(xd, *_cuda(o, g, w), eps, ridx.cuda(), *_cuda(s1, sh), order=order,
                                         rsqrt_mode=1, stats=True)
    ox, oh, ovar, _ = O.gate_norm_mod(bits(x), bits(o), bits(g), bits(w), eps, ridx.numpy(), bits(s1), bits(sh),
                                      order=ORDERS[order])
    assert np.array_equal(bits(xd), ox)
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    assert np.array_equal(bits(hout), oh)


def test_gate_norm_mod_default_downstream_bitexact():
    h = _h3mi()
    x, w, s1, sh, g, o, ridx = norm_inputs(48, 5120, 2, seed=99, stress=False)
    xd = x.cuda()
    hout, var, rstd = h.gate_norm_mod_ex(xd, *_cuda(o, g, w), 1e-6, ridx.cuda(), *_cuda(s1, sh), stats=True)
    ox, oh, ovar, _ = O.gate_norm_mod(bits(x), bits(o), bits(g), bits(w), 1e-6, ridx.numpy(), bits(s1), bits(sh),
                                      order=h.order_info(0), rstd=rstd.cpu().numpy())
    assert np.array_equal(bits(xd), ox)
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    assert np.array_equal(bits(hout), oh)
    x2 = x.cuda()
    h2 = h.gate_norm_mod_(x2, *_cuda(o, g, w), 1e-6, ridx.cuda(), *_cuda(s1, sh))
    assert torch.equal(h2, hout) and torch.equal(x2, xd)


@pytest.mark.parametrize("S,N,R", [(64, 5120, 1), (33, 5376, 3), (7, 4, 2), (1000, 1028, 5)])
def test_gate_matches_oracle_and_eager(S, N, R):
    h = _h3mi()
    x, _, _, _, g, o, ridx = norm_inputs(S, N, R, seed=S * N, stress=False)
    xd = x.cuda()
    h.gate_(xd, o.cuda(), g.cuda(), ridx.cuda())
    assert np.array_equal(bits(xd), O.gate(bits(x), bits(o), bits(g), ridx.numpy()))
    # PyTorch eager on the GPU: x[rows].addcmul_(o[rows], g[r])
    ref = x.cuda()
    for r in range(R):
        rows = (ridx == r).nonzero().flatten().cuda()
        sub = ref[rows]
        sub.addcmul_(o.cuda()[rows], g.cuda()[r])
        ref[rows] = sub
    assert torch.equal(xd, ref)


def test_out_of_range_ridx_rows_untouched():
    h = _h3mi()
    x, w, s1, sh, g, o, ridx = norm_inputs(8, 512, 2, seed=4, stress=False)
    ridx[3] = 7
    ridx[5] = -1
    xd = x.cuda()
    h.gate_(xd, o.cuda(), g.cuda(), ridx.cuda())
    assert torch.equal(xd[3].cpu(), x[3]) and torch.equal(xd[5].cpu(), x[5])


def test_rejects_aliasing_and_bad_shapes():
    h = _h3mi()
    from h3mi._lib import H3miError
    x = torch.randn(4, 64, device="cuda").to(torch.bfloat16)
    g = torch.randn(1, 64, device="cuda").to(torch.bfloat16)
    ridx = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(H3miError):
        h.gate_(x, x, g, ridx)
    with pytest.raises(ValueError):
        h.gate_(x, x[:, :32].contiguous(), g, ridx)
    x6 = torch.randn(4, 66, device="cuda").to(torch.bfloat16)
    with pytest.raises(H3miError):
        h.gate_(x6, x6.clone(), torch.ones(1, 66, device="cuda", dtype=torch.bfloat16), ridx)


# Persistent row-stream kernels (N <= 8192, product order): rows handled by one
# wave span several strides, tables staged in LDS (one table row), mixed table
# rows (two segments: the majority row staged, the rest from global memory),
# random table rows, the widest stream row and the first row past it, fewer
# rows than one workgroup has waves, and more than 256 rows per workgroup
# (the table-row count takes several steps), with one table row and with two
# segments.  gate_norm_mod_ runs one row per workgroup where N is a multiple of
# 1024 (5120, 8192, 1024, 2048 here) or 1024 IT + 256 (5376, 1280, 7424: the
# last 256 elements' elementwise work one element per thread), and the row
# stream otherwise.
STREAM_CASES = [
    ("uniform", 3001, 5120, 1),
    ("few", 5, 5120, 2),
    ("segments", 2603, 5120, 2),
    ("random", 2500, 5376, 3),
    ("uniform", 3000, 5376, 1),
    ("segments", 2603, 5376, 2),
    ("few", 3, 5376, 2),
    ("segments", 1500, 1280, 2),
    ("uniform", 700, 7424, 1),
    ("widest", 1100, 8192, 2),
    ("past", 300, 8196, 1),
    ("tail", 2049, 1028, 1),
    ("uniform", 70001, 1024, 1),
    ("segments", 70001, 1024, 2),
    ("uniform", 600, 2048, 1),
]


def _stream_inputs(kind, S, N, R, seed):
    x, w, s1, sh, g, o, ridx = norm_inputs(S, N, R, seed=seed, stress=False)
    if kind == "segments":  # a short first segment with its own table row
        ridx[:] = 0
        ridx[:301] = 1
    elif kind in ("uniform", "past", "tail"):
        ridx[:] = R - 1
    return x, w, s1, sh, g, o, ridx


@pytest.mark.parametrize("kind,S,N,R", STREAM_CASES)
def test_stream_norm_mod_bitexact(kind, S, N, R):
    h = _h3mi()
    x, w, s1, sh, _, _, ridx = _stream_inputs(kind, S, N, R, seed=S + N + 11)
    hout, var, rstd = h.norm_mod_ex(*_cuda(x, w), 1e-6, ridx.cuda(), *_cuda(s1, sh), rsqrt_mode=1, stats=True)
    oh, ovar, orstd = O.norm_mod(bits(x), bits(w), 1e-6, ridx.numpy(), bits(s1), bits(sh), order=h.order_info(0))
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), orstd.view(np.uint32))
    assert np.array_equal(bits(hout), oh)


@pytest.mark.parametrize("kind,S,N,R", STREAM_CASES)
def test_stream_gate_norm_mod_bitexact(kind, S, N, R):
    h = _h3mi()
    x, w, s1, sh, g, o, ridx = _stream_inputs(kind, S, N, R, seed=2 * S + N)
    xd = x.cuda()
    hout, var, rstd = h.gate_norm_mod_ex(xd, *_cuda(o, g, w), 1e-6, ridx.cuda(), *_cuda(s1, sh), rsqrt_mode=1,
                                         stats=True)
    ox, oh, ovar, _ = O.gate_norm_mod(bits(x), bits(o), bits(g), bits(w), 1e-6, ridx.numpy(), bits(s1), bits(sh),
                                      order=h.order_info(0))
    assert np.array_equal(bits(xd), ox)
    assert np.array_equal(var.cpu().numpy().view(np.uint32), ovar.view(np.uint32))
    assert np.array_equal(bits(hout), oh)


@pytest.mark.parametrize("kind,S,N,R", STREAM_CASES)
def test_stream_gate_bitexact(kind, S, N, R):
    h = _h3mi()
    x, _, _, _, g, o, ridx = _stream_inputs(kind, S, N, R, seed=3 * S + N)
    xd = x.cuda()
    h.gate_(xd, o.cuda(), g.cuda(), ridx.cuda())
    assert np.array_equal(bits(xd), O.gate(bits(x), bits(o), bits(g), ridx.numpy()))


@pytest.mark.parametrize("N,R", [(5120, 2), (1028, 2), (5120, 1), (5376, 1)])
def test_stream_out_of_range_rows_untouched(N, R):
    """Rows whose table index is out of range are left unwritten (h and x),
    both when they are a workgroup's majority and when they are not, with one
    table row (R = 1) as with two."""
    h = _h3mi()
    S = 2100
    x, w, s1, sh, g, o, ridx = norm_inputs(S, N, R, seed=N + R, stress=False)
    ridx[:] = R - 1
    bad = torch.zeros(S, dtype=torch.bool)
    bad[5::7] = True
    bad[1000:1400] = True
    ridx[bad] = torch.where(torch.arange(S)[bad] % 2 == 0, torch.tensor(-1, dtype=torch.int32),
                            torch.tensor(R, dtype=torch.int32))
    good = (~bad).nonzero().flatten().numpy()
    sentinel = torch.full((S, N), 7.0, dtype=torch.bfloat16, device="cuda")
    hout = h.norm_mod_ex(*_cuda(x, w), 1e-6, ridx.cuda(), *_cuda(s1, sh), rsqrt_mode=1, h=sentinel.clone())
    rg = torch.full((len(good),), R - 1, dtype=torch.int32)
    oh, _, _ = O.norm_mod(bits(x)[good], bits(w), 1e-6, rg.numpy(), bits(s1), bits(sh), order=h.order_info(0))
    assert np.array_equal(bits(hout)[good], oh)
    assert torch.equal(hout[bad.cuda()], sentinel[bad.cuda()])
    xd = x.cuda()
    hg = h.gate_norm_mod_ex(xd, *_cuda(o, g, w), 1e-6, ridx.cuda(), *_cuda(s1, sh), rsqrt_mode=1, h=sentinel.clone())
    ox, oh, _, _ = O.gate_norm_mod(bits(x)[good], bits(o)[good], bits(g), bits(w), 1e-6, rg.numpy(), bits(s1),
                                   bits(sh), order=h.order_info(0))
    assert np.array_equal(bits(xd)[good], ox) and np.array_equal(bits(hg)[good], oh)
    assert torch.equal(xd[bad.cuda()], x.cuda()[bad.cuda()]) and torch.equal(hg[bad.cuda()], sentinel[bad.cuda()])
    xg = x.cuda()
    h.gate_(xg, o.cuda(), g.cuda(), ridx.cuda())
    assert np.array_equal(bits(xg)[good], O.gate(bits(x)[good], bits(o)[good], bits(g), rg.numpy()))
    assert torch.equal(xg[bad.cuda()], x.cuda()[bad.cuda()])
