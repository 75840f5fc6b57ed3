"""ConvRot quantizer on the GPU against the oracle.

h3mi.quantize_rowwise_convrot (C ABI h3mi_quant_convrot_i8) stands in for
comfy-kitchen's _C.quantize_int8_rowwise_convrot64 as the reference calls it
(comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95,
tests/bench_linear.py:33-40).  Bar: q and s bit-identical to the oracle's
h3o_convrot_quant (whose agreement with comfy-kitchen is unpinned; the oracle
is pinned to the Hadamard / exp / silu mathematics in
tests/test_oracle_convrot.py).  Covers every kernel shape class (one, two and
four waves per row, partial last pass), SwiGLU inputs, padded row strides,
zero / tiny / outlier / integer-valued rows (the last put many quotients on
half-integers, so the exact-divide branch runs), the real H3 widths at full
row counts (sampled rows), and that nothing is written past q and s.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import bits, gen

pytestmark = pytest.mark.gpu


def _h3mi():
    import h3mi
    return h3mi


def _rows(M, kin, seed, special=True):
    g = gen(seed)
    x = torch.randn(M, kin, generator=g)
    if M * kin > 0:
        n_out = max(1, int(0.001 * M * kin))
        x.view(-1)[torch.randperm(M * kin, generator=g)[:n_out]] *= 20
    if special and M >= 6:
        x[1] = 0                                                    # zero row
        x[2] *= 1e-33                                               # tiny row (w below 2^-100)
        x[3] = torch.randint(-3, 4, (kin,), generator=g).float()   # integers: quotients on half-integers
        x[4] = 1.0                                                  # constant row
        x[5, 11] = 4e4                                              # one dominant element
    return x.to(torch.bfloat16)


def _check(x, act, ldx_pad=0, seed=0):
    h = _h3mi()
    M, kin = x.shape
    if ldx_pad:
        buf = torch.zeros(M, kin + ldx_pad, dtype=torch.bfloat16)
        buf[:, :kin] = x
        xd = buf.cuda()[:, :kin]
    else:
        xd = x.cuda()
    K = kin // 2 if act == "swiglu" else kin
    # guard bytes after q and s: the kernel must not write past them
    qbuf = torch.full((M * K + 4096,), 0x5A, dtype=torch.int8, device="cuda")
    sbuf = torch.full((M + 64,), 7.0, dtype=torch.float32, device="cuda")
    q, s = h.quantize_rowwise_convrot(xd, act, xq=qbuf[: M * K].view(M, K), xs=sbuf[:M].view(M, 1))
    torch.cuda.synchronize()
    oq, os_ = O.convrot_quant(bits(x), act)
    gq, gs = q.cpu().numpy(), s.cpu().numpy().reshape(-1)
    bad = np.argwhere(gq != oq)
    assert bad.size == 0, (f"{len(bad)} q mismatches, first at {bad[:5].tolist()}, per row "
                           f"{np.bincount(bad[:, 0], minlength=M).tolist()[:16]}")
    assert np.array_equal(gs.view(np.uint32), os_.view(np.uint32))
    assert bool((qbuf[M * K:] == 0x5A).all()) and bool((sbuf[M:] == 7.0).all())


@pytest.mark.parametrize("K", [256, 512, 1024, 1280, 5120, 5376, 7168, 8192, 8448, 14336, 16384, 16640, 32768])
def test_convrot_matches_oracle(K):
    print(f"[convrot] act=none K={K}", flush=True)
    _check(_rows(9, K, seed=K), None)


@pytest.mark.parametrize("K", [256, 1024, 5376, 7168, 8448, 14336, 16640, 32768])
def test_convrot_swiglu_matches_oracle(K):
    print(f"[convrot] act=swiglu K={K}", flush=True)
    _check(_rows(9, 2 * K, seed=K + 1), "swiglu")


@pytest.mark.parametrize("act,K,M", [(None, 5376, 2053), (None, 14336, 515), ("swiglu", 5376, 1027),
                                     ("swiglu", 14336, 258), (None, 1024, 4099)])
def test_convrot_many_rows(act, K, M):
    print(f"[convrot] many rows act={act} K={K} M={M}", flush=True)
    _check(_rows(M, 2 * K if act else K, seed=M), act)


@pytest.mark.parametrize("act", [None, "swiglu"])
def test_convrot_padded_row_stride(act):
    print(f"[convrot] padded ldx act={act}", flush=True)
    _check(_rows(13, 2 * 1280 if act else 1280, seed=99), act, ldx_pad=72)


@pytest.mark.parametrize("act,K,M", [(None, 5376, 19200), ("swiglu", 14336, 19200)])
def test_convrot_h3_widths_full_rows_sampled(act, K, M):
    """Real H3 widths at a full token count; the oracle checks 48 spread rows."""
    print(f"[convrot] H3 act={act} K={K} M={M}", flush=True)
    h = _h3mi()
    kin = 2 * K if act else K
    x = _rows(M, kin, seed=K, special=False).cuda()
    q, s = h.quantize_rowwise_convrot(x, act)
    q2, s2 = h.quantize_rowwise_convrot(x, act)
    assert torch.equal(q, q2) and torch.equal(s, s2)
    rows = np.unique(np.linspace(0, M - 1, 48).astype(np.int64))
    oq, os_ = O.convrot_quant(bits(x[rows]), act)
    assert np.array_equal(q[rows].cpu().numpy(), oq)
    assert np.array_equal(s[rows].cpu().numpy().reshape(-1).view(np.uint32), os_.view(np.uint32))


def test_convrot_swiglu_special_values_match_oracle():
    """SwiGLU rows whose a half holds zeros, subnormals, values around 2^-25
    (where e^-|a| rounds to 1), around 32 and 128 (where 1 + e^-|a| rounds to
    1 and the exponent's argument clamps at -86) and huge values of both
    signs, quantized against the oracle."""
    K = 1024
    g = gen(5)
    # magnitudes stay below ~1e30 so that no 256-element Hadamard sum overflows
    edges = torch.tensor([0.0, -0.0, 1e-40, -1e-40, 2.0 ** -26, 2.0 ** -25, -(2.0 ** -25), 2.0 ** -24, 31.9, 32.0,
                          -32.0, 127.0, -127.0, 128.0, -128.0, 200.0, -200.0, 1.0e30, -1.0e30, 86.0, -86.0, -90.0])
    x = torch.randn(8, 2 * K, generator=g)
    x[:, :K] = edges[torch.randint(0, len(edges), (8, K), generator=g)] * (1 + 0 * x[:, :K])
    x[0, :K] = x[0, :K] * 0 + edges.repeat(K // len(edges) + 1)[:K]
    x[1, :K] = 1e-39                       # all subnormal: silu = a / 2
    x[2, :K] = -1.0e30                     # all huge negative: silu = a e^-86
    _check(x.to(torch.bfloat16), "swiglu")


def test_convrot_swiglu_every_bf16_a_value():
    """One SwiGLU product per row: row i has a[0] = the i-th bf16 bit pattern
    (NaN and infinity patterns left out), b[0] = 1, and a = 1, b = 0 elsewhere,
    so s = fl(|silu(a[0])| / 2032) and the other elements are zero products of
    in-range values.  A wave pass whose values all lie in exponent fields
    102-133 reads silu from the kernel's table, the others evaluate it, so this
    covers every table entry and both boundaries, both signs, against the
    oracle."""
    K = 1024
    pat = np.arange(65536, dtype=np.uint32)
    pat = pat[((pat >> 7) & 0xFF) != 0xFF].astype(np.uint16)
    xb = np.zeros((len(pat), 2 * K), np.uint16)
    xb[:, 1:K] = 0x3F80      # a = 1
    xb[:, 0] = pat
    xb[:, K] = 0x3F80        # b[0] = 1, b = 0 elsewhere
    _check(torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16), "swiglu")


def test_convrot_swiglu_concurrent_streams():
    """SwiGLU calls on two streams at once (each call refills the shared silu
    table while the other's quantizer may be reading it): every call's output
    equals the oracle's."""
    h = _h3mi()
    K = 5376
    xs = [_rows(96, 2 * K, seed=40 + i) for i in range(2)]
    want = [O.convrot_quant(bits(x), "swiglu") for x in xs]
    xd = [x.cuda() for x in xs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    torch.cuda.synchronize()
    for _ in range(8):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                outs[i].append(h.quantize_rowwise_convrot(xd[i], "swiglu"))
    torch.cuda.synchronize()
    for i in range(2):
        for q, sc in outs[i]:
            assert np.array_equal(q.cpu().numpy(), want[i][0])
            assert np.array_equal(sc.cpu().numpy().reshape(-1).view(np.uint32), want[i][1].view(np.uint32))


def test_convrot_empty_and_rejects():
    h = _h3mi()
    x = torch.zeros(0, 1024, dtype=torch.bfloat16, device="cuda")
    q, s = h.quantize_rowwise_convrot(x)
    assert q.shape == (0, 1024) and s.shape == (0, 1)
    from h3mi._lib import H3miError
    with pytest.raises(H3miError):
        h.quantize_rowwise_convrot(torch.zeros(4, 1000, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        h.quantize_rowwise_convrot(torch.zeros(4, 1024, dtype=torch.bfloat16, device="cuda"), act="gelu")
