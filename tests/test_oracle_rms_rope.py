"""Pins of the oracle's q/k RMSNorm + split-half RoPE
(oracle/h3_oracle.c: h3o_rms_rope_split_half).

The reference calls comfy-kitchen's ck.rms_rope_split_half_
(comfyui_nodes/minimax-h3-sp/minimax_sp/sp_forward.py:279-296); comfy-kitchen is
not vendored, so agreement with its bytes is unpinned.  The definition is the
eager sequence F.rms_norm -> rotate (pairs (i, i + rot/2)) in fp32 -> bf16.
These tests fix it with torch CPU ops (independent code) given the rstd, the
sum-of-squares order pinned in tests/test_oracle_pins.py, and known answers
that a wrong pairing (interleaved instead of split-half), a wrong table entry
or a wrong untouched tail would change.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_bits(b):
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def _inputs(S, H, D, rot, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(S, H, D, generator=g) * torch.logspace(-1, 1, S)[:, None, None]).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    ang = torch.rand(S, rot // 2, generator=g) * 6.3
    tab = torch.stack([torch.stack([ang.cos(), -ang.sin()], -1), torch.stack([ang.sin(), ang.cos()], -1)], -2)
    return x, w, tab.to(torch.bfloat16)


def _torch_ref(x, w, tab, rot, rstd):
    """Same definition in torch CPU fp32 ops, rstd given per row."""
    S, H, D = x.shape
    y = (w.float() * (torch.from_numpy(rstd).reshape(S, H, 1) * x.float())).to(torch.bfloat16).float()
    out = y.clone()
    h = rot // 2
    if rot:
        a, b = y[..., :h], y[..., h:rot]
        R = tab.float()[:, None]                                   # [S, 1, h, 2, 2]
        out[..., :h] = R[..., 0, 0] * a + R[..., 0, 1] * b
        out[..., h:rot] = R[..., 1, 0] * a + R[..., 1, 1] * b
    return out.to(torch.bfloat16)


@pytest.mark.parametrize("D,rot", [(128, 128), (128, 64), (128, 0), (64, 64), (256, 128), (128, 16)])
def test_matches_torch_cpu_ops_given_rstd(D, rot):
    x, w, tab = _inputs(7, 3, D, rot, seed=D + rot)
    out, rs = O.rms_rope_split_half(_bits(x), _bits(tab), _bits(w), 1e-6, rot)
    ref = _torch_ref(x, w, tab, rot, rs)
    assert np.array_equal(out, _bits(ref))


def test_rstd_is_rn_of_the_pinned_sum():
    x, w, tab = _inputs(5, 2, 128, 128, seed=1)
    _, rs = O.rms_rope_split_half(_bits(x), _bits(tab), _bits(w), 1e-6, 128)
    xf = O.bf16_bits_to_f32(_bits(x)).reshape(10, 128)
    for r in range(10):
        tot = O.row_sumsq(xf[r], (256, 4, 64))
        var = np.float32(np.float32(tot) / np.float32(128)) + np.float32(1e-6)
        assert rs.reshape(-1)[r] == np.float32(O.rsqrt_rn(var))


def test_identity_table_leaves_the_norm():
    x, w, _ = _inputs(4, 2, 128, 128, seed=2)
    eye = torch.zeros(4, 64, 2, 2)
    eye[..., 0, 0] = 1
    eye[..., 1, 1] = 1
    out, _ = O.rms_rope_split_half(_bits(x), _bits(eye.to(torch.bfloat16)), _bits(w), 1e-6, 128)
    plain, _ = O.rms_rope_split_half(_bits(x), None, _bits(w), 1e-6, 0)
    assert np.array_equal(out, plain)


def test_quarter_turn_pairs_split_halves():
    # R = [[0, -1], [1, 0]]: out[i] = -y[i + 64], out[i + 64] = y[i]  (split-half pairing;
    # an interleaved pairing would mix y[2i] and y[2i+1] instead)
    x, w, _ = _inputs(3, 2, 128, 128, seed=3)
    R = torch.zeros(3, 64, 2, 2)
    R[..., 0, 1] = -1
    R[..., 1, 0] = 1
    out, _ = O.rms_rope_split_half(_bits(x), _bits(R.to(torch.bfloat16)), _bits(w), 1e-6, 128)
    y, _ = O.rms_rope_split_half(_bits(x), None, _bits(w), 1e-6, 0)
    assert np.array_equal(out[..., :64], y[..., 64:] ^ np.uint16(0x8000))
    assert np.array_equal(out[..., 64:], y[..., :64])


def test_partial_rotation_leaves_the_tail():
    x, w, tab = _inputs(3, 4, 128, 32, seed=4)
    out, _ = O.rms_rope_split_half(_bits(x), _bits(tab), _bits(w), 1e-6, 32)
    y, _ = O.rms_rope_split_half(_bits(x), None, _bits(w), 1e-6, 0)
    assert np.array_equal(out[..., 32:], y[..., 32:])
    assert not np.array_equal(out[..., :32], y[..., :32])


def test_table_rows_follow_the_token():
    # token 1's table is the identity, token 0's a quarter turn: only token 0 changes
    x, w, _ = _inputs(2, 1, 64, 64, seed=5)
    R = torch.zeros(2, 32, 2, 2)
    R[0, :, 0, 1], R[0, :, 1, 0] = -1, 1
    R[1, :, 0, 0], R[1, :, 1, 1] = 1, 1
    out, _ = O.rms_rope_split_half(_bits(x), _bits(R.to(torch.bfloat16)), _bits(w), 1e-6, 64)
    y, _ = O.rms_rope_split_half(_bits(x), None, _bits(w), 1e-6, 0)
    assert np.array_equal(out[1], y[1]) and not np.array_equal(out[0], y[0])


def test_close_to_float64_rmsnorm_and_rotation():
    x, w, tab = _inputs(6, 2, 128, 128, seed=6)
    out, _ = O.rms_rope_split_half(_bits(x), _bits(tab), _bits(w), 1e-6, 128)
    xd = x.double()
    y = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    R = tab.double()[:, None]
    ref = y.clone()
    ref[..., :64] = R[..., 0, 0] * y[..., :64] + R[..., 0, 1] * y[..., 64:]
    ref[..., 64:] = R[..., 1, 0] * y[..., :64] + R[..., 1, 1] * y[..., 64:]
    got = _from_bits(out).double()
    # y and the output are each rounded to bf16 (8 significant bits): two ulps of the largest value
    assert (got - ref).abs().max().item() <= 2.0 ** -7 * ref.abs().max().item()
