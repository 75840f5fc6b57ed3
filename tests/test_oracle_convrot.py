"""Pins of the oracle's ConvRot quantizer (oracle/h3_oracle.c: h3o_exp_neg,
h3o_silu, h3o_fwht256, h3o_convrot_quant).

The reference calls comfy-kitchen's _C.quantize_int8_rowwise_convrot64
(comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:90-95,
tests/bench_linear.py:33-40); comfy-kitchen is not vendored, so agreement with
its bytes is unpinned.  What these tests fix is the stated definition, against
computations that share no code with the oracle: scipy's Sylvester Hadamard
matrix, float64 exp / silu, hand-derived known answers that a wrong stage
order, pairing, sign or normalisation would change, and the identity the
rotation exists for, (x H / 16)(W H / 16)^T = x W^T.
"""
import math

import numpy as np
import pytest
import scipy.linalg

from oracle import oracle as O

H256 = scipy.linalg.hadamard(256).astype(np.float64)


def _ulps(got, ref):
    ref32 = np.float32(ref)
    return abs(float(got) - ref) / float(np.spacing(np.float32(abs(ref32)) if ref32 != 0 else np.float32(1e-45)))


# ------------------------------------------------------------------ the transform

@pytest.mark.parametrize("j", [0, 1, 2, 3, 5, 16, 17, 100, 128, 255])
def test_fwht_of_unit_vector_is_a_sylvester_column(j):
    e = np.zeros(256, np.float32)
    e[j] = 1.0
    y = O.fwht256(e)
    assert np.array_equal(y.astype(np.float64), H256[:, j])


def test_fwht_matches_dense_hadamard_in_float64():
    rng = np.random.default_rng(0)
    for scale in (1.0, 1e-3, 300.0):
        v = (rng.standard_normal(256) * scale).astype(np.float32)
        v[rng.integers(0, 256, 3)] *= 40.0
        ref = H256 @ v.astype(np.float64)
        got = O.fwht256(v).astype(np.float64)
        bound = 8 * 2.0 ** -24 * np.abs(v).astype(np.float64).sum()
        assert np.all(np.abs(got - ref) <= bound)


def test_fwht_twice_is_256_times_identity():
    rng = np.random.default_rng(1)
    v = rng.standard_normal(256).astype(np.float32)
    back = O.fwht256(O.fwht256(v)) / 256.0
    assert np.allclose(back, v, rtol=0, atol=1e-5)


def test_fwht_stage_order_known_answer():
    # stages h = 1 then h = 2: y0 = rn(rn(1 + 2^-24) + rn(0 + 2^-24)) = rn(1 + 2^-24) = 1;
    # h = 2 first would give rn(1 + rn(2^-24 + 2^-24)) = 1 + 2^-23
    v = np.zeros(256, np.float32)
    v[0], v[1], v[3] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert O.fwht256(v)[0] == np.float32(1.0)


def test_fwht_butterfly_sign_known_answer():
    # (a, b) -> (a + b, a - b): v = [3, 1] gives y0 = 4, y1 = 2 (b - a would give -2)
    v = np.zeros(256, np.float32)
    v[0], v[1] = 3.0, 1.0
    y = O.fwht256(v)
    assert y[0] == 4.0 and y[1] == 2.0 and y[2] == 4.0 and y[3] == 2.0 and y[255] == 2.0


# ------------------------------------------------------------------ exp and silu

def test_exp_neg_within_one_ulp_of_float64():
    xs = np.linspace(-86.0, 0.0, 20001).astype(np.float32)
    got = O.exp_neg(xs)
    worst = max(_ulps(g, math.exp(float(x))) for x, g in zip(xs, got))
    assert worst <= 1.0


def test_exp_neg_special_values():
    assert O.exp_neg(np.float32(0.0)) == 1.0
    assert O.exp_neg(np.float32(-86.5)) == O.exp_neg(np.float32(-86.0))    # argument clamped at -86
    assert O.exp_neg(np.float32(-200.0)) == O.exp_neg(np.float32(-86.0))
    assert abs(float(O.exp_neg(np.float32(-86.0))) - math.exp(-86.0)) < 1e-44
    assert O.exp_neg(np.float32(-math.log(2.0))) == np.float32(0.5)


def test_rcp12_within_half_an_ulp_and_a_bit():
    ds = np.linspace(1.0, 2.0, 50001).astype(np.float32)
    got = O.rcp12(ds)
    worst = max(_ulps(g, 1.0 / float(d)) for d, g in zip(ds, got))
    assert worst <= 0.51
    assert O.rcp12(np.float32(1.0)) == 1.0 and O.rcp12(np.float32(2.0)) == 0.5


def test_silu_within_three_ulps_of_float64():
    xs = np.concatenate([np.linspace(-30, 30, 6001), np.linspace(-1e-3, 1e-3, 201)]).astype(np.float32)
    got = O.silu(xs)
    for x, g in zip(xs, got):
        ref = float(x) / (1.0 + math.exp(-float(x)))
        if ref == 0.0:
            assert g == 0.0
            continue
        assert _ulps(g, ref) <= 3.0, (x, g, ref)


def test_silu_special_values():
    assert O.silu(np.float32(0.0)) == 0.0
    assert math.copysign(1.0, float(O.silu(np.float32(-0.0)))) == -1.0
    assert O.silu(np.float32(30.0)) == np.float32(30.0)       # 1 + e^-30 rounds to 1
    v = float(O.silu(np.float32(-100.0)))                    # exp's argument clamps at -86: -100 e^-86
    assert -1e-35 < v < 0.0 and abs(v - (-100.0 * math.exp(-86.0))) < 1e-40


# ------------------------------------------------------------------ the quantizer

def _silu64(a):
    return a / (1.0 + np.exp(-a))


def _check_against_float64(q, s, u64):
    M, K = u64.shape
    y64 = (u64.reshape(M, K // 256, 256) @ H256.T).reshape(M, K) / 16.0
    s64 = np.abs(y64).max(1) / 127.0
    assert np.all(np.abs(s.astype(np.float64) - s64) <= 4e-6 * s64 + 1e-30)
    t = y64 / s64[:, None]
    sure = np.abs(np.abs(t) - np.floor(np.abs(t)) - 0.5) > 1e-3
    want = np.clip(np.rint(t), -127, 127)
    assert np.array_equal(q[sure], want[sure].astype(np.int8))
    assert np.all(np.abs(q.astype(np.int64) - want) <= 1)


@pytest.mark.parametrize("act", [None, "swiglu"])
def test_convrot_quant_matches_float64_definition(act):
    rng = np.random.default_rng(2)
    M, K = 12, 1024
    kin = 2 * K if act else K
    xf = rng.standard_normal((M, kin)).astype(np.float32)
    xf[rng.random((M, kin)) < 0.002] *= 20.0
    xb = O.f32_to_bf16_bits(xf)
    x64 = O.bf16_bits_to_f32(xb).astype(np.float64)
    u64 = _silu64(x64[:, :K]) * x64[:, K:] if act else x64
    q, s = O.convrot_quant(xb, act)
    _check_against_float64(q, s, u64)


def test_convrot_swiglu_takes_silu_of_the_first_half():
    # a = first half, b = second half: silu(2) * 1 vs silu(1) * 2 differ
    x = np.zeros((1, 512), np.float32)
    x[0, 0], x[0, 256] = 2.0, 1.0
    q, s = O.convrot_quant(O.f32_to_bf16_bits(x), "swiglu")
    expect = 2.0 / (1.0 + math.exp(-2.0)) / 16.0 / 127.0
    assert abs(float(s[0]) - expect) <= 1e-6 * expect
    assert np.all(q[0] == 127)     # one element -> a constant row of y


def test_convrot_zero_row_and_group_locality():
    x = np.zeros((3, 1024), np.float32)
    x[1, 2 * 256 + 7] = 5.0        # one value in group 2
    x[2, :] = 1.0                  # constant row: each group's y is 16 at index 0 and 0 elsewhere
    q, s = O.convrot_quant(O.f32_to_bf16_bits(x))
    assert s[0] == 0.0 and not q[0].any()
    assert not q[1, :512].any() and not q[1, 768:].any()
    assert np.all(np.abs(q[1, 512:768]) == 127)
    assert s[2] == np.float32(np.float32(16.0) / np.float32(127.0))
    assert np.all(q[2].reshape(4, 256)[:, 0] == 127) and not q[2].reshape(4, 256)[:, 1:].any()


def test_convrot_quant_tiny_and_outlier_rows():
    rng = np.random.default_rng(3)
    xf = rng.standard_normal((4, 512)).astype(np.float32)
    xf[0] *= np.float32(1e-33)
    xf[1, 5] = 3e4
    xb = O.f32_to_bf16_bits(xf)
    q, s = O.convrot_quant(xb)
    _check_against_float64(q[1:], s[1:], O.bf16_bits_to_f32(xb)[1:].astype(np.float64))
    assert s[0] > 0 and np.abs(q[0]).max() == 127


def test_rotated_linear_recovers_the_plain_product():
    # the identity ConvRot checkpoints rely on: weights stored as W H / 16 per
    # group, and H H^T = 256 I, so (x H / 16)(W H / 16)^T == x W^T; with int8
    # activations the product agrees to quantization error
    rng = np.random.default_rng(4)
    M, N, K = 8, 16, 768
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = rng.standard_normal((N, K))
    xb = O.f32_to_bf16_bits(x)
    xv = O.bf16_bits_to_f32(xb).astype(np.float64)
    Wr = (W.reshape(N, K // 256, 256) @ H256.T).reshape(N, K) / 16.0
    q, s = O.convrot_quant(xb)
    got = (q.astype(np.float64) * s[:, None]) @ Wr.T
    ref = xv @ W.T
    err = np.abs(got - ref).max()
    assert err < 0.05 * np.abs(ref).max()
