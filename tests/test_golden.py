"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py): the CPU oracle must reproduce them on the CPU,
and the HIP kernels through the C ABI on the GPU, bit for bit."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from util import from_bits, bits

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ORDERS = {"ref": (1, (128, 4, 32)), "w64": (2, (256, 4, 64))}


def _load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def test_oracle_reproduces_w8a8_fixture():
    f = _load("w8a8_m37_n72_k384.npz")
    out, q, s, acc = O.w8a8_linear(f["x"], f["w"], f["ws"])
    assert np.array_equal(q, f["q"]) and np.array_equal(s, f["s"]) and np.array_equal(acc, f["acc"])
    assert np.array_equal(out, f["out"])
    assert np.array_equal(O.epilogue_bf16(acc, s, f["ws"], f["bias"]), f["out_bias"])


@pytest.mark.parametrize("tag", ["ref", "w64"])
def test_oracle_reproduces_norm_fixture(tag):
    f = _load("norms_s6_n5376_r2.npz")
    order = ORDERS[tag][1]
    h, var, rstd = O.norm_mod(f["x"], f["w"], float(f["eps"]), f["ridx"], f["s1"], f["sh"], order=order)
    assert np.array_equal(h, f[f"norm_h_{tag}"]) and np.array_equal(var, f[f"norm_var_{tag}"])
    assert np.array_equal(rstd, f[f"norm_rstd_{tag}"])
    xn, hg, _, _ = O.gate_norm_mod(f["x"], f["o"], f["g"], f["w"], float(f["eps"]), f["ridx"], f["s1"], f["sh"],
                                   order=order)
    assert np.array_equal(xn, f[f"gnm_x_{tag}"]) and np.array_equal(hg, f[f"gnm_h_{tag}"])
    assert np.array_equal(O.gate(f["x"], f["o"], f["g"], f["ridx"]), f["gate_x"])


@pytest.mark.gpu
def test_hip_reproduces_w8a8_fixture():
    import h3mi
    f = _load("w8a8_m37_n72_k384.npz")
    x = from_bits(f["x"], "cuda")
    q, s = h3mi.quantize_rowwise(x)
    assert np.array_equal(q.cpu().numpy(), f["q"]) and np.array_equal(s.cpu().numpy().reshape(-1), f["s"])
    w = torch.from_numpy(f["w"]).cuda()
    assert np.array_equal(h3mi.int8_mm_i32(q, w).cpu().numpy(), f["acc"])
    ws = torch.from_numpy(f["ws"]).cuda()
    assert np.array_equal(bits(h3mi.int8_mm_scaled(q, w, s, ws)), f["out"])
    out = h3mi.w8a8_linear(x, w, ws, bias=from_bits(f["bias"], "cuda"))
    assert np.array_equal(bits(out), f["out_bias"])


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["ref", "w64"])
def test_hip_reproduces_norm_fixture(tag):
    import h3mi
    f = _load("norms_s6_n5376_r2.npz")
    order = ORDERS[tag][0]
    d = {k: from_bits(f[k], "cuda") for k in ("x", "w", "s1", "sh", "g", "o")}
    ridx = torch.from_numpy(f["ridx"]).cuda()
    eps = float(f["eps"])
    h, var, rstd = h3mi.norm_mod_ex(d["x"], d["w"], eps, ridx, d["s1"], d["sh"], order=order, rsqrt_mode=1,
                                    stats=True)
    assert np.array_equal(bits(h), f[f"norm_h_{tag}"])
    assert np.array_equal(var.cpu().numpy(), f[f"norm_var_{tag}"])
    x = d["x"].clone()
    hg = h3mi.gate_norm_mod_ex(x, d["o"], d["g"], d["w"], eps, ridx, d["s1"], d["sh"], order=order, rsqrt_mode=1)
    assert np.array_equal(bits(x), f[f"gnm_x_{tag}"]) and np.array_equal(bits(hg), f[f"gnm_h_{tag}"])
    x = d["x"].clone()
    h3mi.gate_(x, d["o"], d["g"], ridx)
    assert np.array_equal(bits(x), f["gate_x"])
