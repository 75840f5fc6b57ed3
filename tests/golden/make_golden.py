"""Writes the golden fixtures in this folder (run from the repository root:
python tests/golden/make_golden.py).

The reference repository ships no golden vectors for this path, so these are
built here from seeded inputs.  Expected outputs come from the CPU oracle and,
where the arithmetic is exact in torch CPU ops (quantizer, int32 GEMM,
epilogue, gate), are cross-checked against torch before being written; the
norm vectors are additionally tied to the hand-derived known answers in
tests/test_oracle_pins.py.  Inputs follow the workload distributions (bf16
N(0,1) activations with outliers, int8 uniform weights, U(1e-3,1e-2) channel
scales, N(0,0.02) bias) and the stress pattern of the reference's RMSNorm
order search (tests/test_rmsnorm_exact.py:117-124: per-row magnitudes over
1e-2..1e3, 7 hot columns x50, w = 1 + 0.3 N(0,1)).
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from oracle import oracle as O  # noqa: E402
from oracle import torch_cpu  # noqa: E402
from util import bits, gemm_inputs, norm_inputs  # noqa: E402


def w8a8():
    M, N, K = 37, 72, 384
    x, w, ws, bias = gemm_inputs(M, N, K, seed=2026, outliers=0.002)
    x[5] = 0
    out, q, s, acc = O.w8a8_linear(bits(x), w.numpy(), ws.numpy())
    out_b = O.epilogue_bf16(acc, s, ws.numpy(), bits(bias))
    # independent cross-check in torch CPU ops
    tq, ts = torch_cpu.quant_rowwise(x)
    assert np.array_equal(q, tq.numpy()) and np.array_equal(s, ts.reshape(-1).numpy())
    assert np.array_equal(acc, torch._int_mm(tq, w.t()).numpy())
    assert np.array_equal(out_b, bits(torch_cpu.w8a8_linear(x, w, ws, bias)))
    np.savez_compressed(os.path.join(HERE, "w8a8_m37_n72_k384.npz"), x=bits(x), w=w.numpy(), ws=ws.numpy(),
                        bias=bits(bias), q=q, s=s, acc=acc, out=out, out_bias=out_b)


def norms():
    S, N, R, eps = 6, 5376, 2, 1e-5
    x, w, s1, sh, g, o, ridx = norm_inputs(S, N, R, seed=7)
    rec = dict(x=bits(x), w=bits(w), s1=bits(s1), sh=bits(sh), g=bits(g), o=bits(o), ridx=ridx.numpy(),
               eps=np.float32(eps))
    for tag, order in (("ref", (128, 4, 32)), ("w64", (256, 4, 64))):
        h, var, rstd = O.norm_mod(bits(x), bits(w), eps, ridx.numpy(), bits(s1), bits(sh), order=order)
        xn, hg, varg, rstdg = O.gate_norm_mod(bits(x), bits(o), bits(g), bits(w), eps, ridx.numpy(), bits(s1),
                                              bits(sh), order=order)
        rec.update({f"norm_h_{tag}": h, f"norm_var_{tag}": var, f"norm_rstd_{tag}": rstd,
                    f"gnm_x_{tag}": xn, f"gnm_h_{tag}": hg, f"gnm_var_{tag}": varg, f"gnm_rstd_{tag}": rstdg})
    xg = O.gate(bits(x), bits(o), bits(g), ridx.numpy())
    ref = x.clone()
    for r in range(R):
        rows = (ridx == r).nonzero().flatten()
        sub = ref[rows]
        sub.addcmul_(o[rows], g[r])
        ref[rows] = sub
    assert np.array_equal(xg, bits(ref))
    rec["gate_x"] = xg
    np.savez_compressed(os.path.join(HERE, "norms_s6_n5376_r2.npz"), **rec)


if __name__ == "__main__":
    w8a8()
    norms()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
