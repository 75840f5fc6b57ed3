"""The per-token quantizer's quotient for bf16 inputs, checked exhaustively on the CPU.

The GPU kernels (quant8b in minimax-h3-multi-dgx-spark_amd/csrc/common.h, used by the per-token quantizer and the
norm -> quantizer fusion) form rne(fl(x / s)) without a divide: q0 = fl(x r), the exact remainder fma(-q0, s, x), one
correction fma(rem, r, q0).  tests/quant_exact_check.c runs that sequence in IEEE single precision (each operation
rounded as written) against the IEEE divide for every bf16 amax with s in [2^-100, 2^126] and every bf16 x in
[0, amax], the whole domain those kernels send down this path.  A planted mistake (no correction step) must fail.
The ConvRot quantizer's values are fp32, so its residual edge (kQuantEdge) gets a randomized check instead
(tests/quant_edge_check.c), which an edge below the error bound must fail.
"""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "quant_exact_check.c")


def _build(tmp_path, src_text=None):
    src = SRC
    if src_text is not None:
        src = str(tmp_path / "planted.c")
        with open(src, "w") as f:
            f.write(src_text)
    exe = str(tmp_path / ("chk_planted" if src_text is not None else "chk"))
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-frounding-math", "-o", exe, src,
                    "-lm"], check=True)
    return exe


def _run(exe, lo, hi):
    return subprocess.run([exe, hex(lo), hex(hi)], capture_output=True, text=True, timeout=600)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_quotient_exact_every_bf16(tmp_path):
    exe = _build(tmp_path)
    # the amax range split over worker processes (the check is independent per amax)
    cuts = [1, 0x3C00, 0x4080, 0x4300, 0x4600, 0x4C00, 0x5400, 0x6000, 0x7F80]
    procs = [subprocess.Popen([exe, hex(a), hex(b)], stdout=subprocess.PIPE, text=True) for a, b in zip(cuts, cuts[1:])]
    pairs = 0
    for p in procs:
        out, _ = p.communicate(timeout=600)
        assert p.returncode == 0, out
        pairs += int(out.split("pairs ")[1].split()[0])
    assert pairs == 523237695


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_planted_mistake_fails(tmp_path):
    with open(SRC) as f:
        text = f.read()
    planted = text.replace("const float q1 = fmaf(rem, r, q0);", "const float q1 = q0;")
    assert planted != text
    exe = _build(tmp_path, planted)
    res = _run(exe, 0x4000, 0x4100)  # amax in [2, 8): the uncorrected product misrounds near half-integers
    assert res.returncode == 1 and "mismatch" in res.stdout


EDGE_SRC = os.path.join(HERE, "quant_edge_check.c")


def _build_edge(tmp_path, text=None, name="edge"):
    src = EDGE_SRC
    if text is not None:
        src = str(tmp_path / (name + ".c"))
        with open(src, "w") as f:
            f.write(text)
    exe = str(tmp_path / name)
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-frounding-math", "-o", exe, src,
                    "-lm"], check=True)
    return exe


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_convrot_residual_edge(tmp_path):
    """The ConvRot quantizer's residual edge 0.5 - 2^-16 (kQuantEdge): no sample whose residual passes it rounds
    differently from the IEEE divide, over seeds that put half of the samples next to half-integer quotients."""
    exe = _build_edge(tmp_path)
    for seed in (1, 2, 3):
        res = subprocess.run([exe, str(seed)], capture_output=True, text=True, timeout=300)
        assert res.returncode == 0, res.stdout
        assert "violations 0" in res.stdout


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_convrot_residual_edge_too_loose_fails(tmp_path):
    """An edge of 0.5 - 2^-17 is below the error bound, and the check must catch it."""
    with open(EDGE_SRC) as f:
        text = f.read()
    planted = text.replace("0.5f - 0x1p-16f", "0.5f - 0x1p-17f")
    assert planted != text
    exe = _build_edge(tmp_path, planted, "edge_planted")
    res = subprocess.run([exe, "7"], capture_output=True, text=True, timeout=300)
    assert res.returncode == 1 and "violation" in res.stdout
