"""The drop-in layer on the CPU: install/uninstall/stats contracts, the
eligibility gate, fallbacks, the row-index builder, after-import hooks and
both boot paths, exercised against stand-in upstream modules (tests/fakes).

Counterparts: comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py,
comfyui_nodes/h3-linear-fast/boot/sitecustomize.py,
comfyui_nodes/h3-fuse-graph/h3_fuse_patch.py, h3_fg_profile.py and
boot/h3_fuse_launch.py of the reference.
"""
import importlib
import logging
import os
import subprocess
import sys
import textwrap
import types

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "minimax-h3-multi-dgx-spark_amd")
LF = os.path.join(PKG, "comfyui_nodes", "h3-linear-fast")
FG = os.path.join(PKG, "comfyui_nodes", "h3-fuse-graph")
FAKES = os.path.join(ROOT, "tests", "fakes")


def _fresh(monkeypatch, *mods):
    for p in (FAKES, LF, FG):
        monkeypatch.syspath_prepend(p)
    for name in list(sys.modules):
        if name.split(".")[0] in ("comfy_kitchen", "comfy") or name in mods:
            monkeypatch.delitem(sys.modules, name, raising=False)
    return [importlib.import_module(m) for m in mods]


# ------------------------------------------------------------------ h3-linear-fast

def test_linear_install_needs_env(monkeypatch):
    monkeypatch.delenv("H3_LINEAR_FAST", raising=False)
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    assert lf.install() is False
    assert lf.stats() == {"installed": False, "fast_calls": 0, "fallback_calls": 0, "disabled": False}


def test_linear_install_missing_target(monkeypatch, caplog):
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.setenv("H3_LINEAR_FAST_TARGET", "no_such_pkg.backend")
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    with caplog.at_level(logging.WARNING):
        assert lf.install() is False
    assert "cannot import" in caplog.text


def test_linear_install_fallback_uninstall(monkeypatch):
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.delenv("H3_LINEAR_FAST_TARGET", raising=False)
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    ckc = importlib.import_module("comfy_kitchen.backends.cuda")
    orig = ckc.int8_linear
    assert lf.install() is True and lf.install() is True
    assert ckc.int8_linear is not orig and ckc.int8_linear._h3_linear_fast_orig is orig
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 300, 256, generator=g).to(torch.bfloat16)        # CPU: ineligible
    w = torch.randint(-127, 128, (64, 256), generator=g, dtype=torch.int8)
    ws = 1e-3 + 9e-3 * torch.rand(64, generator=g)
    out = ckc.int8_linear(x, w, ws)
    ref = orig(x, w, ws)
    assert out.shape == (3, 300, 64) and torch.equal(out, ref)
    st = lf.stats()
    assert st["installed"] and st["fallback_calls"] == 1 and st["fast_calls"] == 0
    lf.uninstall()
    assert ckc.int8_linear is orig and lf.stats()["installed"] is False


class _T:
    """Tensor-shaped stand-in for the gate (no data, any device flag)."""

    def __init__(self, shape, dtype, cuda=True, ptr=4096):
        self.shape = tuple(shape)
        self.dtype = dtype
        self.is_cuda = cuda
        self.device = "cuda:0" if cuda else "cpu"
        self.ptr = ptr

    def is_contiguous(self):
        return True

    def data_ptr(self):
        return self.ptr

    def dim(self):
        return len(self.shape)

    def numel(self):
        n = 1
        for s in self.shape:
            n *= s
        return n


@pytest.mark.parametrize("case,expect", [
    (dict(), True),
    (dict(x=_T((4, 128, 5120), torch.bfloat16)), True),                 # 3-D input, m = 512
    (dict(x=_T((255, 5120), torch.bfloat16)), False),                   # m < MIN_M
    (dict(x=_T((512, 5120), torch.float16)), False),                    # not bf16
    (dict(x=_T((512, 5120), torch.bfloat16, cuda=False)), False),       # CPU tensor
    (dict(w=_T((15360, 5120), torch.float16)), False),                  # weight not int8
    (dict(w=_T((15364, 5120), torch.int8)), False),                     # n % 8
    (dict(x=_T((512, 5000), torch.bfloat16), w=_T((64, 5000), torch.int8)), False),  # k % 128
    (dict(residual=object()), False),
    (dict(input_act="gelu"), False),
    (dict(input_act="swiglu"), False),                                  # per-token quantizer fuses no activation
    (dict(convrot=True), False),                                        # no ConvRot quantizer available
    (dict(convrot=True, have_convrot=True), True),
    (dict(convrot=True, have_convrot=True, input_act="swiglu", x=_T((512, 10240), torch.bfloat16)), True),
    (dict(convrot=True, have_convrot=True, groups=128), False),
    (dict(convrot=True, have_convrot=True, x=_T((512, 16384 + 256), torch.bfloat16),
          w=_T((64, 16384 + 256), torch.int8)), False),                 # k above the quantizer's maximum
    (dict(bias=_T((15360,), torch.bfloat16)), False),                   # bias needs H3_LINEAR_FAST_BIAS=1
    (dict(out_dtype=torch.float32), False),
    (dict(w=_T((15360, 5120), torch.int8, cuda=False)), False),         # weight on the host
    (dict(w=_T((15360, 5120), torch.int8, ptr=4104)), False),           # weight not 16-byte aligned
    (dict(ws=_T((1,), torch.float32)), True),                           # per-tensor scale, expanded
    (dict(ws=_T((15360,), torch.float32)), True),
    (dict(ws=_T((7,), torch.float32)), False),                          # neither 1 nor n scales
    (dict(act_w=object()), False),                                      # the per-token path takes no act weight
    # this library's ConvRot quantizer takes no activation weight or epsilon: those calls keep the original
    (dict(convrot=True, have_convrot=True, input_act="swiglu", x=_T((512, 10240), torch.bfloat16), act_w=object()),
     False),
    (dict(convrot=True, have_convrot=True, eps=1e-6), False),
    # comfy-kitchen's quantizer (own_convrot False) takes them, as in the reference
    (dict(convrot=True, have_convrot=True, input_act="swiglu", x=_T((512, 10240), torch.bfloat16), act_w=object(),
          eps=1e-6, own=False), True),
])
def test_linear_eligibility(monkeypatch, case, expect):
    monkeypatch.delenv("H3_LINEAR_FAST_BIAS", raising=False)
    monkeypatch.delenv("H3_LINEAR_FAST_MIN_M", raising=False)
    monkeypatch.setenv("H3_LINEAR_FAST_PLAIN", "1")  # the gate's other rules, with convrot=False calls opted in
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    x = case.get("x", _T((512, 5120), torch.bfloat16))
    w = case.get("w", _T((15360, 5120), torch.int8))
    ok, m, k, n = lf.eligible(x, w, case.get("bias"), case.get("out_dtype"), case.get("convrot", False),
                              case.get("groups", 256), case.get("input_act"), case.get("residual"),
                              have_convrot=case.get("have_convrot", False), max_k_convrot=16384,
                              supported=lambda kk: kk % 128 == 0, input_act_weight=case.get("act_w"),
                              input_act_eps=case.get("eps", 0.0), own_convrot=case.get("own", True),
                              weight_scale=case.get("ws"))
    assert ok is expect
    if ok:
        act_w = 2 if case.get("input_act") == "swiglu" else 1
        assert n == w.shape[0] and k == x.shape[-1] // act_w and m == x.numel() // x.shape[-1]


def test_linear_bias_gate_env(monkeypatch):
    monkeypatch.setenv("H3_LINEAR_FAST_BIAS", "1")
    monkeypatch.setenv("H3_LINEAR_FAST_PLAIN", "1")
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    x = _T((512, 5120), torch.bfloat16)
    w = _T((15360, 5120), torch.int8)
    b = _T((15360,), torch.bfloat16)
    ok = lf.eligible(x, w, b, None, False, 256, None, None, have_convrot=False, max_k_convrot=0,
                     supported=lambda kk: True)[0]
    assert ok
    bad = _T((100,), torch.bfloat16)
    assert not lf.eligible(x, w, bad, None, False, 256, None, None, have_convrot=False, max_k_convrot=0,
                           supported=lambda kk: True)[0]


@pytest.mark.parametrize("plain,takes_plain", [(None, False), ("0", False), ("1", True)])
def test_linear_plain_takeover_env(monkeypatch, plain, takes_plain):
    """The reference's routing by default (H3_LINEAR_FAST_PLAIN unset or 0):
    convrot=False calls go to the original, as at the reference's
    h3_linear_fast_patch.py:64; H3_LINEAR_FAST_PLAIN=1 opts them in.
    convrot=True calls take the fast path either way."""
    if plain is None:
        monkeypatch.delenv("H3_LINEAR_FAST_PLAIN", raising=False)
    else:
        monkeypatch.setenv("H3_LINEAR_FAST_PLAIN", plain)
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    x = _T((512, 5120), torch.bfloat16)
    w = _T((64, 5120), torch.int8)
    kw = dict(have_convrot=True, max_k_convrot=16384, supported=lambda kk: True)
    assert lf.eligible(x, w, None, None, False, 256, None, None, **kw)[0] is takes_plain
    assert lf.eligible(x, w, None, None, True, 256, None, None, **kw)[0]


@pytest.mark.parametrize("mode,up,expect", [("auto", False, (False, True)), ("auto", True, (True, True)),
                                            ("own", True, (False, True)), ("upstream", False, (False, False)),
                                            ("upstream", True, (True, True))])
def test_linear_convrot_quantizer_choice(monkeypatch, mode, up, expect):
    """H3_LINEAR_FAST_CONVROT: auto (default) takes comfy-kitchen's rotation
    quantizer when its extension is there, else this library's; upstream
    without the extension leaves convrot=True calls to the original."""
    monkeypatch.setenv("H3_LINEAR_FAST_CONVROT", mode)
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    ckc = types.SimpleNamespace()
    if up:
        ckc._C = types.SimpleNamespace(quantize_int8_rowwise_convrot64=lambda *a: None)
        for name in ("_wrap_for_dlpack", "_act_weight_arg", "_input_act_code", "_convrot_fused_shared_memory_fits"):
            setattr(ckc, name, lambda *a: None)
        ckc._CONVROT_FUSED_MAX_K = 16384
    q, have = lf._pick_convrot(ckc)
    assert (q is not None, have) == expect


def test_linear_argument_errors_fall_back_per_call(monkeypatch):
    """An argument rejection (ValueError, H3miError EINVAL/EALIGN/EALIAS) is a
    per-call fallback; a launch error disables the fast path."""
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    from h3mi._lib import EALIAS, EALIGN, EINVAL, ELAUNCH, H3miError
    for code in (EINVAL, EALIGN, EALIAS):
        assert lf._argument_error(H3miError(code, "x"))
    assert lf._argument_error(ValueError("shape"))
    assert not lf._argument_error(H3miError(ELAUNCH, "launch"))
    assert not lf._argument_error(RuntimeError("HIP error"))


def test_linear_min_m_env(monkeypatch):
    monkeypatch.setenv("H3_LINEAR_FAST_MIN_M", "1024")
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    w = _T((64, 5120), torch.int8)
    kw = dict(have_convrot=True, max_k_convrot=16384, supported=lambda kk: True)
    assert not lf.eligible(_T((512, 5120), torch.bfloat16), w, None, None, True, 256, None, None, **kw)[0]
    assert lf.eligible(_T((1024, 5120), torch.bfloat16), w, None, None, True, 256, None, None, **kw)[0]


def test_int8_gemm_hip_module_api(monkeypatch):
    (tg,) = _fresh(monkeypatch, "int8_gemm_hip")
    assert tg.supported(5120) and tg.supported(128) and not tg.supported(5000) and not tg.supported(0)
    assert hasattr(tg._int8_mm_scaled_kernel, "best_config")
    assert tg.config_for(32768, 15360, 5120).startswith("d_")


@pytest.mark.parametrize("cfg,pinned", [
    ("128,256,64,3,8", None),                        # the reference's own example (int8_gemm_triton.py:24)
    (" 64, 256,128,3,4", None),
    ("no_such_tile", None),
    ("d_bm128_bn128_bk128_s2_g4_o2", "d_bm128_bn128_bk128_s2_g4_o2"),
])
def test_tile_pin_never_breaks_import_or_install(cfg, pinned):
    """H3_LINEAR_FAST_CFG in the reference's "BM,BN,BK,stages,warps" form (a
    Triton tile with no counterpart here) or an unknown name keeps the
    heuristic with a warning: `import h3mi` and both nodes' install() still
    work.  A configuration name of this library pins it."""
    code = textwrap.dedent("""
        import logging, os, sys
        logging.basicConfig(level=logging.WARNING)
        import h3mi
        from h3mi import gemm
        import h3_linear_fast_patch as lf
        import h3_fuse_patch as fp
        assert lf.install(), 'h3-linear-fast did not install'
        assert fp.install(), 'h3-fuse-graph did not install'
        assert gemm._autotune() is False, 'a pin of any kind turns autotuning off'
        print('NOTE', gemm.fixed_config_note() is not None)
        print('CFG', h3mi.config_for(32768, 15360, 5120))
    """)
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([LF, FG, FAKES, PKG])
    env.update(H3_LINEAR_FAST="1", H3_FUSE="1", H3_LINEAR_FAST_CFG=cfg, H3_LINEAR_FAST_ALLCFG="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = dict(line.split(" ", 1) for line in r.stdout.strip().splitlines() if line[:4] in ("NOTE", "CFG "))
    if pinned is None:
        assert out["NOTE"] == "True" and "H3_LINEAR_FAST_CFG" in r.stderr
        assert out["CFG"] == "d_bm256_bn384_bk128_s2_g8_w8m_l4_a1_sw_res"  # the heuristic's pick
    else:
        assert out["NOTE"] == "False" and out["CFG"] == pinned


def test_sitecustomize_boot_hook(tmp_path):
    """A fresh interpreter with the boot folder on PYTHONPATH patches the
    target right after it is imported, and still runs the shadowed hook."""
    shadow = tmp_path / "shadow"
    shadow.mkdir()
    (shadow / "sitecustomize.py").write_text("import os\nos.environ['SHADOWED_SITECUSTOMIZE_RAN'] = '1'\n")
    code = textwrap.dedent("""
        import os, sys
        import comfy_kitchen.backends.cuda as ckc
        import h3_linear_fast_patch as lf
        assert os.environ.get('SHADOWED_SITECUSTOMIZE_RAN') == '1', 'shadowed sitecustomize not run'
        assert lf.stats()['installed'], lf.stats()
        assert hasattr(ckc.int8_linear, '_h3_linear_fast_orig')
        print('ok')
    """)
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(LF, "boot"), str(shadow), FAKES, PKG])
    env["H3_LINEAR_FAST"] = "1"
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.strip().endswith("ok")


# ------------------------------------------------------------------ h3-fuse-graph

def test_fuse_install_needs_env(monkeypatch):
    monkeypatch.delenv("H3_FUSE", raising=False)
    (fp,) = _fresh(monkeypatch, "h3_fuse_patch")
    assert fp.enabled() is False and fp.install() is False


def test_fuse_row_index(monkeypatch):
    (fp,) = _fresh(monkeypatch, "h3_fuse_patch")
    segs = [(4, 10, 1), (0, 4, 0)]
    r = fp._row_index(segs, 10, torch.device("cpu"))
    assert r.dtype == torch.int32 and r.tolist() == [0] * 4 + [1] * 6
    assert fp._row_index(segs, 10, torch.device("cpu")) is r            # cached
    assert fp._row_index(list(segs), 10, torch.device("cpu")) is r      # by content, not by list identity
    per_row = torch.tensor([2, 0, 1])
    a = fp._row_index([(0, 3, per_row), (3, 5, 3)], 5, torch.device("cpu"))
    per_row[0] = 1                                                       # in-place change: not the cached index
    assert fp._row_index([(0, 3, per_row), (3, 5, 3)], 5, torch.device("cpu")).tolist() == [1, 0, 1, 3, 3]
    assert a.tolist() == [2, 0, 1, 3, 3]
    segs2 = [(0, 3, torch.tensor([2, 0, 1])), (3, 5, 3)]
    assert fp._row_index(segs2, 5, torch.device("cpu")).tolist() == [2, 0, 1, 3, 3]
    assert fp._row_index([(0, 4, 0), (5, 10, 1)], 10, torch.device("cpu")) is None      # gap
    assert fp._row_index([(0, 6, 0), (5, 10, 1)], 10, torch.device("cpu")) is None      # overlap
    assert fp._row_index([(0, 4, 0)], 10, torch.device("cpu")) is None                   # short
    assert fp._row_index([(0, 3, torch.tensor([1, 2]))], 3, torch.device("cpu")) is None  # bad length
    assert fp._row_index([(0, 0, 0), (0, 2, 1)], 2, torch.device("cpu")).tolist() == [1, 1]  # empty segment


def _block(seed=0, dim=64, device="cpu"):
    torch.manual_seed(seed)
    mm = importlib.import_module("comfy.ldm.minimax.model")
    blk = mm.DiTBlock(dim, 4, 2 * dim, tdim=16, device=device)
    for p in blk.parameters():
        p.requires_grad_(False)
    x = torch.randn(24, dim, device=device).to(torch.bfloat16)
    t = torch.randn(2, 16, device=device)
    return mm, blk, x, t


def test_fuse_install_and_cpu_fallback(monkeypatch):
    monkeypatch.setenv("H3_FUSE", "1")
    (fp,) = _fresh(monkeypatch, "h3_fuse_patch")
    mm = importlib.import_module("comfy.ldm.minimax.model")
    orig = mm.DiTBlock.forward
    assert fp.install() is True
    assert mm.DiTBlock.forward._h3_fuse_orig is orig
    _, blk, x, t = _block()
    segs = [(0, 10, 0), (10, 24, 1)]
    with torch.no_grad():
        ref = orig(blk, x.clone(), t, segs, None)
        out = blk(x.clone(), t, segs, None)                                   # CPU -> original forward
    assert torch.equal(out, ref)
    assert fp.stats()["fallback"] == 1 and fp.stats()["fused"] == 0
    fp.uninstall()
    assert mm.DiTBlock.forward is orig


def _eager_kernels(monkeypatch, fk, calls, q_rejects=None, first_error=None):
    """Point the fused-kernel module at eager CPU stand-ins with the kernels'
    arithmetic (the stand-in block's own ops, gathered per row), so the fused
    forward's control flow runs on the CPU.  q_rejects: the exception the
    quantizing second norm raises; first_error: the one the first norm raises."""
    import torch.nn.functional as F

    def norm_mod(x, w, eps, ridx, s1, sh):
        calls.append("norm_mod")
        if first_error is not None:
            raise first_error
        h = F.rms_norm(x, (x.shape[1],), w, eps)
        return h.mul_(s1[ridx]).add_(sh[ridx])

    def norm_mod_q(x, w, eps, ridx, s1, sh, want_h=True):
        calls.append("norm_mod_q")
        if first_error is not None:
            raise first_error
        h = F.rms_norm(x, (x.shape[1],), w, eps).mul_(s1[ridx]).add_(sh[ridx])
        return h, torch.zeros(h.shape, dtype=torch.int8), torch.ones(h.shape[0], 1)

    def gate_norm_mod_(x, o, g, w, eps, ridx, s1, sh):
        calls.append("gate_norm_mod_")
        x.addcmul_(o, g[ridx])
        h = F.rms_norm(x, (x.shape[1],), w, eps)
        return h.mul_(s1[ridx]).add_(sh[ridx])

    def gate_norm_mod_q_(x, o, g, w, eps, ridx, s1, sh, want_h=True):
        calls.append("gate_norm_mod_q_")
        raise q_rejects

    def gate_(x, o, g, ridx):
        calls.append("gate_")
        return x.addcmul_(o, g[ridx])

    for name, f in (("norm_mod", norm_mod), ("norm_mod_q", norm_mod_q), ("gate_norm_mod_", gate_norm_mod_),
                    ("gate_norm_mod_q_", gate_norm_mod_q_), ("gate_", gate_)):
        monkeypatch.setattr(fk, name, f)


def _cpu_fits(x, n1, n2):
    return x.dim() == 2 and x.dtype == torch.bfloat16 and x.is_contiguous() and not torch.is_grad_enabled()


@pytest.mark.parametrize("reject", ["value", "einval"])
def test_fuse_handoff_rejection_falls_back_per_call(monkeypatch, reject):
    """H3_FUSE_QUANT=1: when the quantizing second norm rejects its arguments
    (before any launch, so x is untouched) the forward uses the plain fused
    norm for that call and stays enabled; its output equals the original
    block's.  Stand-in kernels on the CPU."""
    from h3mi._lib import EINVAL, H3miError
    monkeypatch.setenv("H3_FUSE", "1")
    monkeypatch.setenv("H3_FUSE_QUANT", "1")
    (fp, fk) = _fresh(monkeypatch, "h3_fuse_patch", "h3_fuse_kernels")
    calls = []
    err = ValueError("rejected") if reject == "value" else H3miError(EINVAL, "N too large")
    _eager_kernels(monkeypatch, fk, calls, q_rejects=err)
    monkeypatch.setattr(fp, "_fits", _cpu_fits)
    mm, blk, x, t = _block(seed=5)
    orig = mm.DiTBlock.forward
    assert fp.install()
    segs = [(0, 10, 1), (10, 24, 0)]
    with torch.no_grad():
        ref = orig(blk, x.clone(), t, segs, None)
        out = blk(x.clone(), t, segs, None)
        out2 = blk(x.clone(), t, segs, None)
    assert torch.equal(out, ref) and torch.equal(out2, ref)
    assert calls == ["norm_mod_q", "gate_norm_mod_q_", "gate_norm_mod_", "gate_"] * 2
    st = fp.stats()
    assert st["fused"] == 2 and st["fallback"] == 0 and not st["disabled"]
    fp.uninstall()


@pytest.mark.parametrize("handoff", [False, True])
@pytest.mark.parametrize("error,disables", [("value", False), ("einval", False), ("ealias", False),
                                            ("launch", True), ("runtime", True)])
def test_fuse_first_norm_errors(monkeypatch, handoff, error, disables):
    """An argument rejection in the first norm (nothing written yet) runs the
    original forward for that call only; a launch or runtime failure disables
    the fused block for the process."""
    from h3mi._lib import EALIAS, EINVAL, ELAUNCH, H3miError
    monkeypatch.setenv("H3_FUSE", "1")
    monkeypatch.setenv("H3_FUSE_QUANT", "1" if handoff else "0")
    (fp, fk) = _fresh(monkeypatch, "h3_fuse_patch", "h3_fuse_kernels")
    errs = {"value": ValueError("bad"), "einval": H3miError(EINVAL, "x"), "ealias": H3miError(EALIAS, "x"),
            "launch": H3miError(ELAUNCH, "x"), "runtime": RuntimeError("hip")}
    calls = []
    _eager_kernels(monkeypatch, fk, calls, first_error=errs[error])
    monkeypatch.setattr(fp, "_fits", _cpu_fits)
    mm, blk, x, t = _block(seed=6)
    orig = mm.DiTBlock.forward
    assert fp.install()
    segs = [(0, 24, 0)]
    with torch.no_grad():
        ref = orig(blk, x.clone(), t, segs, None)
        out = blk(x.clone(), t, segs, None)
    assert torch.equal(out, ref)
    assert calls == ["norm_mod_q" if handoff else "norm_mod"]
    st = fp.stats()
    assert st["fused"] == 0 and st["fallback"] == 1 and st["disabled"] is disables
    fp.uninstall()


def test_fuse_handoff_row_rule(monkeypatch):
    """The hand-off runs only for rows the fused quantizer takes (a multiple of
    8, at most 8192 elements)."""
    (fp,) = _fresh(monkeypatch, "h3_fuse_patch")
    assert fp._handoff_fits(5120) and fp._handoff_fits(5376) and fp._handoff_fits(8192) and fp._handoff_fits(8)
    assert not fp._handoff_fits(8200) and not fp._handoff_fits(10240) and not fp._handoff_fits(5124)
    assert not fp._handoff_fits(0)


def test_after_import_hook(monkeypatch, tmp_path):
    (fp,) = _fresh(monkeypatch, "h3_fuse_patch")
    pkg = tmp_path / "h3hookpkg"
    pkg.mkdir()
    (pkg / "__init__.py").write_text("")
    (pkg / "target.py").write_text("VALUE = 41\n")
    monkeypatch.syspath_prepend(str(tmp_path))
    seen = []
    fp.after_import(lambda n: n == "h3hookpkg.target", lambda m: seen.append(m.VALUE + 1))
    importlib.import_module("h3hookpkg.target")
    assert seen == [42]
    import h3_import_hooks as hooks
    assert hooks.pending() == 0 and hooks._watcher not in sys.meta_path   # fired once, watcher gone
    # a module that is already imported gets the call at once
    fp.after_import(lambda n: n == "h3hookpkg.target", lambda m: seen.append(m.VALUE))
    assert seen == [42, 41] and hooks.pending() == 0


def test_after_import_failed_import_keeps_the_hook(monkeypatch, tmp_path):
    """A watched module whose body raises leaves its hook waiting; the next
    successful import fires it."""
    (fp,) = _fresh(monkeypatch, "h3_fuse_patch")
    import h3_import_hooks as hooks
    (tmp_path / "h3hook_flaky.py").write_text("import os\nif os.environ.get('H3HOOK_FAIL'): raise ImportError('x')\n"
                                              "VALUE = 5\n")
    monkeypatch.syspath_prepend(str(tmp_path))
    monkeypatch.setenv("H3HOOK_FAIL", "1")
    seen = []
    fp.after_import(lambda n: n == "h3hook_flaky", lambda m: seen.append(m.VALUE))
    with pytest.raises(ImportError):
        importlib.import_module("h3hook_flaky")
    assert seen == [] and hooks.pending() == 1
    monkeypatch.delenv("H3HOOK_FAIL")
    sys.modules.pop("h3hook_flaky", None)
    importlib.import_module("h3hook_flaky")
    assert seen == [5] and hooks.pending() == 0


def test_fuse_launcher_boot(tmp_path):
    """boot/h3_fuse_launch.py runs a worker script as __main__ with the block
    patched as soon as the model module is imported."""
    worker = tmp_path / "worker.py"
    worker.write_text(textwrap.dedent("""
        import sys
        import comfy.ldm.minimax.model as mm
        assert hasattr(mm.DiTBlock.forward, '_h3_fuse_orig'), 'not patched'
        assert sys.argv[1:] == ['--flag', 'v'], sys.argv
        print('worker ok')
    """))
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([FAKES, PKG])
    env["H3_FUSE"] = "1"
    r = subprocess.run([sys.executable, "-s", os.path.join(FG, "boot", "h3_fuse_launch.py"), str(worker), "--flag", "v"],
                       env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "worker ok" in r.stdout


def test_fg_profile_timing_and_trace(monkeypatch, tmp_path, caplog):
    monkeypatch.setenv("H3_FG_PROFILE", "2")
    monkeypatch.setenv("H3_FG_PROFILE_DIR", str(tmp_path))
    monkeypatch.setenv("H3_FG_PROFILE_TAG", "t")
    (prof,) = _fresh(monkeypatch, "h3_fg_profile")
    mm = importlib.import_module("comfy.ldm.minimax.model")
    orig = mm.MiniMaxH3Model._forward
    prof.install()
    assert mm.MiniMaxH3Model._forward._h3_fg_orig is orig
    _, blk, x, t = _block()
    model = mm.MiniMaxH3Model([blk])
    with torch.no_grad(), caplog.at_level(logging.WARNING):
        model._forward(x.clone(), t, [(0, 24, 0)])
        model._forward(x.clone(), t, [(0, 24, 0)])
    assert "forward 1" in caplog.text
    assert (tmp_path / "t-r0-fwd2.json").exists() and (tmp_path / "t-r0-fwd2.txt").exists()
    sp = types.SimpleNamespace(sp_forward=lambda *a: 7)
    prof.install_sp(sp)
    assert sp.sp_forward() == 7


def test_node_packages_import(monkeypatch):
    """ComfyUI imports each node folder's __init__: both expose empty node
    mappings and call install() (a no-op without the enabling variables)."""
    monkeypatch.delenv("H3_LINEAR_FAST", raising=False)
    monkeypatch.delenv("H3_FUSE", raising=False)
    _fresh(monkeypatch)
    for d, name in ((LF, "h3lf_node"), (FG, "h3fg_node")):
        spec = importlib.util.spec_from_file_location(name, os.path.join(d, "__init__.py"),
                                                      submodule_search_locations=[d])
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        assert mod.NODE_CLASS_MAPPINGS == {} and mod.NODE_DISPLAY_NAME_MAPPINGS == {}


def test_rope_patch_install_and_cpu_fallback(monkeypatch):
    """H3_FUSE_ROPE=1 points comfy.quant_ops.ck at the HIP version; CPU tensors
    are not taken and go to the original, whose result is returned unchanged."""
    monkeypatch.setenv("H3_FUSE_ROPE", "1")
    (rp,) = _fresh(monkeypatch, "h3_rope_patch")
    qo = importlib.import_module("comfy.quant_ops")
    orig_, orig = qo.ck.rms_rope_split_half_, qo.ck.rms_rope_split_half
    assert rp.install() and qo.ck.rms_rope_split_half_ is not orig_ and qo.ck.rms_rope_split_half is not orig
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 5, 2, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 5, 2, 64, generator=g).to(torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    tab = torch.zeros(1, 5, 32, 2, 2, dtype=torch.bfloat16)
    tab[..., 0, 0] = tab[..., 1, 1] = 1
    q2, k2 = q.clone(), k.clone()
    qo.ck.rms_rope_split_half_(q, k, tab, w, w, epsilon=1e-6, rot_dim=64)
    orig_(q2, k2, tab, w, w, epsilon=1e-6, rot_dim=64)
    assert torch.equal(q, q2) and torch.equal(k, k2)
    assert rp.stats()["fallback_calls"] == 1 and rp.stats()["fast_calls"] == 0
    assert not rp.eligible(q, k, tab, w, w, 64)                        # CPU tensors
    rp.uninstall()
    assert qo.ck.rms_rope_split_half_ is orig_ and qo.ck.rms_rope_split_half is orig


def test_rope_patch_needs_env(monkeypatch):
    monkeypatch.delenv("H3_FUSE_ROPE", raising=False)
    (rp,) = _fresh(monkeypatch, "h3_rope_patch")
    assert rp.install() is False and not rp.stats()["installed"]
