"""The drop-in patches on the GPU against the stand-in upstream modules:
the patched int8_linear and DiTBlock.forward must return exactly what the
original (eager) functions return, count their calls, and fall back / disable
themselves as the reference does."""
import importlib
import os
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

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


def test_linear_fast_path_bitexact(monkeypatch):
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.setenv("H3_LINEAR_FAST_PLAIN", "1")  # convrot=False calls: opt-in
    monkeypatch.setenv("H3_LINEAR_FAST_BIAS", "1")
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    ckc = importlib.import_module("comfy_kitchen.backends.cuda")
    orig = ckc.int8_linear
    assert lf.install()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 640, 1024, generator=g).to(torch.bfloat16).cuda()
    w = torch.randint(-127, 128, (768, 1024), generator=g, dtype=torch.int8).cuda()
    ws = (1e-3 + 9e-3 * torch.rand(768, generator=g)).cuda()
    b = (0.02 * torch.randn(768, generator=g)).to(torch.bfloat16).cuda()
    for bias in (None, b):
        out = ckc.int8_linear(x, w, ws, bias)
        ref = orig(x, w, ws, bias)
        assert out.shape == (2, 640, 768) and torch.equal(out, ref)
    st = lf.stats()
    assert st["fast_calls"] == 2 and st["fallback_calls"] == 0
    small = ckc.int8_linear(x[:, :100], w, ws)                        # m = 200 < MIN_M
    assert torch.equal(small, orig(x[:, :100], w, ws)) and lf.stats()["fallback_calls"] == 1
    lf.uninstall()


def test_linear_kernel_error_disables(monkeypatch):
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.setenv("H3_LINEAR_FAST_PLAIN", "1")  # convrot=False calls: opt-in
    (lf, tg) = _fresh(monkeypatch, "h3_linear_fast_patch", "int8_gemm_hip")
    ckc = importlib.import_module("comfy_kitchen.backends.cuda")
    orig = ckc.int8_linear
    assert lf.install()

    def boom(*a, **k):
        raise RuntimeError("forced failure")

    monkeypatch.setattr(tg, "int8_mm_scaled", boom)
    x = torch.randn(512, 256, device="cuda").to(torch.bfloat16)
    w = torch.randint(-127, 128, (64, 256), dtype=torch.int8, device="cuda")
    ws = torch.rand(64, device="cuda") * 1e-2
    assert torch.equal(ckc.int8_linear(x, w, ws), orig(x, w, ws))
    assert lf.stats()["disabled"] is True
    calls = ckc.CALLS["int8_linear"]
    ckc.int8_linear(x, w, ws)                                          # sticky: straight to the original
    assert ckc.CALLS["int8_linear"] == calls + 1 and lf.stats()["fallback_calls"] >= 1
    lf.uninstall()


@pytest.mark.parametrize("segs_kind", ["one", "two", "per_row"])
def test_fused_block_matches_eager(monkeypatch, segs_kind):
    monkeypatch.setenv("H3_FUSE", "1")
    (fp,) = _fresh(monkeypatch, "h3_fuse_patch")
    mm = importlib.import_module("comfy.ldm.minimax.model")
    orig = mm.DiTBlock.forward
    torch.manual_seed(0)
    dim, S = 512, 300
    blk = mm.DiTBlock(dim, 8, 2 * dim, tdim=64, device="cuda")
    with torch.no_grad():
        blk.norm1.weight.copy_((1 + 0.02 * torch.randn(dim, device="cuda")).to(torch.bfloat16))
        blk.norm2.weight.copy_((1 + 0.02 * torch.randn(dim, device="cuda")).to(torch.bfloat16))
    x = torch.randn(S, dim, device="cuda").to(torch.bfloat16)
    t = torch.randn(3, 64, device="cuda")
    segs = {"one": [(0, S, 0)], "two": [(0, 100, 2), (100, S, 1)],
            "per_row": [(0, 50, torch.randint(0, 3, (50,), device="cuda")), (50, S, 0)]}[segs_kind]
    assert fp.install()
    with torch.no_grad():
        ref = orig(blk, x.clone(), t, segs, None)
        out = blk(x.clone(), t, segs, None)
    assert fp.stats()["fused"] == 1 and fp.stats()["fallback"] == 0
    assert torch.equal(out, ref), int((out != ref).sum())
    fp.uninstall()


def test_fused_block_grad_and_layout_fallbacks(monkeypatch):
    monkeypatch.setenv("H3_FUSE", "1")
    (fp,) = _fresh(monkeypatch, "h3_fuse_patch")
    mm = importlib.import_module("comfy.ldm.minimax.model")
    torch.manual_seed(1)
    blk = mm.DiTBlock(256, 4, 512, tdim=32, device="cuda")
    for p in blk.parameters():
        p.requires_grad_(False)
    x = torch.randn(64, 256, device="cuda").to(torch.bfloat16)
    t = torch.randn(1, 32, device="cuda")
    assert fp.install()
    with torch.no_grad():
        blk(x.clone(), t, [(0, 60, 0)], None)                        # segments do not cover the rows
        wide = torch.zeros(64, 512, device="cuda", dtype=torch.bfloat16)
        wide[:, :256] = x
        blk(wide[:, :256], t, [(0, 64, 0)], None)                    # not contiguous
    blk(x.clone(), t, [(0, 64, 0)], None)                            # grad enabled
    st = fp.stats()
    assert st["fallback"] == 3 and st["fused"] == 0
    fp.uninstall()


def test_fused_block_quant_handoff(monkeypatch):
    """H3_FUSE_QUANT=1: the fused norms also quantize h and offer it to the
    INT8 linear that opens the attention and MLP calls; that linear skips its
    quantizer (prequant_calls) and the block output stays exactly the eager
    block's with the original int8_linear."""
    monkeypatch.setenv("H3_FUSE", "1")
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.setenv("H3_LINEAR_FAST_PLAIN", "1")  # convrot=False calls: opt-in
    (fp, lf) = _fresh(monkeypatch, "h3_fuse_patch", "h3_linear_fast_patch")
    mm = importlib.import_module("comfy.ldm.minimax.model")
    ckc = importlib.import_module("comfy_kitchen.backends.cuda")
    orig_lin, orig_fwd = ckc.int8_linear, mm.DiTBlock.forward
    mode = {"lin": orig_lin}

    def lin(x, mod):
        return mode["lin"](x, mod.w8, mod.ws8)

    torch.manual_seed(3)
    dim, S = 512, 320
    blk = mm.DiTBlock(dim, 8, 2 * dim, tdim=64, device="cuda", linear=lin)
    for m in (blk.attn.qkv_proj, blk.attn.out_proj, blk.mlp.fc1, blk.mlp.fc2):
        dout, din = m.weight.shape
        m.w8 = torch.randint(-127, 128, (dout, din), dtype=torch.int8, device="cuda")
        m.ws8 = torch.rand(dout, device="cuda") * 1e-2
    with torch.no_grad():
        blk.norm1.weight.copy_((1 + 0.02 * torch.randn(dim, device="cuda")).to(torch.bfloat16))
        blk.norm2.weight.copy_((1 + 0.02 * torch.randn(dim, device="cuda")).to(torch.bfloat16))
    x = torch.randn(S, dim, device="cuda").to(torch.bfloat16)
    t = torch.randn(2, 64, device="cuda")
    segs = [(0, 40, 1), (40, S, 0)]
    with torch.no_grad():
        ref = orig_fwd(blk, x.clone(), t, segs, None)
    assert lf.install() and fp.install()
    mode["lin"] = ckc.int8_linear                                         # the patched function
    with torch.no_grad():
        monkeypatch.setenv("H3_FUSE_QUANT", "0")
        out0 = blk(x.clone(), t, segs, None)
        assert lf._state["prequant_calls"] == 0
        monkeypatch.setenv("H3_FUSE_QUANT", "1")
        out1 = blk(x.clone(), t, segs, None)
    assert torch.equal(out0, ref) and torch.equal(out1, ref)
    st = lf.stats()
    assert lf._state["prequant_calls"] == 2 and st["fast_calls"] == 8 and st["fallback_calls"] == 0
    assert fp.stats()["fused"] == 2
    fp.uninstall()
    lf.uninstall()


@pytest.mark.parametrize("act", [None, "swiglu"])
def test_linear_convrot_path(monkeypatch, act):
    """convrot=True calls (the only ones the reference's fast path takes,
    comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:64) run the HIP ConvRot
    quantizer + GEMM; the output equals the oracle chain convrot_quant ->
    gemm_i32 -> epilogue_bf16 bit for bit.  The stand-in original has no
    ConvRot path, so a call the fast path declines raises."""
    import numpy as np
    from oracle import oracle as O
    from util import bits
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.delenv("H3_LINEAR_FAST_CONVROT", raising=False)
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    ckc = importlib.import_module("comfy_kitchen.backends.cuda")
    assert lf.install()
    g = torch.Generator().manual_seed(7)
    M, K, N = 300, 1280, 256
    kin = 2 * K if act else K
    x = torch.randn(3, M // 3, kin, generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    ws = 1e-3 + 9e-3 * torch.rand(N, generator=g)
    out = ckc.int8_linear(x.cuda(), w.cuda(), ws.cuda(), None, torch.bfloat16, convrot=True, convrot_groupsize=256,
                          input_act=act)
    assert out.shape == (3, M // 3, N)
    q, s = O.convrot_quant(bits(x.reshape(M, kin)), act)
    ref = O.epilogue_bf16(O.gemm_i32(q, w.numpy()), s, ws.numpy())
    assert np.array_equal(bits(out.reshape(M, N)), ref)
    assert lf.stats()["fast_calls"] == 1 and lf.stats()["fallback_calls"] == 0
    with pytest.raises(NotImplementedError):
        ckc.int8_linear(x.cuda(), w.cuda(), ws.cuda(), None, torch.bfloat16, convrot=True, convrot_groupsize=128,
                        input_act=act)
    lf.uninstall()


def test_rope_patch_matches_eager(monkeypatch):
    """H3_FUSE_ROPE=1: comfy.quant_ops.ck.rms_rope_split_half_ (the call at
    comfyui_nodes/minimax-h3-sp/minimax_sp/sp_forward.py:292-293) runs the HIP
    kernel in place on q / k views of the qkv buffer and returns exactly what
    the eager original returns; the out-of-place form too."""
    monkeypatch.setenv("H3_FUSE_ROPE", "1")
    (rp,) = _fresh(monkeypatch, "h3_rope_patch")
    qo = importlib.import_module("comfy.quant_ops")
    orig_, orig = qo.ck.rms_rope_split_half_, qo.ck.rms_rope_split_half
    assert rp.install()
    g = torch.Generator().manual_seed(3)
    S, H, D = 70, 4, 128
    buf = torch.randn(S, 3 * H * D, generator=g).to(torch.bfloat16).cuda()
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    ang = torch.rand(S, D // 2, generator=g) * 6.3
    tab = torch.stack([torch.stack([ang.cos(), -ang.sin()], -1), torch.stack([ang.sin(), ang.cos()], -1)], -2)
    tab = tab.to(torch.bfloat16)[None].cuda()
    ref = buf.clone()
    q, k = buf[:, :H * D].view(1, S, H, D), buf[:, H * D:2 * H * D].view(1, S, H, D)
    rq, rk = ref[:, :H * D].view(1, S, H, D), ref[:, H * D:2 * H * D].view(1, S, H, D)
    qo.ck.rms_rope_split_half_(q, k, tab, qw, kw, epsilon=1e-6, rot_dim=D)
    orig_(rq, rk, tab, qw, kw, epsilon=1e-6, rot_dim=D)
    assert torch.equal(buf, ref)
    q2 = torch.randn(1, S, H, D, generator=g).to(torch.bfloat16).cuda()
    k2 = torch.randn(1, S, H, D, generator=g).to(torch.bfloat16).cuda()
    a = qo.ck.rms_rope_split_half(q2, k2, tab, qw, kw, epsilon=1e-6, rot_dim=D)
    b = orig(q2, k2, tab, qw, kw, epsilon=1e-6, rot_dim=D)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    st = rp.stats()
    assert st["fast_calls"] == 2 and st["fallback_calls"] == 0
    rp.uninstall()


@pytest.mark.parametrize("shape", [(1,), ()])
def test_linear_per_tensor_weight_scale(monkeypatch, shape):
    """A per-tensor weight scale (one element, or a 0-d tensor) is expanded to
    every output channel before the GEMM (reference
    comfyui_nodes/h3-linear-fast/h3_linear_fast_patch.py:97-99); the output
    equals the stand-in original's, which broadcasts the same scale."""
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.setenv("H3_LINEAR_FAST_PLAIN", "1")  # convrot=False calls: opt-in
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    ckc = importlib.import_module("comfy_kitchen.backends.cuda")
    orig = ckc.int8_linear
    assert lf.install()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(640, 1024, generator=g).to(torch.bfloat16).cuda()
    w = torch.randint(-127, 128, (512, 1024), generator=g, dtype=torch.int8).cuda()
    ws = torch.full(shape, 3.7e-3).cuda()
    out = ckc.int8_linear(x, w, ws)
    assert torch.equal(out, orig(x, w, ws))
    assert lf.stats()["fast_calls"] == 1 and lf.stats()["fallback_calls"] == 0
    lf.uninstall()


def test_linear_act_weight_goes_to_the_original(monkeypatch):
    """convrot=True calls with an activation weight or epsilon cannot be served
    by this library's ConvRot quantizer (it has neither), so they reach the
    original (the stand-in raises for any ConvRot call); a plain call with an
    activation weight too."""
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.delenv("H3_LINEAR_FAST_CONVROT", raising=False)
    (lf,) = _fresh(monkeypatch, "h3_linear_fast_patch")
    ckc = importlib.import_module("comfy_kitchen.backends.cuda")
    assert lf.install()
    x = torch.randn(512, 2 * 1024, device="cuda").to(torch.bfloat16)
    w = torch.randint(-127, 128, (256, 1024), dtype=torch.int8, device="cuda")
    ws = torch.rand(256, device="cuda") * 1e-2
    aw = torch.ones(1024, dtype=torch.bfloat16, device="cuda")
    calls = ckc.CALLS["int8_linear"]
    with pytest.raises(NotImplementedError):
        ckc.int8_linear(x, w, ws, None, torch.bfloat16, convrot=True, input_act="swiglu", input_act_weight=aw)
    with pytest.raises(NotImplementedError):
        ckc.int8_linear(x, w, ws, None, torch.bfloat16, convrot=True, input_act="swiglu", input_act_eps=1e-6)
    assert ckc.CALLS["int8_linear"] == calls + 2
    assert lf.stats()["fast_calls"] == 0 and lf.stats()["fallback_calls"] == 2 and not lf.stats()["disabled"]
    lf.uninstall()


def test_linear_argument_rejection_is_per_call(monkeypatch):
    """An argument error raised by the HIP entry points falls back for that call
    only; the fast path stays enabled for the next call."""
    monkeypatch.setenv("H3_LINEAR_FAST", "1")
    monkeypatch.setenv("H3_LINEAR_FAST_PLAIN", "1")  # convrot=False calls: opt-in
    (lf, tg) = _fresh(monkeypatch, "h3_linear_fast_patch", "int8_gemm_hip")
    ckc = importlib.import_module("comfy_kitchen.backends.cuda")
    orig = ckc.int8_linear
    assert lf.install()
    real = tg.int8_mm_scaled
    state = {"n": 0}

    def reject_once(*a, **k):
        state["n"] += 1
        if state["n"] == 1:
            raise ValueError("rejected")
        return real(*a, **k)

    monkeypatch.setattr(tg, "int8_mm_scaled", reject_once)
    x = torch.randn(512, 256, device="cuda").to(torch.bfloat16)
    w = torch.randint(-127, 128, (64, 256), dtype=torch.int8, device="cuda")
    ws = torch.rand(64, device="cuda") * 1e-2
    assert torch.equal(ckc.int8_linear(x, w, ws), orig(x, w, ws))
    assert lf.stats()["fallback_calls"] == 1 and not lf.stats()["disabled"]
    assert torch.equal(ckc.int8_linear(x, w, ws), orig(x, w, ws))
    assert lf.stats()["fast_calls"] == 1
    lf.uninstall()


def test_host_tensors_are_rejected_before_any_launch():
    """Every tensor operand must be on the GPU of x: a host tensor raises
    ValueError in the Python layer (the C ABI cannot tell host addresses from
    device ones)."""
    import h3mi
    x = torch.randn(64, 512, device="cuda").to(torch.bfloat16)
    w = torch.ones(512, dtype=torch.bfloat16)
    ridx = torch.zeros(64, dtype=torch.int32)
    tab = torch.zeros(1, 512, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        h3mi.norm_mod(x, w, 1e-6, ridx.cuda(), tab, tab)
    with pytest.raises(ValueError):
        h3mi.norm_mod(x, w.cuda(), 1e-6, ridx, tab, tab)
    with pytest.raises(ValueError):
        h3mi.gate_(x, x.clone(), tab.cpu(), ridx.cuda())
    xq = torch.zeros(64, 512, dtype=torch.int8, device="cuda")
    wq = torch.zeros(128, 512, dtype=torch.int8, device="cuda")
    with pytest.raises(ValueError):
        h3mi.int8_mm_scaled(xq, wq, torch.ones(64, 1), torch.ones(128, device="cuda"))
    with pytest.raises(ValueError):
        h3mi.int8_mm_scaled(xq, wq, torch.ones(64, 1, device="cuda"), torch.ones(128))
    with pytest.raises(ValueError):
        h3mi.quantize_rowwise(x, xs=torch.empty(64, 1))
