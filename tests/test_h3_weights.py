"""The H3 checkpoint-format harness on the CPU: keys, shapes and scale handling
of a synthetic safetensors file laid out like the reference's checkpoint
(tests/bench_linear.py:12,25-29)."""
import pytest
import torch

from h3mi import h3_weights as HW


def _write(tmp_path, layers, per_tensor=False):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(5)
    tensors, ref = {}, {}
    for name in layers:
        k, n = HW.SHAPES[name]
        w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        s = torch.rand(1 if per_tensor else n, 1, generator=g) * 1e-2
        kw, ks = HW.keys(name, block=3)
        tensors[kw], tensors[ks] = w, s.to(torch.bfloat16)
        ref[name] = (w, s.to(torch.bfloat16))
    path = tmp_path / "h3_int8.safetensors"
    save_file(tensors, str(path))
    return path, ref


def test_keys_follow_the_checkpoint_layout():
    assert HW.keys("qkv") == ("blocks.0.attn.qkv_proj.weight", "blocks.0.attn.qkv_proj.weight_scale")
    assert HW.keys("fc2", 49) == ("blocks.49.mlp.fc2.weight", "blocks.49.mlp.fc2.weight_scale")
    with pytest.raises(KeyError):
        HW.keys("proj")


def test_shapes_are_the_h3_dims():
    assert HW.SHAPES["qkv"] == (HW.HIDDEN, 3 * HW.HEADS * HW.HEAD_DIM)
    assert HW.SHAPES["out"] == (HW.HEADS * HW.HEAD_DIM, HW.HIDDEN)
    assert HW.SHAPES["fc1"][1] == 2 * HW.SHAPES["fc2"][0]  # fc1 feeds SwiGLU, whose output is fc2's input
    for k, n in HW.SHAPES.values():
        assert k % 128 == 0 and n % 4 == 0  # the GEMM's shape rules


@pytest.mark.parametrize("per_tensor", [False, True])
def test_load_linear(tmp_path, per_tensor):
    path, ref = _write(tmp_path, ["out", "fc2"], per_tensor=per_tensor)
    for name in ["out", "fc2"]:
        w, ws = HW.load_linear(str(path), name, block=3)
        assert torch.equal(w, ref[name][0])
        n = HW.SHAPES[name][1]
        assert ws.dtype == torch.float32 and ws.shape == (n,)
        assert torch.equal(ws, ref[name][1].reshape(-1).float().expand(n))
    with pytest.raises(KeyError):
        HW.load_linear(str(path), "qkv", block=3)  # not in the file


def test_load_rejects_wrong_shape(tmp_path):
    from safetensors.torch import save_file
    kw, ks = HW.keys("out")
    save_file({kw: torch.zeros(8, 16, dtype=torch.int8), ks: torch.ones(8)}, str(tmp_path / "bad.safetensors"))
    with pytest.raises(ValueError):
        HW.load_linear(str(tmp_path / "bad.safetensors"), "out")
