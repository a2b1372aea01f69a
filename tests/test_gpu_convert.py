"""The checkpoint quantizer and quantize_module on the GPU: the triples they write are
bit-exact with the oracle's quantizer (mlx's algorithm, mode 1) on the same bf16
values, the kept tensors are byte-identical, and the output file serves MfLinear
through the loader."""
import numpy as np
import torch
import pytest
from safetensors import safe_open
from safetensors.torch import save_file

import wuxianhuabu_amd as mx
from tests.gpu_util import assert_tight, host_bf16, host_f32_of_bf16, host_words

pytestmark = pytest.mark.gpu


def _bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("bits,gs", [(4, 64), (6, 64), (2, 32), (3, 128), (5, 64), (8, 32),
                                     (6, 128), (4, 32)])
def test_quantize_checkpoint_matches_oracle(dev, O, tmp_path, bits, gs):
    g = torch.Generator().manual_seed(bits)
    src_t = {
        "blocks.0.norm.weight": torch.randn(256, generator=g).bfloat16(),
        "blocks.0.adaln_proj.linear.weight": torch.randn(384, 8, generator=g).bfloat16(),
        "adaln_t_table": torch.randn(33, 8, generator=g),
        "blocks.0.attn.qkv.weight": (torch.randn(192, 256, generator=g) * 0.02).bfloat16(),
        "blocks.0.attn.qkv.bias": torch.randn(192, generator=g).bfloat16(),
        "blocks.0.odd.weight": torch.randn(10, 96, generator=g).bfloat16(),
        "blocks.0.mlp.fc2.weight": (torch.randn(64, 384, generator=g) * 0.02).bfloat16(),
        "blocks.0.empty.weight": torch.zeros(0, 128).bfloat16(),
    }
    src, dst = tmp_path / "dense.safetensors", tmp_path / "q.safetensors"
    save_file(src_t, str(src))
    stats = mx.quantize_checkpoint(src, dst, group_size=gs, bits=bits, device=dev)
    quant = {k for k, v in src_t.items() if mx.should_quant("BF16" if v.dtype == torch.bfloat16
                                                            else "F32", tuple(v.shape), gs)}
    assert stats["quantized"] == len(quant) and stats["kept"] == len(src_t) - len(quant)
    if gs == 64:
        assert len(quant) == 3  # qkv, fc2 and the empty weight; the [384, 8] table is kept
    with safe_open(str(dst), framework="pt") as f:
        keys = set(f.keys())
        for k, v in src_t.items():
            if k in quant:
                assert {k, k + ".scales", k + ".biases"} <= keys
                wq = f.get_tensor(k).view(torch.int32).numpy().view(np.uint32)
                s = _bf16_bits(f.get_tensor(k + ".scales"))
                b = _bf16_bits(f.get_tensor(k + ".biases"))
                n, kd = v.shape
                assert wq.shape == (n, kd * bits // 32) and s.shape == b.shape == (n, kd // gs)
                if n == 0:
                    continue
                ref = O.quantize(v.float().numpy().reshape(v.shape), gs, bits, mode=1)
                np.testing.assert_array_equal(wq, ref["wq"].reshape(wq.shape), err_msg=k)
                np.testing.assert_array_equal(s, ref["scales_bf16"].reshape(s.shape), err_msg=k)
                np.testing.assert_array_equal(b, ref["biases_bf16"].reshape(b.shape), err_msg=k)
            else:
                assert torch.equal(f.get_tensor(k), v), k
    # the output serves the loader: parameter inference and a layer's forward
    with mx.SafetensorsFile(dst, device=dev) as f:
        if (bits, gs) in ((4, 64), (6, 64)):  # widths that fit one (bits, gs) pair only, or
            assert f.infer_quant_params() == (bits, 64)  # resolved by code statistics
        lin = mx.MfLinear.load(f, "blocks.0.attn.qkv", 256)
        assert lin.is_quantized and lin.bits == bits and lin.group_size == gs
        assert lin.bias is not None
        x = O.normal_bf16(5, 70 * 256).reshape(70, 256)
        xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(dev)
        y = host_f32_of_bf16(lin(xd))
        ref = O.quantize(src_t["blocks.0.attn.qkv.weight"].float().numpy(), gs, bits, mode=1)
        bias = _bf16_bits(src_t["blocks.0.attn.qkv.bias"])
        assert_tight(y, O.qmm_f64_bf16w(x, ref["wq"], ref["scales_bf16"], ref["biases_bf16"], gs,
                                        bits, bias=bias), "converted layer")


def test_quantize_module_zimage_filter(dev, O):
    """quantize(model:filter:) with the Z-Image filter (`Weights.swift:12-37`): the
    precision-sensitive layers stay dense, every other Linear becomes a quantized layer
    whose weights are mlx's quantization of the bf16 weight."""
    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv = torch.nn.Linear(128, 384)
            self.out = torch.nn.Linear(128, 128, bias=False)
            self.adaLN_modulation = torch.nn.Sequential(torch.nn.SiLU(), torch.nn.Linear(64, 256))

    class Net(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.x_embedder = torch.nn.Linear(64, 128)
            self.layers = torch.nn.ModuleList([Block(), Block()])
            self.final_layer = torch.nn.Linear(128, 64)
            self.norm = torch.nn.LayerNorm(128)

    torch.manual_seed(0)
    net = Net().to(dev).bfloat16()
    dense = {n: m.weight.detach().clone() for n, m in net.named_modules()
             if isinstance(m, torch.nn.Linear)}

    def keep_hi(path):
        return (any(path.startswith(p) for p in ("x_embedder", "final_layer", "t_embedder",
                                                  "cap_embedder_linear")) or
                path.endswith("adaLN_modulation.1"))

    done = mx.quantize_module(net, lambda path, m: None if keep_hi(path) else (64, 6, "affine"))
    assert done == ["layers.0.qkv", "layers.0.out", "layers.1.qkv", "layers.1.out"]
    assert isinstance(net.x_embedder, torch.nn.Linear)
    assert isinstance(net.final_layer, torch.nn.Linear)
    assert isinstance(net.layers[0].adaLN_modulation[1], torch.nn.Linear)
    for path in done:
        q = net.get_submodule(path).q
        assert isinstance(q, mx.QuantizedLinear) and q.bits == 6 and q.group_size == 64
        w = dense[path].float().cpu().numpy()
        ref = O.quantize(w, 64, 6, mode=1)
        np.testing.assert_array_equal(host_words(q.weight), ref["wq"], err_msg=path)
        np.testing.assert_array_equal(host_bf16(q.scales), ref["scales_bf16"], err_msg=path)
    x = torch.randn(80, 128, device=dev).bfloat16()
    blk = net.layers[0]
    y = blk.qkv(x)
    assert tuple(y.shape) == (80, 384)
    assert blk.out.q.bias is None
    ref = mx.quantized_matmul(x, blk.qkv.q.weight, blk.qkv.q.scales, blk.qkv.q.biases,
                              group_size=64, bits=6, bias=blk.qkv.q.bias)
    assert torch.equal(y, ref)
