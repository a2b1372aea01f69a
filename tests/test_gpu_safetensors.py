"""Device reads of libmxq's safetensors reader (mmap -> two pinned staging buffers ->
hipMemcpyAsync): bytes equal the file's across chunk boundaries and back-to-back reads
that reuse the staging buffers, and modules loaded from a file equal the same modules
built from the tensors in memory."""
import pytest
import torch
from safetensors.torch import save_file

import wuxianhuabu_amd as mx

pytestmark = pytest.mark.gpu


def test_device_reads_match_file_bytes(dev, tmp_path):
    g = torch.Generator().manual_seed(1)
    t = {"big": torch.randint(-2 ** 31, 2 ** 31 - 1, (10_000_003,), generator=g,
                              dtype=torch.int64).to(torch.int32).view(torch.uint32),
         "mid": torch.randn(4097, 1031, generator=g).bfloat16(),
         "small": torch.randn(7, generator=g),
         "empty": torch.zeros(0, 3)}
    path = tmp_path / "w.safetensors"
    save_file(t, str(path))
    with mx.SafetensorsFile(path, device=dev) as f:
        got = {k: f.get_uncached(k) for k in ("big", "mid", "small", "empty", "big")}
        torch.cuda.synchronize()
        for k, v in got.items():
            assert v.device.type == "cuda"
            a = v.cpu().reshape(-1)
            b = t[k].reshape(-1)
            if a.numel():
                assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), k
            else:
                assert b.numel() == 0


def test_modules_load_from_file(dev, tmp_path):
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    hidden, ffn = 512, 768
    tensors = {}
    for name, n, k in (("blk.mlp.fc1", 2 * ffn, hidden), ("blk.mlp.fc2", hidden, ffn)):
        w = torch.randn(n, k, generator=g, device=dev) * 0.05
        wq, s, b = mx.quantized(w, 64, 6, scales_dtype=torch.bfloat16, mode="minmax")
        tensors[name + ".weight"] = wq
        tensors[name + ".weight.scales"] = s   # the H3 spelling
        tensors[name + ".weight.biases"] = b
        tensors[name + ".bias"] = (torch.randn(n, generator=g, device=dev) * 0.1).bfloat16()
    path = tmp_path / "h3.safetensors"
    save_file({k: v.cpu() for k, v in tensors.items()}, str(path))
    x = torch.randn(300, hidden, generator=g, device=dev).bfloat16()
    mem = mx.H3MlpW.load(tensors, "blk.mlp", hidden, ffn)
    with mx.SafetensorsFile(path, device=dev) as f:
        assert f.infer_quant_params() == (6, 64)
        disk = mx.H3MlpW.load(f, "blk.mlp", hidden, ffn)
        assert torch.equal(disk(x), mem(x))
        lin = mx.MfLinear.load(f, "blk.mlp.fc2", in_features=ffn)
        xin = torch.randn(40, ffn, generator=g, device=dev).bfloat16()
        assert torch.equal(lin(xin), mem.fc2(xin))
