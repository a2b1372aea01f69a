"""The checkpoint quantizer's host side: the should_quant rule, the planned output
header, and byte-exact copies of the tensors it keeps (no quantization runs here;
tests/test_gpu_convert.py covers the triples)."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

import wuxianhuabu_amd as mx
from wuxianhuabu_amd import convert


@pytest.mark.parametrize("dtype,shape,expect", [
    ("BF16", (5376, 5376), True),      # a DiT projection
    ("BF16", (96768, 8), False),       # pruned adaLN factor table: last dim 8 < 64
    ("F32", (1025, 8), False),         # timestep table, F32
    ("F32", (4096, 4096), False),      # F32 kept at full precision
    ("F16", (4096, 4096), False),
    ("BF16", (5376,), False),          # 1-D norm weight / bias
    ("BF16", (2, 64, 64), False),      # 3-D
    ("BF16", (10, 96), False),         # 96 % 64 != 0
    ("BF16", (10, 64), True),          # exactly one group
    ("BF16", (10, 63), False),
    ("BF16", (0, 128), True),          # empty rows still form a 2-D BF16 tensor
])
def test_should_quant_rule(dtype, shape, expect):
    """`quantize_h3_g64.py:92-99`: BF16 and 2-D and last dim >= 64 and % 64 == 0."""
    assert convert.should_quant(dtype, shape) is expect


def test_should_quant_follows_group_size():
    assert convert.should_quant("BF16", (4, 96), group_size=32)
    assert not convert.should_quant("BF16", (4, 96), group_size=64)
    assert not convert.should_quant("BF16", (4, 64), group_size=128)


def _mixed_source(path):
    g = torch.Generator().manual_seed(0)
    t = {
        "blk.norm.weight": torch.randn(256, generator=g).bfloat16(),
        "blk.adaln.linear.weight": torch.randn(96, 8, generator=g).bfloat16(),
        "adaln_t_table": torch.randn(17, 8, generator=g),
        "blk.lin.weight": torch.randn(192, 256, generator=g).bfloat16(),
        "blk.lin.bias": torch.randn(192, generator=g).bfloat16(),
        "blk.odd.weight": torch.randn(10, 96, generator=g).bfloat16(),
        "blk.f16.weight": torch.randn(8, 64, generator=g).half(),
        "blk.cube": torch.randn(2, 4, 64, generator=g).bfloat16(),
        "blk.up.weight": torch.randn(64, 128, generator=g).bfloat16(),
    }
    save_file(t, str(path))
    return t


def test_dry_run_counts_and_size(tmp_path):
    src = tmp_path / "src.safetensors"
    _mixed_source(src)
    stats = mx.quantize_checkpoint(src, tmp_path / "never.safetensors", bits=4, dry_run=True)
    assert stats["quantized"] == 2 and stats["kept"] == 7 and stats["entries"] == 13
    assert not (tmp_path / "never.safetensors").exists()
    with mx.SafetensorsFile(src, device="cpu") as f:
        header, data = convert._header(convert._plan(f, 64, 4))
    # 2 triples (192x256 and 64x128, 4-bit) + the 7 kept tensors
    kept = (256 * 2 + 96 * 8 * 2 + 17 * 8 * 4 + 192 * 2 + 10 * 96 * 2 + 8 * 64 * 2 +
            2 * 4 * 64 * 2)
    trip = sum(n * k // 2 + 2 * n * (k // 64) * 2 for n, k in ((192, 256), (64, 128)))
    assert data == kept + trip
    assert stats["bytes"] == 8 + len(header) + data and len(header) % 8 == 0


def test_header_plan_layout(tmp_path):
    """Entries in source order, the triple as k / k.scales / k.biases, contiguous
    offsets from 0, U32 codes [N, K*bits/32], BF16 scales and biases [N, K/gs]."""
    src = tmp_path / "src.safetensors"
    _mixed_source(src)
    with mx.SafetensorsFile(src, device="cpu") as f:
        order = f.keys()
        raw, total = convert._header(convert._plan(f, 64, 6))
    h = json.loads(raw)
    assert h.pop("__metadata__") == {"format": "mlx"}
    expect_keys = []
    for k in order:
        expect_keys += [k, k + ".scales", k + ".biases"] if k in ("blk.lin.weight",
                                                                  "blk.up.weight") else [k]
    assert list(h) == expect_keys
    assert h["blk.lin.weight"]["dtype"] == "U32"
    assert h["blk.lin.weight"]["shape"] == [192, 256 * 6 // 32]
    assert h["blk.lin.weight.scales"] == {"dtype": "BF16", "shape": [192, 4],
                                          "data_offsets": h["blk.lin.weight.scales"]
                                          ["data_offsets"]}
    off = 0
    for k in expect_keys:
        lo, hi = h[k]["data_offsets"]
        assert lo == off and hi >= lo
        off = hi
    assert off == total


def test_kept_tensors_copied_byte_for_byte(tmp_path):
    """A file with nothing to quantize converts without a GPU; the output reads back
    through the safetensors package and through libmxq's loader, byte for byte."""
    src, dst = tmp_path / "src.safetensors", tmp_path / "out" / "dst.safetensors"
    g = torch.Generator().manual_seed(1)
    t = {"a": torch.randn(5, 8, generator=g).bfloat16(), "b": torch.randn(3, 7, generator=g),
         "c": torch.arange(12, dtype=torch.int64).reshape(3, 4),
         "d": torch.randn(7, generator=g).half(), "e": torch.zeros(0, 4)}
    save_file(t, str(src))
    stats = mx.quantize_checkpoint(src, dst, device="cpu")
    assert stats["quantized"] == 0 and stats["kept"] == 5
    assert stats["bytes"] == dst.stat().st_size
    with safe_open(str(dst), framework="pt") as f:
        assert sorted(f.keys()) == sorted(t)
        for k, v in t.items():
            assert torch.equal(f.get_tensor(k), v), k
    with mx.SafetensorsFile(dst, device="cpu") as f:
        for k, v in t.items():
            assert bytes(f.read_bytes(k)) == v.contiguous().view(torch.uint8).numpy().tobytes()
    n = struct.unpack("<Q", dst.read_bytes()[:8])[0]
    assert n % 8 == 0


def test_read_bytes_any_dtype(tmp_path):
    p = tmp_path / "x.safetensors"
    save_file({"f8": torch.ones(4).to(torch.float8_e4m3fn)}, str(p))
    with mx.SafetensorsFile(p, device="cpu") as f:
        assert f.info("f8")[0] == "F8_E4M3"
        assert f.read_bytes("f8").tolist() == [0x38] * 4


def test_filter_answers():
    """quantize(model:filter:)'s filter returns nil or (groupSize, bits, mode)."""
    p = convert._params
    assert p(None, 64, 4, "mlx_edge") is None and p(False, 64, 4, "mlx_edge") is None
    assert p(True, 64, 4, "mlx_edge") == (64, 4, "mlx_edge")
    assert p((32, 8), 64, 4, "mlx_edge") == (32, 8, "mlx_edge")
    assert p((128, 6, "affine"), 64, 4, "minmax") == (128, 6, "mlx_edge")
    assert p((64,), 64, 4, "minmax") == (64, 4, "minmax")


def test_quantize_module_keeps_what_the_filter_rejects():
    m = torch.nn.Sequential(torch.nn.Linear(64, 32), torch.nn.ReLU(),
                            torch.nn.Sequential(torch.nn.Linear(32, 16)))
    assert mx.quantize_module(m, filter=lambda path, mod: None) == []
    assert isinstance(m[0], torch.nn.Linear) and isinstance(m[2][0], torch.nn.Linear)
    # no filter: only Linears whose input width the group size divides (64 and 32 are not
    # multiples of 128)
    assert mx.quantize_module(m, group_size=128) == []


def test_cli_dry_run(tmp_path, capsys):
    src = tmp_path / "src.safetensors"
    _mixed_source(src)
    assert convert.main(["--src", str(src), "--dst", str(tmp_path / "o.safetensors"),
                         "--dry-run"]) == 0
    out = capsys.readouterr().out
    assert "quantize 2 (6 entries), keep 7, 13 entries" in out
    np.testing.assert_equal((tmp_path / "o.safetensors").exists(), False)
