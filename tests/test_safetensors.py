"""The safetensors reader of libmxq (mxq_st_*) and SafetensorsFile, on the CPU.

The header parser is checked against the `safetensors` package's own reader (an
independent implementation) on files it wrote, and against hand-made malformed files.
Quantization parameters are inferred from files holding the oracle's quantized triples."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

import wuxianhuabu_amd as mx


def _u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).view(torch.uint32)


def _bf16(u16):
    return torch.from_numpy(np.ascontiguousarray(u16, np.uint16).view(np.int16)).view(
        torch.bfloat16)


def test_header_and_bytes_match_the_safetensors_package(tmp_path):
    g = torch.Generator().manual_seed(0)
    t = {
        "blocks.0.attn.qkv.weight": _u32(np.arange(96 * 24).reshape(96, 24)),
        "blocks.0.attn.qkv.scales": torch.randn(96, 4, generator=g).bfloat16(),
        "blocks.0.attn.qkv.biases": torch.randn(96, 4, generator=g).bfloat16(),
        "norm.weight": torch.randn(4096, generator=g),
        "emb": torch.randn(3, 5, 7, generator=g).half(),
        "idx": torch.arange(10, dtype=torch.int64),
        "mask": torch.tensor([True, False, True]),
        "empty": torch.zeros(0, 4),
        "scalar": torch.tensor(2.5),
        "名字.权重": torch.ones(2, 2),
    }
    path = tmp_path / "m.safetensors"
    save_file(t, str(path), metadata={"format": "mlx", "nested": json.dumps({"a": [1, 2]})})
    f = mx.SafetensorsFile(path, device="cpu")
    with safe_open(str(path), "pt") as ref:
        assert sorted(f.keys()) == sorted(ref.keys())
        for k in ref.keys():
            sl = ref.get_slice(k)
            dt, shape, nbytes = f.info(k)
            assert dt == sl.get_dtype() and list(shape) == list(sl.get_shape()), k
            got = f.get(k)
            want = ref.get_tensor(k)
            assert got.dtype == want.dtype and tuple(got.shape) == tuple(want.shape)
            assert nbytes == want.numel() * want.element_size()
            raw = lambda a: a.reshape(-1).view(torch.uint8) if a.numel() else a.reshape(-1)
            assert torch.equal(raw(got), raw(want)), k
    w, s, b = f.get_quantized("blocks.0.attn.qkv")
    assert w.dtype == torch.uint32 and tuple(s.shape) == (96, 4)
    assert f.get("missing") is None and f.get_quantized("norm") is None
    f.close()
    with pytest.raises(ValueError, match="closed"):
        f.info("norm.weight")


def test_weight_dot_scales_spelling(tmp_path):
    path = tmp_path / "h3.safetensors"
    save_file({"fc1.weight": _u32(np.ones((8, 6))), "fc1.weight.scales": torch.ones(8, 1).bfloat16(),
               "fc1.weight.biases": torch.zeros(8, 1).bfloat16()}, str(path))
    with mx.SafetensorsFile(path, device="cpu") as f:
        w, s, b = f.get_quantized("fc1")
        assert tuple(w.shape) == (8, 6) and tuple(b.shape) == (8, 1)


def _raw(tmp_path, header, data=b"", n=None):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    p = tmp_path / "bad.safetensors"
    p.write_bytes(struct.pack("<Q", len(h) if n is None else n) + h + data)
    return p


@pytest.mark.parametrize("case", ["tiny", "length", "json", "range", "size", "dup", "deep",
                                  "offsets", "missing", "end_overflow", "begin_overflow",
                                  "unknown_dtype_range", "size_overflow"])
def test_malformed_files_are_rejected(tmp_path, case):
    ok = {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    if case == "tiny":
        p = tmp_path / "t.safetensors"
        p.write_bytes(b"\x01\x00")
    elif case == "length":
        p = _raw(tmp_path, ok, b"\0" * 8, n=10 ** 6)
    elif case == "json":
        p = _raw(tmp_path, b"{not json}", b"\0" * 8)
    elif case == "range":
        p = _raw(tmp_path, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}},
                 b"\0" * 8)
    elif case == "size":
        p = _raw(tmp_path, {"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}},
                 b"\0" * 8)
    elif case == "dup":
        p = _raw(tmp_path, b'{"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}, '
                           b'"a": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}',
                 b"\0" * 2)
    elif case == "deep":
        p = _raw(tmp_path, b'{"__metadata__": ' + b"[" * 200 + b"]" * 200 + b"}")
    elif case == "offsets":
        p = _raw(tmp_path, {"a": {"dtype": "F32", "shape": [2], "data_offsets": [8, 0]}},
                 b"\0" * 8)
    elif case == "end_overflow":  # offset + start would wrap past INT64_MAX
        p = _raw(tmp_path, {"a": {"dtype": "U8", "shape": [64],
                                  "data_offsets": [2 ** 63 - 101, 2 ** 63 - 37]}}, b"\0" * 8)
    elif case == "begin_overflow":
        p = _raw(tmp_path, {"a": {"dtype": "U8", "shape": [0],
                                  "data_offsets": [2 ** 63 - 2, 2 ** 63 - 2]}}, b"\0" * 8)
    elif case == "unknown_dtype_range":  # a dtype without a known size is range-checked too
        p = _raw(tmp_path, {"a": {"dtype": "XX", "shape": [4],
                                  "data_offsets": [0, 2 ** 63 - 10]}}, b"\0" * 8)
    elif case == "size_overflow":  # element count x item size past INT64_MAX
        p = _raw(tmp_path, {"a": {"dtype": "F64", "shape": [2 ** 62],
                                  "data_offsets": [0, 8]}}, b"\0" * 8)
    else:
        p = tmp_path / "none.safetensors"
    with pytest.raises(ValueError, match=r"\[safetensors\]"):
        mx.SafetensorsFile(p, device="cpu")


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 32), (2, 128), (6, 64), (3, 128), (5, 32)])
@pytest.mark.parametrize("mode", [0, 1])
def test_infer_quant_params(tmp_path, O, bits, gs, mode):
    """Files whose widths fit several (bits, group_size) pairs resolve to the true one."""
    K, N = 2048, 48
    rng = np.random.default_rng(bits * 10 + gs + mode)
    t = {}
    for i in range(3):
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        q = O.quantize(w, gs, bits, mode=mode)
        t[f"l{i}.weight"] = _u32(q["wq"])
        t[f"l{i}.scales"] = _bf16(q["scales_bf16"])
        t[f"l{i}.biases"] = _bf16(q["biases_bf16"])
    t["norm.weight"] = torch.ones(K)
    path = tmp_path / "q.safetensors"
    save_file(t, str(path))
    with mx.SafetensorsFile(path, device="cpu") as f:
        assert f.infer_quant_params() == (bits, gs)
        lin = mx.MfLinear.load(f, "l1", in_features=K)
        assert (lin.bits, lin.group_size, lin.out_dim) == (bits, gs, N)


def test_no_quantized_layers(tmp_path):
    path = tmp_path / "d.safetensors"
    save_file({"w.weight": torch.ones(4, 4)}, str(path))
    with mx.SafetensorsFile(path, device="cpu") as f:
        assert f.infer_quant_params() is None
