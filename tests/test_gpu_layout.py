"""Packer, unpacker, quantizer and dequantizer on the GPU: bit-exact against
the oracle (integer and byte work; no tolerance)."""
import ctypes

import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from wuxianhuabu_amd import _lib
from tests.gpu_util import (dev_bf16, dev_f32, dev_u8, dev_words, host_bf16, host_words)

pytestmark = pytest.mark.gpu

BITS = [2, 3, 4, 5, 6, 8]


@pytest.mark.parametrize("bits", BITS)
def test_pack_unpack_bit_exact(dev, O, bits):
    rng = np.random.default_rng(100 + bits)
    for N, K in [(1, 32), (7, 256), (33, 96), (5, 4096)]:
        codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
        wq = mx.pack(dev_u8(codes, dev), bits)
        ref = O.pack_words(codes, bits)
        assert np.array_equal(host_words(wq), ref), (N, K)
        back = mx.unpack(wq, bits)
        assert np.array_equal(back.cpu().numpy(), codes), (N, K)
        # unpack of arbitrary words (every bit pattern is a valid stream)
        words = rng.integers(0, 2**32, size=ref.shape, dtype=np.uint64).astype(np.uint32)
        assert np.array_equal(mx.unpack(dev_words(words, dev), bits).cpu().numpy(),
                              O.unpack(words, K, bits))


def test_pack_golden(dev, golden):
    for case in golden["pack"]:
        codes = np.array(case["codes"], np.uint8)
        wq = mx.pack(dev_u8(codes, dev), case["bits"])
        assert host_words(wq).tolist() == case["words"], case["kind"]


def test_pack_masks_out_of_range_codes(dev, O):
    codes = np.full((2, 64), 0xFF, np.uint8)
    assert np.array_equal(host_words(mx.pack(dev_u8(codes, dev), 4)),
                          O.pack_words(np.full((2, 64), 15, np.uint8), 4))


def _quantize_via_abi(w_dev, w_dtype, N, K, gs, bits, mode, sb_dtype, dev):
    wq = torch.empty((N, K * bits // 32), dtype=torch.uint32, device=dev)
    tdt = torch.float32 if sb_dtype == _lib.MXQ_FLOAT32 else torch.bfloat16
    s = torch.empty((N, K // gs), dtype=tdt, device=dev)
    b = torch.empty_like(s)
    L = _lib.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(L.mxq_quantize(ctypes.c_void_p(w_dev.data_ptr()), w_dtype, N, K, gs, bits, mode,
                              ctypes.c_void_p(wq.data_ptr()), ctypes.c_void_p(s.data_ptr()),
                              ctypes.c_void_p(b.data_ptr()), sb_dtype, st))
    return wq, s, b


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("mode", [0, 1])
def test_quantize_bit_exact(dev, O, bits, gs, mode):
    N, K = 9, 4 * 128
    w = O.normal_f32(500 + bits * 7 + gs, N * K, 0.001, 0.02).reshape(N, K)
    ref = O.quantize(w, gs, bits, mode=mode)
    # fp32 weights -> bf16 scales/biases
    wq, s, b = _quantize_via_abi(dev_f32(w, dev), 0, N, K, gs, bits, mode, 1, dev)
    assert np.array_equal(host_words(wq), ref["wq"])
    assert np.array_equal(host_bf16(s), ref["scales_bf16"])
    assert np.array_equal(host_bf16(b), ref["biases_bf16"])
    # fp32 weights -> fp32 scales/biases
    wq, s, b = _quantize_via_abi(dev_f32(w, dev), 0, N, K, gs, bits, mode, 0, dev)
    assert np.array_equal(host_words(wq), ref["wq"])
    assert np.array_equal(s.cpu().numpy(), ref["scales_f32"])
    assert np.array_equal(b.cpu().numpy(), ref["biases_f32"])
    # bf16 weights: the oracle sees the same bf16 values in fp32
    wb = O.bf16_rne(w)
    ref_b = O.quantize(O.bf16_to_f32(wb), gs, bits, mode=mode)
    wq, s, b = mx.quantized(dev_bf16(wb, dev), gs, bits, mode="minmax" if mode == 0 else "mlx_edge")
    assert np.array_equal(host_words(wq), ref_b["wq"])
    assert np.array_equal(host_bf16(s), ref_b["scales_bf16"])
    assert np.array_equal(host_bf16(b), ref_b["biases_bf16"])


def test_quantized_defaults_to_mlx_edge(dev, O):
    """The drop-in quantized(w, groupSize:, bits:) uses mlx's quantizer unless told
    otherwise (the reference's checkpoints come from mx.quantize,
    `model/minimax h3/tools/quantize_h3_g64.py:132`), and so does
    QuantizedLinear.from_linear."""
    N, K = 16, 256
    w = O.normal_f32(77, N * K, 0.0, 0.02).reshape(N, K)
    ref = O.quantize(w, 64, 6, mode=1)
    wq, s, b = mx.quantized(dev_f32(w, dev), 64, 6, scales_dtype=torch.bfloat16)
    assert np.array_equal(host_words(wq), ref["wq"])
    assert np.array_equal(host_bf16(s), ref["scales_bf16"])
    assert np.array_equal(host_bf16(b), ref["biases_bf16"])
    lin = mx.QuantizedLinear.from_linear(dev_f32(w, dev).bfloat16(), group_size=64, bits=6)
    ref_b = O.quantize(O.bf16_to_f32(O.bf16_rne(w)), 64, 6, mode=1)
    assert np.array_equal(host_words(lin.weight), ref_b["wq"])


def test_quantize_golden(dev, golden):
    for c in golden["quantize"]:
        w = np.array(c["w"], np.float32).reshape(c["N"], c["K"])
        wq, s, b = _quantize_via_abi(dev_f32(w, dev), 0, c["N"], c["K"], c["gs"], c["bits"], 0,
                                     1, dev)
        codes = mx.unpack(wq, c["bits"]).cpu().numpy().ravel().tolist()
        assert codes == c["codes"], (c["kind"], c["bits"], c["gs"])
        assert host_bf16(s).ravel().tolist() == c["scales_bf16"]
        assert host_bf16(b).ravel().tolist() == c["biases_bf16"]


def test_quantize_leading_dims_and_errors(dev, O):
    w = O.normal_f32(3, 2 * 3 * 128, 0, 0.02).reshape(2, 3, 128)
    wq, s, b = mx.quantized(dev_f32(w, dev), 64, 4, mode="minmax")
    assert tuple(wq.shape) == (2, 3, 16) and tuple(s.shape) == (2, 3, 2)
    ref = O.quantize(w.reshape(6, 128), 64, 4)
    assert np.array_equal(host_words(wq).reshape(6, 16), ref["wq"])
    with pytest.raises(ValueError, match="group size"):
        mx.quantized(dev_f32(w, dev), 48, 4)
    with pytest.raises(ValueError, match="bits"):
        mx.quantized(dev_f32(w, dev), 64, 7)
    with pytest.raises(ValueError, match="divisible"):
        mx.quantized(dev_f32(w[..., :96], dev), 64, 4)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_dequantize_bit_exact(dev, O, bits, gs):
    N, K = 11, 512
    w = O.normal_f32(900 + bits + gs, N * K, 0, 0.02).reshape(N, K)
    q = O.quantize(w, gs, bits)
    f_ref, b_ref = O.dequantize(q["wq"], q["scales_bf16"], q["biases_bf16"], K, gs, bits)
    wq = dev_words(q["wq"], dev)
    s = dev_bf16(q["scales_bf16"], dev)
    b = dev_bf16(q["biases_bf16"], dev)
    out_bf = mx.dequantized(wq, s, b, gs, bits)
    assert out_bf.dtype == torch.bfloat16
    assert np.array_equal(host_bf16(out_bf), b_ref)
    out_f = mx.dequantized(wq, s, b, gs, bits, dtype=torch.float32)
    assert np.array_equal(out_f.cpu().numpy(), f_ref)


def test_dequantize_fp32_scales(dev, O):
    N, K, gs, bits = 4, 256, 64, 6
    w = O.normal_f32(77, N * K, 0, 0.02).reshape(N, K)
    wq, s, b = mx.quantized(dev_f32(w, dev), gs, bits, mode="minmax")  # fp32 scales/biases
    out = mx.dequantized(wq, s, b, gs, bits)
    assert out.dtype == torch.float32
    q = O.quantize(w, gs, bits)
    sf = np.repeat(q["scales_f32"], gs, axis=1).astype(np.float64)
    bf = np.repeat(q["biases_f32"], gs, axis=1).astype(np.float64)
    # q*s+b is exact in fp64 here, so one rounding to fp32 equals fmaf(q, s, b)
    ref = (q["codes"] * sf + bf).astype(np.float32)
    assert np.array_equal(out.cpu().numpy(), ref)


def test_quantize_dequantize_round_trip_error(dev, O):
    """Size-independent property at a full config size: |w - deq(q(w))| <= s/2."""
    N, K, gs, bits = 16384, 4096, 64, 6
    w = torch.randn(N, K, device=dev, generator=torch.Generator(device=dev).manual_seed(2003)) * 0.02
    wq, s, b = mx.quantized(w, gs, bits, mode="minmax")
    deq = mx.dequantized(wq, s, b, gs, bits)
    err = (w - deq).abs().view(N, K // gs, gs)
    assert bool((err <= s.abs().unsqueeze(-1) / 2 * (1 + 1e-5) + 1e-7).all())
    codes = mx.unpack(wq, bits)
    assert int(codes.max()) == 63 and int(codes.min()) == 0
    # repacking the unpacked codes reproduces the words exactly
    assert torch.equal(mx.pack(codes, bits).view(torch.int32), wq.view(torch.int32))
