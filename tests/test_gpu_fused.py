"""Activations fused into the tiled MFMA kernel's epilogue (GELU-tanh, SwiGLU) against the
oracle: the fp64 matmul over the bf16-rounded weights (orc_qmm_f64_bf16w), then the fp64
activation (tests/test_fused_oracle pins those against torch's float64 functions).

Tolerance: the fused kernel rounds once, after the activation, so the tight bound of
tests/gpu_util.assert_tight applies to act(reference); the north-star metric
max|y - r| / max|r| <= 2e-2 is checked against act(exact fp64 matmul). Shapes cover the
64-, 128- and 256-row tiles, the remainder launch, ragged N, odd K steps, gs 32/64/128,
bias and no bias."""
import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from tests.gpu_util import assert_tight, dev_bf16, dev_words, host_f32_of_bf16, spec_metric
from tests.test_gpu_matmul import make_case

pytestmark = pytest.mark.gpu


def _rows(M):
    return np.unique(np.array([0, 1, M // 3, M // 2, M - 2, M - 1]).clip(0, M - 1))


@pytest.mark.parametrize("M,N,K,bits,gs", [(9, 130, 256, 6, 64), (100, 288, 640, 4, 32),
                                           (300, 200, 640, 6, 128), (1000, 100, 1088, 8, 64),
                                           (2148, 8192, 576, 6, 64)])
def test_gelu_fused(dev, O, M, N, K, bits, gs):
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M + N + K, with_bias=(bits != 8))
    tw = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits)
    y = mx.tiled_matmul(dev_bf16(x, dev), tw, activation="gelu_tanh",
                        bias=None if bias is None else dev_bf16(bias, dev))
    assert tuple(y.shape) == (M, N)
    rows = _rows(M)
    got = host_f32_of_bf16(y)[rows]
    pre = O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows, threads=16)
    assert_tight(got, O.gelu_tanh_f64(pre), f"gelu M={M} N={N} K={K}")
    exact = O.gelu_tanh_f64(O.qmm_f64(x, wq, s, b, gs, bits, bias=bias, rows=rows, threads=16))
    assert spec_metric(got, exact) <= 2e-2


@pytest.mark.parametrize("M,F,K,bits,gs", [(9, 64, 256, 6, 64), (130, 100, 576, 4, 32),
                                           (257, 2048, 512, 6, 64), (300, 48, 640, 5, 128),
                                           (2148, 4096, 576, 6, 64)])
def test_swiglu_fused(dev, O, M, F, K, bits, gs):
    N = 2 * F
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M + F + K, with_bias=(F != 2048))
    tw = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits, swiglu=True)
    np.testing.assert_array_equal(tw.data.cpu().numpy(), O.tile_swiglu(wq, s, b, K, gs, bits))
    y = mx.tiled_matmul(dev_bf16(x, dev), tw, activation="swiglu",
                        bias=None if bias is None else dev_bf16(bias, dev))
    assert tuple(y.shape) == (M, F)
    rows = _rows(M)
    got = host_f32_of_bf16(y)[rows]
    pre = O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows, threads=16)
    assert_tight(got, O.swiglu_f64(pre), f"swiglu M={M} F={F} K={K}")
    exact = O.swiglu_f64(O.qmm_f64(x, wq, s, b, gs, bits, bias=bias, rows=rows, threads=16))
    assert spec_metric(got, exact) <= 2e-2


def test_fused_matches_unfused_chain(dev, O):
    """The fused outputs equal the unfused chain (matmul rounded to bf16, then the activation
    in fp32 and a second rounding) to within the unfused chain's extra rounding."""
    M, F, K, gs, bits = 600, 512, 1024, 64, 6
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    w = torch.randn(2 * F, K, generator=g, device=dev) * 0.02
    bias = (torch.randn(2 * F, generator=g, device=dev) * 0.1).bfloat16()
    wq, s, b = mx.quantized(w, gs, bits, scales_dtype=torch.bfloat16, mode="minmax")
    plain = mx.tiled_matmul(x, mx.tile(wq, s, b, gs, bits), bias=bias).float()
    gelu = mx.tiled_matmul(x, mx.tile(wq, s, b, gs, bits), bias=bias, activation="gelu_tanh")
    ref = torch.nn.functional.gelu(plain, approximate="tanh")
    assert ((gelu.float() - ref).abs() <= 2 ** -7 * ref.abs() + 1e-3).all()
    sw = mx.tiled_matmul(x, mx.tile(wq, s, b, gs, bits, swiglu=True), bias=bias,
                         activation="swiglu")
    ref = torch.nn.functional.silu(plain[:, :F]) * plain[:, F:]
    assert ((sw.float() - ref).abs() <= 2 ** -6 * ref.abs() + 1e-3).all()


def test_fused_errors(dev, O):
    M, N, K, gs, bits = 16, 64, 128, 64, 4
    x, wq, s, b, _ = make_case(O, M, N, K, gs, bits, seed=5)
    xd = dev_bf16(x, dev)
    tw = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits)
    tp = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits, swiglu=True)
    with pytest.raises(ValueError, match="swiglu"):
        mx.tiled_matmul(xd, tw, activation="swiglu")
    with pytest.raises(ValueError, match="swiglu"):
        mx.tiled_matmul(xd, tp)
    with pytest.raises(ValueError, match="unknown activation"):
        mx.tiled_matmul(xd, tw, activation="relu")
    with pytest.raises(ValueError, match="MFMA"):
        mx.tiled_matmul(xd, tw, activation="gelu_tanh", path="qmv")
    x7, wq7, s7, b7, _ = make_case(O, 2, 63, K, gs, bits, seed=6)
    with pytest.raises(ValueError, match="even number of rows"):
        mx.tile(dev_words(wq7, dev), dev_bf16(s7, dev), dev_bf16(b7, dev), gs, bits,
                swiglu=True)


def test_ltx_ffn_module(dev):
    """LTXFFN (GELU fused into proj_in) against the same two layers run unfused."""
    ffn = mx.LTXFFN(512, 2048, bias=True, group_size=64, bits=4, device=dev, seed=3)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    ffn.proj_in.bias = (torch.randn(2048, generator=g, device=dev) * 0.1).bfloat16()
    ffn.proj_out.bias = (torch.randn(512, generator=g, device=dev) * 0.1).bfloat16()
    x = torch.randn(333, 512, generator=g, device=dev).bfloat16()
    y = ffn(x)
    mid = torch.nn.functional.gelu(ffn.proj_in(x).float(), approximate="tanh").bfloat16()
    ref = ffn.proj_out(mid).float()
    assert tuple(y.shape) == (333, 512)
    assert ((y.float() - ref).abs().max() / ref.abs().max()).item() < 1e-2


def test_h3_mlp_module(dev):
    """H3MlpW.load from a weights mapping (fc1 2*ffn x hidden, fc2 hidden x ffn, 6-bit):
    silu(gate) * up fused into fc1 against the unfused split / silu / multiply chain."""
    hidden, ffn = 256, 384
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    tensors = {}
    for name, n, k in (("mlp.fc1", 2 * ffn, hidden), ("mlp.fc2", hidden, ffn)):
        w = torch.randn(n, k, generator=g, device=dev) * 0.05
        wq, s, b = mx.quantized(w, 64, 6, scales_dtype=torch.bfloat16, mode="minmax")
        tensors[name + ".weight"], tensors[name + ".scales"], tensors[name + ".biases"] = wq, s, b
        tensors[name + ".bias"] = (torch.randn(n, generator=g, device=dev) * 0.1).bfloat16()
    mlp = mx.H3MlpW.load(tensors, "mlp", hidden, ffn)
    assert mlp.fc1.bits == 6 and mlp.fc1.group_size == 64
    x = torch.randn(2, 150, hidden, generator=g, device=dev).bfloat16()
    y = mlp(x)
    h = mlp.fc1.forward(x).float()
    ref = mlp.fc2.forward((torch.nn.functional.silu(h[..., :ffn]) * h[..., ffn:]).bfloat16())
    assert tuple(y.shape) == (2, 150, hidden)
    assert ((y.float() - ref.float()).abs().max() / ref.float().abs().max()).item() < 1e-2
