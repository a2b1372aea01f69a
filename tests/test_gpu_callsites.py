"""The reference's own call-site shapes of the quantized linear (6-bit H3, 4-bit Gemma-4),
beyond the benchmark configurations:

  H3 attention qkv   K=5376  N=21504   `model/minimax h3/H3Transformer.swift:430,448`
  H3 attention out   K=7168  N=5376    `:434,580`
  H3 MLP fc1         K=5376  N=2x14336 with silu(gate)*up fused (output 14336)  `:614-627`
  H3 MLP fc2         K=14336 N=5376    `:614-627`
  H3 adaLN GEMV      K=2688  N=96768 at M = 1, 2, 6 unique timesteps  `:366-402`
  LTX to_gate_logits N=32 with bias    `model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:188`
  Gemma-4 logits     M=1 K=3840 N=262144, 4-bit, full output
                     `model/3模块/ltx2.5专属/gemma4文本-(ltx专属).swift:306-312`

Token count 2100 for the MFMA shapes: eight 256-row tiles and a 52-row remainder launch.
Sampled rows (seeded, plus the last row and the launch seam) against the fp64 oracle:
tight against the weights as the kernel rounds them, and max|y - r| / max|r| <= 2e-2
against the exact result; the GEMV outputs are checked whole.
"""
import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from tests.gpu_util import assert_tight, host_bf16, host_f32_of_bf16, host_words, spec_metric
from tests.test_gpu_configs import _acts, _check, _rows, _weights

pytestmark = pytest.mark.gpu

M_TOKENS = 2100


@pytest.mark.parametrize("name,K,N", [("H3 qkv", 5376, 21504), ("H3 out", 7168, 5376),
                                      ("H3 fc2", 14336, 5376)])
def test_h3_projections(dev, O, name, K, N):
    x = _acts(dev, M_TOKENS, K, 4100 + K)
    wq, s, b = _weights(dev, N, K, 5100 + N, 6)
    y = mx.tiled_matmul(x, mx.tile(wq, s, b, 64, 6))
    _check(O, x, wq, s, b, y, _rows(M_TOKENS, 48, K), 64, 6, name)
    y_mlx = mx.quantized_matmul(x, wq, s, b, group_size=64, bits=6, path="qmm")
    assert torch.equal(y, y_mlx), f"{name}: tiled and MLX-layout kernels differ"


def test_h3_fc1_swiglu(dev, O):
    K, F = 5376, 14336
    x = _acts(dev, M_TOKENS, K, 4200)
    wq, s, b = _weights(dev, 2 * F, K, 5200, 6)
    y = mx.tiled_matmul(x, mx.tile(wq, s, b, 64, 6, swiglu=True), activation="swiglu")
    assert tuple(y.shape) == (M_TOKENS, F)
    rows = _rows(M_TOKENS, 32, 7)
    xh = host_bf16(x[torch.as_tensor(rows, device=dev)])
    wqh, sh, bh = host_words(wq), host_bf16(s), host_bf16(b)
    got = host_f32_of_bf16(y)[rows]
    assert_tight(got, O.swiglu_f64(O.qmm_f64_bf16w(xh, wqh, sh, bh, 64, 6, threads=16)),
                 "H3 fc1 swiglu")
    assert spec_metric(got, O.swiglu_f64(O.qmm_f64(xh, wqh, sh, bh, 64, 6, threads=16))) <= 2e-2


@pytest.mark.parametrize("M", [1, 2, 6])
def test_h3_adaln_gemv(dev, O, M):
    K, N = 2688, 96768
    x = _acts(dev, M, K, 4300 + M)
    wq, s, b = _weights(dev, N, K, 5300, 6)
    tw = mx.tile(wq, s, b, 64, 6)
    for y, what in ((mx.tiled_matmul(x, tw), "tiled"),
                    (mx.quantized_matmul(x, wq, s, b, group_size=64, bits=6), "MLX layout")):
        _check(O, x, wq, s, b, y, np.arange(M), 64, 6, f"adaLN M={M} ({what})",
               exact_only=True)


def test_ltx_gate_logits_n32_bias(dev, O):
    M, K, N = M_TOKENS, 4096, 32
    x = _acts(dev, M, K, 4400)
    wq, s, b = _weights(dev, N, K, 5400, 6)
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    bias = (torch.randn(N, generator=g, device=dev) * 0.1).bfloat16()
    lin = mx.QuantizedLinear.from_weights(wq, s, b, bias=bias, group_size=64, bits=6)
    y = lin(x)
    rows = _rows(M, 64, 11)
    xh = host_bf16(x[torch.as_tensor(rows, device=dev)])
    wqh, sh, bh, biash = host_words(wq), host_bf16(s), host_bf16(b), host_bf16(bias)
    got = host_f32_of_bf16(y)[rows]
    assert_tight(got, O.qmm_f64_bf16w(xh, wqh, sh, bh, 64, 6, bias=biash, threads=16),
                 "to_gate_logits")
    assert spec_metric(got, O.qmm_f64(xh, wqh, sh, bh, 64, 6, bias=biash, threads=16)) <= 2e-2


def test_gemma4_tied_logits(dev, O):
    K, N = 3840, 262144
    x = _acts(dev, 1, K, 4500)
    wq, s, b = _weights(dev, N, K, 5500, 4)
    tw = mx.tile(wq, s, b, 64, 4)
    for y, what in ((mx.tiled_matmul(x, tw), "tiled"),
                    (mx.quantized_matmul(x, wq, s, b, group_size=64, bits=4), "MLX layout")):
        _check(O, x, wq, s, b, y, np.arange(1), 64, 4, f"gemma4 logits ({what})",
               exact_only=True)
