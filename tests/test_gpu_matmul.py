"""Quantized matmul on the GPU (MFMA qmm and split-K GEMV) against the oracle.

Tolerances (written here):
  * tight: against orc_qmm_f64_bf16w (weights rounded to bf16 exactly as the
    MFMA kernel consumes them) for the qmm path, and against the exact fp64
    oracle for the GEMV path (which applies scale and bias in fp32 per group):
    |y - r| <= 2^-8 |r| + 1e-4 max|r|  (one bf16 output rounding + fp32 sums);
  * spec: max|y - r| / max|r| <= 2e-2 against the exact fp64 oracle.
"""
import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from tests.gpu_util import (assert_tight, cosine, dev_bf16, dev_words, host_f32_of_bf16,
                            spec_metric)

pytestmark = pytest.mark.gpu


def make_case(O, M, N, K, gs, bits, seed, with_bias=False, wstd=0.02):
    w = O.normal_f32(2000 + seed, N * K, 0, wstd).reshape(N, K)
    q = O.quantize(w, gs, bits)
    x = O.normal_bf16(1000 + seed, M * K).reshape(M, K)
    bias = O.bf16_rne(O.normal_f32(3000 + seed, N, 0, 0.5)) if with_bias else None
    return x, q["wq"], q["scales_bf16"], q["biases_bf16"], bias


def run(dev, x, wq, s, b, bias, gs, bits, path="auto"):
    y = mx.quantized_matmul(dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev),
                            dev_bf16(b, dev), transpose=True, group_size=gs, bits=bits,
                            bias=None if bias is None else dev_bf16(bias, dev), path=path)
    return host_f32_of_bf16(y)


def test_golden_cases_all_paths(dev, O, golden):
    for c in golden["qmm"]:
        N, K, M, gs, bits = c["N"], c["K"], c["M"], c["gs"], c["bits"]
        wq = np.array(c["words"], np.uint32).reshape(N, K * bits // 32)
        s = np.array(c["scales_bf16"], np.uint16).reshape(N, K // gs)
        b = np.array(c["biases_bf16"], np.uint16).reshape(N, K // gs)
        x = np.array(c["x_bf16"], np.uint16).reshape(M, K)
        bias = None if c["bias_bf16"] is None else np.array(c["bias_bf16"], np.uint16)
        y64 = np.array(c["y_f64"]).reshape(M, N)
        ref_w = O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias)
        for path in ("auto", "qmm", "qmv"):
            y = run(dev, x, wq, s, b, bias, gs, bits, path)
            ref = ref_w if path == "qmm" else y64
            assert_tight(y, ref, f"golden bits={bits} gs={gs} path={path}")
            assert spec_metric(y, y64) <= 2e-2


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [1, 2, 3, 8, 12, 16, 24, 32])
def test_qmv_parity(dev, O, bits, gs, M):
    N, K = 96, 512
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits * 100 + gs + M,
                                  with_bias=(M % 2 == 1))
    y = run(dev, x, wq, s, b, bias, gs, bits, path="qmv")
    ref = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias)
    assert_tight(y, ref, f"qmv bits={bits} gs={gs} M={M}")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M,N,K", [(1, 100, 2048), (5, 200, 2176), (32, 72, 4224)])
def test_qmv_eight_wave_split(dev, O, bits, gs, M, N, K):
    """Fewer than 512 workgroups and K >= 2048: the GEMV splits K over 8 waves per
    workgroup instead of 4 (K = 2176 and 4224 are 34 and 66 steps of 64 codes, which do
    not divide evenly over the waves)."""
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits * 31 + gs + M + K,
                                  with_bias=(M != 5))
    y = run(dev, x, wq, s, b, bias, gs, bits, path="qmv")
    ref = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias)
    assert_tight(y, ref, f"qmv 8 waves bits={bits} gs={gs} M={M} N={N} K={K}")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("M", [1, 2, 5, 8])
@pytest.mark.parametrize("N,K", [(96, 96), (40, 544), (17000, 160)])
def test_qmv_k_odd_multiple_of_32(dev, O, bits, M, N, K):
    """K an odd multiple of 32 (gs = 32) does not fill whole 64-code steps: the
    GEMV takes the lane-per-chunk kernel, with the K range split over the 4 waves
    (small N) or one wave per row set (N = 17000 at M <= 2: 8-row sets, >= 2048 waves)."""
    gs = 32
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits * 7 + M + K,
                                  with_bias=(M % 2 == 0))
    y = run(dev, x, wq, s, b, bias, gs, bits, path="qmv")
    ref = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias)
    assert_tight(y, ref, f"qmv K={K} bits={bits} M={M} N={N}")
    assert spec_metric(y, ref) <= 2e-2


@pytest.mark.parametrize("N", [1, 32, 33, 4000, 6000])
def test_qmv_row_counts_and_split(dev, O, N):
    """Small N uses the 4-wave K split, large N one wave per row set."""
    M, K, gs, bits = 2, 1024, 64, 6
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=N, with_bias=True)
    y = run(dev, x, wq, s, b, bias, gs, bits, path="qmv")
    assert_tight(y, O.qmm_f64(x, wq, s, b, gs, bits, bias=bias), f"qmv N={N}")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M,K", [(200, 768), (100, 1024), (200, 640)])
def test_qmm_parity_bits_gs(dev, O, bits, gs, M, K):
    """K % 256 == 0 runs the ring-pipelined kernel (256- and 128-token tiles);
    K = 640 runs the two-deep kernel."""
    N = 288
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits + gs + M, with_bias=True)
    y = run(dev, x, wq, s, b, bias, gs, bits, path="qmm")
    assert_tight(y, O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias), f"qmm {bits}/{gs}")
    exact = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias)
    assert spec_metric(y, exact) <= 2e-2
    assert cosine(y, exact) > 0.9999


@pytest.mark.parametrize("M,N,K,gs", [
    (9, 256, 256, 64),     # just above the GEMV limit
    (64, 512, 4096, 64),   # BM=64 tile
    (100, 300, 128, 64),   # ragged M and N (N not a multiple of 16)
    (129, 33, 64, 32),     # BM=256 tile, N smaller than one wave's share
    (300, 256, 96, 32),    # K=96: half a K step at the tail
    (257, 260, 16384, 128),  # long K
])
def test_qmm_shapes(dev, O, M, N, K, gs):
    bits = 6
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M + N + K, with_bias=(N % 2 == 0))
    y = run(dev, x, wq, s, b, bias, gs, bits, path="qmm")
    assert_tight(y, O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias), f"qmm {M}x{N}x{K}")


@pytest.mark.parametrize("bits", [3, 5])
def test_qmm_odd_widths_k_tail(dev, O, bits):
    """3- and 5-bit runs of 32 codes are whole words; K=96 leaves a half step."""
    M, N, K, gs = 40, 64, 96, 32
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits)
    y = run(dev, x, wq, s, b, bias, gs, bits, path="auto")  # M > 32: the MFMA kernel
    assert_tight(y, O.qmm_f64_bf16w(x, wq, s, b, gs, bits), f"odd width {bits}")


def test_dispatch_boundary_is_consistent(dev, O):
    K, N, gs, bits = 512, 128, 64, 4
    x, wq, s, b, _ = make_case(O, 16, N, K, gs, bits, seed=5)
    full = run(dev, x, wq, s, b, None, gs, bits, path="qmm")
    for M in (1, 8, 9, 16):
        y = run(dev, x[:M], wq, s, b, None, gs, bits)
        assert spec_metric(y, full[:M]) < 1e-2


def test_leading_dims_and_empty(dev, O):
    K, N, gs, bits = 256, 64, 64, 4
    x, wq, s, b, _ = make_case(O, 10, N, K, gs, bits, seed=9)
    xd = dev_bf16(x, dev).view(2, 5, K)
    y = mx.quantized_matmul(xd, dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev),
                            group_size=gs, bits=bits)
    assert tuple(y.shape) == (2, 5, N)
    # 10 tokens: the GEMV, which applies the unrounded weights (the exact reference)
    assert_tight(host_f32_of_bf16(y).reshape(10, N),
                 O.qmm_f64(x, wq, s, b, gs, bits), "leading dims")
    empty = mx.quantized_matmul(xd[:0], dev_words(wq, dev), dev_bf16(s, dev),
                                dev_bf16(b, dev), group_size=gs, bits=bits)
    assert tuple(empty.shape) == (0, 5, N)


def test_matmul_shape_errors(dev, O):
    K, N, gs, bits = 256, 64, 64, 4
    x, wq, s, b, _ = make_case(O, 4, N, K, gs, bits, seed=10)
    X, W, S, B = dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev)
    with pytest.raises(ValueError, match="incompatible"):
        mx.quantized_matmul(X, W, S, B, group_size=gs, bits=6)
    with pytest.raises(ValueError, match="incompatible"):
        mx.quantized_matmul(X, W, S[:, :2], B[:, :2], group_size=gs, bits=bits)
    with pytest.raises(NotImplementedError):
        mx.quantized_matmul(X, W, S, B, transpose=False, group_size=gs, bits=bits)
    with pytest.raises(ValueError, match="bfloat16"):
        mx.quantized_matmul(X.float(), W, S, B, group_size=gs, bits=bits)


def test_runs_on_caller_stream(dev, O):
    K, N, gs, bits = 512, 256, 64, 6
    x, wq, s, b, _ = make_case(O, 300, N, K, gs, bits, seed=11)
    X, W, S, B = dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev)
    st = torch.cuda.Stream(device=dev)
    st.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(st):
        y = mx.quantized_matmul(X, W, S, B, group_size=gs, bits=bits)
        y2 = mx.quantized_matmul(X[:2], W, S, B, group_size=gs, bits=bits)
    st.synchronize()
    assert_tight(host_f32_of_bf16(y), O.qmm_f64_bf16w(x, wq, s, b, gs, bits), "stream")
    assert_tight(host_f32_of_bf16(y2), O.qmm_f64(x[:2], wq, s, b, gs, bits), "stream gemv")


def test_quantized_linear_module(dev, O):
    K, N = 512, 192
    w = O.normal_f32(44, N * K, 0, 0.02).reshape(N, K)
    bias = O.bf16_rne(O.normal_f32(45, N, 0, 0.1))
    lin = mx.QuantizedLinear.from_linear(torch.from_numpy(w).to(dev), bias=dev_bf16(bias, dev),
                                         group_size=64, bits=6, mode="minmax")
    assert lin.shape == (N, K)
    q = O.quantize(w, 64, 6)
    for M in (2, 50):
        x = O.normal_bf16(46 + M, M * K).reshape(M, K)
        # fp32 weights quantize to fp32 scales; the module keeps bf16 for the kernel
        lin_b = mx.QuantizedLinear.from_weights(lin.weight, lin.scales.bfloat16(),
                                                lin.biases.bfloat16(), lin.bias, 64, 6)
        y = host_f32_of_bf16(lin_b(dev_bf16(x, dev)))
        ref = O.qmm_f64_bf16w(x, q["wq"], q["scales_bf16"], q["biases_bf16"], 64, 6, bias=bias)
        assert spec_metric(y, ref) < 5e-3
    fresh = mx.QuantizedLinear(256, 64, bias=True, group_size=64, bits=4, device=dev, seed=0)
    assert fresh.weight.dtype == torch.uint32 and tuple(fresh.scales.shape) == (64, 4)
    out = fresh(torch.zeros(3, 256, dtype=torch.bfloat16, device=dev))
    assert tuple(out.shape) == (3, 64) and float(out.abs().max()) == 0.0


@pytest.mark.parametrize("spelling", ["mlx", "hf"])
def test_mflinear_load_and_forward(dev, O, spelling):
    K, N, gs, bits = 4096, 128, 64, 6
    x, wq, s, b, bias = make_case(O, 5, N, K, gs, bits, seed=12, with_bias=True)
    p = "blocks.0.attn.qkv_proj"
    tensors = {p + ".weight": dev_words(wq, dev), p + ".bias": dev_bf16(bias, dev)}
    if spelling == "mlx":
        tensors.update({p + ".scales": dev_bf16(s, dev), p + ".biases": dev_bf16(b, dev)})
    else:
        tensors.update({p + ".weight.scales": dev_bf16(s, dev),
                        p + ".weight.biases": dev_bf16(b, dev)})
    lin = mx.MfLinear.load(tensors, p, in_features=K)
    assert lin.is_quantized and lin.bits == 6 and lin.group_size == 64 and lin.out_dim == N
    y = host_f32_of_bf16(lin(dev_bf16(x, dev).float()))  # forward casts x to bf16
    assert_tight(y, O.qmm_f64(x, wq, s, b, gs, bits, bias=bias), "MfLinear")


def test_strided_inputs_are_accepted(dev, O):
    """mlx takes any strides; the Python surface copies views to row-major."""
    K, N, gs, bits = 256, 64, 64, 4
    x, wq, s, b, _ = make_case(O, 12, N, K, gs, bits, seed=13)
    xt = dev_bf16(x, dev).t().contiguous().t()  # same values, column-major strides
    assert not xt.is_contiguous()
    y = mx.quantized_matmul(xt, dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev),
                            group_size=gs, bits=bits)
    assert_tight(host_f32_of_bf16(y), O.qmm_f64(x, wq, s, b, gs, bits), "strided")  # GEMV
