"""Tiled weight layout on the GPU: the tiler against the oracle's writer, and
the tiled kernels against the MLX-layout kernels and the fp64 oracle.

Tolerances: the tiled MFMA kernel shares every arithmetic step with the
MLX-layout MFMA kernel (only where the weight bits are fetched from differs),
so for M > 64 and K % 64 == 0 (where the MLX-layout path runs the same kernel)
the outputs must be bit-identical. Elsewhere the tight bound of
tests/gpu_util.assert_tight applies against the oracle (orc_qmm_f64_bf16w for
the MFMA kernels, orc_qmm_f64 for the GEMV), and max|y - r| / max|r| <= 2e-2
against the exact fp64 oracle.
"""
import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from tests.gpu_util import (assert_tight, dev_bf16, dev_words, host_bf16, host_f32_of_bf16,
                            host_words, spec_metric)
from tests.test_gpu_matmul import make_case

pytestmark = pytest.mark.gpu

BITS = [2, 3, 4, 5, 6, 8]
GS = [32, 64, 128]


def _tile(dev, wq, s, b, gs, bits):
    return mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits)


def _tiled_run(dev, x, tw, bias, path="auto"):
    y = mx.tiled_matmul(dev_bf16(x, dev), tw,
                        bias=None if bias is None else dev_bf16(bias, dev), path=path)
    return y


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", GS)
def test_tile_matches_oracle_bytes(dev, O, bits, gs):
    N, K = 100, 384
    _, wq, s, b, _ = make_case(O, 1, N, K, gs, bits, seed=bits * 7 + gs)
    tw = _tile(dev, wq, s, b, gs, bits)
    ref = O.tile(wq, s, b, K, gs, bits)
    got = tw.data.cpu().numpy()
    assert got.shape == ref.shape
    np.testing.assert_array_equal(got, ref)


def test_tile_full_size_matches_oracle(dev, O):
    """The benchmark weight geometry (16384 x 4096, 6-bit, gs 64)."""
    N, K, gs, bits = 16384, 4096, 64, 6
    rng = np.random.default_rng(7)
    wq = rng.integers(0, 2 ** 32, size=(N, K * bits // 32), dtype=np.uint32)
    s = rng.integers(0, 2 ** 16, size=(N, K // gs), dtype=np.uint16)
    b = rng.integers(0, 2 ** 16, size=(N, K // gs), dtype=np.uint16)
    tw = _tile(dev, wq, s, b, gs, bits)
    np.testing.assert_array_equal(tw.data.cpu().numpy(), O.tile(wq, s, b, K, gs, bits))


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", GS)
@pytest.mark.parametrize("M,K", [(200, 768), (100, 1024), (300, 640)])
def test_tiled_qmm_bit_identical_to_mlx_layout(dev, O, bits, gs, M, K):
    N = 288
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits * 31 + gs + K,
                                  with_bias=(bits % 2 == 0))
    tw = _tile(dev, wq, s, b, gs, bits)
    y_t = _tiled_run(dev, x, tw, bias, path="qmm")
    y_m = mx.quantized_matmul(dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev),
                              dev_bf16(b, dev), group_size=gs, bits=bits,
                              bias=None if bias is None else dev_bf16(bias, dev), path="qmm")
    np.testing.assert_array_equal(host_bf16(y_t), host_bf16(y_m))
    rows = np.arange(0, M, 7)
    ref = O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows)
    assert_tight(host_f32_of_bf16(y_t)[rows], ref, f"tiled qmm bits={bits} gs={gs}")


@pytest.mark.parametrize("bits,gs", [(6, 64), (4, 32), (3, 64)])
@pytest.mark.parametrize("K", [576, 640])
@pytest.mark.parametrize("M,N", [(2100, 8200), (2100, 8192), (2148, 8192)])
def test_tiled_qmm_several_tiles_per_workgroup(dev, O, bits, gs, K, M, N):
    """More tiles than CUs, ragged in M (and N), with an odd (576 / 64 = 9) and an even
    number of K steps: the persistent kernel carries its load streams and unpack parity
    across tile boundaries. On a 256-CU device, 2100 x 8200 runs 9 x 33 tiles of 256 rows
    in one launch; 2100 x 8192 (8 x 32 full tiles) and 2148 x 8192 move the 52- and
    100-row remainders to a second launch of 64- and 128-row tiles."""
    g = torch.Generator(device=dev)
    g.manual_seed(bits * 1000 + K)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    w = torch.randn(N, K, generator=g, device=dev) * 0.02
    bias = (torch.randn(N, generator=g, device=dev) * 0.1).bfloat16()
    wq, s, b = mx.quantized(w, gs, bits, scales_dtype=torch.bfloat16, mode="minmax")
    y_t = mx.tiled_matmul(x, mx.tile(wq, s, b, gs, bits), bias=bias, path="qmm")
    y_m = mx.quantized_matmul(x, wq, s, b, group_size=gs, bits=bits, bias=bias, path="qmm")
    assert torch.equal(y_t, y_m), f"bits={bits} gs={gs} K={K}: tiled and MLX-layout differ"
    rows = np.array([0, 255, 256, 1023, 2047, 2048, M - 1])
    ref = O.qmm_f64_bf16w(host_bf16(x[torch.as_tensor(rows, device=dev)]), host_words(wq),
                          host_bf16(s), host_bf16(b), gs, bits, bias=host_bf16(bias), threads=16)
    assert_tight(host_f32_of_bf16(y_t)[rows], ref, f"tiled qmm bits={bits} gs={gs} K={K}")


@pytest.mark.parametrize("bits,gs", [(6, 64), (4, 32), (8, 128)])
def test_tiled_qmm_large_scales(dev, O, bits, gs):
    """Scales of magnitude 2^104 and above (s * 2^24 overflows fp32) take the
    kernel's plain unpack for their whole record; records around them keep the
    fast one. Outputs stay bit-identical to the MLX-layout kernel and within the
    tight bound of the oracle. Activations are scaled down so y stays finite."""
    M, N, K = 300, 192, 512
    rng = np.random.default_rng(bits * 10 + gs)
    codes = rng.integers(0, 2 ** bits, size=(N, K), dtype=np.uint32)
    wq = O.pack_words(codes, bits)
    ng = K // gs
    e = rng.integers(-8, 9, size=(N, ng))
    big = rng.random((N, ng)) < 0.1                       # about one group in ten
    e[big] = rng.integers(104, 118, size=int(big.sum()))
    sgn = np.where(rng.random((N, ng)) < 0.5, -1.0, 1.0)
    s = O.bf16_rne((sgn * np.ldexp(1.0 + rng.random((N, ng)), e)).astype(np.float32))
    b = O.bf16_rne((-0.5 * (2 ** bits) * O.bf16_to_f32(s)).astype(np.float32))
    x = O.bf16_rne(np.ldexp(rng.standard_normal((M, K)), -118).astype(np.float32))
    tw = _tile(dev, wq, s, b, gs, bits)
    y_t = _tiled_run(dev, x, tw, None, path="qmm")
    y_m = mx.quantized_matmul(dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev),
                              dev_bf16(b, dev), group_size=gs, bits=bits, path="qmm")
    np.testing.assert_array_equal(host_bf16(y_t), host_bf16(y_m))
    y = host_f32_of_bf16(y_t)
    assert np.isfinite(y).all()
    assert_tight(y, O.qmm_f64_bf16w(x, wq, s, b, gs, bits), f"large scales bits={bits} gs={gs}")


@pytest.mark.parametrize("M,N,K", [(9, 64, 64), (33, 1, 128), (64, 130, 192), (65, 200, 320),
                                   (129, 63, 256), (257, 300, 512), (1000, 100, 1088)])
def test_tiled_qmm_shapes(dev, O, M, N, K):
    gs, bits = 64, 6
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M + N + K, with_bias=True)
    tw = _tile(dev, wq, s, b, gs, bits)
    y = host_f32_of_bf16(_tiled_run(dev, x, tw, bias, path="qmm"))
    assert_tight(y, O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias),
                 f"tiled qmm M={M} N={N} K={K}")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", GS)
@pytest.mark.parametrize("M", [1, 2, 5, 8, 9, 16, 20, 32])
def test_tiled_qmv_parity(dev, O, bits, gs, M):
    N, K = 200, 512
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits * 100 + gs + M + 1,
                                  with_bias=(M % 2 == 1))
    tw = _tile(dev, wq, s, b, gs, bits)
    y = host_f32_of_bf16(_tiled_run(dev, x, tw, bias, path="qmv"))
    ref = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias)
    assert_tight(y, ref, f"tiled qmv bits={bits} gs={gs} M={M}")
    assert spec_metric(y, ref) <= 2e-2


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", GS)
@pytest.mark.parametrize("M,N,K", [(1, 100, 2048), (5, 200, 2176), (32, 72, 4224)])
def test_tiled_qmv_eight_wave_split(dev, O, bits, gs, M, N, K):
    """The tiled GEMV with K split over 8 waves (fewer than 512 workgroups, K >= 2048)."""
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits * 37 + gs + M + K,
                                  with_bias=(M != 5))
    tw = _tile(dev, wq, s, b, gs, bits)
    y = host_f32_of_bf16(_tiled_run(dev, x, tw, bias, path="qmv"))
    ref = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias)
    assert_tight(y, ref, f"tiled qmv 8 waves bits={bits} gs={gs} M={M} N={N} K={K}")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", GS)
def test_workspace_matmul_bit_identical(dev, O, bits, gs):
    """quantized_matmul(path="auto") at M >= 1024 tiles the MLX-layout weight into a
    workspace and runs the tiled kernel: the same bits as the MLX-layout MFMA kernel.
    A workspace one byte short, or none, takes mxq_quantized_matmul itself."""
    import ctypes
    M, N, K = 1100, 300, 640
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits * 13 + gs, with_bias=True)
    xd, wd, sd, bd, biasd = (dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev),
                             dev_bf16(b, dev), dev_bf16(bias, dev))
    y_auto = mx.quantized_matmul(xd, wd, sd, bd, group_size=gs, bits=bits, bias=biasd)
    y_qmm = mx.quantized_matmul(xd, wd, sd, bd, group_size=gs, bits=bits, bias=biasd, path="qmm")
    np.testing.assert_array_equal(host_bf16(y_auto), host_bf16(y_qmm))
    L = mx.lib()
    need = L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits)
    assert need == L.mxq_tiled_bytes(N, K, gs, bits) > 0
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws = torch.empty(need + 16, dtype=torch.uint8, device=dev)
    # full size, one byte short, none, and a workspace that is not 16-byte aligned
    for nbytes, shift in ((need, 0), (need - 1, 0), (0, 0), (need, 4)):
        y = torch.empty_like(y_qmm)
        wptr = ctypes.c_void_p(ws.data_ptr() + shift)
        assert L.mxq_quantized_matmul_ws(P(xd), M, K, P(wd), P(sd), P(bd), N, 1, gs, bits,
                                         P(biasd), P(y), wptr, nbytes, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(y, y_qmm), f"workspace {nbytes} of {need} bytes, offset {shift}"
    rows = np.arange(0, M, 37)
    assert_tight(host_f32_of_bf16(y_auto)[rows],
                 O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows),
                 f"workspace matmul bits={bits} gs={gs}")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", GS)
def test_mlx_qmv_bit_identical_to_tiled_qmv(dev, O, bits, gs):
    """For K % 64 == 0 the MLX-layout GEMV is the tiled GEMV kernel reading the
    MLX layout in place: same wave split, same per-step arithmetic, so the
    outputs agree bit for bit (ragged N, every token count). K = 192 gives rows
    of 24 * bits bytes, not whole 16-byte chunks for odd widths: the batch's
    coalesced loads then straddle row ends. The MLX form loads each batch's scales and
    biases as one window per row: K = 320 (5 groups of 64 per row, so the window's
    alignment differs between rows), 2688 and 1856 (waves whose batches start at odd
    steps, gs = 128 groups split between batches), 3840 (the Gemma-4 logits K). 16-token
    passes (M = 12, 16) at N = 16384 run 4 waves per workgroup over long K spans, where
    even widths take 2-step batches. N = 19, 285 and 41 with K = 1408 and 3456 leave an odd
    number of scale halfwords in the last row block at gs = 128 (odd rows times odd groups):
    its last scale shares a dword with bytes past the buffer, which a dword load reads as
    zero, so the kernel loads that one on its own."""
    for (M, N, K) in [(1, 200, 1024), (2, 200, 1024), (3, 200, 1024), (5, 200, 1024),
                      (8, 200, 1024), (2, 130, 192), (7, 130, 192), (1, 130, 320),
                      (2, 200, 2688), (5, 70, 1856), (3, 300, 3840), (9, 200, 1024),
                      (16, 130, 2688), (17, 200, 1024), (32, 96, 3840),
                      (16, 16384, 2048), (12, 16384, 2560),
                      (8, 19, 1408), (2, 285, 3456), (27, 41, 1408)]:
        if K % gs:
            continue
        x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=bits * 17 + gs + M,
                                      with_bias=(M % 2 == 1))
        tw = _tile(dev, wq, s, b, gs, bits)
        y_t = _tiled_run(dev, x, tw, bias, path="qmv")
        y_m = mx.quantized_matmul(dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev),
                                  dev_bf16(b, dev), group_size=gs, bits=bits,
                                  bias=None if bias is None else dev_bf16(bias, dev), path="qmv")
        np.testing.assert_array_equal(host_bf16(y_t), host_bf16(y_m),
                                      err_msg=f"bits={bits} gs={gs} M={M} K={K}")


@pytest.mark.parametrize("N,K", [(1, 64), (63, 128), (65, 4096), (24576 // 8, 4096),
                                 (300, 11264)])
def test_tiled_qmv_shapes(dev, O, N, K):
    M, gs, bits = 2, 64, 6
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=N + K, with_bias=True)
    tw = _tile(dev, wq, s, b, gs, bits)
    y = host_f32_of_bf16(_tiled_run(dev, x, tw, bias, path="qmv"))
    assert_tight(y, O.qmm_f64(x, wq, s, b, gs, bits, bias=bias), f"tiled qmv N={N} K={K}")


def test_tiled_dispatch_boundary(dev, O):
    """M = 8 runs the GEMV, M = 9 the MFMA kernel; both agree with the oracle."""
    N, K, gs, bits = 130, 512, 64, 4
    for M in (8, 9):
        x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M)
        tw = _tile(dev, wq, s, b, gs, bits)
        y = host_f32_of_bf16(_tiled_run(dev, x, tw, bias))
        ref = O.qmm_f64(x, wq, s, b, gs, bits)
        assert spec_metric(y, ref) <= 2e-2


def test_tiled_leading_dims_and_errors(dev, O):
    N, K, gs, bits = 64, 256, 64, 4
    x, wq, s, b, _ = make_case(O, 6, N, K, gs, bits, seed=3)
    tw = _tile(dev, wq, s, b, gs, bits)
    x3 = dev_bf16(x, dev).reshape(2, 3, K)
    y = mx.tiled_matmul(x3, tw)
    assert tuple(y.shape) == (2, 3, N)
    y0 = mx.tiled_matmul(torch.empty(0, K, dtype=torch.bfloat16, device=dev), tw)
    assert tuple(y0.shape) == (0, N)
    with pytest.raises(ValueError, match="does not match"):
        mx.tiled_matmul(torch.zeros(2, K + 64, dtype=torch.bfloat16, device=dev), tw)
    with pytest.raises(ValueError, match="bfloat16"):
        mx.tiled_matmul(torch.zeros(2, K, dtype=torch.float32, device=dev), tw)
    # K = 96 cannot be tiled (K % 64 != 0)
    _, wq2, s2, b2, _ = make_case(O, 1, N, 96, 32, bits, seed=4)
    with pytest.raises(ValueError, match="multiple of 64"):
        _tile(dev, wq2, s2, b2, 32, bits)


def test_quantized_linear_uses_tiled_copy(dev, O):
    """The module's tiled call equals the MLX-layout operator bit for bit
    (M > 64), and tiled=False runs the MLX-layout kernels."""
    N, K, gs, bits, M = 192, 512, 64, 6, 130
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=77, with_bias=True)
    args = (dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), dev_bf16(bias, dev))
    lin = mx.QuantizedLinear.from_weights(*args, group_size=gs, bits=bits)
    xd = dev_bf16(x, dev)
    y = lin(xd)
    assert lin.tiled_weight() is not None
    ref = mx.quantized_matmul(xd, *args[:3], group_size=gs, bits=bits, bias=args[3])
    assert torch.equal(y, ref)
    plain = mx.QuantizedLinear.from_weights(*args, group_size=gs, bits=bits, tiled=False)
    assert plain.tiled_weight() is None
    assert torch.equal(plain(xd), ref)
    # update() drops the stale tiled copy
    lin.update({"weight": args[0], "scales": args[1], "biases": args[2]})
    assert lin._tw is None
    assert torch.equal(lin(xd), ref)
