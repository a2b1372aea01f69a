"""mxq_quantized_matmul past the GEMV's range (M > 32) on the MLX layout: the weight is
tiled into a stream-ordered workspace from the library's pool and the tiled kernel runs.
Checked through the C ABI against the in-place MFMA kernel (mxq_qmm) and the
caller-workspace entry point (mxq_quantized_matmul_ws), bit for bit, and against the
fp64 oracle on sampled rows; 3- and 5-bit codes (whose in-place form is the GEMV kernel)
against the oracle; two streams used at once; under graph capture the call allocates
nothing (the in-place kernel runs) and every replay gives the same bits.
"""
import ctypes

import numpy as np
import pytest
import torch

from wuxianhuabu_amd import _lib

from gpu_util import assert_tight, dev_bf16, dev_words, host_f32_of_bf16
from test_gpu_matmul import make_case

pytestmark = pytest.mark.gpu

P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731


def _sp(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _inputs(O, dev, M, N, K, gs, bits, seed, with_bias=True):
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=seed, with_bias=with_bias)
    d = (dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev),
         dev_bf16(bias, dev) if bias is not None else None)
    return (x, wq, s, b, bias), d


def _plain(L, d, M, N, K, gs, bits, y, stream=None):
    xd, wd, sd, bd, biasd = d
    return L.mxq_quantized_matmul(P(xd), M, K, P(wd), P(sd), P(bd), N, 1, gs, bits, P(biasd),
                                  P(y), _sp(stream))


def _in_place(L, d, M, N, K, gs, bits, y):
    xd, wd, sd, bd, biasd = d
    return L.mxq_qmm(P(xd), M, K, P(wd), P(sd), P(bd), N, gs, bits, P(biasd), P(y), _sp())


@pytest.mark.parametrize("M,N,K,gs,bits", [(1536, 2048, 2048, 64, 6), (1100, 1000, 1024, 32, 4),
                                           (2048, 768, 4096, 128, 8), (1024, 512, 1536, 64, 2)])
def test_pooled_workspace_matches_in_place_kernel(dev, O, M, N, K, gs, bits):
    L = _lib.lib()
    assert L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits) > 0
    host, d = _inputs(O, dev, M, N, K, gs, bits, seed=M + bits)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    y_in = torch.empty_like(y)
    y_ws = torch.empty_like(y)
    assert _plain(L, d, M, N, K, gs, bits, y) == _lib.MXQ_OK, L.mxq_last_error()
    assert _in_place(L, d, M, N, K, gs, bits, y_in) == _lib.MXQ_OK
    need = L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    xd, wd, sd, bd, biasd = d
    assert L.mxq_quantized_matmul_ws(P(xd), M, K, P(wd), P(sd), P(bd), N, 1, gs, bits, P(biasd),
                                     P(y_ws), P(ws), need, _sp()) == _lib.MXQ_OK
    torch.cuda.synchronize()
    assert torch.equal(y, y_in), f"pooled vs in-place M={M} N={N} K={K} gs={gs} bits={bits}"
    assert torch.equal(y, y_ws)
    rows = np.unique(np.r_[np.arange(0, M, 61), M - 1])
    x, wq, s, b, bias = host
    assert_tight(host_f32_of_bf16(y)[rows],
                 O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows),
                 f"pooled M={M} N={N} K={K} gs={gs} bits={bits}")


@pytest.mark.parametrize("M,N,K,gs,bits", [(33, 512, 1024, 64, 6), (48, 2048, 2048, 64, 4),
                                           (100, 700, 1536, 32, 8), (300, 1000, 2048, 128, 2),
                                           (640, 384, 4096, 64, 6)])
def test_pooled_small_m_matches_in_place_kernel(dev, O, M, N, K, gs, bits):
    """Below the caller-workspace threshold (M < 1024) the pooled call still tiles."""
    L = _lib.lib()
    assert L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits) == 0
    host, d = _inputs(O, dev, M, N, K, gs, bits, seed=M * 3 + bits)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    y_in = torch.empty_like(y)
    assert _plain(L, d, M, N, K, gs, bits, y) == _lib.MXQ_OK, L.mxq_last_error()
    assert _in_place(L, d, M, N, K, gs, bits, y_in) == _lib.MXQ_OK
    torch.cuda.synchronize()
    assert torch.equal(y, y_in), f"pooled vs in-place M={M} N={N} K={K} gs={gs} bits={bits}"
    x, wq, s, b, bias = host
    rows = np.unique(np.r_[np.arange(0, M, 7), M - 1])
    assert_tight(host_f32_of_bf16(y)[rows],
                 O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows),
                 f"pooled M={M} N={N} K={K} gs={gs} bits={bits}")


@pytest.mark.parametrize("M,bits,gs", [(40, 3, 64), (1100, 5, 32), (300, 3, 128)])
def test_pooled_3_and_5_bit_codes(dev, O, M, bits, gs):
    """3- and 5-bit codes (runs of 32 codes are whole words, not 16-byte chunks): the
    pooled call against the in-place kernel, bit for bit, and the oracle."""
    L = _lib.lib()
    N, K = 520, 1024
    host, d = _inputs(O, dev, M, N, K, gs, bits, seed=M + 7 * bits)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    y_in = torch.empty_like(y)
    assert _plain(L, d, M, N, K, gs, bits, y) == _lib.MXQ_OK, L.mxq_last_error()
    assert _in_place(L, d, M, N, K, gs, bits, y_in) == _lib.MXQ_OK
    torch.cuda.synchronize()
    assert torch.equal(y, y_in), f"pooled vs in-place M={M} bits={bits} gs={gs}"
    x, wq, s, b, bias = host
    rows = np.unique(np.r_[np.arange(0, M, 11), M - 1])
    assert_tight(host_f32_of_bf16(y)[rows],
                 O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows),
                 f"pooled M={M} bits={bits} gs={gs}")


def test_pooled_workspace_two_streams_and_repeated_sizes(dev, O):
    """Calls on two streams at once (each stream's workspace is its own) and calls of
    growing and shrinking size in a row (the pool reuses what earlier calls freed)."""
    L = _lib.lib()
    shapes = [(1536, 2048, 2048, 64, 6), (1280, 1024, 1024, 64, 4)]
    cases = [_inputs(O, dev, *sh, seed=40 + i) for i, sh in enumerate(shapes)]
    refs = []
    for (M, N, K, gs, bits), (_, d) in zip(shapes, cases):
        r = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        assert _in_place(L, d, M, N, K, gs, bits, r) == _lib.MXQ_OK
        refs.append(r)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.full_like(r, float("nan")) for r in refs]
    for _ in range(3):
        for (M, N, K, gs, bits), (_, d), y, st in zip(shapes, cases, outs, streams):
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            assert _plain(L, d, M, N, K, gs, bits, y, stream=st) == _lib.MXQ_OK, L.mxq_last_error()
        torch.cuda.synchronize()
        for y, r in zip(outs, refs):
            assert torch.equal(y, r)
    # the same stream, sizes alternating
    for i in (0, 1, 0, 1, 1, 0):
        (M, N, K, gs, bits), (_, d) = shapes[i], cases[i]
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        assert _plain(L, d, M, N, K, gs, bits, y) == _lib.MXQ_OK
        torch.cuda.synchronize()
        assert torch.equal(y, refs[i]), f"call {i}"


def test_pooled_workspace_refuses_bad_arguments_before_allocating(dev, O):
    L = _lib.lib()
    M, N, K, gs, bits = 1536, 2048, 2048, 64, 6
    _, d = _inputs(O, dev, M, N, K, gs, bits, seed=7, with_bias=False)
    xd, wd, sd, bd, _ = d
    y = torch.full((M, N), 3.0, dtype=torch.bfloat16, device=dev)
    rc = L.mxq_quantized_matmul(None, M, K, P(wd), P(sd), P(bd), N, 1, gs, bits, None, P(y), _sp())
    assert rc == _lib.MXQ_ERR_NULL
    # y 2-byte aligned: refused by the argument checks, before any allocation or launch
    rc = L.mxq_quantized_matmul(P(xd), M, K, P(wd), P(sd), P(bd), N, 1, gs, bits, None,
                                ctypes.c_void_p(y.data_ptr() + 2), _sp())
    assert rc == _lib.MXQ_ERR_ALIGNMENT
    torch.cuda.synchronize()
    assert bool((y == 3.0).all())


def test_pooled_call_under_graph_capture_runs_in_place(dev, O):
    """Captured, the call allocates nothing and runs the in-place kernel; three replays
    with eager calls of the pooled path between them give the eager bits each time."""
    L = _lib.lib()
    M, N, K, gs, bits = 1536, 1024, 2048, 64, 6
    _, d = _inputs(O, dev, M, N, K, gs, bits, seed=11)
    _, d2 = _inputs(O, dev, 1100, 1024, 1024, 32, 4, seed=12)
    ref = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    assert _plain(L, d, M, N, K, gs, bits, ref) == _lib.MXQ_OK
    torch.cuda.synchronize()
    y = torch.full_like(ref, float("nan"))
    y2 = torch.empty(1100, 1024, dtype=torch.bfloat16, device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = _plain(L, d, M, N, K, gs, bits, y)
    assert rc == _lib.MXQ_OK, L.mxq_last_error()
    for i in range(3):
        y.fill_(float("nan"))
        assert _plain(L, d2, 1100, 1024, 1024, 32, 4, y2) == _lib.MXQ_OK
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {i}"
