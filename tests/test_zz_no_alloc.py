"""mxq_quantized_matmul_noalloc (its workspace is a static device array, one per GPU)
against mxq_quantized_matmul_ws (a caller workspace), through the C ABI.

Two calls in a row, the second with a smaller input, give the bits of the workspace
entry point each time (the array keeps the first call's tiled weight; the second
call overwrites what it uses). A small M takes the plain operator; a weight whose
tiled copy exceeds the array is refused before anything is enqueued. Captured in a HIP
graph (the callers it is for), every replay gives the same bits.
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


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _inputs(O, dev, M, N, K, gs, bits, seed):
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=seed, with_bias=True)
    d = (dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev),
         dev_bf16(bias, dev))
    return (x, wq, s, b, bias), d


def _noalloc(L, d, M, N, K, gs, bits, y):
    xd, wd, sd, bd, biasd = d
    return L.mxq_quantized_matmul_noalloc(P(xd), M, K, P(wd), P(sd), P(bd), N, 1, gs, bits,
                                          P(biasd), P(y), _stream())


def _with_workspace(L, d, M, N, K, gs, bits, y):
    xd, wd, sd, bd, biasd = d
    need = L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=y.device)
    rc = L.mxq_quantized_matmul_ws(P(xd), M, K, P(wd), P(sd), P(bd), N, 1, gs, bits, P(biasd),
                                   P(y), P(ws), max(need, 0), _stream())
    torch.cuda.synchronize()
    return rc, need


def test_noalloc_matches_workspace_entry_point(dev, O):
    L = _lib.lib()
    # the second call is smaller in every dimension, with another width and group size
    for (M, N, K, gs, bits, seed) in [(1536, 4096, 2048, 64, 6, 5), (1100, 1000, 1024, 32, 4, 6)]:
        host, d = _inputs(O, dev, M, N, K, gs, bits, seed)
        need = L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits)
        assert 0 < need <= _lib.MXQ_NOALLOC_SCRATCH_BYTES
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        assert _noalloc(L, d, M, N, K, gs, bits, y) == _lib.MXQ_OK, L.mxq_last_error()
        torch.cuda.synchronize()
        y_ws = torch.empty_like(y)
        rc, _ = _with_workspace(L, d, M, N, K, gs, bits, y_ws)
        assert rc == _lib.MXQ_OK
        assert torch.equal(y, y_ws), f"M={M} N={N} K={K} bits={bits} gs={gs}"
        rows = np.arange(0, M, 97)
        x, wq, s, b, bias = host
        assert_tight(host_f32_of_bf16(y)[rows],
                     O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows),
                     f"noalloc M={M} N={N} K={K} bits={bits} gs={gs}")


def test_noalloc_small_m_is_the_plain_operator(dev, O):
    L = _lib.lib()
    M, N, K, gs, bits = 4, 512, 1024, 64, 6
    host, d = _inputs(O, dev, M, N, K, gs, bits, 9)
    assert L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits) == 0
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    y_ref = torch.empty_like(y)
    assert _noalloc(L, d, M, N, K, gs, bits, y) == _lib.MXQ_OK
    xd, wd, sd, bd, biasd = d
    assert L.mxq_quantized_matmul(P(xd), M, K, P(wd), P(sd), P(bd), N, 1, gs, bits, P(biasd),
                                  P(y_ref), _stream()) == _lib.MXQ_OK
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)


def test_noalloc_refuses_a_weight_above_the_scratch(dev):
    L = _lib.lib()
    M, N, K, gs, bits = 1024, 24576, 4096, 64, 6   # tiled: 384 x 64 x 3328 B = 81.8 MB
    need = L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits)
    assert need > _lib.MXQ_NOALLOC_SCRATCH_BYTES
    # real buffers of the right sizes, so a regression could not touch foreign memory
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    wq = torch.zeros(N, K * bits // 32, dtype=torch.int32, device=dev)
    s = torch.zeros(N, K // gs, dtype=torch.bfloat16, device=dev)
    y = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=dev)
    rc = L.mxq_quantized_matmul_noalloc(P(x), M, K, P(wq), P(s), P(s), N, 1, gs, bits, None,
                                        P(y), _stream())
    assert rc == _lib.MXQ_ERR_INVALID
    assert b"scratch" in L.mxq_last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())


def test_noalloc_under_graph_capture(dev, O):
    """The calls it is for: captured in a HIP graph (nothing allocated, no memset node),
    the graph replayed three times with eager work and synchronizations between the
    replays (an eager call on another weight overwrites the shared array each time);
    every replay gives the workspace entry point's bits."""
    L = _lib.lib()
    M, N, K, gs, bits = 1536, 2048, 2048, 64, 6
    _, d = _inputs(O, dev, M, N, K, gs, bits, 21)
    _, d2 = _inputs(O, dev, 1100, 1024, 1024, 32, 4, 22)
    y_ref = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    rc, _ = _with_workspace(L, d, M, N, K, gs, bits, y_ref)
    assert rc == _lib.MXQ_OK
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    y2 = torch.empty(1100, 1024, dtype=torch.bfloat16, device=dev)
    # outside capture first: the library looks up the array's address and the CU count once
    assert _noalloc(L, d, M, N, K, gs, bits, y) == _lib.MXQ_OK
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = _noalloc(L, d, M, N, K, gs, bits, y)
    assert rc == _lib.MXQ_OK, L.mxq_last_error()
    for i in range(3):
        y.fill_(float("nan"))
        assert _noalloc(L, d2, 1100, 1024, 1024, 32, 4, y2) == _lib.MXQ_OK
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"replay {i}"
