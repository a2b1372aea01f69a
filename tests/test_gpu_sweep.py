"""Seeded sweep of random geometries through every matmul path, against the fp64 oracle.

Forty cases drawn once from a fixed seed: code width, group size, K (a multiple of 32 and
of the group size, up to 4096), N up to 600, M mostly small (the GEMV's range and its
boundary) and sometimes up to 300, with and without bias. For each case:
- the MLX-layout GEMV (`path="qmv"`, M <= 32) within the tight bound of the exact oracle
  (the GEMV multiplies the codes in fp32);
- the MLX-layout MFMA kernel (`path="qmm"`) within the tight bound of the oracle over the
  bf16-rounded weight (the kernel's operands);
- the dispatching call (`path="auto"`) within max|y - r| / max|r| <= 2e-2 of the exact oracle;
- for K % 64 == 0, the tiled layout: its GEMV bit-identical to the MLX-layout GEMV, and
  above 64 tokens (where the MLX layout runs the same MFMA kernel) its MFMA kernel
  bit-identical to the MLX layout's (they share the arithmetic; only where the weight bits
  come from differs); below, within the tight bound of the bf16-weight oracle.
"""
import numpy as np
import pytest

import wuxianhuabu_amd as mx
from tests.gpu_util import assert_tight, dev_bf16, dev_words, host_bf16, host_f32_of_bf16, spec_metric
from tests.test_gpu_matmul import make_case

pytestmark = pytest.mark.gpu


def _cases(n=40, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        bits = int(rng.choice([2, 3, 4, 5, 6, 8]))
        gs = int(rng.choice([32, 64, 128]))
        K = int(rng.integers(1, 4096 // gs + 1)) * gs
        N = int(rng.integers(1, 601))
        M = int(rng.integers(1, 41)) if rng.random() < 0.7 else int(rng.integers(41, 301))
        if M * N * K > 40_000_000:
            continue
        out.append((M, N, K, gs, bits, bool(rng.random() < 0.5)))
    return out


CASES = _cases()


@pytest.mark.parametrize("M,N,K,gs,bits,with_bias", CASES,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}-g{c[3]}-b{c[4]}" for c in CASES])
def test_random_geometry_all_paths(dev, O, M, N, K, gs, bits, with_bias):
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M * 7 + N * 3 + K + bits,
                                  with_bias=with_bias)
    xd, wd, sd, bd = dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev)
    biasd = None if bias is None else dev_bf16(bias, dev)
    what = f"M={M} N={N} K={K} gs={gs} bits={bits} bias={with_bias}"
    exact = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias)
    run = lambda path: mx.quantized_matmul(xd, wd, sd, bd, group_size=gs, bits=bits,  # noqa: E731
                                           bias=biasd, path=path)
    y_mfma = run("qmm")
    assert_tight(host_f32_of_bf16(y_mfma), O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias),
                 f"qmm {what}")
    y_auto = host_f32_of_bf16(run("auto"))
    assert spec_metric(y_auto, exact) <= 2e-2, f"auto {what}"
    y_gemv = None
    if M <= mx._lib.MXQ_QMV_MAX_M:
        y_gemv = run("qmv")
        assert_tight(host_f32_of_bf16(y_gemv), exact, f"qmv {what}")
    if K % 64 == 0:
        tw = mx.tile(wd, sd, bd, gs, bits)
        y_t = mx.tiled_matmul(xd, tw, bias=biasd, path="qmm")
        if M > 64:
            np.testing.assert_array_equal(host_bf16(y_t), host_bf16(y_mfma),
                                          err_msg=f"tiled qmm {what}")
        else:
            assert_tight(host_f32_of_bf16(y_t), O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias),
                         f"tiled qmm {what}")
        if y_gemv is not None:
            y_tv = mx.tiled_matmul(xd, tw, bias=biasd, path="qmv")
            np.testing.assert_array_equal(host_bf16(y_tv), host_bf16(y_gemv),
                                          err_msg=f"tiled qmv {what}")
