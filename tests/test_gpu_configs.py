"""The benchmark configurations at their full sizes, on both weight layouts.

c0  6-bit  M=256   K=2048  N=2048   every output row checked
c1  6-bit  M=3600  K=4096  N=4096   256 sampled rows + the last row + the launch seam
c2  6-bit  M=2     K=4096  N=24576  (GEMV) every output checked
c3  6-bit  M=14400 K=4096  N=16384 (up) and K=16384 N=4096 on GELU_tanh(h) (down), 256 sampled
    rows + the last row + rows 14335/14336 (the 256-row / 64-row launch seam)
c4  4-bit  one DiT block's linear chain at M=14400 (kv at M=512), weights resident, 128
    sampled rows per layer + the last row + the seam

Inputs are seeded on the GPU (x from seed 1000+c, W from 2000+c, W2 from 3000+c),
weights are quantized by the GPU quantizer (bit-exact with the oracle, see
test_gpu_layout), and the packed triple plus the sampled activation rows come back
to the host, where the oracle recomputes those rows. Tolerances as in
test_gpu_matmul: tight against orc_qmm_f64_bf16w (MFMA kernels) or orc_qmm_f64
(GEMV), and max|y - r| / max|r| <= 2e-2 against the exact fp64 oracle. Where both
layouts run the same MFMA kernel (K % 64 == 0, M > 64), their outputs must be
bit-identical.
"""
import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from tests.gpu_util import assert_tight, host_bf16, host_words, spec_metric

pytestmark = pytest.mark.gpu


def _weights(dev, N, K, seed, bits, gs=64):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = torch.randn(N, K, generator=g, device=dev) * 0.02
    wq, s, b = mx.quantized(w, gs, bits, scales_dtype=torch.bfloat16, mode="minmax")
    return wq, s, b


def _acts(dev, M, K, seed, gelu=False):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    if gelu:
        x = torch.nn.functional.gelu(x.float(), approximate="tanh").bfloat16()
    return x


def _rows(M, n, seed):
    """n seeded rows, the last row and the rows either side of the seam between the
    256-row tiles and the remainder (a second launch of 64- or 128-row tiles)."""
    if M <= n:
        return np.arange(M)
    rng = np.random.default_rng(seed)
    seam = (M // 256) * 256
    extra = [M - 1] + ([seam - 1, seam] if 0 < seam < M else [])
    return np.unique(np.concatenate([rng.choice(M, n, replace=False), extra]))


def _check(O, x, wq, s, b, y, rows, gs, bits, what, exact_only=False):
    xh = host_bf16(x[torch.as_tensor(rows, device=x.device)])
    wqh, sh, bh = host_words(wq), host_bf16(s), host_bf16(b)
    yh = y[torch.as_tensor(rows, device=y.device)].float().cpu().numpy().astype(np.float64)
    ref = O.qmm_f64(xh, wqh, sh, bh, gs, bits, threads=16)
    if exact_only:
        assert_tight(yh, ref, what)
    else:
        assert_tight(yh, O.qmm_f64_bf16w(xh, wqh, sh, bh, gs, bits, threads=16), what)
    assert spec_metric(yh, ref) <= 2e-2, what


def _both_layouts(dev, O, M, K, N, bits, seed_x, seed_w, nrows, what, gelu=False):
    x = _acts(dev, M, K, seed_x, gelu)
    wq, s, b = _weights(dev, N, K, seed_w, bits)
    # the MLX-layout kernels themselves (path="auto" tiles the weight first at large M)
    y_mlx = mx.quantized_matmul(x, wq, s, b, group_size=64, bits=bits,
                                path="qmv" if M <= 8 else "qmm")
    tw = mx.tile(wq, s, b, 64, bits)
    y_t = mx.tiled_matmul(x, tw)
    rows = _rows(M, nrows, seed_x)
    gemv = M <= 8
    _check(O, x, wq, s, b, y_mlx, rows, 64, bits, what + " (MLX layout)", exact_only=gemv)
    _check(O, x, wq, s, b, y_t, rows, 64, bits, what + " (tiled)", exact_only=gemv)
    if not gemv and M > 64:
        assert torch.equal(y_mlx, y_t), what + ": tiled and MLX-layout kernels differ"
    return x, y_t


def test_c0(dev, O):
    _both_layouts(dev, O, 256, 2048, 2048, 6, 1000, 2000, 256, "c0")


def test_c1(dev, O):
    _both_layouts(dev, O, 3600, 4096, 4096, 6, 1001, 2001, 256, "c1")


def test_c2_gemv(dev, O):
    _both_layouts(dev, O, 2, 4096, 24576, 6, 1002, 2002, 2, "c2")


def test_c3_up(dev, O):
    _both_layouts(dev, O, 14400, 4096, 16384, 6, 1003, 2003, 256, "c3 up")


def test_c3_down_on_gelu(dev, O):
    _both_layouts(dev, O, 14400, 16384, 4096, 6, 1003, 3003, 256, "c3 down", gelu=True)


def test_c4_chain_4bit(dev, O):
    """The block's chain with every weight resident (both layouts held at once)."""
    chain = [("qkv", 14400, 4096, 12288), ("out", 14400, 4096, 4096),
             ("xq", 14400, 4096, 4096), ("xkv", 512, 4096, 8192),
             ("up", 14400, 4096, 16384), ("down", 14400, 16384, 4096)]
    layers = []
    for i, (name, M, K, N) in enumerate(chain):
        wq, s, b = _weights(dev, N, K, 2004 + 100 * i, 4)
        layers.append((name, M, K, N, wq, s, b, mx.tile(wq, s, b, 64, 4)))
    for i, (name, M, K, N, wq, s, b, tw) in enumerate(layers):
        x = _acts(dev, M, K, 1004 + 100 * i, gelu=(name == "down"))
        y_mlx = mx.quantized_matmul(x, wq, s, b, group_size=64, bits=4, path="qmm")
        y_t = mx.tiled_matmul(x, tw)
        assert torch.equal(y_mlx, y_t), f"c4 {name}: layouts differ"
        _check(O, x, wq, s, b, y_t, _rows(M, 128, 1004 + i), 64, 4, f"c4 {name}")
