"""LoRA fused into the tiled MFMA kernel (`model/minimax h3/H3Common.swift:369-375, 405-434`:
out + sum_i scale_i (x a_i) b_i), against the oracle.

The kernel consumes xa = x [a_1 | a_2 | ...] (bf16, a library GEMM) and bt = [scale_i b_i]^T
(bf16); the tight check runs the fp64 matmul over the bf16-rounded weights plus xa . bt^T in
fp64 on exactly those operands, then the fp64 activation; the north-star metric compares
with the exact fp64 chain sum_i scale_i (x a_i) b_i. Shapes cover 64/128/256-row tiles, the
remainder launch, ragged N, odd K steps, ranks padded to 16, several adapters, and each
activation (SwiGLU with its [gate; up] rows)."""
import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from tests.gpu_util import assert_tight, dev_bf16, dev_words, host_f32_of_bf16, spec_metric
from tests.test_gpu_matmul import make_case

pytestmark = pytest.mark.gpu

_ACT = {None: lambda O, v: v, "gelu_tanh": lambda O, v: O.gelu_tanh_f64(v),
        "swiglu": lambda O, v: O.swiglu_f64(v)}


def _adapters(dev, K, N, ranks, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    refs = []
    for i, r in enumerate(ranks):
        a = (torch.randn(K, r, generator=g, device=dev) * 0.05).bfloat16()
        b = (torch.randn(r, N, generator=g, device=dev) * 0.05).bfloat16()
        refs.append((a, b, 0.5 + 0.25 * i))
    return refs


@pytest.mark.parametrize("M,N,K,bits,gs,act,ranks", [
    (9, 130, 256, 6, 64, None, [8]),
    (100, 288, 576, 4, 32, "gelu_tanh", [16, 4]),
    (300, 256, 640, 6, 128, "swiglu", [32]),
    (700, 200, 1088, 8, 64, None, [64, 64]),
    (2148, 8192, 576, 6, 64, "gelu_tanh", [16]),
])
def test_lora_fused(dev, O, M, N, K, bits, gs, act, ranks):
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M + N + K + len(ranks),
                                  with_bias=True)
    swiglu = act == "swiglu"
    tw = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits, swiglu=swiglu)
    refs = _adapters(dev, K, N, ranks, seed=M)
    lora = mx.LoraAdapters(refs)
    assert lora.R % 16 == 0 and lora.rank == sum(ranks)
    xd = dev_bf16(x, dev)
    y = mx.tiled_matmul(xd, tw, bias=dev_bf16(bias, dev), activation=act, lora=lora)
    rows = np.unique(np.array([0, 1, M // 2, M - 1]))
    got = host_f32_of_bf16(y)[rows]
    xa = host_f32_of_bf16(lora.xa(xd))[rows]
    bt = host_f32_of_bf16(lora.bt)
    base = O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows, threads=16)
    assert_tight(got, _ACT[act](O, base + xa @ bt.T), f"lora M={M} act={act}")
    xf = host_f32_of_bf16(xd)[rows]
    delta = sum(sc * (xf @ host_f32_of_bf16(a)) @ host_f32_of_bf16(bb) for a, bb, sc in refs)
    exact = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias, rows=rows, threads=16) + delta
    assert spec_metric(got, _ACT[act](O, exact)) <= 2e-2


def test_mflinear_lora_matches_unfused(dev):
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    K, N, M = 512, 384, 200
    w = torch.randn(N, K, generator=g, device=dev) * 0.05
    wq, s, b = mx.quantized(w, 64, 4, scales_dtype=torch.bfloat16, mode="minmax")
    t = {"l.weight": wq, "l.scales": s, "l.biases": b,
         "l.bias": (torch.randn(N, generator=g, device=dev) * 0.1).bfloat16()}
    fused = mx.MfLinear.load(t, "l", K).set_lora(_adapters(dev, K, N, [16, 8], 5))
    plain = mx.MfLinear.load(t, "l", K).set_lora(_adapters(dev, K, N, [16, 8], 5))
    plain.tiled = False
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    a, r = fused(x).float(), plain(x).float()
    # the unfused chain rounds the base output and the sum separately (an ulp of the
    # larger intermediate where base and LoRA term cancel): compare max-normalised
    assert ((a - r).abs().max() / r.abs().max()).item() < 1e-2


def test_h3_mlp_with_fc1_lora(dev):
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    hidden, ffn = 256, 384
    t = {}
    for name, n, k in (("m.fc1", 2 * ffn, hidden), ("m.fc2", hidden, ffn)):
        wq, s, b = mx.quantized(torch.randn(n, k, generator=g, device=dev) * 0.05, 64, 6,
                                scales_dtype=torch.bfloat16, mode="minmax")
        t[name + ".weight"], t[name + ".scales"], t[name + ".biases"] = wq, s, b
    mlp = mx.H3MlpW.load(t, "m", hidden, ffn)
    mlp.fc1.set_lora(_adapters(dev, hidden, 2 * ffn, [32], 1))
    x = torch.randn(130, hidden, generator=g, device=dev).bfloat16()
    y = mlp(x).float()
    h = mlp.fc1.forward(x).float()
    ref = mlp.fc2.forward((torch.nn.functional.silu(h[:, :ffn]) * h[:, ffn:]).bfloat16()).float()
    assert ((y - ref).abs().max() / ref.abs().max()).item() < 1e-2


def test_lora_errors(dev, O):
    M, N, K, gs, bits = 16, 64, 128, 64, 4
    x, wq, s, b, _ = make_case(O, M, N, K, gs, bits, seed=7)
    tw = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits)
    bad = mx.LoraAdapters(_adapters(dev, K + 64, N, [16], 2))
    with pytest.raises(ValueError, match="LoRA shapes"):
        mx.tiled_matmul(dev_bf16(x, dev), tw, lora=bad)
    with pytest.raises(ValueError, match="lora"):
        mx.LoraAdapters([])
    L = mx.lib()
    import ctypes
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    xd = dev_bf16(x, dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = L.mxq_qmm_tiled_lora(p(xd), M, K, p(tw.data), N, gs, bits, None, 0, p(xd), p(xd), 8,
                              p(y), None)
    assert rc == mx._lib.MXQ_ERR_INVALID and b"multiple of 16" in L.mxq_last_error()
