"""Seeded sweeps of random geometries through the drop-in entry point, the quantizer, the
dequantizer and the fused epilogues, against the oracle.

- `mxq_quantized_matmul` (the drop-in call on the MLX layout: GEMV, pooled tiling or the
  in-place MFMA kernel by shape), 24 cases with M from 1 to 2000, checked on sampled rows
  within the tight bound of the exact oracle (GEMV) or of the bf16-weight oracle (MFMA
  kernels), whichever kernel the shape selects;
- `quantized` (both quantizers, fp32 and bf16 scales) and `dequantized`, 16 cases each,
  bit for bit;
- the tiled MFMA kernel with GELU-tanh or SwiGLU fused, 12 cases, and with LoRA adapters
  (one or two, ranks 1-39, each activation), 8 cases, on sampled rows.
"""
import ctypes

import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from wuxianhuabu_amd import _lib
from tests.gpu_util import (assert_tight, dev_bf16, dev_f32, dev_words, host_bf16,
                            host_f32_of_bf16, host_words, spec_metric)
from tests.test_gpu_matmul import make_case

pytestmark = pytest.mark.gpu
P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731


def _draw(rng, k_max=4096):
    bits = int(rng.choice([2, 3, 4, 5, 6, 8]))
    gs = int(rng.choice([32, 64, 128]))
    K = int(rng.integers(1, k_max // gs + 1)) * gs
    return bits, gs, K


def _dropin_cases(n=24, seed=7):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        bits, gs, K = _draw(rng)
        M = int(np.exp(rng.uniform(0, np.log(2000))))
        N = int(rng.integers(1, 1201))
        if M * N * K <= 1_500_000_000:
            out.append((M, N, K, gs, bits, bool(rng.random() < 0.5)))
    return out


DROPIN = _dropin_cases()


def _tight_either(y, refs, what):
    errs = []
    for r in refs:
        try:
            assert_tight(y, r, what)
            return
        except AssertionError as e:
            errs.append(str(e))
    raise AssertionError(" / ".join(errs))


@pytest.mark.parametrize("M,N,K,gs,bits,with_bias", DROPIN,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}-g{c[3]}-b{c[4]}" for c in DROPIN])
def test_dropin_random_geometry(dev, O, M, N, K, gs, bits, with_bias):
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M + 5 * N + K + bits,
                                  with_bias=with_bias)
    xd, wd, sd, bd = dev_bf16(x, dev), dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev)
    biasd = None if bias is None else dev_bf16(bias, dev)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.mxq_quantized_matmul(P(xd), M, K, P(wd), P(sd), P(bd), N, 1, gs, bits, P(biasd),
                                P(y), st)
    assert rc == _lib.MXQ_OK, L.mxq_last_error()
    torch.cuda.synchronize()
    rows = np.unique(np.r_[np.linspace(0, M - 1, min(M, 24)).astype(int), M - 1])
    got = host_f32_of_bf16(y)[rows]
    exact = O.qmm_f64(x, wq, s, b, gs, bits, bias=bias, rows=rows)
    what = f"drop-in M={M} N={N} K={K} gs={gs} bits={bits}"
    _tight_either(got, [O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows), exact],
                  what)
    assert spec_metric(got, exact) <= 2e-2, what


def _quant_cases(n=16, seed=11):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 65)),) + _draw(rng, 2048) + (int(rng.integers(0, 2)),)
            for _ in range(n)]


QUANT = _quant_cases()


@pytest.mark.parametrize("N,bits,gs,K,mode", QUANT,
                         ids=[f"N{c[0]}-b{c[1]}-g{c[2]}-K{c[3]}-m{c[4]}" for c in QUANT])
def test_quantize_dequantize_random_geometry(dev, O, N, bits, gs, K, mode):
    w = O.normal_f32(N * 131 + K + bits, N * K, 0.003, 0.05).reshape(N, K)
    ref = O.quantize(w, gs, bits, mode=mode)
    name = "minmax" if mode == 0 else "mlx_edge"
    for sdt, key in ((torch.bfloat16, "bf16"), (torch.float32, "f32")):
        wq, s, b = mx.quantized(dev_f32(w, dev), gs, bits, mode=name, scales_dtype=sdt)
        assert np.array_equal(host_words(wq), ref["wq"]), f"codes N={N} K={K} {name}"
        hs = host_bf16(s) if key == "bf16" else s.cpu().numpy()
        hb = host_bf16(b) if key == "bf16" else b.cpu().numpy()
        assert np.array_equal(hs, ref[f"scales_{key}"]) and np.array_equal(hb, ref[f"biases_{key}"])
    f_ref, b_ref = O.dequantize(ref["wq"], ref["scales_bf16"], ref["biases_bf16"], K, gs, bits)
    out = mx.dequantized(dev_words(ref["wq"], dev), dev_bf16(ref["scales_bf16"], dev),
                         dev_bf16(ref["biases_bf16"], dev), gs, bits)
    assert np.array_equal(host_bf16(out), b_ref)
    out_f = mx.dequantized(dev_words(ref["wq"], dev), dev_bf16(ref["scales_bf16"], dev),
                           dev_bf16(ref["biases_bf16"], dev), gs, bits, dtype=torch.float32)
    assert np.array_equal(out_f.cpu().numpy(), f_ref)


def _fused_cases(n=12, seed=13):
    """K a multiple of 64 and of the group size (the tiled layout's steps)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        bits = int(rng.choice([2, 3, 4, 5, 6, 8]))
        gs = int(rng.choice([32, 64, 128]))
        step = max(64, gs)
        K = int(rng.integers(1, 2048 // step + 1)) * step
        out.append((int(rng.integers(1, 601)), int(rng.integers(1, 400)) * 2, K, gs, bits,
                    "gelu_tanh" if i % 2 == 0 else "swiglu"))
    return out


FUSED = _fused_cases()


@pytest.mark.parametrize("M,N,K,gs,bits,act", FUSED,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}-g{c[3]}-b{c[4]}-{c[5]}" for c in FUSED])
def test_fused_epilogue_random_geometry(dev, O, M, N, K, gs, bits, act):
    assert K % 64 == 0 and K % gs == 0
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M + N + K, with_bias=True)
    tw = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits,
                 swiglu=act == "swiglu")
    y = mx.tiled_matmul(dev_bf16(x, dev), tw, activation=act, bias=dev_bf16(bias, dev))
    rows = np.unique(np.r_[np.linspace(0, M - 1, min(M, 16)).astype(int), M - 1])
    got = host_f32_of_bf16(y)[rows]
    f = O.gelu_tanh_f64 if act == "gelu_tanh" else O.swiglu_f64
    pre = O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows)
    assert_tight(got, f(pre), f"{act} M={M} N={N} K={K} gs={gs} bits={bits}")
    exact = f(O.qmm_f64(x, wq, s, b, gs, bits, bias=bias, rows=rows))
    assert spec_metric(got, exact) <= 2e-2


def _lora_cases(n=8, seed=17):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        bits = int(rng.choice([2, 3, 4, 5, 6, 8]))
        gs = int(rng.choice([32, 64, 128]))
        K = int(rng.integers(1, 2048 // 128 + 1)) * 128
        ranks = [int(r) for r in rng.integers(1, 40, size=int(rng.integers(1, 3)))]
        act = [None, "gelu_tanh", "swiglu"][i % 3]
        out.append((int(rng.integers(1, 900)), int(rng.integers(1, 300)) * 2, K, gs, bits, act,
                    ranks))
    return out


LORA = _lora_cases()


@pytest.mark.parametrize("M,N,K,gs,bits,act,ranks", LORA,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}-g{c[3]}-b{c[4]}-{c[5]}" for c in LORA])
def test_lora_random_geometry(dev, O, M, N, K, gs, bits, act, ranks):
    from tests.test_gpu_lora import _ACT, _adapters
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=M + N + K, with_bias=True)
    tw = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits,
                 swiglu=act == "swiglu")
    refs = _adapters(dev, K, N, ranks, seed=M + K)
    lora = mx.LoraAdapters(refs)
    xd = dev_bf16(x, dev)
    y = mx.tiled_matmul(xd, tw, bias=dev_bf16(bias, dev), activation=act, lora=lora)
    rows = np.unique(np.r_[np.linspace(0, M - 1, min(M, 12)).astype(int), M - 1])
    got = host_f32_of_bf16(y)[rows]
    xa = host_f32_of_bf16(lora.xa(xd))[rows]
    base = O.qmm_f64_bf16w(x, wq, s, b, gs, bits, bias=bias, rows=rows)
    assert_tight(got, _ACT[act](O, base + xa @ host_f32_of_bf16(lora.bt).T),
                 f"lora M={M} N={N} K={K} gs={gs} bits={bits} act={act} ranks={ranks}")
