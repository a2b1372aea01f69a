"""Untiling and the single resident copy.

mxq_untile / mxq_untile_swiglu turn a tiled buffer back into the MLX triple.
They are checked bit for bit on buffers written by the oracle's tiler (orc_tile,
every bit pattern of codes, scales and biases), so they are pinned against the
format and not only against the HIP tiler; round trips through the HIP tiler run at
the benchmark geometry. The module types keep one copy: once tiled, the MLX
triple is dropped and rebuilt on demand, and the bytes the layer holds equal
those of the triple it was given.
"""
import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from tests.gpu_util import dev_bf16, dev_words, host_bf16, host_words
from tests.test_gpu_matmul import make_case

pytestmark = pytest.mark.gpu

BITS = [2, 3, 4, 5, 6, 8]
GS = [32, 64, 128]


def _random_triple(N, K, gs, bits, seed):
    rng = np.random.default_rng(seed)
    wq = rng.integers(0, 2 ** 32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = rng.integers(0, 2 ** 16, size=(N, K // gs), dtype=np.uint16)
    b = rng.integers(0, 2 ** 16, size=(N, K // gs), dtype=np.uint16)
    return wq, s, b


def _assert_triple(got, wq, s, b, what):
    gw, gsc, gb = got
    np.testing.assert_array_equal(host_words(gw), wq, err_msg=what + " codes")
    np.testing.assert_array_equal(host_bf16(gsc), s, err_msg=what + " scales")
    np.testing.assert_array_equal(host_bf16(gb), b, err_msg=what + " biases")


# K steps per case: 6 (one full and one partial block of the kernel's 4-step groups),
# 1 and 5 (a single step; a remainder of one step), 4 (one exact group)
_SHAPES = [(100, 384), (1, 64), (65, 320), (128, 256), (3, 640)]


@pytest.mark.parametrize("bits,gs,N,K", [(bits, gs, N, K) for bits in BITS for gs in GS
                                         for N, K in _SHAPES if K % gs == 0])
def test_untile_inverts_oracle_tile(dev, O, bits, gs, N, K):
    wq, s, b = _random_triple(N, K, gs, bits, seed=bits * 101 + gs + N + K)
    buf = torch.from_numpy(O.tile(wq, s, b, K, gs, bits)).to(dev)
    got = mx.untile(mx.TiledWeight(buf, N, K, gs, bits))
    _assert_triple(got, wq, s, b, f"bits={bits} gs={gs} N={N} K={K}")


@pytest.mark.parametrize("bits,gs", [(6, 64), (4, 32), (3, 128), (8, 64)])
@pytest.mark.parametrize("N", [140, 128, 2])
def test_untile_swiglu_inverts_oracle_tile(dev, O, bits, gs, N):
    K = 384  # six K steps: one full and one partial group of the kernel's 4-step blocks
    wq, s, b = _random_triple(N, K, gs, bits, seed=bits + gs + N)
    buf = torch.from_numpy(O.tile_swiglu(wq, s, b, K, gs, bits)).to(dev)
    got = mx.untile(mx.TiledWeight(buf, N, K, gs, bits, swiglu=True))
    _assert_triple(got, wq, s, b, f"swiglu bits={bits} gs={gs} N={N}")


def test_untile_round_trip_full_size(dev):
    """The benchmark weight (16384 x 4096, 6-bit, gs 64) and the down projection's
    (4096 x 16384): tile then untile returns the same bits."""
    for N, K in ((16384, 4096), (4096, 16384)):
        g = torch.Generator(device=dev)
        g.manual_seed(N + K)
        wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K * 6 // 32), generator=g,
                           device=dev, dtype=torch.int32).view(torch.uint32)
        s = torch.randint(0, 2 ** 16, (N, K // 64), generator=g, device=dev,
                          dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
        b = torch.randint(0, 2 ** 16, (N, K // 64), generator=g, device=dev,
                          dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
        w2, s2, b2 = mx.untile(mx.tile(wq, s, b, 64, 6))
        assert torch.equal(w2.view(torch.int32), wq.view(torch.int32)), (N, K)
        assert torch.equal(s2.view(torch.int16), s.view(torch.int16)), (N, K)
        assert torch.equal(b2.view(torch.int16), b.view(torch.int16)), (N, K)


def test_untile_rejects_odd_swiglu_and_bad_geometry(dev):
    buf = torch.zeros(mx.lib().mxq_tiled_bytes(3, 64, 64, 4), dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="even"):
        mx.untile(mx.TiledWeight(buf, 3, 64, 64, 4, swiglu=True))
    with pytest.raises(ValueError, match="multiple of 64"):
        mx.untile(mx.TiledWeight(buf, 3, 96, 32, 4))
    with pytest.raises(ValueError, match="TiledWeight"):
        mx.untile(buf)


def _held_bytes(*tensors):
    return sum(t.numel() * t.element_size() for t in tensors if t is not None)


def test_quantized_linear_holds_one_copy(dev, O):
    """After the first call the layer holds the tiled copy only; its bytes equal the
    triple's (N a multiple of 64, gs 64), the parameters read back bit for bit, and
    assigning a parameter goes back to the triple, bit-identical results throughout."""
    N, K, gs, bits, M = 256, 1024, 64, 6, 130
    x, wq, s, b, bias = make_case(O, M, N, K, gs, bits, seed=5, with_bias=True)
    lin = mx.QuantizedLinear.from_weights(dev_words(wq, dev), dev_bf16(s, dev),
                                          dev_bf16(b, dev), dev_bf16(bias, dev), gs, bits)
    triple_bytes = _held_bytes(*lin._triple)
    xd = dev_bf16(x, dev)
    ref = mx.quantized_matmul(xd, *lin._triple, group_size=gs, bits=bits, bias=lin.bias)
    y = lin(xd)
    assert torch.equal(y, ref)
    assert lin._triple is None and lin._tw is not None
    assert lin._tw.nbytes == triple_bytes
    _assert_triple((lin.weight, lin.scales, lin.biases), wq, s, b, "read back")
    assert lin._triple is None, "reading a parameter must not keep a second copy"
    # dequantized() over the rebuilt parameters equals it over the original triple
    deq = mx.dequantized(lin.weight, lin.scales, lin.biases, gs, bits)
    assert torch.equal(deq, mx.dequantized(dev_words(wq, dev), dev_bf16(s, dev),
                                           dev_bf16(b, dev), gs, bits))
    # assigning one parameter replaces the triple; the next call tiles it again
    lin.biases = dev_bf16(b, dev)
    assert lin._tw is None and lin._triple is not None
    assert torch.equal(lin(xd), ref) and lin._triple is None
    # the GEMV on the held copy equals the GEMV on a fresh tiling of the original bits
    fresh = mx.tile(dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev), gs, bits)
    assert torch.equal(lin(xd[:2]), mx.tiled_matmul(xd[:2], fresh, bias=lin.bias))


def test_quantized_linear_device_memory_is_one_weight(dev, O):
    """Device bytes allocated by the layer are one weight's worth before and after
    tiling (the caller drops its own references to the triple)."""
    N, K, gs, bits = 4096, 4096, 64, 6
    torch.cuda.synchronize()
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    w = torch.randn(N, K, generator=g, device=dev).bfloat16()
    x = torch.randn(256, K, generator=g, device=dev).bfloat16()
    base = torch.cuda.memory_allocated(dev)
    lin = mx.QuantizedLinear.from_linear(w, None, gs, bits)
    del w
    torch.cuda.synchronize()
    weight_bytes = N * K * bits // 8 + 2 * N * (K // gs) * 2
    before = torch.cuda.memory_allocated(dev)
    y = lin(x)
    torch.cuda.synchronize()
    after = torch.cuda.memory_allocated(dev) - y.numel() * y.element_size()
    assert after == before, (before, after)
    assert lin._tw.nbytes == weight_bytes
    del lin, y
    assert torch.cuda.memory_allocated(dev) <= base


def test_mflinear_and_h3mlp_hold_one_copy(dev, O, tmp_path):
    """MfLinear.load from a file keeps no cached copy; H3MlpW's fc1 holds its gate/up
    pairs in place of the triple, and fc1.w reads back in [gate; up] order."""
    from safetensors.torch import save_file
    H, F, gs, bits = 256, 384, 64, 4
    tensors = {}
    parts = {}
    for name, n, k in (("mlp.fc1", 2 * F, H), ("mlp.fc2", H, F)):
        _, wq, s, b, _ = make_case(O, 1, n, k, gs, bits, seed=n + k)
        parts[name] = (wq, s, b)
        tensors[name + ".weight"] = torch.from_numpy(wq.view(np.int32)).view(torch.uint32)
        tensors[name + ".scales"] = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
        tensors[name + ".biases"] = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    path = tmp_path / "mlp.safetensors"
    save_file(tensors, str(path))
    with mx.SafetensorsFile(path, device=dev) as f:
        mlp = mx.H3MlpW.load(f, "mlp", H, F)
        assert len(f._cache) == 0, "load must read around the file's cache"
    x = torch.randn(100, H, device=dev).bfloat16()
    y = mlp(x)
    fc1, fc2 = mlp.fc1, mlp.fc2
    assert fc1._triple is None and fc1._tw.swiglu
    assert fc2._triple is None and fc2._tw is not None and not fc2._tw.swiglu
    _assert_triple((fc1.w, fc1.scales, fc1.biases), *parts["mlp.fc1"], "fc1 pairs")
    _assert_triple((fc2.w, fc2.scales, fc2.biases), *parts["mlp.fc2"], "fc2")
    # fc1 called on its own while held in pairs: MLX-layout kernels on the rebuilt triple
    y1 = fc1(x)
    wq, s, b = parts["mlp.fc1"]
    ref1 = mx.quantized_matmul(x, dev_words(wq, dev), dev_bf16(s, dev), dev_bf16(b, dev),
                               group_size=gs, bits=bits)
    assert torch.equal(y1, ref1)
    assert fc1._tw.swiglu, "a direct fc1 call must leave the pairs copy in place"
    assert torch.equal(mlp(x), y)
