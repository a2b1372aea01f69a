"""The fp64 activation references and the paired (SwiGLU) tiling of the oracle, pinned on
the CPU: against torch's own float64 implementations of the same functions, closed forms,
and the tiled reader of tests/tiled_util."""
import numpy as np
import pytest
import torch

from tests.tiled_util import untile


def test_gelu_tanh_f64_matches_torch(O):
    v = np.linspace(-12.0, 12.0, 4801)
    ref = torch.nn.functional.gelu(torch.from_numpy(v), approximate="tanh").numpy()
    np.testing.assert_allclose(O.gelu_tanh_f64(v), ref, rtol=1e-13, atol=1e-15)
    assert O.gelu_tanh_f64(0.0) == 0.0
    assert abs(O.gelu_tanh_f64(10.0) - 10.0) < 1e-12 and abs(O.gelu_tanh_f64(-10.0)) < 1e-12
    # plain GELU (erf form) agrees to about 1e-3 absolute: the approximation itself
    exact = torch.nn.functional.gelu(torch.from_numpy(v)).numpy()
    assert np.abs(O.gelu_tanh_f64(v) - exact).max() < 2e-3


def test_silu_and_swiglu_f64(O):
    v = np.linspace(-30.0, 30.0, 6001)
    ref = torch.nn.functional.silu(torch.from_numpy(v)).numpy()
    np.testing.assert_allclose(O.silu_f64(v), ref, rtol=1e-13, atol=1e-15)
    # silu(v) - silu(-v) = v
    np.testing.assert_allclose(O.silu_f64(v) - O.silu_f64(-v), v, rtol=0, atol=1e-12)
    y = np.random.default_rng(0).standard_normal((3, 10))
    g, u = y[:, :5], y[:, 5:]
    np.testing.assert_allclose(O.swiglu_f64(y), g / (1 + np.exp(-g)) * u, rtol=1e-15)


@pytest.mark.parametrize("N", [64, 200, 2 * 100])
def test_tile_swiglu_pairs_gate_and_up_rows(O, N):
    """Row block rb of the paired tiling reads back as gate rows 32rb.. then up rows
    N/2 + 32rb.., with zero rows where a half runs past N/2."""
    K, gs, bits = 128, 64, 6
    rng = np.random.default_rng(N)
    wq = rng.integers(0, 2 ** 32, size=(N, K * bits // 32), dtype=np.uint32)
    s = rng.integers(1, 2 ** 15, size=(N, K // gs), dtype=np.uint16)
    b = rng.integers(1, 2 ** 15, size=(N, K // gs), dtype=np.uint16)
    t = O.tile_swiglu(wq, s, b, K, gs, bits)
    assert t.nbytes == O.tiled_bytes(N, K, gs, bits)
    F = N // 2
    nrows = ((F + 31) // 32) * 64
    wq2, s2, b2 = untile(t, nrows, K, gs, bits)
    for rb in range((F + 31) // 32):
        for r in range(32):
            j = rb * 32 + r
            for h, src in ((0, j), (1, F + j)):
                row = rb * 64 + h * 32 + r
                if j < F:
                    assert np.array_equal(wq2[row], wq[src]) and np.array_equal(s2[row], s[src])
                    assert np.array_equal(b2[row], b[src])
                else:
                    assert not wq2[row].any() and not s2[row].any() and not b2[row].any()
