"""The H3 block row ops on the GPU against the oracle (tests/test_blockops_oracle pins it).

Tolerance: the kernels round the normalised value to bf16 and the result once more; their
fp32 rstd can differ from the oracle's in the last bit, which can move the intermediate
rounding by one bf16 step (up to 2^-7 relative just above a power of two). Bound: one bf16
step of the result, 2^-7 |ref|, plus one of each term that carries the intermediate value,
2^-7 times their magnitude, + 1e-6 of the scale."""
import numpy as np
import pytest
import torch

import wuxianhuabu_amd as mx
from tests.gpu_util import dev_bf16, host_f32_of_bf16

pytestmark = pytest.mark.gpu


def _rand(O, rng, shape, s=1.0, m=0.0):
    return O.bf16_rne((rng.standard_normal(shape) * s + m).astype(np.float32))


def _close(y, ref, carry, what):
    y, ref, carry = (np.asarray(a, np.float64) for a in (y, ref, carry))
    bound = 2.0 ** -7 * (np.abs(ref) + np.abs(carry)) + 1e-6 * max(np.abs(ref).max(), 1e-30)
    bad = np.abs(y - ref) > bound
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside; worst " \
                          f"{np.abs(y - ref).max():.3e}"


@pytest.mark.parametrize("S,hidden,rows", [(300, 5376, 3), (7, 100, 2), (64, 4096, 1)])
def test_norm_modscale(dev, O, S, hidden, rows):
    rng = np.random.default_rng(S + hidden)
    x = _rand(O, rng, (S, hidden), 2.0)
    w = _rand(O, rng, hidden, 0.3, 1.0)
    sh = _rand(O, rng, (rows, hidden), 0.5)
    sc = _rand(O, rng, (rows, hidden), 0.5)
    runs = [(0, S // 3, rows - 1), (S // 3, S, 0)]
    rm = mx.build_row_mod_map(S, runs, device=dev)
    y = mx.fused_norm_modscale(dev_bf16(x, dev), dev_bf16(w, dev), dev_bf16(sh, dev),
                               dev_bf16(sc, dev), rm, eps=1e-6)
    m = rm.view(torch.int32).cpu().numpy()
    ref = O.norm_modscale_f64(x, w, sh, sc, m, 1e-6)
    carry = O.rmsnorm_bf16(x, w, 1e-6) * (O.bf16_to_f32(sc)[m] + 1)
    _close(host_f32_of_bf16(y), ref, carry, f"norm_modscale S={S} hidden={hidden}")
    # one modulation row for all token rows (the final head)
    y1 = mx.fused_norm_modscale_row(dev_bf16(x, dev), dev_bf16(w, dev), dev_bf16(sh[:1], dev),
                                    dev_bf16(sc[:1], dev), eps=1e-6)
    ref1 = O.norm_modscale_f64(x, w, sh[:1], sc[:1], None, 1e-6)
    carry1 = O.rmsnorm_bf16(x, w, 1e-6) * (O.bf16_to_f32(sc[:1]) + 1)
    _close(host_f32_of_bf16(y1), ref1, carry1, "norm_modscale_row")


@pytest.mark.parametrize("S,hidden,rows", [(300, 5376, 3), (9, 37, 2)])
def test_mod_gate(dev, O, S, hidden, rows):
    rng = np.random.default_rng(S * hidden)
    x, o = _rand(O, rng, (S, hidden)), _rand(O, rng, (S, hidden))
    g = _rand(O, rng, (rows, hidden), 0.5)
    rm = mx.build_row_mod_map(S, [(0, S, rows - 1)], device=dev)
    y = mx.fused_mod_gate(dev_bf16(x, dev), dev_bf16(g, dev), dev_bf16(o, dev), rm)
    ref = O.mod_gate_f64(x, o, g, rm.view(torch.int32).cpu().numpy())
    _close(host_f32_of_bf16(y), ref, 0 * ref, f"mod_gate S={S} hidden={hidden}")


@pytest.mark.parametrize("S,H,hd,rot,tdt", [(50, 24, 128, 96, torch.float32),
                                             (33, 3, 72, 64, torch.bfloat16),
                                             (8, 2, 256, 256, torch.float32),
                                             (5, 4, 64, 0, torch.float32),
                                             (3, 2, 500, 100, torch.bfloat16)])
def test_rmsnorm_rope(dev, O, S, H, hd, rot, tdt):
    rng = np.random.default_rng(S + H + hd)
    x = _rand(O, rng, (S, H, hd), 1.5)
    w = _rand(O, rng, hd, 0.2, 1.0)
    rh = rot // 2
    th = rng.uniform(0, 6.3, (S, max(rh, 1)))[:, :rh]
    c, s = torch.from_numpy(np.cos(th)).to(tdt), torch.from_numpy(np.sin(th)).to(tdt)
    y = mx.fused_rmsnorm_rope(dev_bf16(x, dev).reshape(1, S, H, hd), dev_bf16(w, dev),
                              c.to(dev).reshape(1, S, 1, rh), s.to(dev).reshape(1, S, 1, rh),
                              rot, eps=1e-6)
    assert tuple(y.shape) == (1, S, H, hd)
    cf, sf = c.float().numpy(), s.float().numpy()
    ref = O.rmsnorm_rope_f64(x, w, cf, sf, rot, 1e-6)
    n = O.rmsnorm_bf16(x, w, 1e-6).astype(np.float64)
    carry = np.abs(n).copy()
    carry[..., :rh] = np.abs(n[..., :rh] * cf[:, None]) + np.abs(n[..., rh:rot] * sf[:, None])
    carry[..., rh:rot] = np.abs(n[..., rh:rot] * cf[:, None]) + np.abs(n[..., :rh] * sf[:, None])
    _close(host_f32_of_bf16(y.reshape(S, H, hd)), ref, carry, f"rope S={S} hd={hd} rot={rot}")


def test_blockops_errors(dev):
    x = torch.zeros(4, 8, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="bfloat16"):
        mx.fused_mod_gate(x.float(), x, x)
    with pytest.raises(ValueError, match=r"rot"):
        mx.fused_rmsnorm_rope(x.reshape(1, 4, 1, 8), x[0], torch.zeros(4, 5, device=dev),
                              torch.zeros(4, 5, device=dev), 10)


def _sweep(n, seed):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 400)), int(rng.integers(1, 6000)), int(rng.integers(1, 5)))
            for _ in range(n)]


@pytest.mark.parametrize("S,hidden,rows", _sweep(10, 23))
def test_norm_modscale_and_mod_gate_random_geometry(dev, O, S, hidden, rows):
    """Seeded random token counts, widths (odd ones included) and modulation rows, with
    runs of rows mapped to random modulation rows."""
    rng = np.random.default_rng(S * 7 + hidden)
    x = _rand(O, rng, (S, hidden), 2.0)
    w = _rand(O, rng, hidden, 0.3, 1.0)
    sh = _rand(O, rng, (rows, hidden), 0.5)
    sc = _rand(O, rng, (rows, hidden), 0.5)
    cut = int(rng.integers(0, S + 1))
    runs = [(0, cut, int(rng.integers(0, rows))), (cut, S, int(rng.integers(0, rows)))]
    rm = mx.build_row_mod_map(S, [r for r in runs if r[1] > r[0]], device=dev)
    m = rm.view(torch.int32).cpu().numpy()
    y = mx.fused_norm_modscale(dev_bf16(x, dev), dev_bf16(w, dev), dev_bf16(sh, dev),
                               dev_bf16(sc, dev), rm, eps=1e-6)
    carry = O.rmsnorm_bf16(x, w, 1e-6) * (O.bf16_to_f32(sc)[m] + 1)
    _close(host_f32_of_bf16(y), O.norm_modscale_f64(x, w, sh, sc, m, 1e-6), carry,
           f"norm_modscale S={S} hidden={hidden} rows={rows}")
    o = _rand(O, rng, (S, hidden))
    g = _rand(O, rng, (rows, hidden), 0.5)
    y = mx.fused_mod_gate(dev_bf16(x, dev), dev_bf16(g, dev), dev_bf16(o, dev), rm)
    ref = O.mod_gate_f64(x, o, g, m)
    _close(host_f32_of_bf16(y), ref, 0 * ref, f"mod_gate S={S} hidden={hidden} rows={rows}")
