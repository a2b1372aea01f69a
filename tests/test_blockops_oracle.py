"""The oracle's restatement of the H3 block row ops, pinned on the CPU: against torch's
float64 rms_norm, the rotation written as complex multiplication, and closed forms; plus the
host-side row map of plan.runs."""
import numpy as np
import torch

import wuxianhuabu_amd as mx


def _bf16(a, O):
    return O.bf16_rne(np.asarray(a, np.float32))


def test_rmsnorm_matches_torch(O):
    rng = np.random.default_rng(0)
    x = _bf16(rng.standard_normal((64, 5376)) * 3, O)
    w = _bf16(rng.standard_normal(5376) * 0.5 + 1, O)
    got = O.rmsnorm_bf16(x, w, 1e-6)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(O.bf16_to_f32(x).astype(np.float64)),
                                       (5376,), torch.from_numpy(O.bf16_to_f32(w).astype(np.float64)),
                                       eps=1e-6).numpy()
    ref_b = O.bf16_to_f32(O.bf16_rne(ref.astype(np.float32)))
    ulp = np.abs(ref_b) * 2.0 ** -7 + 1e-30
    assert (np.abs(got - ref_b) <= ulp).all()          # at most one bf16 step apart
    assert (got == ref_b).mean() > 0.99                 # and almost always equal
    # constant rows: x * rsqrt(x^2 + eps) * w = sign(x) * w (eps negligible)
    c = _bf16(np.full((2, 8), [[2.0], [-0.5]]), O)
    wc = _bf16(np.arange(1, 9) / 8, O)
    np.testing.assert_allclose(O.rmsnorm_bf16(c, wc, 0.0),
                               np.sign([[2.0], [-0.5]]) * O.bf16_to_f32(wc), rtol=2 ** -8)


def test_rope_is_complex_rotation(O):
    rng = np.random.default_rng(1)
    S, H, hd, rot = 5, 3, 128, 96
    x = _bf16(rng.standard_normal((S, H, hd)), O)
    w = _bf16(np.ones(hd), O)
    th = rng.uniform(0, 6.3, (S, rot // 2))
    out = O.rmsnorm_rope_f64(x, w, np.cos(th), np.sin(th), rot, 1e-6)
    n = O.rmsnorm_bf16(x, w, 1e-6).astype(np.float64)
    z = (n[..., : rot // 2] + 1j * n[..., rot // 2: rot]) * np.exp(1j * th)[:, None, :]
    np.testing.assert_allclose(out[..., : rot // 2], z.real, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out[..., rot // 2: rot], z.imag, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(out[..., rot:], n[..., rot:])   # tail passes through
    # pair norms are preserved; angle 0 is the plain norm
    np.testing.assert_allclose(out[..., :48] ** 2 + out[..., 48:96] ** 2,
                               n[..., :48] ** 2 + n[..., 48:96] ** 2, rtol=1e-12)
    zero = O.rmsnorm_rope_f64(x, w, np.ones((S, 48)), np.zeros((S, 48)), rot, 1e-6)
    np.testing.assert_array_equal(zero, n)


def test_modscale_and_gate_closed_forms(O):
    rng = np.random.default_rng(2)
    x = _bf16(rng.standard_normal((6, 40)), O)
    w = _bf16(rng.standard_normal(40), O)
    z = _bf16(np.zeros((2, 40)), O)
    np.testing.assert_array_equal(O.norm_modscale_f64(x, w, z, z, [0, 1, 1, 0, 1, 0], 1e-5),
                                  O.rmsnorm_bf16(x, w, 1e-5))
    sc = _bf16(rng.standard_normal((2, 40)), O)
    sh = _bf16(rng.standard_normal((2, 40)), O)
    rm = np.array([1, 1, 0, 0, 1, 0])
    n = O.rmsnorm_bf16(x, w, 1e-5).astype(np.float64)
    want = n * (O.bf16_to_f32(sc)[rm] + 1) + O.bf16_to_f32(sh)[rm]
    np.testing.assert_allclose(O.norm_modscale_f64(x, w, sh, sc, rm, 1e-5), want, rtol=1e-15)
    o = _bf16(rng.standard_normal((6, 40)), O)
    np.testing.assert_array_equal(O.mod_gate_f64(x, o, z, rm), O.bf16_to_f32(x))
    one = _bf16(np.ones((1, 40)), O)
    np.testing.assert_allclose(O.mod_gate_f64(x, o, one, None),
                               O.bf16_to_f32(x).astype(np.float64) + O.bf16_to_f32(o), rtol=0)


def test_build_row_mod_map():
    m = mx.build_row_mod_map(10, [(0, 3, 2), (3, 7, 0), (7, 20, 1)], device="cpu")
    assert m.view(torch.int32).tolist() == [2, 2, 2, 0, 0, 0, 0, 1, 1, 1]
    assert mx.build_row_mod_map(4, [(2, 1, 5)], device="cpu").view(torch.int32).tolist() == [0] * 4
