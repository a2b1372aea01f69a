"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

Every check here compares the oracle with something it was not derived from:
the goldens of tests/golden/make_golden.py (big-integer bitstreams, exact
rational bf16 rounding, numpy float32 quantizer, numpy fp64 matmul), closed
forms written out by hand (Appendix-style known answers), the reference's own
4-bit unpacker (`model/minimax h3/H3Common.swift:389-394`) restated, and
special cases that reduce to an integer GEMM or to row sums. A final group
plants mistakes in copies of the oracle's inputs/outputs and checks that the
comparisons above would catch them.
"""
import math

import numpy as np
import pytest


def f64_of_bf16(bits):
    bits = np.asarray(bits, dtype=np.uint32)
    return (bits << 16).view(np.float32).astype(np.float64)


# ---------------------------------------------------------------- generator
def test_generator_matches_golden(O, golden):
    for g in golden["generator"]:
        f = O.normal_f32(g["seed"], g["n"], g["mean"], g["std"])
        assert f.tolist() == g["f32"], g["seed"]
        b = O.normal_bf16(g["seed"], g["n"], g["mean"], g["std"])
        assert b.tolist() == g["bf16"], g["seed"]


def test_splitmix_stream_matches_golden(O, golden):
    import ctypes
    for g in golden["generator"]:
        st = ctypes.c_uint64(g["seed"])
        got = [O.lib().orc_splitmix64_next(ctypes.byref(st)) for _ in range(4)]
        assert [str(v) for v in got] == g["splitmix"]


def test_generator_statistics(O):
    z = O.normal_f32(42, 200_000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert abs(((z - z.mean()) ** 3).mean()) < 0.02


# ---------------------------------------------------------------- bf16
def test_bf16_rounding_matches_exact_rationals(O, golden):
    for e in golden["bf16"]:
        v = e["f32"]
        v = math.inf if v == "inf" else (-math.inf if v == "-inf" else v)
        assert int(O.lib().orc_bf16_rne(v)) == e["bits"], v


def test_bf16_roundtrip_exact_for_bf16_values(O):
    bits = np.arange(0, 0x7F80, 37, dtype=np.uint16)
    assert np.array_equal(O.bf16_rne(O.bf16_to_f32(bits)), bits)


# ---------------------------------------------------------------- packing
def test_pack_matches_bigint_golden(O, golden):
    for case in golden["pack"]:
        codes = np.array(case["codes"], dtype=np.uint8)
        words = np.array(case["words"], dtype=np.uint32)
        assert np.array_equal(O.pack_bitwise(codes, case["bits"]), words), case["kind"]
        assert np.array_equal(O.pack_words(codes, case["bits"]), words), case["kind"]
        assert np.array_equal(O.unpack(words, case["K"], case["bits"]), codes), case["kind"]


def test_six_bit_known_answer(O):
    # codes 0..15 in one 3-word period, words written out from the layout:
    # word0 = codes 0..4 at 6i, low 2 bits of code 5 at bit 30;
    # word1 = high 4 bits of code 5, codes 6..9 at 6i-32, low 4 bits of 10 at 28;
    # word2 = high 2 bits of code 10, codes 11..15 at 6i-64.
    w0 = (0 << 0) | (1 << 6) | (2 << 12) | (3 << 18) | (4 << 24) | ((5 & 3) << 30)
    w1 = (5 >> 2) | (6 << 4) | (7 << 10) | (8 << 16) | (9 << 22) | ((10 & 0xF) << 28)
    w2 = (10 >> 4) | (11 << 2) | (12 << 8) | (13 << 14) | (14 << 20) | (15 << 26)
    codes = np.arange(16, dtype=np.uint8)[None, :]  # 16 codes = 96 bits = 3 words
    got = O.pack_bitwise(codes, 6)
    assert got[0].tolist() == [w0, w1, w2]
    assert O.pack_words(codes, 6)[0].tolist() == [w0, w1, w2]


def test_four_bit_known_answer(O):
    codes = np.arange(8, dtype=np.uint8)[None, :]
    assert O.pack_words(codes, 4)[0].tolist() == [0x76543210]
    assert O.pack_bitwise(codes, 4)[0].tolist() == [0x76543210]


def test_eight_and_two_bit_known_answers(O):
    assert O.pack_words(np.array([[0x11, 0x22, 0x33, 0x44]], np.uint8), 8)[0].tolist() == [0x44332211]
    codes = np.array([[1, 2, 3, 0] * 4], np.uint8)  # 2-bit: 0b00111001 per byte
    assert O.pack_words(codes, 2)[0].tolist() == [0x39393939]


def reference_unpack_4bit(words, out_dim, in_dim, group_size):
    """`H3Common.swift:386-398`: words [out, groups, gs/8, 1] >> (j*4) & 0xF."""
    groups = in_dim // group_size
    npw = 32 // 4
    w = words.reshape(out_dim, groups, group_size // npw, 1).astype(np.uint32)
    shifts = (np.arange(npw, dtype=np.uint32) * 4).reshape(1, 1, 1, npw)
    nib = (w >> shifts) & 0xF
    return nib.reshape(out_dim, in_dim)


def test_unpack_agrees_with_reference_4bit_unpacker(O):
    rng = np.random.default_rng(5)
    words = rng.integers(0, 2**32, size=(6, 64), dtype=np.uint64).astype(np.uint32)
    ref = reference_unpack_4bit(words, 6, 512, 64)
    assert np.array_equal(O.unpack(words, 512, 4), ref)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_pack_roundtrip_random(O, bits):
    rng = np.random.default_rng(bits)
    for N, K in [(1, 32), (5, 96), (3, 640)]:
        codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
        wq = O.pack_words(codes, bits)
        assert np.array_equal(wq, O.pack_bitwise(codes, bits))
        assert np.array_equal(O.unpack(wq, K, bits), codes)


def test_pack_rejects_bad_widths(O):
    with pytest.raises(ValueError):
        O.pack_words(np.zeros((1, 32), np.uint8), 7)
    with pytest.raises(ValueError):
        O.pack_words(np.zeros((1, 10), np.uint8), 6)


# ---------------------------------------------------------------- quantizer
def test_quantize_matches_golden(O, golden):
    for c in golden["quantize"]:
        w = np.array(c["w"], dtype=np.float32).reshape(c["N"], c["K"])
        q = O.quantize(w, c["gs"], c["bits"], mode=0)
        assert q["codes"].ravel().tolist() == c["codes"], (c["kind"], c["bits"], c["gs"])
        assert q["scales_bf16"].ravel().tolist() == c["scales_bf16"]
        assert q["biases_bf16"].ravel().tolist() == c["biases_bf16"]
        assert q["scales_f32"].ravel().tolist() == [np.float32(v) for v in c["scales_f32"]]
        assert q["biases_f32"].ravel().tolist() == [np.float32(v) for v in c["biases_f32"]]
        codes = np.array(c["codes"], np.uint8).reshape(c["N"], c["K"])
        assert np.array_equal(q["wq"], O.pack_bitwise(codes, c["bits"]))


def test_quantize_degenerate_group(O):
    w = np.full((1, 64), 0.25, np.float32)
    q = O.quantize(w, 64, 4, mode=0)
    assert not q["codes"].any()
    assert q["biases_f32"][0, 0] == np.float32(0.25)
    assert q["scales_f32"][0, 0] == np.float32(1e-7)


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
def test_quantize_error_bound_minmax(O, bits):
    w = O.normal_f32(99, 8 * 256, 0, 0.02).reshape(8, 256)
    q = O.quantize(w, 64, bits, mode=0)
    s = np.repeat(q["scales_f32"], 64, axis=1).astype(np.float64)
    b = np.repeat(q["biases_f32"], 64, axis=1).astype(np.float64)
    what = q["codes"] * s + b
    assert np.all(np.abs(w - what) <= s / 2 * (1 + 1e-5) + 1e-9)
    assert q["codes"].max() == (1 << bits) - 1 and q["codes"].min() == 0


@pytest.mark.parametrize("bits", [3, 4, 6, 8])
def test_quantize_edge_mode_invariants(O, bits):
    """mlx edge mode is recalled, not imported: only invariants are checked."""
    w = O.normal_f32(123, 16 * 128, 0.003, 0.02).reshape(16, 128)
    q = O.quantize(w, 64, bits, mode=1)
    n = (1 << bits) - 1
    assert q["codes"].max() <= n
    s = np.repeat(q["scales_f32"], 64, axis=1).astype(np.float64)
    b = np.repeat(q["biases_f32"], 64, axis=1).astype(np.float64)
    what = q["codes"] * s + b
    err = np.abs(w - what)
    unclipped = (q["codes"] > 0) & (q["codes"] < n)
    assert np.all(err[unclipped] <= np.abs(s[unclipped]) / 2 * (1 + 1e-4) + 1e-9)
    # the larger-magnitude extreme of each group is the edge: code 0, exact
    for r in range(16):
        for g in range(2):
            grp = w[r, g * 64:(g + 1) * 64]
            mn, mx = grp.min(), grp.max()
            edge_i = int(np.argmin(grp)) if abs(mn) > abs(mx) else int(np.argmax(grp))
            assert q["codes"][r, g * 64 + edge_i] == 0
            assert q["biases_f32"][r, g] in (np.float32(grp[edge_i]), np.float32(0))


# ---------------------------------------------------------------- dequant
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_dequantize_exact_closed_form(O, bits):
    w = O.normal_f32(7 + bits, 4 * 128, 0, 0.02).reshape(4, 128)
    q = O.quantize(w, 32, bits)
    f, bf = O.dequantize(q["wq"], q["scales_bf16"], q["biases_bf16"], 128, 32, bits)
    s = np.repeat(f64_of_bf16(q["scales_bf16"]), 32, axis=1)
    b = np.repeat(f64_of_bf16(q["biases_bf16"]), 32, axis=1)
    exact = q["codes"].astype(np.float64) * s + b  # exact in fp64
    assert np.array_equal(f, exact.astype(np.float32))  # one rounding == fmaf
    assert np.array_equal(bf, O.bf16_rne(exact.astype(np.float32)))


# ---------------------------------------------------------------- matmul
def _golden_qmm_args(c):
    N, K, M, gs = c["N"], c["K"], c["M"], c["gs"]
    wq = np.array(c["words"], np.uint32).reshape(N, K * c["bits"] // 32)
    s = np.array(c["scales_bf16"], np.uint16).reshape(N, K // gs)
    b = np.array(c["biases_bf16"], np.uint16).reshape(N, K // gs)
    x = np.array(c["x_bf16"], np.uint16).reshape(M, K)
    bias = None if c["bias_bf16"] is None else np.array(c["bias_bf16"], np.uint16)
    y = np.array(c["y_f64"]).reshape(M, N)
    return x, wq, s, b, bias, y


def test_qmm_f64_matches_numpy_golden(O, golden):
    for c in golden["qmm"]:
        x, wq, s, b, bias, y = _golden_qmm_args(c)
        got = O.qmm_f64(x, wq, s, b, c["gs"], c["bits"], bias=bias)
        assert np.allclose(got, y, rtol=1e-12, atol=1e-12), (c["bits"], c["gs"])
        # packed words in the golden are the big-integer stream of the codes
        codes = np.array(c["codes"], np.uint8).reshape(c["N"], c["K"])
        assert np.array_equal(O.pack_words(codes, c["bits"]), wq)


def test_qmm_row_subset(O, golden):
    c = golden["qmm"][2]
    x, wq, s, b, bias, y = _golden_qmm_args(c)
    got = O.qmm_f64(x, wq, s, b, c["gs"], c["bits"], bias=bias, rows=[4, 0, 2])
    assert np.allclose(got, y[[4, 0, 2]], rtol=1e-12, atol=1e-12)


def test_qmm_unit_scale_zero_bias_is_integer_gemm(O):
    rng = np.random.default_rng(3)
    M, N, K, gs, bits = 4, 6, 192, 64, 6
    codes = rng.integers(0, 64, size=(N, K), dtype=np.uint8)
    wq = O.pack_bitwise(codes, bits)
    s = np.full((N, K // gs), 0x3F80, np.uint16)  # 1.0
    b = np.zeros((N, K // gs), np.uint16)          # 0.0
    x = O.normal_bf16(17, M * K).reshape(M, K)
    y = O.qmm_f64(x, wq, s, b, gs, bits)
    ref = f64_of_bf16(x) @ codes.astype(np.float64).T
    assert np.array_equal(y, ref) or np.allclose(y, ref, rtol=1e-15, atol=0)
    y2 = O.qmm_f64_bf16w(x, wq, s, b, gs, bits)  # integer weights <= 63 are bf16-exact
    assert np.allclose(y2, ref, rtol=1e-15, atol=0)


def test_qmm_bias_only_is_group_row_sums(O):
    M, N, K, gs, bits = 3, 5, 256, 64, 4
    wq = np.zeros((N, K * bits // 32), np.uint32)  # all codes 0
    rng = np.random.default_rng(8)
    s = O.bf16_rne(rng.uniform(0.001, 0.01, size=(N, K // gs)).astype(np.float32))
    b = O.bf16_rne(rng.uniform(-0.1, 0.1, size=(N, K // gs)).astype(np.float32))
    x = O.normal_bf16(19, M * K).reshape(M, K)
    y = O.qmm_f64(x, wq, s, b, gs, bits)
    xs = f64_of_bf16(x).reshape(M, K // gs, gs).sum(axis=2)  # [M, G]
    ref = xs @ f64_of_bf16(b).T
    assert np.allclose(y, ref, rtol=1e-13, atol=1e-13)


def test_mlx_cpu_restatement_close_to_exact(O):
    M, N, K, gs, bits = 2, 64, 512, 64, 6
    w = O.normal_f32(5, N * K, 0, 0.02).reshape(N, K)
    q = O.quantize(w, gs, bits)
    x = O.normal_bf16(6, M * K).reshape(M, K)
    ref = O.qmm_f64(x, q["wq"], q["scales_bf16"], q["biases_bf16"], gs, bits)
    f32acc = O.bf16_to_f32(O.qmm_mlx_cpu(x, q["wq"], q["scales_bf16"], q["biases_bf16"], gs,
                                        bits, accum=1))
    bfacc = O.bf16_to_f32(O.qmm_mlx_cpu(x, q["wq"], q["scales_bf16"], q["biases_bf16"], gs,
                                       bits, accum=0, threads=4))
    scale = np.abs(ref).max()
    assert np.abs(f32acc - ref).max() / scale < 1e-2
    assert np.abs(bfacc - ref).max() / scale < 5e-2  # bf16 accumulation is noisy
    # bf16w reference is within bf16 weight rounding of the exact one
    r2 = O.qmm_f64_bf16w(x, q["wq"], q["scales_bf16"], q["biases_bf16"], gs, bits)
    assert np.abs(r2 - ref).max() / scale < 5e-3


def _one_row(O, codes, s_bf16, b_bf16, x_bf16, gs, bits):
    K = len(codes)
    wq = O.pack_words(np.array(codes, np.uint8).reshape(1, K), bits)
    s = np.full((1, K // gs), s_bf16, np.uint16)
    b = np.full((1, K // gs), b_bf16, np.uint16)
    x = np.array(x_bf16, np.uint16).reshape(1, K)
    return [int(O.qmm_mlx_cpu(x, wq, s, b, gs, bits, accum=a)[0, 0]) for a in (0, 1)]


def test_mlx_cpu_restatement_accumulates_in_bf16(O):
    """x = 1, s = 1, b = 0, q = 1, K = 512: a bf16 running sum reaches 256 and stays
    there (256 + 1 is a tie between 256 and 258 and rounds to the even 256); an fp32
    sum reaches 512. An fp32-accumulating restatement fails the first assertion."""
    one = 0x3F80
    bf, f32 = _one_row(O, [1] * 512, one, 0, [one] * 512, 64, 6)
    assert bf == 0x4380  # 256.0
    assert f32 == 0x4400  # 512.0


def test_mlx_cpu_restatement_rounds_scale_times_code_first(O):
    """w = bf16(bf16(s * q) + b): with s = 1 + 2^-7, q = 3, b = -3, s*q = 3.0234375 is a
    tie that rounds to 3.03125, so w = 0.03125; one rounding of s*q + b gives
    0.0234375 (exact in bf16). x = [1, 0, 0, ...] picks w_0 as the output."""
    codes = [3] + [0] * 63
    x = [0x3F80] + [0] * 63
    bf, f32 = _one_row(O, codes, 0x3F81, 0xC040, x, 64, 6)
    assert bf == 0x3D00  # 0.03125
    assert f32 == 0x3CC0  # 0.0234375


def test_gelu_tanh_closed_form(O):
    xs = np.array([0.0, 1.0, -1.0, 3.0, -3.0], np.float32)
    got = O.bf16_to_f32(O.gelu_tanh_bf16(O.bf16_rne(xs)))
    c = math.sqrt(2 / math.pi)
    ref = [0.5 * v * (1 + math.tanh(c * (v + 0.044715 * v ** 3))) for v in xs]
    assert np.allclose(got, ref, rtol=2 ** -8, atol=1e-6)
    assert got[0] == 0.0


# ---------------------------------------------------------------- planted mistakes
def test_checks_catch_msb_first_unpacking(O, golden):
    """The MSB-first order of `模型加载-通用.swift:256-266` must fail the goldens."""
    case = next(c for c in golden["pack"] if c["bits"] == 4 and c["kind"] == "random")
    words = np.array(case["words"], np.uint32)
    msb = np.stack([(words >> (32 - 4 - 4 * j)) & 0xF for j in range(8)], axis=-1)
    msb = msb.reshape(words.shape[0], -1)
    assert not np.array_equal(msb, np.array(case["codes"]))


def test_checks_catch_swapped_scales_biases(O, golden):
    c = golden["qmm"][0]
    x, wq, s, b, bias, y = _golden_qmm_args(c)
    bad = O.qmm_f64(x, wq, b, s, c["gs"], c["bits"], bias=bias)
    assert not np.allclose(bad, y, rtol=1e-3)


def test_checks_catch_off_by_one_group(O, golden):
    c = golden["qmm"][1]
    x, wq, s, b, bias, y = _golden_qmm_args(c)
    s_shift = np.roll(s, 1, axis=1)
    bad = O.qmm_f64(x, wq, s_shift, b, c["gs"], c["bits"], bias=bias)
    assert not np.allclose(bad, y, rtol=1e-3)
