"""CPU checks of the oracle's tiled-layout writer (orc_tile).

The tiled layout is this library's own load-time format, so there is no
reference vector for it: the writer is pinned by reading every code word and
scale/bias back through an independent reshape-based reader, and by the size
formula computed by hand."""
import numpy as np
import pytest

from tests.tiled_util import padded, untile

BITS = [2, 3, 4, 5, 6, 8]
GS = [32, 64, 128]


def _triple(O, N, K, gs, bits, seed):
    w = O.normal_f32(seed, N * K).reshape(N, K)
    q = O.quantize(w, gs, bits)
    return q["wq"], q["scales_bf16"], q["biases_bf16"]


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", GS)
def test_tile_round_trip(O, bits, gs):
    N, K = 100, 256  # ragged row block, four K steps
    wq, s, b = _triple(O, N, K, gs, bits, 11 + bits + gs)
    t = O.tile(wq, s, b, K, gs, bits)
    assert t.size == O.tiled_bytes(N, K, gs, bits)
    rwq, rs, rb = untile(t, N, K, gs, bits)
    np.testing.assert_array_equal(rwq, padded(wq, N))
    np.testing.assert_array_equal(rs, padded(s, N))
    np.testing.assert_array_equal(rb, padded(b, N))


@pytest.mark.parametrize("N,K,gs,bits,expect", [
    (64, 64, 64, 4, 64 * 4 * 8 + 256),          # one record
    (65, 128, 32, 6, 2 * 2 * (512 * 6 + 512)),  # two row blocks, two K steps
    (16384, 4096, 64, 6, 256 * 64 * (3072 + 256)),
    (1, 192, 128, 3, 3 * (1536 + 256)),
])
def test_tiled_bytes(O, N, K, gs, bits, expect):
    assert O.tiled_bytes(N, K, gs, bits) == expect


def test_tiled_bytes_rejects(O):
    assert O.tiled_bytes(64, 96, 32, 4) < 0   # K not a multiple of 64
    assert O.tiled_bytes(64, 64, 16, 4) < 0   # group size
    assert O.tiled_bytes(64, 64, 64, 7) < 0   # bits


def test_tile_code_positions(O):
    """A single set code bit lands at the documented byte: row 37 (half 1,
    r 5), code 100 (K step 1, code half 1, unit 37, index 4 in its run) of a
    6-bit weight: bit 24 of run word 0 -> plane 0, word 0 of unit 37."""
    N, K, bits, gs = 64, 128, 6, 64
    codes = np.zeros((N, K), np.uint8)
    codes[37, 100] = 1
    wq = O.pack_words(codes, bits)
    z = np.zeros((N, K // gs), np.uint16)
    t = O.tile(wq, z, z, K, gs, bits)
    rec = 512 * bits + 256
    off = 1 * rec + 1 * 256 * bits + 0 * 1024 + 37 * 16 + 0
    assert np.flatnonzero(t).tolist() == [off + 3]   # bit 24 = byte 3, bit 0
    assert t[off + 3] == 1


def test_tile_mistake_detected(O):
    """A plant: swapping the two code halves of a unit must fail the reader."""
    N, K, gs, bits = 64, 64, 64, 4
    wq, s, b = _triple(O, N, K, gs, bits, 5)
    t = O.tile(wq, s, b, K, gs, bits).copy()
    units = t[:1024].reshape(64, 16).copy()
    t[:1024] = np.concatenate([units[32:], units[:32]]).reshape(-1)
    rwq, _, _ = untile(t, N, K, gs, bits)
    assert not np.array_equal(rwq, wq)
