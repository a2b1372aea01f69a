"""Reader of the tiled weight layout written with array reshapes.

It shares no code with the oracle's bit-scatter writer (`orc_tile`) or with
the HIP tiler: it views the record bytes through the documented geometry and
returns the MLX-layout triple they hold, so `untile(tile(t)) == t` checks the
writer against an independent statement of the format.
"""
import numpy as np


def geometry(N, K, gs, bits):
    gps = 2 if gs == 32 else 1
    rec = 512 * bits + 256 * gps
    return (N + 63) // 64, K // 64, rec, gps


def untile(buf, N, K, gs, bits):
    """tiled bytes -> (wq uint32 [Npad, K*bits/32], scales, biases uint16 [Npad, K/gs]).

    Npad = 64 * ceil(N/64): padding rows come back too, so callers can check
    they are zero."""
    RB, nk, rec, gps = geometry(N, K, gs, bits)
    # records are step-major: record (rb, kk) at (kk * RB + rb) * rec
    T = np.asarray(buf, np.uint8).reshape(nk, RB, rec).transpose(1, 0, 2)
    FP, RW = bits // 4, bits % 4
    codes = T[:, :, :512 * bits].reshape(RB, nk, 2, 256 * bits)
    parts = []
    if FP:
        P = np.ascontiguousarray(codes[..., :FP * 1024]).view(np.uint32)
        P = P.reshape(RB, nk, 2, FP, 64, 4).transpose(0, 1, 2, 4, 3, 5)
        parts.append(P.reshape(RB, nk, 2, 64, 4 * FP))
    if RW:
        R = np.ascontiguousarray(codes[..., FP * 1024:]).view(np.uint32)
        parts.append(R.reshape(RB, nk, 2, 64, RW))
    words = np.concatenate(parts, axis=-1)  # [RB, nk, h, u, bits]
    words = words.reshape(RB, nk, 2, 2, 32, bits)  # u = r + 32 g -> (g, r)
    wq = words.transpose(0, 2, 4, 1, 3, 5).reshape(RB * 64, nk * 2 * bits)
    sb = np.ascontiguousarray(T[:, :, 512 * bits:]).view(np.uint32)
    sb = sb.reshape(RB, nk, 2, 32, gps).transpose(0, 2, 3, 1, 4).reshape(RB * 64, nk * gps)
    if gs == 128:
        # one dword per 64 codes; both K steps of a group must agree
        assert np.array_equal(sb[:, 0::2], sb[:, 1::2]), "gs=128 halves disagree"
        sb = sb[:, 0::2]
    return wq, (sb & 0xFFFF).astype(np.uint16), (sb >> 16).astype(np.uint16)


def padded(a, N):
    """a [N, ...] zero-padded to 64*ceil(N/64) rows."""
    Np = (N + 63) // 64 * 64
    out = np.zeros((Np,) + a.shape[1:], a.dtype)
    out[:N] = a
    return out
