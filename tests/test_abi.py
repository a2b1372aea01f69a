"""C-ABI checks that need no GPU: the library loads, exports every symbol that
include/mxq.h declares, and rejects bad arguments on the host before any
launch (the error paths of mlx's quantize / quantized_matmul)."""
import ctypes
import os
import re
import subprocess

import pytest

from wuxianhuabu_amd import _lib, weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mxq.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mxq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_api():
    syms = declared_symbols()
    assert syms == sorted(_lib.SIGNATURES), syms


def test_library_exports_every_declared_symbol(mxq_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (mxq_\w+)", out))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing
    for s in declared_symbols():
        assert getattr(mxq_lib, s) is not None


def test_version_and_status_strings(mxq_lib):
    assert mxq_lib.mxq_abi_version() == _lib.ABI_VERSION
    assert mxq_lib.mxq_status_string(_lib.MXQ_ERR_INVALID) == b"MXQ_ERR_INVALID"
    assert mxq_lib.mxq_status_string(-99) == b"MXQ_ERR_UNKNOWN"


def _fake(addr=0x10000):
    return ctypes.c_void_p(addr)


def _qmm(L, M=16, K=256, N=64, gs=64, bits=4, transpose=1, x=_fake(), wq=_fake(),
         s=_fake(), b=_fake(), y=_fake(), bias=None):
    return L.mxq_quantized_matmul(x, M, K, wq, s, b, N, transpose, gs, bits, bias, y, None)


def test_matmul_rejects_bad_bits(mxq_lib):
    assert _qmm(mxq_lib, bits=7) == _lib.MXQ_ERR_INVALID
    assert b"number of bits 7" in mxq_lib.mxq_last_error()


def test_matmul_rejects_bad_group_size(mxq_lib):
    assert _qmm(mxq_lib, gs=16) == _lib.MXQ_ERR_INVALID
    assert b"group size 16" in mxq_lib.mxq_last_error()


def test_matmul_rejects_k_not_multiple_of_group(mxq_lib):
    assert _qmm(mxq_lib, K=96, gs=64) == _lib.MXQ_ERR_INVALID
    assert b"divisible" in mxq_lib.mxq_last_error()


def test_matmul_rejects_transpose_false(mxq_lib):
    assert _qmm(mxq_lib, transpose=0) == _lib.MXQ_ERR_UNSUPPORTED


def test_matmul_rejects_null_and_misaligned(mxq_lib):
    assert _qmm(mxq_lib, x=None) == _lib.MXQ_ERR_NULL
    assert _qmm(mxq_lib, M=1, y=None) == _lib.MXQ_ERR_NULL
    assert _qmm(mxq_lib, wq=_fake(0x10002)) == _lib.MXQ_ERR_ALIGNMENT
    assert _qmm(mxq_lib, M=2, x=_fake(0x10001)) == _lib.MXQ_ERR_ALIGNMENT


def test_matmul_empty_is_noop(mxq_lib):
    # no pointer is touched and no kernel is launched for M == 0 or N == 0
    assert _qmm(mxq_lib, M=0, x=None, y=None) == _lib.MXQ_OK
    assert _qmm(mxq_lib, N=0, x=None, y=None) == _lib.MXQ_OK


def test_matmul_caps_k(mxq_lib):
    # the kernels' 32-bit activation offsets (row * K * 2 for up to 256 rows) stay below
    # 2^31 only up to K = 2^22; above, every matmul entry point refuses before launching
    L = mxq_lib
    f = _fake()
    big, ok = (1 << 22) + 64, 1 << 22
    assert _qmm(L, K=big) == _lib.MXQ_ERR_INVALID
    assert b"2^22" in L.mxq_last_error()
    assert _qmm(L, K=ok, M=0) == _lib.MXQ_OK
    assert L.mxq_qmm(f, 16, big, f, f, f, 64, 64, 4, None, f, None) == _lib.MXQ_ERR_INVALID
    assert L.mxq_qmv(f, 2, big, f, f, f, 64, 64, 4, None, f, None) == _lib.MXQ_ERR_INVALID
    for fn in (L.mxq_qmm_tiled, L.mxq_qmv_tiled, L.mxq_quantized_matmul_tiled):
        assert fn(f, 2, big, f, 64, 64, 4, None, f, None) == _lib.MXQ_ERR_INVALID
        assert b"2^22" in L.mxq_last_error()
        assert fn(None, 0, ok, None, 64, 64, 4, None, None, None) == _lib.MXQ_OK


def test_qmv_rejects_large_m(mxq_lib):
    L = mxq_lib
    rc = L.mxq_qmv(_fake(), _lib.MXQ_QMV_MAX_M + 1, 256, _fake(), _fake(), _fake(), 64, 64, 4, None,
                   _fake(), None)
    assert rc == _lib.MXQ_ERR_INVALID


def test_quantize_and_dequantize_validation(mxq_lib):
    L = mxq_lib
    f = _fake()
    assert L.mxq_quantize(f, 0, 4, 96, 64, 4, 0, f, f, f, 0, None) == _lib.MXQ_ERR_INVALID
    assert L.mxq_quantize(f, 2, 4, 128, 64, 4, 0, f, f, f, 0, None) == _lib.MXQ_ERR_INVALID
    assert L.mxq_quantize(f, 0, 4, 128, 64, 4, 9, f, f, f, 0, None) == _lib.MXQ_ERR_INVALID
    assert L.mxq_quantize(None, 0, 4, 128, 64, 4, 0, f, f, f, 0, None) == _lib.MXQ_ERR_NULL
    assert L.mxq_quantize(None, 0, 0, 128, 64, 4, 0, None, None, None, 0, None) == _lib.MXQ_OK
    assert L.mxq_dequantize(f, f, f, 1, 4, 128, 48, 4, f, 1, None) == _lib.MXQ_ERR_INVALID
    assert L.mxq_pack(f, 1, 10, 6, f, None) == _lib.MXQ_ERR_INVALID
    assert L.mxq_unpack(f, 1, 32, 7, f, None) == _lib.MXQ_ERR_INVALID


def test_tiled_validation(mxq_lib):
    L = mxq_lib
    f = _fake()
    assert L.mxq_tiled_bytes(16384, 4096, 64, 6) == 256 * 64 * (512 * 6 + 256)
    assert L.mxq_tiled_bytes(100, 256, 32, 3) == 2 * 4 * (512 * 3 + 512)
    assert L.mxq_tiled_bytes(64, 96, 32, 4) == _lib.MXQ_ERR_INVALID   # K % 64
    assert b"multiple of 64" in L.mxq_last_error()
    assert L.mxq_tiled_bytes(64, 128, 64, 7) == _lib.MXQ_ERR_INVALID
    assert L.mxq_tile(None, f, f, 64, 128, 64, 4, f, None) == _lib.MXQ_ERR_NULL
    assert L.mxq_tile(None, None, None, 0, 128, 64, 4, None, None) == _lib.MXQ_OK
    for fn in (L.mxq_qmm_tiled, L.mxq_qmv_tiled, L.mxq_quantized_matmul_tiled):
        assert fn(f, 2, 96, f, 64, 32, 4, None, f, None) == _lib.MXQ_ERR_INVALID
        assert fn(f, 2, 128, f, 64, 64, 5 + 2, None, f, None) == _lib.MXQ_ERR_INVALID
        assert fn(f, 2, 128, None, 64, 64, 4, None, f, None) == _lib.MXQ_ERR_NULL
        assert fn(None, 0, 128, None, 64, 64, 4, None, None, None) == _lib.MXQ_OK
    # the tiled buffer must be 16-byte aligned (the kernels read it with b128 loads)
    odd = ctypes.c_void_p(f.value + 4)
    assert L.mxq_qmm_tiled(f, 2, 128, odd, 64, 64, 4, None, f, None) == _lib.MXQ_ERR_ALIGNMENT
    assert L.mxq_qmv_tiled(f, _lib.MXQ_QMV_MAX_M + 1, 128, f, 64, 64, 4, None, f,
                           None) == _lib.MXQ_ERR_INVALID


def test_errors_are_thread_local(mxq_lib):
    import threading
    assert _qmm(mxq_lib, bits=7) == _lib.MXQ_ERR_INVALID
    seen = []
    t = threading.Thread(target=lambda: seen.append(mxq_lib.mxq_last_error()))
    t.start()
    t.join()
    assert seen == [b""]
    assert b"bits 7" in mxq_lib.mxq_last_error()


def test_python_check_maps_errors(mxq_lib):
    _qmm(mxq_lib, bits=7)
    with pytest.raises(ValueError, match="bits 7"):
        _lib.check(_lib.MXQ_ERR_INVALID)
    _qmm(mxq_lib, transpose=0)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.MXQ_ERR_UNSUPPORTED)


# ---------------------------------------------------------------- host-side geometry
def test_get_quantized_accepts_both_key_spellings():
    a = {"p.weight": 1, "p.scales": 2, "p.biases": 3}
    assert weights.get_quantized(a, "p") == (1, 2, 3)
    b = {"p.weight": 1, "p.weight.scales": 2, "p.weight.biases": 3}
    assert weights.get_quantized(b, "p") == (1, 2, 3)
    assert weights.get_quantized({"p.weight": 1}, "p") is None
    assert weights.get_quantized({}, "p") is None


def test_infer_geometry():
    assert weights.infer_geometry(768, 64, 4096) == (6, 64)   # 6-bit H3 checkpoint
    assert weights.infer_geometry(512, 64, 4096) == (4, 64)   # 4-bit LTX / repack
    assert weights.infer_geometry(2048, 256, 16384) == (4, 64)
    with pytest.raises(ValueError):
        weights.infer_geometry(700, 64, 4096)
    with pytest.raises(ValueError):
        weights.infer_geometry(896, 64, 4096)  # 7 bits


def test_header_candidates_include_six_bit():
    # [N, 768] words with [N, 64] scales: 6-bit gs64 (K=4096) is one reading,
    # 3-bit gs128 (K=8192) the other; the reference helper (bits {2,4,8}) finds none
    assert weights.header_candidates(768, 64) == [(3, 128), (6, 64)]
    # the shape relation alone is ambiguous for 4-bit files
    assert weights.header_candidates(512, 64) == [(2, 128), (4, 64), (8, 32)]


def test_matmul_workspace_size(mxq_lib):
    """The workspace is the tiled copy of the weight, only where tiling pays off:
    M >= 1024 and K % 64 == 0 (every width; the results are bit-identical)."""
    L = mxq_lib
    ws = L.mxq_quantized_matmul_workspace_size
    assert ws(14400, 16384, 4096, 64, 6) == L.mxq_tiled_bytes(16384, 4096, 64, 6) > 0
    for bits in (2, 3, 4, 5, 8):
        assert ws(1024, 300, 640, 32, bits) == L.mxq_tiled_bytes(300, 640, 32, bits)
    assert ws(1023, 16384, 4096, 64, 6) == 0     # too few tokens
    assert ws(4096, 300, 96, 32, 6) == 0         # K not a multiple of 64
    assert ws(4096, 0, 640, 64, 4) == 0
    assert ws(4096, 300, 640, 64, 7) < 0         # unsupported width: an MXQ_ERR_* code
    assert ws(-1, 300, 640, 64, 4) < 0


def test_matmul_workspace_overlap_is_rejected(mxq_lib):
    """A workspace sharing bytes with an operand is refused before anything is
    launched (the pointers below are never dereferenced)."""
    L = mxq_lib
    M, N, K, gs, bits = 1024, 64, 128, 64, 4
    need = L.mxq_quantized_matmul_workspace_size(M, N, K, gs, bits)
    assert need > 0
    base = 1 << 40
    x, wq, sc, bi, bias, y = (base + i * (1 << 30) for i in range(6))
    cases = {
        "x": x + 64,                                # starts inside x
        "wq": wq - need + 4 * 16,                   # ends inside the codes
        "scales": sc, "biases": bi, "bias": bias,
        "y": y + M * N * 2 - 16,                    # starts in y's last 16 bytes
    }
    for name, ws in cases.items():
        rc = L.mxq_quantized_matmul_ws(x, M, K, wq, sc, bi, N, 1, gs, bits, bias, y, ws, need,
                                       None)
        assert rc == _lib.MXQ_ERR_INVALID, name
        assert b"overlaps" in L.mxq_last_error(), name
