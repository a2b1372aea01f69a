"""ctypes binding of the CPU oracle (oracle/libmxq_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product (wuxianhuabu_amd)
never imports this module.
"""
import ctypes
import os
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmxq_oracle.so")

_lib = None

_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    _lib = _bind(ctypes.CDLL(LIB_PATH))
    return _lib


_native = None
NATIVE_FLAGS = ["-O3", "-march=native", "-fopenmp", "-fPIC", "-std=c11"]


def native_lib():
    """The oracle compiled for the CPU this process runs on (gcc with NATIVE_FLAGS, into
    a temporary directory), for the CPU baseline's timing; None where gcc is missing or
    the build fails (the caller then times the prebuilt x86-64-v3 library)."""
    global _native
    if _native is None:
        try:
            out = os.path.join(tempfile.mkdtemp(prefix="mxq_oracle_native_"),
                               "libmxq_oracle_native.so")
            subprocess.run(["gcc", *NATIVE_FLAGS, "-shared", "-o", out,
                            os.path.join(HERE, "mxq_oracle.c"), "-lm"],
                           check=True, capture_output=True, timeout=120)
            _native = _bind(ctypes.CDLL(out))
        except (OSError, subprocess.SubprocessError):
            _native = False
    return _native or None


def _bind(L):
    L.orc_version.restype = _int
    L.orc_splitmix64_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    L.orc_splitmix64_next.restype = ctypes.c_uint64
    L.orc_normal_f32.argtypes = [ctypes.c_uint64, _i64, ctypes.c_double, ctypes.c_double, _f32p]
    L.orc_normal_bf16.argtypes = [ctypes.c_uint64, _i64, ctypes.c_double, ctypes.c_double, _u16p]
    L.orc_bf16_rne.argtypes = [ctypes.c_float]
    L.orc_bf16_rne.restype = ctypes.c_uint16
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_bf16_to_f32.restype = ctypes.c_float
    L.orc_bf16_to_f32_n.argtypes = [_u16p, _i64, _f32p]
    L.orc_f32_to_bf16_n.argtypes = [_f32p, _i64, _u16p]
    for name in ("orc_pack_bitwise", "orc_pack_words"):
        getattr(L, name).argtypes = [_u8p, _i64, _i64, _int, _u32p]
        getattr(L, name).restype = _int
    L.orc_unpack.argtypes = [_u32p, _i64, _i64, _int, _u8p]
    L.orc_unpack.restype = _int
    L.orc_quantize.argtypes = [_f32p, _i64, _i64, _int, _int, _int, _u8p, _u32p, _u16p, _u16p,
                               _f32p, _f32p]
    L.orc_quantize.restype = _int
    L.orc_dequantize.argtypes = [_u32p, _u16p, _u16p, _i64, _i64, _int, _int, _f32p, _u16p]
    L.orc_dequantize.restype = _int
    for name in ("orc_qmm_f64", "orc_qmm_f64_bf16w"):
        getattr(L, name).argtypes = [_u16p, _i64, _i64, _u32p, _u16p, _u16p, _i64, _int, _int,
                                     _vp, _vp, _i64, _int, _f64p]
        getattr(L, name).restype = _int
    L.orc_qmm_mlx_cpu.argtypes = [_u16p, _i64, _i64, _u32p, _u16p, _u16p, _i64, _int, _int,
                                  _int, _vp, _i64, _int, _u16p]
    L.orc_qmm_mlx_cpu.restype = _int
    L.orc_gelu_tanh_bf16.argtypes = [_u16p, _i64, _u16p]
    L.orc_tiled_bytes.argtypes = [_i64, _i64, _int, _int]
    L.orc_tiled_bytes.restype = _i64
    L.orc_tile.argtypes = [_u32p, _u16p, _u16p, _i64, _i64, _int, _int, _u8p]
    L.orc_tile.restype = _int
    return L


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments")


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- generator / bf16 ------------------------------------------------------
def normal_f32(seed, n, mean=0.0, std=1.0):
    out = np.empty(int(n), np.float32)
    lib().orc_normal_f32(seed, n, mean, std, out)
    return out


def normal_bf16(seed, n, mean=0.0, std=1.0):
    out = np.empty(int(n), np.uint16)
    lib().orc_normal_bf16(seed, n, mean, std, out)
    return out


def bf16_rne(a):
    a = _c(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_to_bf16_n(a.reshape(-1), a.size, out.reshape(-1))
    return out


def bf16_to_f32(a):
    a = _c(a, np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().orc_bf16_to_f32_n(a.reshape(-1), a.size, out.reshape(-1))
    return out


# ---- layout ----------------------------------------------------------------
def pack_bitwise(codes, bits):
    codes = _c(codes, np.uint8)
    N, K = codes.shape
    wq = np.empty((N, K * bits // 32), np.uint32)
    _check(lib().orc_pack_bitwise(codes, N, K, bits, wq), "pack_bitwise")
    return wq


def pack_words(codes, bits):
    codes = _c(codes, np.uint8)
    N, K = codes.shape
    wq = np.empty((N, K * bits // 32), np.uint32)
    _check(lib().orc_pack_words(codes, N, K, bits, wq), "pack_words")
    return wq


def unpack(wq, K, bits):
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    codes = np.empty((N, K), np.uint8)
    _check(lib().orc_unpack(wq, N, K, bits, codes), "unpack")
    return codes


def tiled_bytes(N, K, gs, bits):
    return int(lib().orc_tiled_bytes(N, K, gs, bits))


def tile(wq, scales, biases, K, gs, bits):
    """MLX-layout triple (bf16 bits for scales/biases) -> tiled bytes (uint8)."""
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    nbytes = tiled_bytes(N, K, gs, bits)
    _check(0 if nbytes >= 0 else -1, "tiled_bytes")
    out = np.empty(nbytes, np.uint8)
    _check(lib().orc_tile(wq, _c(scales, np.uint16), _c(biases, np.uint16), N, K, gs, bits,
                          out), "tile")
    return out


# ---- quantizer / dequant -----------------------------------------------------
def quantize(w, gs, bits, mode=0):
    w = _c(w, np.float32)
    N, K = w.shape
    G = K // gs
    out = {
        "codes": np.empty((N, K), np.uint8),
        "wq": np.empty((N, K * bits // 32), np.uint32),
        "scales_bf16": np.empty((N, G), np.uint16),
        "biases_bf16": np.empty((N, G), np.uint16),
        "scales_f32": np.empty((N, G), np.float32),
        "biases_f32": np.empty((N, G), np.float32),
    }
    _check(lib().orc_quantize(w, N, K, gs, bits, mode, out["codes"], out["wq"],
                              out["scales_bf16"], out["biases_bf16"], out["scales_f32"],
                              out["biases_f32"]), "quantize")
    return out


def dequantize(wq, scales, biases, K, gs, bits):
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    f = np.empty((N, K), np.float32)
    b = np.empty((N, K), np.uint16)
    _check(lib().orc_dequantize(wq, _c(scales, np.uint16), _c(biases, np.uint16), N, K, gs,
                                bits, f, b), "dequantize")
    return f, b


# ---- matmul references ---------------------------------------------------------
def _rows_arg(rows):
    if rows is None:
        return None, 0, None
    r = np.ascontiguousarray(rows, dtype=np.int64)
    return r.ctypes.data_as(ctypes.c_void_p), len(r), r


def _qmm64(fn, x, wq, scales, biases, gs, bits, bias, rows, threads):
    x = _c(x, np.uint16)
    wq = _c(wq, np.uint32)
    M, K = x.shape
    N = wq.shape[0]
    rp, nr, keep = _rows_arg(rows)
    nrows = M if rows is None else nr
    y = np.empty((nrows, N), np.float64)
    bias_keep = None if bias is None else _c(bias, np.uint16)
    bp = None if bias_keep is None else bias_keep.ctypes.data_as(ctypes.c_void_p)
    _check(fn(x, M, K, wq, _c(scales, np.uint16), _c(biases, np.uint16), N, gs, bits, bp, rp,
              nr, threads, y), fn.__name__)
    del keep
    return y


def qmm_f64(x, wq, scales, biases, gs, bits, bias=None, rows=None, threads=8):
    return _qmm64(lib().orc_qmm_f64, x, wq, scales, biases, gs, bits, bias, rows, threads)


def qmm_f64_bf16w(x, wq, scales, biases, gs, bits, bias=None, rows=None, threads=8):
    return _qmm64(lib().orc_qmm_f64_bf16w, x, wq, scales, biases, gs, bits, bias, rows, threads)


def qmm_mlx_cpu(x, wq, scales, biases, gs, bits, accum=0, rows=None, threads=1, L=None):
    """L: the library to run (default the prebuilt oracle; native_lib() for timing)."""
    L = L or lib()
    x = _c(x, np.uint16)
    wq = _c(wq, np.uint32)
    M, K = x.shape
    N = wq.shape[0]
    rp, nr, keep = _rows_arg(rows)
    nrows = M if rows is None else nr
    y = np.empty((nrows, N), np.uint16)
    _check(L.orc_qmm_mlx_cpu(x, M, K, wq, _c(scales, np.uint16), _c(biases, np.uint16), N,
                             gs, bits, accum, rp, nr, threads, y), "qmm_mlx_cpu")
    del keep
    return y


def gelu_tanh_bf16(a):
    a = _c(a, np.uint16)
    out = np.empty(a.shape, np.uint16)
    lib().orc_gelu_tanh_bf16(a.reshape(-1), a.size, out.reshape(-1))
    return out


# ---------------------------------------------------------------- fused activations (fp64)
def gelu_tanh_f64(a):
    """0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))) in fp64: mlx's geluApproximate, applied
    to the LTX feed-forward's first projection (`model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:392-401`)."""
    v = np.asarray(a, np.float64)
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


def silu_f64(a):
    """v * sigmoid(v) in fp64."""
    v = np.asarray(a, np.float64)
    return v / (1.0 + np.exp(-v))


def swiglu_f64(y):
    """silu(gate) * up of a fused fc1 output y [..., 2F] whose halves are gate and up
    (`model/minimax h3/H3Transformer.swift:620-629`: splitEqual(y, 2, axis 1), silu(h0) * h1)."""
    y = np.asarray(y, np.float64)
    F = y.shape[-1] // 2
    return silu_f64(y[..., :F]) * y[..., F:]


def swiglu_rows(N):
    """Source row of each row of the paired tiling of an [N, K] gate/up weight (N even):
    row block rb holds rows 32rb.. of the gate half, then rows N/2 + 32rb.. of the up half;
    -1 marks the zero rows that pad a half past N/2."""
    F = N // 2
    nb = (F + 31) // 32
    rows = np.full(nb * 64, -1, np.int64)
    for rb in range(nb):
        for r in range(32):
            j = rb * 32 + r
            if j < F:
                rows[rb * 64 + r] = j
                rows[rb * 64 + 32 + r] = F + j
    return rows


def tile_swiglu(wq, scales, biases, K, gs, bits):
    """The paired tiling: tile() of the row-permuted triple (zero rows for the padding)."""
    wq, scales, biases = _c(wq, np.uint32), _c(scales, np.uint16), _c(biases, np.uint16)
    rows = swiglu_rows(wq.shape[0])
    pick = lambda a: np.where((rows >= 0)[:, None], a[np.maximum(rows, 0)], 0).astype(a.dtype)
    return tile(pick(wq), pick(scales), pick(biases), K, gs, bits)


# ---------------------------------------------------------------- H3 block row ops
def _f32_of(u16):
    return bf16_to_f32(np.asarray(u16, np.uint16))


def rmsnorm_bf16(x, w, eps):
    """rmsNormLast as the fused kernels evaluate it (`model/minimax h3/H3Common.swift:502-508`;
    `网络算子-融合-RMSNormRoPE-通用.swift:52-82`): fp32 mean of squares, rsqrt, x * rstd * w
    in fp32, rounded to bf16. x, w bf16 bits; returns float32 values of the bf16 result."""
    xf = _f32_of(x)
    wf = _f32_of(w)
    var = (xf.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    rstd = (1.0 / np.sqrt(var + eps)).astype(np.float32)
    return bf16_to_f32(bf16_rne((xf * rstd) * wf))


def norm_modscale_f64(x, w, shift, scale, row_map, eps):
    """fusedNormModscale before its last rounding (`网络算子-融合-RMSNormRoPE-通用.swift:132-167`):
    n * (scale[m] + 1) + shift[m] with n = rmsnorm_bf16."""
    n = rmsnorm_bf16(x, w, eps).astype(np.float64)
    m = np.zeros(n.shape[0], np.int64) if row_map is None else np.asarray(row_map, np.int64)
    return n * (_f32_of(scale)[m].astype(np.float64) + 1.0) + _f32_of(shift)[m]


def mod_gate_f64(x, other, gate, row_map):
    """fusedModGate before its rounding (:177-199): x + other * gate[m]."""
    m = np.zeros(np.asarray(x).shape[0], np.int64) if row_map is None else \
        np.asarray(row_map, np.int64)
    return _f32_of(x).astype(np.float64) + _f32_of(other).astype(np.float64) * _f32_of(gate)[m]


def rmsnorm_rope_f64(x, w, cos, sin, rot, eps):
    """fusedRmsnormRope before its last rounding (:41-110; applyRopePub, `H3Common.swift:555-569`):
    x [S, H, hd] bf16 bits, cos / sin [S, rot/2] float; pairs (j, j + rot/2) rotate, the tail
    passes through."""
    n = rmsnorm_bf16(x, w, eps).astype(np.float64)
    rh = rot // 2
    out = n.copy()
    c = np.asarray(cos, np.float64)[:, None, :]
    s = np.asarray(sin, np.float64)[:, None, :]
    x1, x2 = n[..., :rh], n[..., rh:rot]
    out[..., :rh] = x1 * c - x2 * s
    out[..., rh:rot] = x2 * c + x1 * s
    return out
