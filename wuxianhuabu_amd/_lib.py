"""ctypes binding of libmxq.so (the C ABI in include/mxq.h).

The HIP library is the only implementation: if libmxq.so is missing or does not
load, every operation raises; there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmxq.so")

MXQ_OK = 0
MXQ_ERR_INVALID = -1
MXQ_ERR_UNSUPPORTED = -2
MXQ_ERR_ALIGNMENT = -3
MXQ_ERR_NULL = -4
MXQ_ERR_HIP = -5

MXQ_FLOAT32 = 0
MXQ_BFLOAT16 = 1
MXQ_MODE_MINMAX = 0
MXQ_MODE_MLX_EDGE = 1
MXQ_QMV_MAX_M = 32
MXQ_ACT_NONE = 0
MXQ_ACT_GELU_TANH = 1
MXQ_ACT_SWIGLU = 2
ABI_VERSION = 1
MXQ_NOALLOC_SCRATCH_BYTES = 64 << 20

# every symbol include/mxq.h declares, with (restype, argtypes)
_i64, _int, _vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
SIGNATURES = {
    "mxq_quantize": (_int, [_vp, _int, _i64, _i64, _int, _int, _int, _vp, _vp, _vp, _int, _vp]),
    "mxq_dequantize": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _int, _int, _vp, _int, _vp]),
    "mxq_pack": (_int, [_vp, _i64, _i64, _int, _vp, _vp]),
    "mxq_unpack": (_int, [_vp, _i64, _i64, _int, _vp, _vp]),
    "mxq_quantized_matmul": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _int, _int, _int,
                                    _vp, _vp, _vp]),
    "mxq_quantized_matmul_workspace_size": (_i64, [_i64, _i64, _i64, _int, _int]),
    "mxq_quantized_matmul_ws": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _int, _int, _int,
                                       _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "mxq_quantized_matmul_noalloc": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _int, _int,
                                            _int, _vp, _vp, _vp]),
    "mxq_qmm": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _int, _int, _vp, _vp, _vp]),
    "mxq_qmv": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _int, _int, _vp, _vp, _vp]),
    "mxq_tiled_bytes": (_i64, [_i64, _i64, _int, _int]),
    "mxq_tile": (_int, [_vp, _vp, _vp, _i64, _i64, _int, _int, _vp, _vp]),
    "mxq_tile_swiglu": (_int, [_vp, _vp, _vp, _i64, _i64, _int, _int, _vp, _vp]),
    "mxq_untile": (_int, [_vp, _i64, _i64, _int, _int, _vp, _vp, _vp, _vp]),
    "mxq_untile_swiglu": (_int, [_vp, _i64, _i64, _int, _int, _vp, _vp, _vp, _vp]),
    "mxq_stream_create": (_int, [_vp]),
    "mxq_stream_destroy": (_int, [_vp]),
    "mxq_malloc": (_int, [_vp, ctypes.c_size_t]),
    "mxq_free": (_int, [_vp]),
    "mxq_copy_to_device": (_int, [_vp, _vp, ctypes.c_size_t, _vp]),
    "mxq_copy_to_host": (_int, [_vp, _vp, ctypes.c_size_t, _vp]),
    "mxq_norm_modscale": (_int, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, ctypes.c_float,
                                 _vp, _vp]),
    "mxq_mod_gate": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "mxq_rmsnorm_rope": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _int, _int,
                                ctypes.c_float, _vp, _vp]),
    "mxq_st_open": (_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "mxq_st_close": (None, [_vp]),
    "mxq_st_count": (_i64, [_vp]),
    "mxq_st_key": (ctypes.c_char_p, [_vp, _i64]),
    "mxq_st_info": (_int, [_vp, ctypes.c_char_p, _vp, ctypes.POINTER(_int), _vp,
                           ctypes.POINTER(_i64)]),
    "mxq_st_read_host": (_int, [_vp, ctypes.c_char_p, _vp]),
    "mxq_st_read": (_int, [_vp, ctypes.c_char_p, _vp, _vp]),
    "mxq_quantized_matmul_tiled": (_int, [_vp, _i64, _i64, _vp, _i64, _int, _int, _vp, _vp,
                                          _vp]),
    "mxq_qmm_tiled": (_int, [_vp, _i64, _i64, _vp, _i64, _int, _int, _vp, _vp, _vp]),
    "mxq_qmm_tiled_act": (_int, [_vp, _i64, _i64, _vp, _i64, _int, _int, _vp, _int, _vp, _vp]),
    "mxq_qmm_tiled_lora": (_int, [_vp, _i64, _i64, _vp, _i64, _int, _int, _vp, _int, _vp, _vp,
                                  _i64, _vp, _vp]),
    "mxq_qmv_tiled": (_int, [_vp, _i64, _i64, _vp, _i64, _int, _int, _vp, _vp, _vp]),
    "mxq_last_error": (ctypes.c_char_p, []),
    "mxq_status_string": (ctypes.c_char_p, [_int]),
    "mxq_stream_synchronize": (_int, [_vp]),
    "mxq_abi_version": (_int, []),
}

_lib = None


class MXQError(RuntimeError):
    """A HIP runtime failure reported by libmxq (MXQ_ERR_HIP)."""

    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


def lib():
    """Load libmxq.so once. Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m wuxianhuabu_amd.build` "
            "(there is no fallback implementation)")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    if L.mxq_abi_version() != ABI_VERSION:
        raise RuntimeError("libmxq ABI version mismatch: rebuild the library")
    _lib = L
    return L


def check(status):
    """Turn a libmxq status into the exception mlx would raise."""
    if status == MXQ_OK:
        return
    msg = lib().mxq_last_error().decode("utf-8", "replace")
    if status in (MXQ_ERR_INVALID, MXQ_ERR_ALIGNMENT, MXQ_ERR_NULL):
        raise ValueError(msg)
    if status == MXQ_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise MXQError(status, msg)
