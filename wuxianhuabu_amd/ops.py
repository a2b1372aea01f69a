"""The MLX-Swift quantization operators, over torch device tensors.

Same names, argument meaning and error behaviour as the functions the
reference calls through MLX-Swift:

    quantized(w, group_size=64, bits=4)            mlx `quantized(_:groupSize:bits:)`
        `model/minimax h3/tools/quantize_h3_g64.py:132` (mx.quantize),
        `Packages/z-image-swift/Sources/ZImage/Weights.swift:31`
    dequantized(w, scales, biases, group_size, bits)
        `model/minimax h3/H3Common.swift:382-401` (MfLinear.dequantizedWeight)
    quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits)
        `model/minimax h3/H3Common.swift:358-359` (quantizedMM),
        `model/3模块/ltx2.5专属/gemma4文本-(ltx专属).swift:306-312` (quantizedMatmul)

torch supplies device memory and the current HIP stream; all arithmetic runs in
libmxq.so (HIP, gfx950). Invalid arguments raise ValueError with mlx's wording.
"""
import ctypes

import torch

from . import _lib

_SB_DTYPES = {torch.float32: _lib.MXQ_FLOAT32, torch.bfloat16: _lib.MXQ_BFLOAT16}
_SUPPORTED_BITS = (2, 3, 4, 5, 6, 8)
_SUPPORTED_GS = (32, 64, 128)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _on_gpu(op, *tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"[{op}] all arrays must be on the GPU (got {t.device}).")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"[{op}] all arrays must be on the same device.")


def _dense(t):
    """Row-major copy of a strided view (mlx accepts any strides; the kernels
    read contiguous rows)."""
    return t if t is None or t.is_contiguous() else t.contiguous()


def _check_bits_gs(op, bits, group_size):
    if bits not in _SUPPORTED_BITS:
        raise ValueError(f"[{op}] The requested number of bits {bits} is not supported. "
                         "The supported bits are 2, 3, 4, 5, 6 and 8.")
    if group_size not in _SUPPORTED_GS:
        raise ValueError(f"[{op}] The requested group size {group_size} is not supported. "
                         "The supported group sizes are 32, 64, and 128.")


def _as_words(w):
    if w.dtype == torch.uint32:
        return w
    if w.dtype == torch.int32:
        return w.view(torch.uint32)
    raise ValueError(f"packed weights must be uint32 (got {w.dtype}).")


def quantized(w, group_size=64, bits=4, *, mode="mlx_edge", scales_dtype=None):
    """Quantize w [..., K] along its last axis -> (wq uint32, scales, biases).

    scales/biases have w's dtype (float32 or bfloat16; `scales_dtype` overrides)
    and shape [..., K/group_size]; wq has shape [..., K*bits/32]. Codes come
    from the fp32 scale and bias, which are then rounded to the stored dtype.
    mode "mlx_edge" (the default, as mlx's quantize): the sign-aware edge quantizer,
    the group's larger-magnitude extreme on code 0 exactly; mode "minmax":
    scale=(max-min)/(2^bits-1), bias=min (the recipe of the benchmark workloads).
    """
    _check_bits_gs("quantize", bits, group_size)
    if w.ndim < 2:
        raise ValueError(f"[quantize] The matrix to be quantized must have at least 2 "
                         f"dimensions but it has only {w.ndim}.")
    K = w.shape[-1]
    if K % group_size != 0:
        raise ValueError(f"[quantize] The last dimension of the matrix needs to be divisible "
                         f"by the quantization group size {group_size}. However the provided "
                         f"matrix has shape {tuple(w.shape)}")
    if w.dtype not in _SB_DTYPES:
        raise ValueError(f"[quantize] Only float32 and bfloat16 weights are supported "
                         f"(got {w.dtype}).")
    modes = {"minmax": _lib.MXQ_MODE_MINMAX, "mlx_edge": _lib.MXQ_MODE_MLX_EDGE}
    if mode not in modes:
        raise ValueError(f"[quantize] unknown mode {mode!r}")
    _on_gpu("quantize", w)
    w = _dense(w)
    lead = tuple(w.shape[:-1])
    rows = w.numel() // K if K else 0
    sdt = w.dtype if scales_dtype is None else scales_dtype
    if sdt not in _SB_DTYPES:
        raise ValueError(f"[quantize] scales must be float32 or bfloat16 (got {sdt}).")
    wq = torch.empty(lead + (K * bits // 32,), dtype=torch.uint32, device=w.device)
    scales = torch.empty(lead + (K // group_size,), dtype=sdt, device=w.device)
    biases = torch.empty_like(scales)
    _lib.check(_lib.lib().mxq_quantize(_ptr(w), _SB_DTYPES[w.dtype], rows, K, group_size, bits,
                                       modes[mode], _ptr(wq), _ptr(scales), _ptr(biases),
                                       _SB_DTYPES[sdt], _stream(w)))
    return wq, scales, biases


def dequantized(w, scales, biases, group_size=64, bits=4, *, dtype=None):
    """w = q*scale + bias -> [..., K] in scales' dtype (or `dtype`)."""
    _check_bits_gs("dequantize", bits, group_size)
    w = _as_words(w)
    _on_gpu("dequantize", w, scales, biases)
    w, scales, biases = _dense(w), _dense(scales), _dense(biases)
    K = w.shape[-1] * 32 // bits
    if w.shape[-1] * 32 % bits != 0:
        raise ValueError("[dequantize] The packed width is not a whole number of codes.")
    if scales.shape != biases.shape or tuple(scales.shape[:-1]) != tuple(w.shape[:-1]) or \
            scales.shape[-1] * group_size != K:
        raise ValueError(f"[dequantize] Shape of scales and biases does not match the matrix "
                         f"given the quantization parameters. Provided matrix of shape "
                         f"{tuple(w.shape)} and scales/biases of shape {tuple(scales.shape)} "
                         f"with group_size={group_size} and bits={bits}.")
    if scales.dtype not in _SB_DTYPES or biases.dtype != scales.dtype:
        raise ValueError("[dequantize] scales and biases must both be float32 or bfloat16.")
    out_dtype = scales.dtype if dtype is None else dtype
    if out_dtype not in _SB_DTYPES:
        raise ValueError("[dequantize] output dtype must be float32 or bfloat16.")
    rows = w.numel() // w.shape[-1] if w.shape[-1] else 0
    out = torch.empty(tuple(w.shape[:-1]) + (K,), dtype=out_dtype, device=w.device)
    _lib.check(_lib.lib().mxq_dequantize(_ptr(w), _ptr(scales), _ptr(biases),
                                         _SB_DTYPES[scales.dtype], rows, K, group_size, bits,
                                         _ptr(out), _SB_DTYPES[out_dtype], _stream(w)))
    return out


def _matmul_shapes(op, x, w, scales, biases, group_size, bits, bias):
    _check_bits_gs(op, bits, group_size)
    w = _as_words(w)
    _on_gpu(op, x, w, scales, biases, bias)
    if w.ndim != 2:
        raise ValueError(f"[{op}] The weight matrix must be 2-D (got {w.ndim}-D).")
    N = w.shape[0]
    K = x.shape[-1]
    if w.shape[1] * 32 != K * bits:
        raise ValueError(f"[{op}] The shapes of the weight and scales are incompatible "
                         f"based on bits and group_size. w.shape() == {tuple(w.shape)} and "
                         f"x.shape() == {tuple(x.shape)} with bits={bits}")
    if tuple(scales.shape) != (N, K // group_size) or scales.shape != biases.shape or \
            K % group_size != 0:
        raise ValueError(f"[{op}] The shapes of the weight and scales are incompatible "
                         f"based on bits and group_size. w.shape() == {tuple(w.shape)} and "
                         f"scales.shape() == {tuple(scales.shape)} with group_size="
                         f"{group_size} and bits={bits}")
    if x.dtype != torch.bfloat16 or scales.dtype != torch.bfloat16 or \
            biases.dtype != torch.bfloat16:
        raise ValueError(f"[{op}] x, scales and biases must be bfloat16 "
                         f"(got {x.dtype}, {scales.dtype}, {biases.dtype}).")
    if bias is not None and (bias.dtype != torch.bfloat16 or tuple(bias.shape) != (N,)):
        raise ValueError(f"[{op}] bias must be bfloat16 of shape ({N},).")
    return _dense(x), _dense(w), _dense(scales), _dense(biases), _dense(bias), N, K


def quantized_matmul(x, w, scales, biases, transpose=True, group_size=64, bits=4, *,
                     bias=None, path="auto"):
    """y [..., N] = x [..., K] @ dequantized(w)^T (+ bias), bf16 in/out, fp32 accumulate.

    path: "auto" (GEMV for M <= MXQ_QMV_MAX_M = 32, MFMA above), "qmm" or "qmv" to force a kernel.
    With "auto" and many tokens (mxq_quantized_matmul_workspace_size > 0) the weight is
    tiled into a temporary buffer first and the tiled MFMA kernel runs: the same
    result bits, in less time.
    """
    op = "quantized_matmul"
    x, w, scales, biases, bias, N, K = _matmul_shapes(op, x, w, scales, biases, group_size,
                                                      bits, bias)
    lead = tuple(x.shape[:-1])
    M = x.numel() // K if K else 0
    y = torch.empty(lead + (N,), dtype=torch.bfloat16, device=x.device)
    L = _lib.lib()
    args = (_ptr(x), M, K, _ptr(w), _ptr(scales), _ptr(biases), N)
    if path == "auto":
        ws_bytes = L.mxq_quantized_matmul_workspace_size(M, N, K, group_size, bits) \
            if transpose else 0
        ws = torch.empty(max(int(ws_bytes), 0), dtype=torch.uint8, device=x.device) \
            if ws_bytes > 0 else None
        rc = L.mxq_quantized_matmul_ws(*args, 1 if transpose else 0, group_size, bits,
                                       _ptr(bias), _ptr(y), _ptr(ws),
                                       0 if ws is None else ws.numel(), _stream(x))
    elif not transpose:
        raise NotImplementedError("[quantized_matmul] transpose=False is not implemented.")
    elif path == "qmm":
        rc = L.mxq_qmm(*args, group_size, bits, _ptr(bias), _ptr(y), _stream(x))
    elif path == "qmv":
        rc = L.mxq_qmv(*args, group_size, bits, _ptr(bias), _ptr(y), _stream(x))
    else:
        raise ValueError(f"unknown path {path!r}")
    _lib.check(rc)
    return y


class TiledWeight:
    """A packed weight reordered into the tiled load-time layout (uint8 device
    buffer) plus its geometry. Built once by `tile()`; read by `tiled_matmul`.
    Holds the same bits as the MLX triple, so results are identical."""

    __slots__ = ("data", "N", "K", "group_size", "bits", "swiglu")

    def __init__(self, data, N, K, group_size, bits, swiglu=False):
        self.data, self.N, self.K = data, int(N), int(K)
        self.group_size, self.bits = int(group_size), int(bits)
        # rows [gate; up] tiled in pairs (mxq_tile_swiglu): only activation="swiglu"
        self.swiglu = bool(swiglu)

    @property
    def device(self):
        return self.data.device

    @property
    def nbytes(self):
        return self.data.numel()


def tiled_supported(K, group_size, bits, scales_dtype=torch.bfloat16):
    """Whether `tile()` accepts this geometry (K % 64 == 0, bf16 scales)."""
    return (K > 0 and K % 64 == 0 and K % group_size == 0 and bits in _SUPPORTED_BITS and
            group_size in _SUPPORTED_GS and scales_dtype == torch.bfloat16)


def tile(w, scales, biases, group_size=64, bits=4, *, swiglu=False):
    """MLX-layout triple -> TiledWeight (one device pass, no requantization).

    swiglu=True: the weight's rows are [gate; up] (a fused fc1, N even) and are
    tiled in pairs for tiled_matmul(..., activation="swiglu")."""
    _check_bits_gs("tile", bits, group_size)
    w = _as_words(w)
    _on_gpu("tile", w, scales, biases)
    if w.ndim != 2:
        raise ValueError(f"[tile] The weight matrix must be 2-D (got {w.ndim}-D).")
    N, K = int(w.shape[0]), int(w.shape[1]) * 32 // bits
    if w.shape[1] * 32 % bits != 0 or tuple(scales.shape) != (N, K // group_size) or \
            scales.shape != biases.shape:
        raise ValueError(f"[tile] Shape of scales and biases does not match the matrix given "
                         f"the quantization parameters (w {tuple(w.shape)}, scales "
                         f"{tuple(scales.shape)}, group_size={group_size}, bits={bits}).")
    if scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
        raise ValueError("[tile] scales and biases must be bfloat16.")
    L = _lib.lib()
    nbytes = L.mxq_tiled_bytes(N, K, group_size, bits)
    if nbytes < 0:
        _lib.check(int(nbytes))
    w, scales, biases = _dense(w), _dense(scales), _dense(biases)
    data = torch.empty(int(nbytes), dtype=torch.uint8, device=w.device)
    fn = L.mxq_tile_swiglu if swiglu else L.mxq_tile
    _lib.check(fn(_ptr(w), _ptr(scales), _ptr(biases), N, K, group_size, bits, _ptr(data),
                  _stream(w)))
    return TiledWeight(data, N, K, group_size, bits, swiglu)


def untile(tw):
    """TiledWeight -> the MLX-layout triple (wq uint32 [N, K*bits/32], bf16 scales and
    biases [N, K/group_size]) holding the same bits as the triple it was tiled from
    (swiglu weights come back with their [gate; up] row order)."""
    if not isinstance(tw, TiledWeight):
        raise ValueError(f"[untile] expected a TiledWeight (got {type(tw).__name__}).")
    dev = tw.device
    wq = torch.empty((tw.N, tw.K * tw.bits // 32), dtype=torch.uint32, device=dev)
    scales = torch.empty((tw.N, tw.K // tw.group_size), dtype=torch.bfloat16, device=dev)
    biases = torch.empty_like(scales)
    L = _lib.lib()
    fn = L.mxq_untile_swiglu if tw.swiglu else L.mxq_untile
    _lib.check(fn(_ptr(tw.data), tw.N, tw.K, tw.group_size, tw.bits, _ptr(wq), _ptr(scales),
                  _ptr(biases), _stream(tw.data)))
    return wq, scales, biases


_ACTIVATIONS = {None: _lib.MXQ_ACT_NONE, "gelu_tanh": _lib.MXQ_ACT_GELU_TANH,
                "swiglu": _lib.MXQ_ACT_SWIGLU}


class LoraAdapters:
    """LoRA adapters of one linear layer, prepared for the fused kernel: the
    reference's LoraSlot of LoraRef(a [in, r], b [r, out], scale)
    (`model/minimax h3/H3Common.swift:405-434`), whose term is
    sum_i scale_i * (x a_i) b_i. Held as a_cat [in, R] = [a_1 | a_2 | ...] and
    bt [out, R] = [scale_1 b_1; scale_2 b_2; ...]^T in bf16, R padded with zeros
    to a multiple of 16."""

    __slots__ = ("a_cat", "bt", "R", "rank")

    def __init__(self, refs):
        refs = list(refs)
        if not refs:
            raise ValueError("[lora] no adapters given.")
        a0, b0, _ = refs[0]
        din, dout = int(a0.shape[0]), int(b0.shape[1])
        for a, b, _ in refs:
            if a.ndim != 2 or b.ndim != 2 or a.shape[0] != din or b.shape[1] != dout or \
                    a.shape[1] != b.shape[0]:
                raise ValueError("[lora] every adapter needs a [in, r] and b [r, out] with the "
                                 "same in and out.")
        self.rank = sum(int(a.shape[1]) for a, _, _ in refs)
        self.R = (self.rank + 15) // 16 * 16
        if self.R > 4096:
            raise ValueError(f"[lora] total rank {self.rank} above 4096.")
        dev = a0.device
        a_cat = torch.zeros(din, self.R, dtype=torch.bfloat16, device=dev)
        bt = torch.zeros(dout, self.R, dtype=torch.bfloat16, device=dev)
        o = 0
        for a, b, scale in refs:
            r = int(a.shape[1])
            a_cat[:, o:o + r] = a.to(torch.bfloat16)
            bt[:, o:o + r] = (b.float() * float(scale)).t().to(torch.bfloat16)
            o += r
        self.a_cat, self.bt = a_cat, bt

    def xa(self, x2d):
        """x [M, in] bf16 -> x a_cat [M, R] bf16 (a plain library GEMM)."""
        return torch.matmul(x2d, self.a_cat).contiguous()


def tiled_matmul(x, tw, *, bias=None, path="auto", activation=None, lora=None):
    """quantized_matmul(x, w, scales, biases, transpose=True, ...) on a TiledWeight.

    path: "auto" (GEMV for M <= MXQ_QMV_MAX_M = 32, MFMA above), "qmm" or "qmv".
    activation (fused into the MFMA kernel's epilogue, applied in fp32 before the
    one bf16 rounding; any M): None, "gelu_tanh" (geluApprox between the LTX
    feed-forward projections), or "swiglu" (silu(gate) * up of a weight tiled
    with swiglu=True; the output has N/2 columns).
    lora: LoraAdapters whose term is added to the MFMA kernel's accumulators
    before the bias, the activation and the rounding (any M)."""
    op = "quantized_matmul"
    if not isinstance(tw, TiledWeight):
        raise ValueError(f"[{op}] expected a TiledWeight (got {type(tw).__name__}).")
    if activation not in _ACTIVATIONS:
        raise ValueError(f"[{op}] unknown activation {activation!r}.")
    if (activation == "swiglu") != tw.swiglu:
        raise ValueError(f"[{op}] activation='swiglu' needs, and only accepts, a weight tiled "
                         f"with swiglu=True.")
    _on_gpu(op, x, tw.data, bias)
    if x.shape[-1] != tw.K:
        raise ValueError(f"[{op}] x.shape[-1] == {x.shape[-1]} does not match the weight's "
                         f"input dimension {tw.K}.")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"[{op}] x must be bfloat16 (got {x.dtype}).")
    if bias is not None and (bias.dtype != torch.bfloat16 or tuple(bias.shape) != (tw.N,)):
        raise ValueError(f"[{op}] bias must be bfloat16 of shape ({tw.N},).")
    x, bias = _dense(x), _dense(bias)
    M = x.numel() // tw.K
    n_out = tw.N // 2 if activation == "swiglu" else tw.N
    y = torch.empty(tuple(x.shape[:-1]) + (n_out,), dtype=torch.bfloat16, device=x.device)
    L = _lib.lib()
    if activation is not None or lora is not None:
        if path == "qmv":
            raise ValueError(f"[{op}] fused activations and LoRA run on the MFMA kernel "
                             f"(path 'qmm').")
        xa = bt = None
        R = 0
        if lora is not None:
            if not isinstance(lora, LoraAdapters):
                raise ValueError(f"[{op}] lora must be LoraAdapters.")
            if tuple(lora.a_cat.shape) != (tw.K, lora.R) or tuple(lora.bt.shape) != (tw.N, lora.R):
                raise ValueError(f"[{op}] LoRA shapes do not match the weight [{tw.N}, {tw.K}].")
            xa, bt, R = lora.xa(x.reshape(M, tw.K)), lora.bt, lora.R
        _lib.check(L.mxq_qmm_tiled_lora(_ptr(x), M, tw.K, _ptr(tw.data), tw.N, tw.group_size,
                                        tw.bits, _ptr(bias), _ACTIVATIONS[activation],
                                        _ptr(xa), _ptr(bt), R, _ptr(y), _stream(x)))
        return y
    fns = {"auto": "mxq_quantized_matmul_tiled", "qmm": "mxq_qmm_tiled",
           "qmv": "mxq_qmv_tiled"}
    if path not in fns:
        raise ValueError(f"unknown path {path!r}")
    fn = getattr(L, fns[path])
    _lib.check(fn(_ptr(x), M, tw.K, _ptr(tw.data), tw.N, tw.group_size, tw.bits, _ptr(bias),
                  _ptr(y), _stream(x)))
    return y


# camelCase aliases, as the Swift surface spells them
quantizedMatmul = quantized_matmul
quantizedMM = quantized_matmul


def pack(codes, bits):
    """codes uint8 [..., K] -> wq uint32 [..., K*bits/32] (MLX bitstream)."""
    if codes.dtype != torch.uint8:
        raise ValueError("[pack] codes must be uint8.")
    _on_gpu("pack", codes)
    codes = _dense(codes)
    K = codes.shape[-1]
    rows = codes.numel() // K if K else 0
    wq = torch.empty(tuple(codes.shape[:-1]) + (K * bits // 32,), dtype=torch.uint32,
                     device=codes.device)
    _lib.check(_lib.lib().mxq_pack(_ptr(codes), rows, K, bits, _ptr(wq), _stream(codes)))
    return wq


def unpack(w, bits):
    """wq uint32 [..., W] -> codes uint8 [..., W*32/bits]."""
    w = _dense(_as_words(w))
    _on_gpu("unpack", w)
    K = w.shape[-1] * 32 // bits
    rows = w.numel() // w.shape[-1] if w.shape[-1] else 0
    codes = torch.empty(tuple(w.shape[:-1]) + (K,), dtype=torch.uint8, device=w.device)
    _lib.check(_lib.lib().mxq_unpack(_ptr(w), rows, K, bits, _ptr(codes), _stream(w)))
    return codes
