"""Row-wise ops of the H3 DiT block that feed and consume its quantized linears, over
libmxq's kernels (mxq_norm_modscale, mxq_mod_gate, mxq_rmsnorm_rope), with the reference's
names and meanings (`model/2网络算子/网络算子-融合-RMSNormRoPE-通用.swift:41-343`):

    fused_norm_modscale(x, weight, shift, scale, row_map, eps)   rmsNormLast + modScaleShift
    fused_norm_modscale_row(x, weight, shift, scale, eps)        one modulation row
    fused_mod_gate(x, gate, other, row_map)                      x + other * gate[row]
    fused_rmsnorm_rope(x, weight, cos, sin, rot, eps)            rmsNormLast + applyRopePub
    build_row_mod_map(count, runs)                               plan.runs -> row map

x, weight, shift, scale, gate, other: bf16 on the GPU; cos / sin: fp32 or bf16.
"""
import ctypes

import torch

from . import _lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _bf16(op, **ts):
    for name, t in ts.items():
        if t.dtype != torch.bfloat16:
            raise ValueError(f"[{op}] {name} must be bfloat16 (got {t.dtype}).")
        if t.device.type != "cuda":
            raise ValueError(f"[{op}] {name} must be on the GPU.")


def build_row_mod_map(count, runs, device="cuda"):
    """`H3FusedKernels.buildRowModMap`: rows [start, end) of each run take its modRow
    (runs as (start, end, mod_row)); rows outside every run take 0."""
    m = torch.zeros(count, dtype=torch.int64)
    for start, end, mod_row in runs:
        s, e = max(0, min(count, int(start))), max(0, min(count, int(end)))
        if e > s:
            m[s:e] = int(mod_row)
    return m.to(torch.int32).to(device).view(torch.uint32)


def _map_arg(op, row_map, S):
    if row_map is None:
        return None
    if row_map.dtype not in (torch.uint32, torch.int32) or row_map.numel() != S:
        raise ValueError(f"[{op}] row_map must be uint32 of length {S}.")
    return row_map.contiguous()


def fused_norm_modscale(x, weight, shift, scale, row_map=None, eps=1e-5):
    """out = (rmsnorm(x) * weight) * (scale[m] + 1) + shift[m], x [S, hidden]."""
    op = "norm_modscale"
    _bf16(op, x=x, weight=weight, shift=shift, scale=scale)
    S, hidden = x.shape[0], x.shape[-1]
    if x.ndim != 2 or shift.ndim != 2 or shift.shape != scale.shape or \
            shift.shape[1] != hidden or weight.numel() != hidden:
        raise ValueError(f"[{op}] expected x [S, hidden], weight [hidden], shift/scale "
                         f"[rows, hidden] (got {tuple(x.shape)}, {tuple(weight.shape)}, "
                         f"{tuple(shift.shape)}, {tuple(scale.shape)}).")
    x, weight, shift, scale = (t.contiguous() for t in (x, weight, shift, scale))
    m = _map_arg(op, row_map, S)
    out = torch.empty_like(x)
    _lib.check(_lib.lib().mxq_norm_modscale(_ptr(x), S, hidden, _ptr(weight), _ptr(shift),
                                            _ptr(scale), shift.shape[0], _ptr(m),
                                            ctypes.c_float(eps), _ptr(out), _stream(x)))
    return out


def fused_norm_modscale_row(x, weight, shift, scale, eps=1e-5):
    """One modulation row for every token row (`fusedNormModscaleRow`, the final head)."""
    return fused_norm_modscale(x, weight, shift.reshape(1, -1), scale.reshape(1, -1), None,
                               eps)


def fused_mod_gate(x, gate, other, row_map=None):
    """out = x + other * gate[m], x and other [S, hidden], gate [rows, hidden]."""
    op = "mod_gate"
    _bf16(op, x=x, gate=gate, other=other)
    if x.shape != other.shape or x.ndim != 2 or gate.ndim != 2 or gate.shape[1] != x.shape[1]:
        raise ValueError(f"[{op}] expected x, other [S, hidden] and gate [rows, hidden].")
    S, hidden = x.shape
    x, gate, other = (t.contiguous() for t in (x, gate, other))
    m = _map_arg(op, row_map, S)
    out = torch.empty_like(x)
    _lib.check(_lib.lib().mxq_mod_gate(_ptr(x), _ptr(other), S, hidden, _ptr(gate),
                                       gate.shape[0], _ptr(m), _ptr(out), _stream(x)))
    return out


def fused_rmsnorm_rope(x, weight, cos, sin, rot, eps=1e-5):
    """x [1, S, H, hd] (or [S, H, hd]) -> same shape: rmsNormLast over hd, then the split-
    half rotary on dims [0, rot) with cos / sin [S, rot/2] (any leading 1s)."""
    op = "rmsnorm_rope"
    _bf16(op, x=x, weight=weight)
    shape = x.shape
    if x.ndim == 4:
        if shape[0] != 1:
            raise ValueError(f"[{op}] x must be [1, S, H, hd] (got {tuple(shape)}).")
        x3 = x.reshape(shape[1:])
    elif x.ndim == 3:
        x3 = x
    else:
        raise ValueError(f"[{op}] x must be [1, S, H, hd] or [S, H, hd].")
    S, H, hd = x3.shape
    rh = rot // 2
    c = cos.reshape(-1, rh) if rh else cos
    s = sin.reshape(-1, rh) if rh else sin
    if rh and (c.shape[0] != S or s.shape != c.shape or c.dtype != s.dtype):
        raise ValueError(f"[{op}] cos / sin must hold [S, rot/2] = [{S}, {rh}] of one dtype.")
    if c.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"[{op}] cos / sin must be float32 or bfloat16.")
    dt = _lib.MXQ_FLOAT32 if c.dtype == torch.float32 else _lib.MXQ_BFLOAT16
    x3, weight, c, s = (t.contiguous() for t in (x3, weight, c, s))
    out = torch.empty_like(x3)
    _lib.check(_lib.lib().mxq_rmsnorm_rope(_ptr(x3), S, H, hd, _ptr(weight), _ptr(c), _ptr(s),
                                           dt, rot, ctypes.c_float(eps), _ptr(out),
                                           _stream(x3)))
    return out.reshape(shape)
