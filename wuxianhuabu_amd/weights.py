"""Host-side handling of the quantized triple: key lookup and geometry.

get_quantized(weights, prefix)
    `model/minimax h3/H3Common.swift:249-258` (H3Weights.getQuantized): accepts
    both `prefix.scales/.biases` (mlx-serve) and `prefix.weight.scales/.weight.biases`
    (comfy/HF style).
infer_geometry(w_cols, s_cols, in_features)
    `model/minimax h3/H3Common.swift:317-323`: bits = 32*wCols/in,
    groupSize = in/sCols, validated against what the kernels accept.
header_candidates(w_cols, s_cols)
    the shape constraint of `model/3模块/模型加载-通用.swift:178-219`
    (w2*32/bits == s2*gs), over every width mlx supports. The reference helper
    only tries bits {2,4,8} and so never recognises a 6-bit file (:214); this one
    includes 3, 5 and 6.
"""

SUPPORTED_BITS = (2, 3, 4, 5, 6, 8)
SUPPORTED_GS = (32, 64, 128)


def get_quantized(weights, prefix):
    """(weight, scales, biases) for `prefix`, or None if the triple is absent."""
    w = weights.get(prefix + ".weight")
    if w is None:
        return None
    s, b = weights.get(prefix + ".scales"), weights.get(prefix + ".biases")
    if s is not None and b is not None:
        return w, s, b
    s, b = weights.get(prefix + ".weight.scales"), weights.get(prefix + ".weight.biases")
    if s is not None and b is not None:
        return w, s, b
    return None


def infer_geometry(w_cols, s_cols, in_features):
    """(bits, group_size) of a packed [out, w_cols] weight with [out, s_cols] scales."""
    if in_features <= 0 or s_cols <= 0:
        raise ValueError("bad file: non-positive in_features or scales width")
    if (32 * w_cols) % in_features or in_features % s_cols:
        raise ValueError(f"bad file: packed width {w_cols} and scales width {s_cols} do not "
                         f"describe {in_features} input features")
    bits = 32 * w_cols // in_features
    gs = in_features // s_cols
    if bits not in SUPPORTED_BITS or gs not in SUPPORTED_GS:
        raise ValueError(f"bad file: inferred bits={bits}, group_size={gs} not supported")
    return bits, gs


def header_candidates(w_cols, s_cols):
    """All (bits, group_size) pairs consistent with the packed and scales widths."""
    out = []
    for bits in SUPPORTED_BITS:
        for gs in SUPPORTED_GS:
            numer = w_cols * 32
            if numer % bits == 0 and numer // bits == s_cols * gs:
                out.append((bits, gs))
    return out
