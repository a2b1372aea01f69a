"""wuxianhuabu_amd — MI355X-native MLX affine group-quantized linear.

The quantized-linear hot path of the reference's MLX-Swift DiT backbones,
rebuilt in HIP for gfx950 behind the same operator surface:

    quantized, dequantized, quantized_matmul (quantizedMatmul / quantizedMM),
    QuantizedLinear, MfLinear, the fused feed-forward blocks LTXFFN and H3MlpW,
    and SafetensorsFile (the on-disk triples, read straight into HBM)

Device memory and streams come from torch; every kernel lives in libmxq.so,
whose C ABI is include/mxq.h.
"""
from ._lib import LIB_PATH, MXQError, lib  # noqa: F401
from .nn import H3MlpW, LTXFFN, MfLinear, QuantizedLinear  # noqa: F401
from .stfile import SafetensorsFile  # noqa: F401
from .blockops import (build_row_mod_map, fused_mod_gate, fused_norm_modscale,  # noqa: F401
                       fused_norm_modscale_row, fused_rmsnorm_rope)
from .ops import (LoraAdapters, TiledWeight, dequantized, pack, quantized,  # noqa: F401
                  quantized_matmul,
                  quantizedMatmul, quantizedMM, tile, tiled_matmul, tiled_supported, unpack,
                  untile)
from .weights import get_quantized, header_candidates, infer_geometry  # noqa: F401
from .convert import (QuantizedLinearModule, quantize_checkpoint, quantize_module,  # noqa: F401
                      should_quant)

__all__ = [
    "quantized", "dequantized", "quantized_matmul", "quantizedMatmul", "quantizedMM",
    "pack", "unpack", "tile", "untile", "tiled_matmul", "tiled_supported", "TiledWeight",
    "LoraAdapters",
    "QuantizedLinear", "MfLinear", "LTXFFN", "H3MlpW", "SafetensorsFile", "get_quantized",
    "infer_geometry", "header_candidates", "lib", "LIB_PATH", "MXQError",
    "fused_norm_modscale", "fused_norm_modscale_row", "fused_mod_gate", "fused_rmsnorm_rope",
    "build_row_mod_map", "quantize_checkpoint", "quantize_module", "QuantizedLinearModule",
    "should_quant",
]
