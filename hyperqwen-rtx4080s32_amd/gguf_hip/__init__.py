"""gguf_hip - the GGUF quantized linear path on MI355X (gfx950): a C-ABI HIP library
(libgqk.so, include/gguf_hip.h) behind the vLLM GGUF plugin's linear-method surface.

    from gguf_hip import GGUFLinearMethod, dequantize, ggml_dequantize
"""
from .ops import (  # noqa: F401
    GGUF_TYPES, TYPE_NAMES, GroupedLayer, dequantize, dequantize_tiles, fused_mul_mat_gguf,
    fused_mul_mat_gguf_grouped, ggml_dequantize, mul_mat_grouped, pack_layer, plan, prepare_grouped_layer,
    quant_shape, repack_tiles, tiles_bytes, type_info, type_planes, unrepack_tiles,
)
from .linear import GGUFLinearMethod  # noqa: F401
