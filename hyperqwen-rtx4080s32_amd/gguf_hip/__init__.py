"""gguf_hip - the GGUF quantized linear path on MI355X (gfx950): a C-ABI HIP library
(libgqk.so, include/gguf_hip.h) behind the vLLM GGUF plugin's linear-method surface.

    from gguf_hip import GGUFLinearMethod, dequantize, ggml_dequantize
    from gguf_hip import GGUFFile, load_grouped_layers      # GGUF v3 files -> grouped layers
"""
from .ops import (  # noqa: F401
    GGUF_TYPES, TYPE_NAMES, GroupedLayer, dequantize, dequantize_tiles, drop_cached_layers, fused_mul_mat_gguf,
    fused_mul_mat_gguf_grouped, ggml_dequantize, grouped_layer_from_packed, mul_mat_grouped, pack_layer, plan,
    prepare_grouped_layer,
    quant_shape, repack_tiles, tiles_bytes, type_info, type_planes, unrepack_tiles,
)
from .linear import GGUFLinearMethod  # noqa: F401
from .gguf_file import GGUFFile, GGUFTensor, ggml_type_size, layer_runs, load_grouped_layers  # noqa: F401
