"""The plugin's kernel-dispatch module, on libgqk: the names the patched vLLM GGUF linear method
imports from ``vllm_gguf_plugin.triton.gluon.interface`` (``gguf-plugin/patches/gguf-gluon-dispatch.patch:13``,
``gguf-plugin/patches/gguf-iq3s-tiles.patch:15-19``, ``gguf-plugin/patches/gguf-tiles-all-types.patch:12-17``,
``gguf-plugin/patches/gguf-tiles-grouped.patch:18-22``), with the meanings of
``gguf-plugin/gluon/interface.py``.  Pointing that import at this module switches the plugin to
the MI355X path without touching its linear method.

Every call runs the HIP library (there is no CPU path).  Differences from the Gluon module, all
at the level of what a caller can observe:

* every GGUF type here has one kernel family for every row count (GEMV up to 16 rows, the mid
  form up to 32, MFMA GEMM above), so ``GLUON_DEQUANT_TYPES`` is empty and the row-count limits
  only matter to callers that choose paths by them;
* ``gluon_mul_mat`` on raw rows (``gguf-plugin/gluon/interface.py:74-80``) repacks a weight to the
  tile layout on its first call and keeps the tiles and launch plans in a cache attached to the
  weight's base tensor (the storage the view belongs to, e.g. the layer's parameter), keyed by the
  view's offset, shape, strides, type and the base's version counter - the reference keys its
  layer caches by the layer's own metadata for the same reason (a freed layer's table must not
  serve another, ``gguf-plugin/gluon/tiles_grouped.py:271-275``).  Later calls allocate only the
  output: no repack, no host-to-device copy, capturable in a HIP graph.  The reference decodes the
  raw rows in place; here the cache holds a tile copy beside them (the weight's size again in
  HBM, freed by ``ops.drop_cached_layers``), and a first call made under graph capture raises.
  The split-K / stream-K launches share the device's workspace (``ops.device_workspace``), so
  calls that may overlap in time on different streams need a workspace of their own
  (``ops.mul_mat_grouped(..., workspace=)``).
"""
from __future__ import annotations

import torch

from . import ops

GGML_TYPE_Q4_0 = ops.Q4_0
GGML_TYPE_Q5_0 = ops.Q5_0
GGML_TYPE_Q8_0 = ops.Q8_0
GGML_TYPE_Q2_K = ops.Q2_K
GGML_TYPE_Q3_K = ops.Q3_K
GGML_TYPE_Q4_K = ops.Q4_K
GGML_TYPE_Q5_K = ops.Q5_K
GGML_TYPE_Q6_K = ops.Q6_K
GGML_TYPE_IQ4_NL = ops.IQ4_NL
GGML_TYPE_IQ3_S = ops.IQ3_S
GGML_TYPE_IQ4_XS = ops.IQ4_XS

GLUON_TYPES = frozenset(ops.GGUF_TYPES)          # the types with a kernel (every row count)
GLUON_INT8_TYPES = frozenset()                   # no int8-activation form: activations stay bf16
GLUON_TILE_TYPES = frozenset(ops.GGUF_TYPES)     # the types the loader holds in the tile layout
GLUON_DEQUANT_TYPES = frozenset()                # no run falls back to dequantize + a library GEMM
GLUON_MAX_ROWS = 16                              # rows of the decode GEMV form
GLUON_MAX_ROWS_GROUPED = 32                      # rows of the streaming forms (GEMV, then the mid form)
GLUON_ARRIVAL_ROWS = 128                         # rows of the 128 x 128 GEMM tile form


def _rec_bytes(weight_type: int) -> int:
    return ops.type_info(weight_type)[2]


def _tile_view(flat: torch.Tensor, n_out: int, K: int, weight_type: int) -> torch.Tensor:
    """The reference's 4-D tile shape [n_tiles, nb, 64, bytes per row per record] over our buffer."""
    return flat.view(-(-n_out // 64), K // 256, 64, _rec_bytes(weight_type))


def gluon_mul_mat(x: torch.Tensor, weight: torch.Tensor, weight_type: int, n_out: int) -> torch.Tensor:
    """x bf16 [M, K]; weight the raw GGUF rows uint8 [n_out, row bytes] (any row stride: a merged
    layer's shard view is fine); returns [M, n_out] in x's dtype (``gguf-plugin/gluon/interface.py:74-80``)."""
    if weight_type not in GLUON_TYPES:
        raise NotImplementedError(f"no kernel for GGUF type {weight_type}")
    if x.shape[0] == 0:
        return torch.empty((0, n_out), dtype=x.dtype, device=x.device)
    return ops.mul_mat_grouped(x, ops.cached_layer(weight, weight_type, n_out, "rows"))


def repack_tiles(W: torch.Tensor, n_out: int, weight_type: int) -> torch.Tensor:
    """Raw rows -> the tile layout as the reference shapes it, [n_tiles, nb, 64, bytes per row per
    256 weights] (``gguf-plugin/gluon/tiles.py:128-130``); the bytes are this library's plane-major tiles."""
    flat = ops.repack_tiles(W, n_out, weight_type)
    _, K = ops.quant_shape(weight_type, n_out, W.shape[1])
    return _tile_view(flat, n_out, K, weight_type)


def repack_iq3s_tiles(W: torch.Tensor, n_out: int) -> torch.Tensor:
    return repack_tiles(W, n_out, GGML_TYPE_IQ3_S)


def dequantize_tiles(tiles: torch.Tensor, n_out: int, K: int, weight_type: int, dtype=torch.bfloat16) -> torch.Tensor:
    """[n_out, K] weights of dtype from the tiles, one pass (``gguf-plugin/gluon/tiles.py:141-149``)."""
    return ops.dequantize_tiles(tiles.reshape(-1), n_out, K, weight_type, dtype)


def dequantize_iq3s_tiles(tiles: torch.Tensor, n_out: int, K: int, dtype=torch.bfloat16) -> torch.Tensor:
    return dequantize_tiles(tiles, n_out, K, GGML_TYPE_IQ3_S, dtype)


def gluon_mul_mat_tiles(x: torch.Tensor, tiles: torch.Tensor, n_out: int, weight_type: int) -> torch.Tensor:
    """x bf16 [M, K]; tiles one shard's tile layout; [M, n_out] in x's dtype, any M
    (``gguf-plugin/gluon/interface.py:98-110``)."""
    if x.shape[0] == 0:
        return torch.empty((0, n_out), dtype=x.dtype, device=x.device)
    return ops.mul_mat_grouped(x, ops.cached_layer(tiles, weight_type, n_out, "tiles"))


def gluon_mul_mat_iq3s_tiles(x: torch.Tensor, tiles: torch.Tensor, n_out: int) -> torch.Tensor:
    return gluon_mul_mat_tiles(x, tiles, n_out, GGML_TYPE_IQ3_S)


def prepare_grouped_layer(tiles_list: list[torch.Tensor], n_outs: list[int], wtypes: list[int]):
    """The loader's step for a run of shards (``gguf-plugin/gluon/tiles_grouped.py:253-267``):
    (packed buffer, the shards' tiles as views into it, the descriptor tables, the launch plans,
    nb, the run's bytes per 256 weights).  The last two are what the reference returns; the plans
    travel in the reference's ``desc_splits`` slot (a list of ints)."""
    nb = None
    for t, n, wt in zip(tiles_list, n_outs, wtypes):
        k = t.numel() // (-(-n // 64) * 64) // _rec_bytes(wt)
        if nb is not None and k != nb:
            raise ValueError(f"prepare_grouped_layer: shards with {nb} and {k} super-blocks per row")
        nb = k
    gl = ops.prepare_grouped_layer([t.reshape(-1) for t in tiles_list], list(n_outs), list(wtypes), nb * 256)
    views = [_tile_view(v, n, gl.K, wt) for v, n, wt in zip(gl.views, n_outs, wtypes)]
    block_bytes = int(round(gl.packed.numel() / (sum(-(-n // 64) * 64 for n in n_outs) * nb)))
    return gl.packed, views, gl.descs, gl.plans, nb, block_bytes


def gluon_mul_mat_tiles_grouped(x: torch.Tensor, packed: torch.Tensor, descs: list[torch.Tensor],
                                desc_splits: list[int], tiles: list[torch.Tensor], n_outs: list[int],
                                weight_types: list[int], nb: int, block_bytes: int) -> torch.Tensor:
    """A layer's run of shards in one launch (``gguf-plugin/gluon/interface.py:141-188``): x bf16
    [M, K]; the rest as ``prepare_grouped_layer`` returned it; [M, sum(n_outs)] in x's dtype."""
    if x.dim() != 2 or x.shape[1] != nb * 256:
        raise ValueError(f"gluon_mul_mat_tiles_grouped: x {tuple(x.shape)} does not match K={nb * 256}")
    gl = ops.GroupedLayer(packed, list(tiles), list(n_outs), list(weight_types), nb * 256, list(descs),
                          list(desc_splits), ops.device_workspace(packed.device))
    return ops.mul_mat_grouped(x, gl)
