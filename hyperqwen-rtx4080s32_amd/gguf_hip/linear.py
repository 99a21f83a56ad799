"""GGUFLinearMethod on libgqk: the plugin's linear-method surface for the GGUF layer.

Mirrors the patched ``vllm_gguf_plugin/quantization/linear.py`` as the reference's patches show
it (the plugin itself is not vendored):

* post-load: ``_create_tiles`` + ``_create_groups`` (``gguf-plugin/patches/gguf-tiles-all-types.patch:59-131``,
  ``gguf-plugin/patches/gguf-tiles-grouped.patch:84-115``) become ``process_weights_after_loading``:
  every shard (or the whole weight of a single-type layer) is repacked to the tile layout, the
  run of shards is packed into one buffer with its launch plans, and the raw rows are freed.
  All eleven quantized types are tile types here, so a merged layer of them is one run (one
  launch); an unquantized shard between them splits it into runs.
* ``apply(layer, x, bias)`` (``gguf-plugin/patches/gguf-tiles-grouped.patch:131-171``,
  ``gguf-plugin/patches/gguf-iq3s-tiles.patch:98-136``): same-type or grouped -> one op, with
  a bf16 bias fused into the kernel's epilogue; a shard of a type without a kernel here (an
  unquantized one) splits the layer into runs, and each run and each such shard writes its
  own column slice of one output, then ``out.add_(bias)``.  M = 0 returns an empty [0, N] tensor.

Layer attributes read (the plugin's): ``weight`` uint8 [N, K_bytes] with ``shard_id`` and
``shard_offset_map`` {idx: (start, end, size)}; ``weight_type.weight_type`` and
``weight_type.shard_weight_type``; optional ``gguf_shards`` {idx: contiguous raw rows} for
mixed-type merged layers (``gguf-plugin/patches/gguf-shard-tensors.patch:17-50``).  Attributes
written: ``gguf_tiles`` {idx: tile view}, ``gguf_tiles_rows``, ``gguf_tiles_types``,
``gguf_groups`` {first idx: GroupedLayer}.
"""
from __future__ import annotations

import torch

from . import ops


def _ordered_shard_ids(shard_id: list) -> list:
    # the merged qkv layer is ordered q, k, v (gguf-plugin/patches/gguf-tiles-grouped.patch:121-122)
    return ["q", "k", "v"] if "q" in shard_id else list(shard_id)


class GGUFLinearMethod:
    """Linear method for GGUF weights on MI355X (gfx950)."""

    def __init__(self, target_wgs: int = 0):
        self.target_wgs = target_wgs

    # ---- load time -------------------------------------------------------------------------
    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        """Repack, pack and plan the layer once; idempotent."""
        if getattr(layer, "gguf_groups", None) is not None:
            return
        fallback = layer.weight_type.weight_type
        shard_types = getattr(layer.weight_type, "shard_weight_type", {}) or {}
        gguf_shards = getattr(layer, "gguf_shards", None)
        tiles, rows, types, raws = {}, {}, {}, {}
        if gguf_shards is not None:
            order = _ordered_shard_ids(list(gguf_shards))
            for idx in order:
                wt = shard_types.get(idx, fallback)
                shard = gguf_shards[idx]
                if wt in ops.GGUF_TYPES and shard.numel() > 0:
                    raws[idx], rows[idx], types[idx] = shard, shard.shape[0], wt
        else:
            w = layer.weight.data
            shard_id = getattr(layer.weight, "shard_id", None)
            wtypes = {shard_types.get(i, fallback) for i in shard_id} if shard_id else {fallback}
            wt = next(iter(wtypes))
            if len(wtypes) == 1 and wt in ops.GGUF_TYPES and w.numel() > 0:
                order = ["__all__"]
                raws["__all__"], rows["__all__"], types["__all__"] = w, w.shape[0], wt
            else:
                order = []
        # runs of consecutive shards with a kernel here (a shard of another type between them
        # stays on its own path), as the reference's _create_groups
        # (gguf-plugin/patches/gguf-tiles-grouped.patch:84-115)
        runs, cur = [], []
        for i in order:
            if i in raws:
                cur.append(i)
            elif cur:
                runs.append(cur)
                cur = []
        if cur:
            runs.append(cur)
        groups = {}
        if runs:
            K = {ops.quant_shape(types[i], rows[i], raws[i].shape[1])[1] for r in runs for i in r}
            if len(K) != 1:
                raise ValueError(f"process_weights_after_loading: shards with different K {sorted(K)}")
            K = K.pop()
        for run in runs:
            for i in run:
                tiles[i] = ops.repack_tiles(raws[i], rows[i], types[i])
            gl = ops.prepare_grouped_layer([tiles[i] for i in run], [rows[i] for i in run], [types[i] for i in run], K,
                                           self.target_wgs)
            for i, v in zip(run, gl.views):
                tiles[i] = v
            groups[run[0]] = (gl, run)
            # the raw rows are freed: every call of these shards runs on the tiles
            if gguf_shards is not None:
                for i in run:
                    gguf_shards[i] = torch.empty(0, dtype=torch.uint8, device=raws[i].device)
            else:
                layer.weight.data = torch.empty(0, dtype=torch.uint8, device=raws["__all__"].device)
        layer.gguf_tiles, layer.gguf_tiles_rows, layer.gguf_tiles_types = tiles, rows, types
        layer.gguf_groups = groups

    # ---- call time -------------------------------------------------------------------------
    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        groups = getattr(layer, "gguf_groups", None)
        if groups is None:
            self.process_weights_after_loading(layer)
            groups = layer.gguf_groups
        if "__all__" in groups:
            return ops.mul_mat_grouped(x, groups["__all__"][0], bias)   # bias fused into the epilogue
        else:
            shard_id = getattr(layer.weight, "shard_id", None) or list(getattr(layer, "gguf_shards", {}) or {})
            fallback = layer.weight_type.weight_type
            shard_types = getattr(layer.weight_type, "shard_weight_type", {}) or {}
            gguf_shards = getattr(layer, "gguf_shards", None)
            order = _ordered_shard_ids(shard_id)
            if len(groups) == 1 and set(next(iter(groups.values()))[1]) == set(order):
                # every shard is in the one grouped run: one launch, bias fused
                return ops.mul_mat_grouped(x, next(iter(groups.values()))[0], bias)
            # the pieces in shard order: grouped runs, and shards on their own path
            pieces, i = [], 0
            while i < len(order):
                idx = order[i]
                if idx in groups:
                    gl, run = groups[idx]
                    pieces.append((gl.n_total, gl, None, None))
                    i += len(run)
                    continue
                wt = shard_types.get(idx, fallback)
                if gguf_shards is not None:
                    shard = gguf_shards[idx]
                else:
                    start, end, size = layer.weight.shard_offset_map[idx]
                    shard = layer.weight[start:end, :size]
                pieces.append((shard.shape[0], None, shard, wt))
                i += 1
            if x.dtype == torch.bfloat16:
                # every piece writes its own column slice of one output (no concatenation)
                out = torch.empty((x.shape[0], sum(p[0] for p in pieces)), dtype=x.dtype, device=x.device)
                c = 0
                for n, gl, shard, wt in pieces:
                    if gl is not None:
                        ops.mul_mat_grouped(x, gl, out=out[:, c:c + n])
                    else:
                        out[:, c:c + n] = ops.fused_mul_mat_gguf(x, shard, wt)
                    c += n
            else:
                result = [ops.mul_mat_grouped(x, gl) if gl is not None else ops.fused_mul_mat_gguf(x, shard, wt)
                          for n, gl, shard, wt in pieces]
                out = result[0] if len(result) == 1 else torch.cat(result, dim=1)
        if bias is not None:
            out.add_(bias)
        return out
