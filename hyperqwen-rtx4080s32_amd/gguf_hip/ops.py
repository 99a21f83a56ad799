"""Torch-facing ops of the GGUF quantized linear path (the plugin's op layer, on libgqk).

Reference surface mirrored here:
* ``ggml_dequantize(W, quant_type, m, n, dtype)`` - the plugin's ``ops.ggml_dequantize``
  (``gguf-plugin/patches/gguf-prefill-dispatch.patch:42-45,60-72``), and the north star's
  ``dequantize(W, type, shape)``.
* ``repack_tiles`` / ``unrepack_tiles`` (``gguf-plugin/gluon/tiles.py:56-130``).
* ``prepare_grouped_layer`` (``gguf-plugin/gluon/tiles_grouped.py:253-267``): the loader's step.
* ``fused_mul_mat_gguf_grouped`` - the graph-opaque custom op with a fake impl, the analogue of
  ``torch.ops.vllm._fused_mul_mat_gguf_tiles_grouped``
  (``gguf-plugin/patches/gguf-tiles-grouped.patch:28-72``); its row-count dispatch (the
  reference's ``gluon_mul_mat_tiles_grouped``, ``gguf-plugin/gluon/interface.py:141-188``) picks
  a precomputed plan, so no table is built inside a captured graph.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib
from ._lib import GqkPlanInfo, GqkShard, check, lib

# GGML type ids served by the library (ggml.h enum)
Q4_0, Q5_0, Q8_0 = 2, 6, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
IQ4_NL, IQ3_S, IQ4_XS = 20, 21, 23
GGUF_TYPES = (Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ3_S, IQ4_XS)
TYPE_NAMES = {Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K",
              Q6_K: "Q6_K", IQ4_NL: "IQ4_NL", IQ3_S: "IQ3_S", IQ4_XS: "IQ4_XS"}
# unquantized GGML types the plugin multiplies as they are (F32, F16, BF16)
UNQUANTIZED_TYPES = (0, 1, 30)

# batch-row buckets of a grouped layer: GEMV plans serve M <= 4, 8, 16; GEMM above
GEMV_BUCKETS = (4, 8, 16)
GEMM_PLAN_M = (32, 64, 128, 129)   # GEMM plans: 32 / 64 x 128 tiles (17..32 / 33..64 rows), 128 x 128 (65..128), 256 x 256 (129+)

_DTYPES = {torch.float32: _lib.GQK_DTYPE_F32, torch.bfloat16: _lib.GQK_DTYPE_BF16, torch.float16: _lib.GQK_DTYPE_F16}


def type_info(weight_type: int) -> tuple[int, int, int, int]:
    """(weights per block, bytes per block, bytes per 256 weights, tile planes) - the library's
    table (gguf.GGML_QUANT_SIZES for the first two)."""
    info = (ctypes.c_int32 * 4)()
    check(lib.gqk_type_info(int(weight_type), info, None), f"type_info({weight_type})")
    return tuple(info)


def type_planes(weight_type: int) -> list[tuple[int, int, int, int, int, int]]:
    """The type's tile planes: (bytes per row, segments, first raw offset, segment bytes, stride,
    column width)."""
    nplanes = type_info(weight_type)[3]
    info = (ctypes.c_int32 * 4)()
    planes = (ctypes.c_int32 * (6 * nplanes))()
    check(lib.gqk_type_info(int(weight_type), info, planes), f"type_info({weight_type})")
    return [tuple(planes[6 * p:6 * p + 6]) for p in range(nplanes)]


def quant_shape(weight_type: int, n: int, row_bytes: int) -> tuple[int, int]:
    """(n, K) of a uint8 [n, row_bytes] GGUF tensor (as the plugin derives it from
    gguf.GGML_QUANT_SIZES, gguf-plugin/patches/gguf-prefill-dispatch.patch:42-44)."""
    bw, bb, _, _ = type_info(weight_type)
    if row_bytes % bb:
        raise ValueError(f"{row_bytes} bytes per row is not a whole number of {bb}-byte blocks of type {weight_type}")
    return n, row_bytes // bb * bw


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{what}: the tensor must be on a GPU (there is no CPU path), got {t.device}")


def _rows_view(W: torch.Tensor, what: str) -> torch.Tensor:
    if W.dtype != torch.uint8 or W.dim() != 2:
        raise ValueError(f"{what}: expected uint8 [rows, bytes], got {W.dtype} {tuple(W.shape)}")
    if W.stride(1) != 1:
        W = W.contiguous()
    return W


def ggml_dequantize(W: torch.Tensor, quant_type: int, m: int, n: int, dtype: torch.dtype | None = None) -> torch.Tensor:
    """The plugin's ``ops.ggml_dequantize``: raw rows uint8 [m, row_bytes] (any row stride) ->
    [m, n] of dtype (default fp16, the plugin's default).  fp32 is bit-exact with gguf-py; bf16 /
    fp16 are its round-to-nearest-even."""
    dtype = torch.float16 if dtype is None else dtype
    if dtype not in _DTYPES:
        raise ValueError(f"ggml_dequantize: dtype {dtype}")
    W = _rows_view(W, "ggml_dequantize")
    _require_gpu(W, "ggml_dequantize")
    out = torch.empty((m, n), dtype=dtype, device=W.device)
    if m == 0 or n == 0:
        return out
    if W.shape[0] < m:
        raise ValueError(f"ggml_dequantize: {W.shape[0]} rows < m={m}")
    check(lib.gqk_dequantize(ctypes.c_void_p(W.data_ptr()), W.stride(0), int(quant_type), m, n,
                             ctypes.c_void_p(out.data_ptr()), out.stride(0), _DTYPES[dtype], _stream(W.device)),
          "ggml_dequantize")
    return out


def dequantize(W: torch.Tensor, weight_type: int, shape: tuple[int, int], dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """The north star's ``dequantize(W, type, shape)``: [n, K] weights of the raw GGUF rows."""
    n, K = shape
    return ggml_dequantize(W, weight_type, n, K, dtype)


def tiles_bytes(weight_type: int, n: int, K: int) -> int:
    return check(lib.gqk_tiles_bytes(int(weight_type), n, K), "tiles_bytes")


def repack_tiles(W: torch.Tensor, n_out: int, weight_type: int) -> torch.Tensor:
    """Raw rows uint8 [n_out, row_bytes] -> the plane-major tile layout (flat uint8)."""
    W = _rows_view(W, "repack_tiles")
    _require_gpu(W, "repack_tiles")
    _, K = quant_shape(weight_type, n_out, W.shape[1])
    tiles = torch.empty(tiles_bytes(weight_type, n_out, K), dtype=torch.uint8, device=W.device)
    check(lib.gqk_repack(ctypes.c_void_p(W.data_ptr()), W.stride(0), int(weight_type), n_out, K,
                         ctypes.c_void_p(tiles.data_ptr()), _stream(W.device)), "repack_tiles")
    return tiles


def unrepack_tiles(tiles: torch.Tensor, n_out: int, K: int, weight_type: int) -> torch.Tensor:
    """The tile layout -> raw rows uint8 [n_out, row_bytes] (bit-exact inverse of repack_tiles)."""
    _require_gpu(tiles, "unrepack_tiles")
    bw, bb, _, _ = type_info(weight_type)
    if tiles.numel() < tiles_bytes(weight_type, n_out, K):
        raise ValueError("unrepack_tiles: buffer smaller than the shard's tiles")
    raw = torch.empty((n_out, K // bw * bb), dtype=torch.uint8, device=tiles.device)
    check(lib.gqk_unrepack(ctypes.c_void_p(tiles.data_ptr()), int(weight_type), n_out, K,
                           ctypes.c_void_p(raw.data_ptr()), raw.stride(0), _stream(tiles.device)), "unrepack_tiles")
    return raw


def dequantize_tiles(tiles: torch.Tensor, n_out: int, K: int, weight_type: int, dtype=torch.bfloat16) -> torch.Tensor:
    """The tiles' weights [n_out, K] (un-repack, then the dequantizer; as the reference's
    dequantize_tiles, gguf-plugin/gluon/tiles.py:141-149)."""
    return dequantize(unrepack_tiles(tiles, n_out, K, weight_type), weight_type, (n_out, K), dtype)


# ----------------------------------------------------------------------------------------------
# grouped layers

def plan(shards: list[tuple[int, int, int]], K: int, M: int, target_wgs: int = 0) -> tuple[GqkPlanInfo, torch.Tensor]:
    """Host plan of a grouped launch: shards = [(type, n, byte offset)] -> (info, int32 table on CPU)."""
    arr = (GqkShard * len(shards))(*[GqkShard(int(t), 0, int(n), int(o)) for t, n, o in shards])
    info = GqkPlanInfo()
    check(lib.gqk_plan(arr, len(shards), K, M, target_wgs, None, 0, ctypes.byref(info)), "plan")
    desc = torch.empty(info.n_desc * 16, dtype=torch.int32)
    check(lib.gqk_plan(arr, len(shards), K, M, target_wgs,
                       ctypes.cast(desc.data_ptr(), ctypes.POINTER(ctypes.c_int32)), desc.numel(), ctypes.byref(info)),
          "plan")
    return info, desc


@dataclass
class GroupedLayer:
    """A run of shards packed into one buffer with the plans of every batch-row bucket (the
    reference's ``layer.gguf_groups[...]`` tuple, gguf-plugin/patches/gguf-tiles-grouped.patch:114-115)."""
    packed: torch.Tensor
    views: list[torch.Tensor]
    n_outs: list[int]
    weight_types: list[int]
    K: int
    descs: list[torch.Tensor] = field(default_factory=list)
    plans: list[int] = field(default_factory=list)    # flattened GqkPlanInfo tuples, one per bucket
    # split-K workspace of the GEMV plans: arrival counters (zeroed once here, left zero by every
    # launch) and fp32 partials; calls on one layer must not overlap in time
    workspace: torch.Tensor | None = None

    @property
    def n_total(self) -> int:
        return sum(self.n_outs)


def prepare_grouped_layer(tiles_list: list[torch.Tensor], n_outs: list[int], wtypes: list[int], K: int,
                          target_wgs: int = 0) -> GroupedLayer:
    """The loader's step for a run of shards already repacked: one packed buffer (the shards'
    tiles back to back; the views replace the separate tensors) and the descriptor tables of
    every batch-row bucket, uploaded once so the op never builds one at call time."""
    for t, n, wt in zip(tiles_list, n_outs, wtypes):
        if t.numel() != tiles_bytes(wt, n, K):
            raise ValueError(f"prepare_grouped_layer: tiles of a {n} x {K} shard of type {wt} have {t.numel()} bytes")
    packed = torch.cat([t.reshape(-1) for t in tiles_list]) if len(tiles_list) > 1 else tiles_list[0].reshape(-1)
    return grouped_layer_from_packed(packed, n_outs, wtypes, K, target_wgs)


def grouped_layer_from_packed(packed: torch.Tensor, n_outs: list[int], wtypes: list[int], K: int,
                              target_wgs: int = 0) -> GroupedLayer:
    """A grouped layer over a buffer that already holds the shards' tiles back to back (the
    GGUF load path uploads each tensor straight into its slice)."""
    sizes = [tiles_bytes(wt, n, K) for n, wt in zip(n_outs, wtypes)]
    if packed.dtype != torch.uint8 or packed.dim() != 1 or packed.numel() != sum(sizes):
        raise ValueError(f"grouped_layer_from_packed: packed must be uint8 [{sum(sizes)}]")
    views, shards, off = [], [], 0
    for size, n, wt in zip(sizes, n_outs, wtypes):
        views.append(packed[off:off + size])
        shards.append((wt, n, off))
        off += size
    gl = GroupedLayer(packed, views, list(n_outs), list(wtypes), K)
    ws = 0
    for m in GEMV_BUCKETS + GEMM_PLAN_M:
        info, desc = plan(shards, K, m, target_wgs)
        gl.descs.append(desc.to(packed.device))
        gl.plans.extend(info.as_tuple())
        ws = max(ws, info.workspace_bytes)
    gl.workspace = torch.zeros(max(ws, 256) // 4, dtype=torch.int32, device=packed.device)
    return gl


def pack_layer(raws: list[torch.Tensor], n_outs: list[int], wtypes: list[int], target_wgs: int = 0) -> GroupedLayer:
    """Raw rows of each shard -> repacked, packed and planned (pack_layer,
    gguf-plugin/gluon/tiles_grouped.py:209-212)."""
    Ks = {quant_shape(wt, n, W.shape[1])[1] for W, n, wt in zip(raws, n_outs, wtypes)}
    if len(Ks) != 1:
        raise ValueError(f"pack_layer: shards have different K {sorted(Ks)}")
    K = Ks.pop()
    return prepare_grouped_layer([repack_tiles(W, n, wt) for W, n, wt in zip(raws, n_outs, wtypes)], n_outs, wtypes, K,
                                 target_wgs)


_NPLAN = len(GqkPlanInfo._fields_)


def _pick_plan(plans: list[int], M: int) -> int:
    """Index of the bucket serving M rows (the reference's row-count dispatch, interface.py:141-188)."""
    for i, m in enumerate(GEMV_BUCKETS):
        if M <= m:
            return i
    for i, m in enumerate(GEMM_PLAN_M[:-1]):
        if M <= m:
            return len(GEMV_BUCKETS) + i
    return len(GEMV_BUCKETS) + len(GEMM_PLAN_M) - 1


def _grouped_into(x: torch.Tensor, packed: torch.Tensor, descs: list[torch.Tensor], plans: list[int],
                  workspace: torch.Tensor, bias: torch.Tensor | None, out: torch.Tensor) -> None:
    M = int(x.shape[0])
    if M == 0:
        return
    i = _pick_plan(plans, M)
    info = GqkPlanInfo.from_tuple(plans[i * _NPLAN:(i + 1) * _NPLAN])
    check(lib.gqk_linear(ctypes.c_void_p(packed.data_ptr()), ctypes.c_void_p(descs[i].data_ptr()), ctypes.byref(info),
                         ctypes.c_void_p(x.data_ptr()), x.stride(0), M, ctypes.c_void_p(out.data_ptr()), out.stride(0),
                         ctypes.c_void_p(bias.data_ptr() if bias is not None else None),
                         ctypes.c_void_p(workspace.data_ptr()), workspace.numel() * workspace.element_size(),
                         _stream(x.device)),
          "fused_mul_mat_gguf_grouped")


def _grouped_impl(x: torch.Tensor, packed: torch.Tensor, descs: list[torch.Tensor], plans: list[int],
                  n_total: int, workspace: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    out = torch.empty((int(x.shape[0]), n_total), dtype=torch.bfloat16, device=x.device)
    _grouped_into(x, packed, descs, plans, workspace, bias, out)
    return out


@torch.library.custom_op("gguf_hip::fused_mul_mat_gguf_grouped", mutates_args=("workspace",))
def fused_mul_mat_gguf_grouped(x: torch.Tensor, packed: torch.Tensor, descs: list[torch.Tensor], plans: list[int],
                               n_total: int, workspace: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """x bf16 [M, K] -> bf16 [M, n_total]: one launch over a grouped layer's shards (columns in
    shard order).  workspace: the layer's split-K counters and partials.  bias: None or bf16
    [n_total], added in the kernel's epilogue before the one rounding to bf16."""
    return _grouped_impl(x, packed, descs, plans, n_total, workspace, bias)


@fused_mul_mat_gguf_grouped.register_fake
def _(x, packed, descs, plans, n_total, workspace, bias=None):
    return torch.empty((x.shape[0], n_total), dtype=torch.bfloat16, device=x.device)


@torch.library.custom_op("gguf_hip::fused_mul_mat_gguf_grouped_out", mutates_args=("workspace", "out"))
def fused_mul_mat_gguf_grouped_out(x: torch.Tensor, packed: torch.Tensor, descs: list[torch.Tensor], plans: list[int],
                                   workspace: torch.Tensor, out: torch.Tensor, bias: torch.Tensor | None = None) -> None:
    """As fused_mul_mat_gguf_grouped, writing into `out` (bf16 [M, n_total], unit column stride:
    e.g. the column slice of a wider layer output that this run's shards own)."""
    _grouped_into(x, packed, descs, plans, workspace, bias, out)


def _ensure_workspace(gl: GroupedLayer, M: int) -> None:
    """Grow the layer's workspace (zero-filled, as the counters need) to what the plan serving M
    rows needs.  GEMV plans are covered at preparation; the large-M GEMM's stream-K partials
    depend on M, so the first call at a larger M grows it (outside any graph capture)."""
    if M <= 0:
        return
    i = _pick_plan(gl.plans, M)
    info = GqkPlanInfo.from_tuple(gl.plans[i * _NPLAN:(i + 1) * _NPLAN])
    need = check(lib.gqk_linear_workspace_bytes(ctypes.byref(info), M), "linear_workspace_bytes")
    have = gl.workspace.numel() * gl.workspace.element_size()
    if need > have:
        gl.workspace = torch.zeros((need + 3) // 4, dtype=torch.int32, device=gl.packed.device)


def mul_mat_grouped(x: torch.Tensor, gl: GroupedLayer, bias: torch.Tensor | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ W^T (+ bias) for a prepared grouped layer, in x's dtype.  The kernels take bf16
    activations; other floating dtypes are rounded to bf16 on the way in and the bf16 result
    is cast back.  A bf16 bias [n_total] is fused into the kernel's epilogue; a bias of another
    dtype is added afterwards in that dtype (as the reference's out.add_(bias)).  out: a bf16
    [M, n_total] view with unit column stride (a column slice of a wider output) to write
    into, for bf16 x; it is returned."""
    _require_gpu(x, "mul_mat_grouped")
    if x.dim() != 2 or x.shape[1] != gl.K:
        raise ValueError(f"mul_mat_grouped: x {tuple(x.shape)} does not match K={gl.K}")
    xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
    if xb.stride(1) != 1 or xb.stride(0) % 8 or xb.data_ptr() % 16:
        xb = xb.contiguous()
    _ensure_workspace(gl, int(xb.shape[0]))
    fused = None
    if bias is not None:
        if bias.shape != (gl.n_total,) or bias.device != x.device:
            raise ValueError(f"mul_mat_grouped: bias {tuple(bias.shape)} on {bias.device}, expected ({gl.n_total},)")
        if bias.dtype == torch.bfloat16:
            fused = bias.contiguous()
    if out is not None:
        if (x.dtype != torch.bfloat16 or out.dtype != torch.bfloat16 or out.shape != (xb.shape[0], gl.n_total)
                or out.device != x.device or (out.numel() and out.stride(1) != 1)):
            raise ValueError(f"mul_mat_grouped: out must be a bf16 [{xb.shape[0]}, {gl.n_total}] view with unit "
                             f"column stride on {x.device}, for bf16 x")
        fused_mul_mat_gguf_grouped_out(xb, gl.packed, gl.descs, gl.plans, gl.workspace, out, fused)
        if bias is not None and fused is None:
            out.add_(bias)
        return out
    y = fused_mul_mat_gguf_grouped(xb, gl.packed, gl.descs, gl.plans, gl.n_total, gl.workspace, fused)
    y = y if x.dtype == torch.bfloat16 else y.to(x.dtype)
    if bias is not None and fused is None:
        y.add_(bias)
    return y


def fused_mul_mat_gguf(x: torch.Tensor, qweight: torch.Tensor, qweight_type: int) -> torch.Tensor:
    """The plugin's module-level op on raw rows (``_fused_mul_mat_gguf``,
    gguf-plugin/patches/gguf-prefill-dispatch.patch:9-50): y = x @ W^T.  Unprepared raw rows are
    repacked for this call (the loader's prepare step does it once instead)."""
    if qweight_type in UNQUANTIZED_TYPES:
        return x @ (qweight if qweight.dtype == x.dtype else qweight.to(x.dtype)).T
    if qweight_type not in GGUF_TYPES:
        raise NotImplementedError(f"Unsupported GGUF quantization type: {qweight_type}")
    n = qweight.shape[0]
    if x.shape[0] == 0:
        return torch.empty((0, n), dtype=x.dtype, device=x.device)
    gl = pack_layer([qweight], [n], [qweight_type])
    return mul_mat_grouped(x, gl)
