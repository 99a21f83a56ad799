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

# batch-row buckets of a grouped layer: the streaming plans serve M <= 4, 8, 16 (GEMV) and 17..32
# (the mid form); GEMM above
GEMV_BUCKETS = (4, 8, 16, 32)
# GEMM plans: 64 x 128 tiles (33..64 rows), 128 x 128 (65..128), 129..384, 385..512 and 513..768
# (256 x 256, or 128 x 128 for a layer with few 256-row groups), 256 x 256 above
GEMM_PLAN_M = (64, 128, 384, 512, 768, 769)
# From this many batch rows mul_mat_grouped takes the reference's dequant regime (its
# gluon_mul_mat_tiles_grouped dequantizes the tiles and runs the vendor bf16 GEMM above 128 rows
# for the types its wide form loses on, gguf-plugin/gluon/interface.py:181-187): each shard is
# decoded once by the tile dequant kernel and multiplied by torch's bf16 GEMM (hipBLASLt) in row
# chunks.  Measured on the gate_up / down shards against the fused GEMM: at 8192 rows 12-44%
# faster on gate_up for Q4_K, Q5_K, Q6_K, IQ4_XS and IQ3_S and, chunked, on `down`; at 4096 rows
# 4-16%; at 2048 rows from even (Q4_K gate_up, the bench's line) to 12%, so the fused kernel keeps
# those.  The chunk: DEQUANT_CHUNK_M rows, or DEQUANT_CHUNK_M_LONG_K for K above
# DEQUANT_LONG_K - the vendor GEMM's 8192-row `down` (K = 17408) ran 2.5x its 4096-row time,
# while gate_up (K = 5120) in two 4096-row chunks took 1.15x its one 8192-row call.
DEQUANT_MIN_M = 4096
DEQUANT_CHUNK_M = 8192
DEQUANT_LONG_K = 8192
DEQUANT_CHUNK_M_LONG_K = 4096

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


def _addr_aligned(t: torch.Tensor, align: int) -> bool:
    """t's first element at an address that is a multiple of align.  Under tracing (FakeTensor,
    torch.compile) a tensor has no address: its byte offset into the storage decides, storages
    being allocated at least 256-byte aligned."""
    if torch.compiler.is_compiling() or isinstance(t, torch._subclasses.fake_tensor.FakeTensor):
        return t.storage_offset() * t.element_size() % align == 0
    return t.data_ptr() % align == 0


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
    # the shape contract first (the C side only sees a row stride, so a view narrower than the
    # rows' bytes would read past its last row)
    if m > 0 and n > 0:
        if W.shape[0] < m:
            raise ValueError(f"ggml_dequantize: {W.shape[0]} rows < m={m}")
        bw, bb, _, _ = type_info(quant_type)
        if n % bw or W.shape[1] < n // bw * bb:
            raise ValueError(f"ggml_dequantize: rows of {W.shape[1]} bytes do not hold {n} weights of type "
                             f"{quant_type} ({bw}-weight blocks of {bb} bytes)")
    _require_gpu(W, "ggml_dequantize")
    out = torch.empty((m, n), dtype=dtype, device=W.device)
    if m == 0 or n == 0:
        return out
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
    """The tiles' weights [n_out, K], decoded straight from the tile layout in one pass (the
    reference's dequantize_tiles / dequantize_iq3s_tiles, gguf-plugin/gluon/tiles.py:141-149,
    gguf-plugin/gluon/iq3s_tile_dequant.py:22-63): the same bits as dequantize of the raw rows."""
    _require_gpu(tiles, "dequantize_tiles")
    if dtype not in _DTYPES:
        raise ValueError(f"dequantize_tiles: dtype {dtype}")
    if tiles.dtype != torch.uint8 or not tiles.is_contiguous() or tiles.numel() < tiles_bytes(weight_type, n_out, K):
        raise ValueError("dequantize_tiles: tiles must be a contiguous uint8 buffer of the shard's tile bytes")
    out = torch.empty((n_out, K), dtype=dtype, device=tiles.device)
    check(lib.gqk_dequantize_tiles(ctypes.c_void_p(tiles.data_ptr()), int(weight_type), n_out, K,
                                   ctypes.c_void_p(out.data_ptr()), out.stride(0), _DTYPES[dtype], _stream(tiles.device)),
          "dequantize_tiles")
    return out


# ----------------------------------------------------------------------------------------------
# grouped layers

def plan(shards: list[tuple[int, int, int]], K: int, M: int, target_wgs: int = 0,
         cus: int = 0) -> tuple[GqkPlanInfo, torch.Tensor]:
    """Host plan of a grouped launch: shards = [(type, n, byte offset)] -> (info, int32 table on CPU).
    cus: compute units of the target device (0: the current device's, as the HIP runtime reports)."""
    arr = (GqkShard * len(shards))(*[GqkShard(int(t), 0, int(n), int(o)) for t, n, o in shards])
    info = GqkPlanInfo()
    check(lib.gqk_plan(arr, len(shards), K, M, target_wgs, cus, None, 0, ctypes.byref(info)), "plan")
    desc = torch.empty(info.n_desc * 16, dtype=torch.int32)
    check(lib.gqk_plan(arr, len(shards), K, M, target_wgs, cus,
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
    # the device's shared split-K / stream-K workspace (device_workspace): arrival counters (zero at
    # rest, left zero by every launch) and fp32 partials; calls sharing it must not overlap in time
    workspace: torch.Tensor | None = None

    @property
    def n_total(self) -> int:
        return sum(self.n_outs)


# one workspace per device, shared by every grouped layer prepared on it
_WORKSPACES: dict[int, torch.Tensor] = {}


def device_workspace(device: torch.device, need: int = 0) -> torch.Tensor:
    """The device's shared workspace: zero-filled int32, at least ``gqk_workspace_bytes_max()``
    bytes (every GEMM plan at any M) and ``need`` (a layer's GEMV plans).  It is made at a layer's
    preparation and never resized or freed while a layer holds it, so the apply path allocates
    nothing and a captured graph's pointer stays valid.  Only a layer whose GEMV plans need more
    (a very large custom wave target) gets a larger one, which then serves the layers prepared
    after it; earlier layers keep theirs."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _WORKSPACES.get(idx)
    if ws is None or ws.numel() * ws.element_size() < need:
        with torch.cuda.device(idx):
            size = max(need, check(lib.gqk_workspace_bytes_max(), "workspace_bytes_max"))
        ws = torch.zeros((size + 3) // 4, dtype=torch.int32, device=torch.device("cuda", idx))
        _WORKSPACES[idx] = ws
    return ws


def prepare_grouped_layer(tiles_list: list[torch.Tensor], n_outs: list[int], wtypes: list[int], K: int,
                          target_wgs: int = 0, cus: int = 0) -> GroupedLayer:
    """The loader's step for a run of shards already repacked: one packed buffer (the shards'
    tiles back to back; the views replace the separate tensors) and the descriptor tables of
    every batch-row bucket, uploaded once so the op never builds one at call time.  cus: the CU
    count the plans are made for (0: the current device's; any count gives plans that run
    correctly on any device)."""
    for t, n, wt in zip(tiles_list, n_outs, wtypes):
        if t.numel() != tiles_bytes(wt, n, K):
            raise ValueError(f"prepare_grouped_layer: tiles of a {n} x {K} shard of type {wt} have {t.numel()} bytes")
    packed = torch.cat([t.reshape(-1) for t in tiles_list]) if len(tiles_list) > 1 else tiles_list[0].reshape(-1)
    return grouped_layer_from_packed(packed, n_outs, wtypes, K, target_wgs, cus)


def grouped_layer_from_packed(packed: torch.Tensor, n_outs: list[int], wtypes: list[int], K: int,
                              target_wgs: int = 0, cus: int = 0) -> GroupedLayer:
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
        info, desc = plan(shards, K, m, target_wgs, cus)
        gl.descs.append(desc.to(packed.device))
        gl.plans.extend(info.as_tuple())
        ws = max(ws, info.workspace_bytes)
    gl.workspace = device_workspace(packed.device, ws)
    return gl


def pack_layer(raws: list[torch.Tensor], n_outs: list[int], wtypes: list[int], target_wgs: int = 0,
               cus: int = 0) -> GroupedLayer:
    """Raw rows of each shard -> repacked, packed and planned (pack_layer,
    gguf-plugin/gluon/tiles_grouped.py:209-212)."""
    Ks = {quant_shape(wt, n, W.shape[1])[1] for W, n, wt in zip(raws, n_outs, wtypes)}
    if len(Ks) != 1:
        raise ValueError(f"pack_layer: shards have different K {sorted(Ks)}")
    K = Ks.pop()
    return prepare_grouped_layer([repack_tiles(W, n, wt) for W, n, wt in zip(raws, n_outs, wtypes)], n_outs, wtypes, K,
                                 target_wgs, cus)


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


def mul_mat_grouped(x: torch.Tensor, gl: GroupedLayer, bias: torch.Tensor | None = None,
                    out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ W^T (+ bias) for a prepared grouped layer, in x's dtype.  The kernels take bf16
    activations; other floating dtypes are rounded to bf16 on the way in and the bf16 result
    is cast back.  A bf16 bias [n_total] is fused into the kernel's epilogue; a bias of another
    dtype is added afterwards in that dtype (as the reference's out.add_(bias)).  out: a bf16
    [M, n_total] view with unit column stride (a column slice of a wider output) to write
    into, for bf16 x; it is returned.  workspace: a zero-filled int32 buffer of at least
    ``gqk_workspace_bytes_max()`` bytes to use instead of the device's shared one (calls that may
    overlap in time on different streams each need their own).  Nothing is allocated here
    besides the output, below DEQUANT_MIN_M rows; from there the regime is the reference's
    dequantize + vendor GEMM (a shard's bf16 weights live for the duration of its GEMMs)."""
    _require_gpu(x, "mul_mat_grouped")
    if x.dim() != 2 or x.shape[1] != gl.K:
        raise ValueError(f"mul_mat_grouped: x {tuple(x.shape)} does not match K={gl.K}")
    xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
    if xb.stride(1) != 1 or xb.stride(0) % 8 or not _addr_aligned(xb, 16):
        xb = xb.contiguous()
    ws = gl.workspace if workspace is None else workspace
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
        if xb.shape[0] >= DEQUANT_MIN_M:
            _dequant_mm_into(xb, gl, out)
            fused = None
        else:
            fused_mul_mat_gguf_grouped_out(xb, gl.packed, gl.descs, gl.plans, ws, out, fused)
        if bias is not None and fused is None:
            out.add_(bias)
        return out
    if xb.shape[0] >= DEQUANT_MIN_M:
        y = torch.empty((xb.shape[0], gl.n_total), dtype=torch.bfloat16, device=x.device)
        _dequant_mm_into(xb, gl, y)
        fused = None
    else:
        y = fused_mul_mat_gguf_grouped(xb, gl.packed, gl.descs, gl.plans, gl.n_total, ws, fused)
    y = y if x.dtype == torch.bfloat16 else y.to(x.dtype)
    if bias is not None and fused is None:
        y.add_(bias)
    return y


def _dequant_mm_into(xb: torch.Tensor, gl: GroupedLayer, y: torch.Tensor) -> None:
    """The dequant regime (DEQUANT_MIN_M rows and more): each shard's weights decoded from its
    tiles to bf16 (the same bits as the fused kernels' decode) and multiplied by torch's bf16 GEMM
    in row chunks, into the shard's columns of y.  Allocates the shard's bf16 weights for the
    duration of its GEMMs."""
    col = 0
    chunk = DEQUANT_CHUNK_M_LONG_K if gl.K > DEQUANT_LONG_K else DEQUANT_CHUNK_M
    for view, n, wt in zip(gl.views, gl.n_outs, gl.weight_types):
        w = dequantize_tiles(view, n, gl.K, wt, torch.bfloat16)
        for r0 in range(0, xb.shape[0], chunk):
            r1 = min(xb.shape[0], r0 + chunk)
            ys = y[r0:r1, col:col + n]
            if ys.is_contiguous():
                torch.mm(xb[r0:r1], w.t(), out=ys)
            else:
                ys.copy_(torch.mm(xb[r0:r1], w.t()))
        del w
        col += n


_CACHE_ATTR = "_gguf_hip_layers"
# views of one base tensor whose layers the cache keeps (a merged qkv / gate_up parameter has 2-3
# shard views); beyond it the least recently used entry is dropped
CACHE_MAX_VIEWS = 8


def cached_layer(weight: torch.Tensor, weight_type: int, n_out: int, kind: str = "rows") -> GroupedLayer:
    """The grouped layer of a weight given as raw GGUF rows (kind "rows", any row stride) or as one
    shard's tiles ("tiles"), made on the first call and kept in a dict attached to the weight's base
    tensor (the storage the view belongs to, e.g. a layer parameter), so it goes with that storage
    and a freed weight's entry can never serve another (the reference keys its caches by the
    layer's own metadata for that reason, gguf-plugin/gluon/tiles_grouped.py:271-275).  The key is
    the view's offset, shape, strides, type and rows, and the entry is rebuilt when the base's
    version counter shows an in-place write.  Later calls allocate nothing and copy nothing.

    Memory: for raw rows the entry holds a repacked copy of the weight (its own size again in
    HBM) beside the raw rows, which stay with their owner; ``drop_cached_layers(weight)`` frees
    it, and at most ``CACHE_MAX_VIEWS`` views of one base tensor are kept (least recently used
    dropped).  The first call on a weight repacks and plans (allocations, a host-to-device copy of
    the plans), so it raises under HIP graph capture: make it once eagerly before capturing."""
    base = weight._base if weight._base is not None else weight
    key = (kind, weight.storage_offset(), tuple(weight.shape), tuple(weight.stride()), int(weight_type), int(n_out),
           str(weight.device))
    cache = getattr(base, _CACHE_ATTR, None)
    if cache is None:
        cache = {}
        setattr(base, _CACHE_ATTR, cache)
    hit = cache.get(key)
    if hit is not None and hit[0] == base._version:
        cache[key] = cache.pop(key)          # most recently used last
        return hit[1]
    if weight.is_cuda and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            "gguf_hip: the first call on a GGUF weight repacks it into the tile layout and uploads its launch "
            "plans (device allocations and a host-to-device copy), which a HIP graph capture cannot record; "
            "call it once eagerly before capturing (later calls allocate only the output)")
    if kind == "rows":
        gl = pack_layer([weight], [n_out], [weight_type])
    elif kind == "tiles":
        per_row = weight.numel() // (-(-n_out // 64) * 64)
        rec = type_info(weight_type)[2]
        if per_row % rec:
            raise ValueError(f"cached_layer: {weight.numel()} tile bytes do not hold {n_out} rows of type {weight_type}")
        flat = weight.reshape(-1) if weight.is_contiguous() else weight.contiguous().reshape(-1)
        gl = grouped_layer_from_packed(flat, [n_out], [weight_type], per_row // rec * 256)
    else:
        raise ValueError(f"cached_layer: kind {kind!r}")
    cache.pop(key, None)
    cache[key] = (base._version, gl)
    while len(cache) > CACHE_MAX_VIEWS:
        cache.pop(next(iter(cache)))
    return gl


def drop_cached_layers(weight: torch.Tensor) -> int:
    """Frees the layers ``cached_layer`` keeps for every view of weight's base tensor (their tile
    copies and plans); returns how many were dropped.  A later call on the weight rebuilds its entry."""
    base = weight._base if weight._base is not None else weight
    cache = getattr(base, _CACHE_ATTR, None)
    if not cache:
        return 0
    n = len(cache)
    cache.clear()
    return n


def fused_mul_mat_gguf(x: torch.Tensor, qweight: torch.Tensor, qweight_type: int) -> torch.Tensor:
    """The plugin's module-level op on raw rows (``_fused_mul_mat_gguf``,
    gguf-plugin/patches/gguf-prefill-dispatch.patch:9-50): y = x @ W^T.  The first call on a weight
    repacks and plans it (``cached_layer``); later calls reuse that and allocate only the output."""
    if qweight_type in UNQUANTIZED_TYPES:
        return x @ (qweight if qweight.dtype == x.dtype else qweight.to(x.dtype)).T
    if qweight_type not in GGUF_TYPES:
        raise NotImplementedError(f"Unsupported GGUF quantization type: {qweight_type}")
    n = qweight.shape[0]
    if x.shape[0] == 0:
        return torch.empty((0, n), dtype=x.dtype, device=x.device)
    return mul_mat_grouped(x, cached_layer(qweight, qweight_type, n, "rows"))
