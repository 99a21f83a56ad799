"""GGUF v3 files through libgqk's C++ reader, and the load path from a file to grouped layers.

The reference's plugin receives its tensors from vLLM's GGUF loader (gguf-py 0.17.1's
``GGUFReader``) and repacks every quantized shard at load time (``_create_tiles`` /
``_create_groups``, gguf-plugin/patches/gguf-tiles-all-types.patch:59-131,
gguf-plugin/patches/gguf-tiles-grouped.patch:84-115).  Here:

    with GGUFFile(path) as f:
        f.fields["general.architecture"], f.tensors[0].name, f.raw("blk.0.ffn_down.weight")
        layers, skipped = load_grouped_layers(f, torch.device("cuda"))

``load_grouped_layers`` groups the tensors of one linear call (q/k/v, gate/up: the shard order
of vLLM's QKVParallelLinear / MergedColumnParallelLinear) into layer runs, uploads each tensor's
raw rows straight into its slice of the run's packed tile buffer (one host-to-device copy and
one repack launch per tensor, gqk_gguf_upload_tiles) and plans the run.
"""
from __future__ import annotations

import ctypes
import re
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import GqkGgufKv, GqkGgufTensor, check, lib
from .ops import GGUF_TYPES, GroupedLayer, _require_gpu, _stream, grouped_layer_from_packed, tiles_bytes

GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32 = range(6)
GGUF_FLOAT32, GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64 = range(6, 13)
_NP = {GGUF_UINT8: np.uint8, GGUF_INT8: np.int8, GGUF_UINT16: np.uint16, GGUF_INT16: np.int16,
       GGUF_UINT32: np.uint32, GGUF_INT32: np.int32, GGUF_FLOAT32: np.float32, GGUF_BOOL: np.bool_,
       GGUF_UINT64: np.uint64, GGUF_INT64: np.int64, GGUF_FLOAT64: np.float64}


def ggml_type_size(ggml_type: int) -> tuple[int, int]:
    """(weights per block, bytes per block): gguf.GGML_QUANT_SIZES[ggml_type]."""
    block, nbytes = ctypes.c_int32(), ctypes.c_int32()
    check(lib.gqk_ggml_type_size(ggml_type, ctypes.byref(block), ctypes.byref(nbytes)), "ggml_type_size")
    return block.value, nbytes.value


@dataclass(frozen=True)
class GGUFTensor:
    """One tensor info.  dims in GGUF order (dims[0] = weights per row); shape = reversed dims,
    so a matrix is (N rows, K)."""
    index: int
    name: str
    ggml_type: int
    dims: tuple[int, ...]
    offset: int     # absolute byte offset of the data in the file
    nbytes: int     # packed bytes (-1: a type without a fixed block size)

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(reversed(self.dims))


class GGUFFile:
    """A memory-mapped GGUF v3 file (read only).  ``fields`` holds the metadata (scalars as
    Python numbers, strings as str, arrays as lists of str or numpy arrays); ``tensors`` the
    tensor infos in file order.  Arrays returned by ``raw`` view the mapping and stay valid
    while the file is open."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib.gqk_gguf_open(str(path).encode(), ctypes.byref(h)), f"gguf_open({path})")
        self._h = h
        self.path = str(path)
        nt, nkv, al, do = (ctypes.c_int64() for _ in range(4))
        ver = ctypes.c_int32()
        check(lib.gqk_gguf_info(h, ctypes.byref(nt), ctypes.byref(nkv), ctypes.byref(al), ctypes.byref(do),
                                ctypes.byref(ver)), "gguf_info")
        self.version, self.alignment, self.data_offset = ver.value, al.value, do.value
        self.fields: dict[str, object] = {}
        for i in range(nkv.value):
            kv = GqkGgufKv()
            check(lib.gqk_gguf_kv_at(h, i, ctypes.byref(kv)), "gguf_kv_at")
            self.fields[kv.key.decode()] = self._value(i, kv)
        self.tensors: list[GGUFTensor] = []
        for i in range(nt.value):
            t = GqkGgufTensor()
            check(lib.gqk_gguf_tensor_at(h, i, ctypes.byref(t)), "gguf_tensor_at")
            self.tensors.append(GGUFTensor(i, t.name.decode(), t.ggml_type, tuple(t.dims[:t.n_dims]), t.offset,
                                           t.nbytes))
        self._by_name = {t.name: t for t in self.tensors}

    def _string(self, i: int, j: int) -> str:
        s, n = ctypes.c_char_p(), ctypes.c_int64()
        check(lib.gqk_gguf_kv_string(self._h, i, j, ctypes.byref(s), ctypes.byref(n)), "gguf_kv_string")
        return ctypes.string_at(s, n.value).decode("utf-8", errors="replace")

    def _value(self, i: int, kv: GqkGgufKv):
        if kv.type == GGUF_STRING:
            return self._string(i, 0)
        if kv.type == GGUF_ARRAY:
            if kv.array_type == GGUF_STRING:
                return [self._string(i, j) for j in range(kv.count)]
            dt = np.dtype(_NP[kv.array_type])
            buf = (ctypes.c_uint8 * (kv.count * dt.itemsize)).from_address(kv.data) if kv.count else b""
            return np.frombuffer(bytes(buf), dtype=dt).copy()
        if kv.type in (GGUF_FLOAT32, GGUF_FLOAT64):
            return float(kv.f64)
        if kv.type == GGUF_BOOL:
            return bool(kv.i64)
        if kv.type == GGUF_UINT64:
            return kv.i64 & 0xFFFFFFFFFFFFFFFF
        return int(kv.i64)

    def _handle(self) -> ctypes.c_void_p:
        if not getattr(self, "_h", None):
            raise ValueError(f"{self.path}: the file is closed")
        return self._h

    def tensor(self, name: str) -> GGUFTensor:
        try:
            return self._by_name[name]
        except KeyError:
            raise KeyError(f"{self.path}: no tensor '{name}'") from None

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as uint8 [rows, bytes per row] (a view of the mapping)."""
        t = self.tensor(name)
        if t.nbytes < 0:
            raise NotImplementedError(f"{name}: GGML type {t.ggml_type} has no fixed block size here")
        info = GqkGgufTensor()
        check(lib.gqk_gguf_tensor_at(self._handle(), t.index, ctypes.byref(info)), "gguf_tensor_at")
        arr = np.ctypeslib.as_array((ctypes.c_uint8 * t.nbytes).from_address(info.data))
        rows = int(np.prod(t.dims[1:])) if len(t.dims) > 1 else 1
        return arr.reshape(rows, t.nbytes // rows)

    def upload_tiles(self, name: str, tiles: torch.Tensor, staging: torch.Tensor) -> None:
        """Raw rows of a quantized matrix -> `tiles` (a uint8 device buffer of exactly the tile
        layout's size) through `staging` (uint8 device, >= the tensor's bytes), on the current stream."""
        t = self.tensor(name)
        _require_gpu(tiles, "upload_tiles")
        _require_gpu(staging, "upload_tiles")
        if len(t.dims) != 2:
            raise ValueError(f"upload_tiles: {name} is not a matrix")
        need = tiles_bytes(t.ggml_type, t.dims[1], t.dims[0])
        if tiles.dtype != torch.uint8 or not tiles.is_contiguous() or tiles.numel() != need:
            raise ValueError(f"upload_tiles: {name} needs a contiguous uint8 tile buffer of {need} bytes")
        check(lib.gqk_gguf_upload_tiles(self._handle(), t.index, ctypes.c_void_p(staging.data_ptr()),
                                        staging.numel() * staging.element_size(), ctypes.c_void_p(tiles.data_ptr()),
                                        _stream(tiles.device)), f"upload_tiles({name})")

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib.gqk_gguf_close(self._h)
            self._h = None

    def __enter__(self) -> "GGUFFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            self.close()


# llama.cpp tensor names whose linear calls vLLM merges, in its shard order
_MERGED = ((("attn_q", "attn_k", "attn_v"), "attn_qkv"), (("ffn_gate", "ffn_up"), "ffn_gate_up"))
_BLK = re.compile(r"^(blk\.\d+\.)([A-Za-z0-9_]+)\.weight$")


def layer_runs(tensors: list[GGUFTensor]) -> list[tuple[str, list[GGUFTensor]]]:
    """The linear calls of a file: 2-D ``*.weight`` tensors, with each block's q/k/v and gate/up
    merged into one run (vLLM's QKVParallelLinear / MergedColumnParallelLinear shard order).
    Runs come in file order of their first tensor.  The token embedding is not a linear call
    (its rows are gathered: gguf-plugin/patches/gguf-tiles-all-types.patch:76-82)."""
    by_name = {t.name: t for t in tensors}
    member_of: dict[str, tuple[str, list[GGUFTensor]]] = {}
    for t in tensors:
        m = _BLK.match(t.name)
        if not m:
            continue
        for parts, run in _MERGED:
            if m.group(2) in parts:
                names = [f"{m.group(1)}{p}.weight" for p in parts]
                if all(n in by_name and len(by_name[n].dims) == 2 for n in names):
                    for n in names:
                        member_of[n] = (m.group(1) + run, [by_name[n] for n in names])
    runs, emitted = [], set()
    for t in tensors:
        if len(t.dims) != 2 or not t.name.endswith(".weight") or t.name == "token_embd.weight":
            continue
        if t.name in member_of:
            run = member_of[t.name]
            if run[0] not in emitted:
                emitted.add(run[0])
                runs.append(run)
            continue
        runs.append((t.name[:-len(".weight")], [t]))
    return runs


def load_grouped_layers(f: GGUFFile, device: torch.device, runs: list[tuple[str, list[GGUFTensor]]] | None = None,
                        target_wgs: int = 0) -> tuple[dict[str, GroupedLayer], dict[str, str]]:
    """Upload and plan every layer run whose tensors are all of a type with a kernel here and
    share one K.  Returns (run name -> GroupedLayer, run name -> why it was skipped); unquantized
    runs (F32/F16/BF16) are skipped too: the linear method multiplies those with torch."""
    device = torch.device(device)
    runs = layer_runs(f.tensors) if runs is None else runs
    layers: dict[str, GroupedLayer] = {}
    skipped: dict[str, str] = {}
    todo = []
    for name, members in runs:
        bad = [t for t in members if t.ggml_type not in GGUF_TYPES]
        if bad:
            skipped[name] = f"GGML type {bad[0].ggml_type} of {bad[0].name} has no kernel here"
            continue
        Ks = {t.dims[0] for t in members}
        if len(Ks) != 1 or next(iter(Ks)) % 256:
            skipped[name] = f"row lengths {sorted(Ks)} (one K, a multiple of 256, per run)"
            continue
        todo.append((name, members))
    if not todo:
        return layers, skipped
    staging = torch.empty(max(t.nbytes for _, ms in todo for t in ms), dtype=torch.uint8, device=device)
    for name, members in todo:
        K = members[0].dims[0]
        sizes = [tiles_bytes(t.ggml_type, t.dims[1], K) for t in members]
        packed = torch.empty(sum(sizes), dtype=torch.uint8, device=device)
        off = 0
        for t, size in zip(members, sizes):
            f.upload_tiles(t.name, packed[off:off + size], staging)
            off += size
        layers[name] = grouped_layer_from_packed(packed, [t.dims[1] for t in members],
                                                 [t.ggml_type for t in members], K, target_wgs)
    torch.cuda.synchronize(device)   # the staging buffer is released on return
    return layers, skipped
