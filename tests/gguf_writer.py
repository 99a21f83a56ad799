"""A minimal GGUF v3 writer for the tests (test infrastructure: the library only reads GGUF).

Writes the published layout: magic "GGUF", u32 version 3, u64 tensor count, u64 key/value
count, key/values (u64-length string key, u32 value type, value), tensor infos (name, u32
n_dims, u64 dims in GGUF order, u32 ggml type, u64 offset relative to the data section),
padding to the alignment, then the tensors' bytes, each at an aligned offset.  ``sparse=True``
writes the headers only and extends the file to its full size without writing the data (a
file-system hole), so a model-sized tensor table costs no disk.
"""
from __future__ import annotations

import struct

import numpy as np

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f", BOOL: "<?",
        UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
# (weights per block, bytes per block) of the GGML types the tests write
TYPE_SIZE = {0: (1, 4), 1: (1, 2), 2: (32, 18), 6: (32, 22), 8: (32, 34), 10: (256, 84), 11: (256, 110),
             12: (256, 144), 13: (256, 176), 14: (256, 210), 16: (256, 66), 17: (256, 74), 18: (256, 98),
             20: (32, 18), 21: (256, 110), 22: (256, 82), 23: (256, 136), 29: (256, 56), 30: (1, 2)}
TYPE_IDS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q5_0": 6, "Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13,
            "Q6_K": 14, "IQ2_XXS": 16, "IQ2_XS": 17, "IQ3_XXS": 18, "IQ4_NL": 20, "IQ3_S": 21, "IQ2_S": 22,
            "IQ4_XS": 23, "IQ1_M": 29, "BF16": 30}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def nbytes(ggml_type: int, dims: tuple[int, ...]) -> int:
    block, size = TYPE_SIZE[ggml_type]
    n = int(np.prod(dims))
    assert dims[0] % block == 0
    return n // block * size


def write_gguf(path, kvs: list[tuple[str, int, object]], tensors: list[tuple[str, tuple[int, ...], int, bytes | None]],
               alignment: int = 32, sparse: bool = False, version: int = 3) -> list[int]:
    """kvs: (key, value type, value); an ARRAY value is (element type, items).  tensors: (name,
    dims in GGUF order, ggml type, raw bytes or None with sparse=True).  Returns each tensor's
    absolute data offset."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kvs))
    for k, vt, v in kvs:
        head += _str(k) + struct.pack("<I", vt) + _value(vt, v)
    rel, off = [], 0
    for name, dims, gt, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        rel.append(off)
        off += nbytes(gt, dims)
    for (name, dims, gt, data), r in zip(tensors, rel):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gt, r)
    data_off = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_off - len(head)))
        if sparse:
            f.truncate(data_off + off)
        else:
            for (name, dims, gt, data), r in zip(tensors, rel):
                assert len(data) == nbytes(gt, dims), name
                f.seek(data_off + r)
                f.write(data)
            f.truncate(data_off + off)
    return [data_off + r for r in rel]
