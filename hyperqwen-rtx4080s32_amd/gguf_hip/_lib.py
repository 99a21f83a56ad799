"""ctypes binding of libgqk.so (the C ABI declared in include/gguf_hip.h).

The library is the only compute path of this package: if it is missing, importing this module
raises, and nothing falls back to a CPU implementation.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgqk.so")

GQK_OK = 0
GQK_ERR_TYPE = -1
GQK_ERR_SHAPE = -2
GQK_ERR_FORM = -3
GQK_ERR_HIP = -4
GQK_ERR_ARG = -5
GQK_FORM_GEMV = 1
GQK_FORM_GEMM = 2
GQK_CTR_BYTES = 262144            # the arrival-counter region at the start of every workspace
GQK_NOALLOC_SCRATCH_BYTES = GQK_CTR_BYTES + (32 << 20)   # gqk_linear_noalloc's per-GPU device array
GQK_DTYPE_F32, GQK_DTYPE_BF16, GQK_DTYPE_F16 = 0, 1, 2

# every entry point include/gguf_hip.h declares
EXPORTS = ("gqk_last_error", "gqk_version", "gqk_type_info", "gqk_dequantize", "gqk_dequantize_tiles",
           "gqk_tiles_bytes", "gqk_repack", "gqk_unrepack", "gqk_plan", "gqk_linear_workspace_bytes",
           "gqk_workspace_bytes_max", "gqk_linear", "gqk_linear_noalloc", "gqk_ggml_type_size",
           "gqk_gguf_open", "gqk_gguf_close", "gqk_gguf_info", "gqk_gguf_tensor_at", "gqk_gguf_find_tensor",
           "gqk_gguf_kv_at", "gqk_gguf_find_kv", "gqk_gguf_kv_string", "gqk_gguf_upload_tiles", "gqk_read_floor")


class GqkShard(ctypes.Structure):
    _fields_ = [("ggml_type", ctypes.c_int32), ("reserved", ctypes.c_int32), ("n", ctypes.c_int64),
                ("offset", ctypes.c_int64)]


class GqkPlanInfo(ctypes.Structure):
    _fields_ = [("form", ctypes.c_int32), ("m_max", ctypes.c_int32), ("g", ctypes.c_int32), ("bm", ctypes.c_int32),
                ("split", ctypes.c_int32), ("n_desc", ctypes.c_int32), ("types_mask", ctypes.c_int32),
                ("nb", ctypes.c_int32), ("nw", ctypes.c_int32), ("ctr_bytes", ctypes.c_int32),
                ("n_total", ctypes.c_int64), ("workspace_bytes", ctypes.c_int64)]

    def as_tuple(self) -> tuple:
        return tuple(getattr(self, f) for f, _ in self._fields_)

    @classmethod
    def from_tuple(cls, t) -> "GqkPlanInfo":
        return cls(*t)


class GqkGgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("ggml_type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("dims", ctypes.c_int64 * 4), ("offset", ctypes.c_int64), ("nbytes", ctypes.c_int64),
                ("data", ctypes.c_void_p)]


class GqkGgufKv(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("type", ctypes.c_int32), ("array_type", ctypes.c_int32),
                ("count", ctypes.c_int64), ("i64", ctypes.c_int64), ("f64", ctypes.c_double),
                ("data", ctypes.c_void_p)]


class GqkError(RuntimeError):
    """A libgqk call failed; ``code`` is the GQK_ERR_* status."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"gguf_hip: the HIP library {LIB_PATH} is not built; run `python -m gguf_hip.build` "
            "(or __graft_entry__.build()) first. There is no CPU fallback.")
    lib = ctypes.CDLL(LIB_PATH)
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    sig = {
        "gqk_last_error": (ctypes.c_char_p, []),
        "gqk_version": (i32, []),
        "gqk_type_info": (i32, [i32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]),
        "gqk_dequantize": (i32, [vp, i64, i32, i64, i64, vp, i64, i32, vp]),
        "gqk_dequantize_tiles": (i32, [vp, i32, i64, i64, vp, i64, i32, vp]),
        "gqk_tiles_bytes": (i64, [i32, i64, i64]),
        "gqk_repack": (i32, [vp, i64, i32, i64, i64, vp, vp]),
        "gqk_unrepack": (i32, [vp, i32, i64, i64, vp, i64, vp]),
        "gqk_plan": (i32, [ctypes.POINTER(GqkShard), i32, i64, i32, i32, i32, ctypes.POINTER(ctypes.c_int32), i64,
                           ctypes.POINTER(GqkPlanInfo)]),
        "gqk_linear_workspace_bytes": (i64, [ctypes.POINTER(GqkPlanInfo), i32]),
        "gqk_workspace_bytes_max": (i64, []),
        "gqk_linear": (i32, [vp, vp, ctypes.POINTER(GqkPlanInfo), vp, i64, i32, vp, i64, vp, vp, i64, vp]),
        "gqk_linear_noalloc": (i32, [vp, vp, ctypes.POINTER(GqkPlanInfo), vp, i64, i32, vp, i64, vp, vp]),
        "gqk_ggml_type_size": (i32, [i32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]),
        "gqk_gguf_open": (i32, [ctypes.c_char_p, ctypes.POINTER(vp)]),
        "gqk_gguf_close": (None, [vp]),
        "gqk_gguf_info": (i32, [vp, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64),
                                ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64),
                                ctypes.POINTER(ctypes.c_int32)]),
        "gqk_gguf_tensor_at": (i32, [vp, i64, ctypes.POINTER(GqkGgufTensor)]),
        "gqk_gguf_find_tensor": (i64, [vp, ctypes.c_char_p]),
        "gqk_gguf_kv_at": (i32, [vp, i64, ctypes.POINTER(GqkGgufKv)]),
        "gqk_gguf_find_kv": (i64, [vp, ctypes.c_char_p]),
        "gqk_gguf_kv_string": (i32, [vp, i64, i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int64)]),
        "gqk_gguf_upload_tiles": (i32, [vp, i64, vp, i64, vp, vp]),
        "gqk_read_floor": (i32, [vp, i64, i32, i32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int, what: str) -> int:
    """Map a GQK status to the reference's exception classes: an unsupported type raises
    NotImplementedError (gguf-plugin/gluon/interface.py:78-79), a broken shape contract
    ValueError, everything else RuntimeError (GqkError)."""
    if rc >= 0:
        return rc
    msg = f"{what}: {lib.gqk_last_error().decode(errors='replace')}"
    if rc == GQK_ERR_TYPE:
        raise NotImplementedError(msg)
    if rc in (GQK_ERR_SHAPE, GQK_ERR_ARG):
        raise ValueError(msg)
    raise GqkError(rc, msg)
