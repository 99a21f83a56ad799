"""Builds the HIP library ``libgqk.so`` in-tree for gfx950 (hipcc, no JIT cache).

    python hyperqwen-rtx4080s32_amd/gguf_hip/build.py     # as a script: no package import, so a
                                                          # stale or missing library is no obstacle
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)                      # hyperqwen-rtx4080s32_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libgqk.so")
SOURCES = ("gqk_api.hip", "gqk_codec.hip", "gqk_gemv.hip", "gqk_gemm.hip", "gqk_gguf.cpp")
ARCH = os.environ.get("GQK_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
    "-I", os.path.join(REPO, "include"), "-I", CSRC,
    # packed fp32 VALU ops stay off (the pool's boxes have shown silent errors from them)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs (no v_accvgpr_read round trips in the GEMV epilogue)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _run(cmd: list[str]) -> None:
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed ({p.returncode}): {' '.join(cmd)}\n{p.stderr[-6000:]}")


def build(jobs: int | None = None) -> str:
    """Compile every source (HIP kernels; the host-only GGUF reader) and link libgqk.so (always rebuilds); returns the library path."""
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=jobs or min(len(cmds), os.cpu_count() or 4)) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(int(sys.argv[1]) if len(sys.argv) > 1 else None))
