"""Writes the golden fixtures under tests/golden/ (run in the build container, where the
reference is mounted read-only at /root/reference; the fixtures are committed, the reference
never travels).

* ``kq_ref_<type>.npz`` (Q8_0=8, Q3_K=11, Q5_K=13, Q6_K=14): random valid rows and their
  fp32 dequantization by the reference's own numpy model ``gguf-plugin/gluon/kq_ref.py``
  (``random_rows`` ``:94-112``, ``parse`` ``:30-80``, ``dequantize`` ``:83-91``), which the
  reference holds bit-exact against gguf-py (``gguf-plugin/test_gguf_rco_cpu.py:345-356``; same
  seed 3 and 6 x 512 shape).  These pin the bit layouts of those four formats; nothing else in
  the reference states them as data.
* ``iq3s_grid_x4.npy``: the 512 IQ3_S grid words as the reference's patch text writes them
  (post-patch lines of ``gguf-plugin/patches/gguf-iq3s-grid-top-magnitude.patch:18-138``, in
  quarter units).
* ``iq4_kvalues.npy``: the IQ4 value table as written at ``gguf-plugin/gluon/iq4xs.py:36``.
* ``qwen35_iq3s_tensors.json``: the tensor table (name, GGUF dims, GGML type) of the published
  IQ3_S model file as the reference records it in ``gguf-plugin/iq3s-tensor-names.json`` (read from
  that file's header; used by the reference's CPU gate, ``gguf-plugin/test_gguf_rco_cpu.py:84-127``).

Usage: ``python tests/golden/make_golden.py`` (everything) or ``... tensors`` (the table only)
"""
from __future__ import annotations

import importlib.util
import json
import os
import re
import sys

import numpy as np

REF = "/root/reference/gguf-plugin"
HERE = os.path.dirname(os.path.abspath(__file__))


def _load_kq_ref():
    spec = importlib.util.spec_from_file_location("kq_ref_reference", os.path.join(REF, "gluon", "kq_ref.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)   # numpy-only module (its only import is numpy, kq_ref.py:8)
    return mod


def grid_from_patch() -> np.ndarray:
    lines = open(os.path.join(REF, "patches", "gguf-iq3s-grid-top-magnitude.patch"), encoding="utf-8").read().splitlines()
    start = next(i for i, line in enumerate(lines) if "iq3xs_grid[512]" in line)
    vals = []
    for line in lines[start + 1:]:
        if line.startswith("-"):          # pre-patch lines
            continue
        if "};" in line:
            break
        vals += [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]{8}", line)]
    assert len(vals) == 512
    return np.array(vals, dtype=np.uint32)


def kvalues_from_text() -> np.ndarray:
    text = open(os.path.join(REF, "gluon", "iq4xs.py"), encoding="utf-8").read()
    m = re.search(r"^KVALUES = \(([^)]*)\)", text, re.M)
    return np.array([int(v) for v in m.group(1).split(",")], dtype=np.int8)


def tensor_table() -> None:
    doc = json.load(open(os.path.join(REF, "iq3s-tensor-names.json"), encoding="utf-8"))
    out = {"file": doc["file"], "architecture": doc["architecture"],
           "tensors": [{"name": t["name"], "dims": t["dims"], "type": t["type"]} for t in doc["tensors"]]}
    with open(os.path.join(HERE, "qwen35_iq3s_tensors.json"), "w", encoding="utf-8") as f:
        f.write('{"file": %s, "architecture": %s, "tensors": [\n' % (json.dumps(out["file"]), json.dumps(out["architecture"])))
        f.write(",\n".join(json.dumps(t) for t in out["tensors"]))
        f.write("\n]}\n")


def main() -> None:
    if sys.argv[1:] == ["tensors"]:
        tensor_table()
        return
    tensor_table()
    kq = _load_kq_ref()
    rng = np.random.default_rng(3)
    for wt in (8, 11, 13, 14):
        raw = kq.random_rows(rng, 6, 512, wt)
        w = kq.dequantize(kq.parse(raw, wt))
        assert w.dtype == np.float32 and w.shape == (6, 512)
        np.savez_compressed(os.path.join(HERE, f"kq_ref_{wt}.npz"), raw=raw, w=w)
    np.save(os.path.join(HERE, "iq3s_grid_x4.npy"), grid_from_patch())
    np.save(os.path.join(HERE, "iq4_kvalues.npy"), kvalues_from_text())
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
