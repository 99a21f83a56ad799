"""CPU tests of the C ABI and host logic: the library loads and exports every declared entry
point, its type tables agree with the oracle's block sizes, the tile planes cover every raw
byte once, and the launch plans / errors follow the contract (no kernel is launched here)."""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import ggml_ref as G

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_exports_every_declared_symbol():
    from gguf_hip import _lib

    hdr = open(os.path.join(REPO, "include", "gguf_hip.h"), encoding="utf-8").read()
    declared = set(re.findall(r"^\s*(?:const\s+char\*|int64_t|int|void)\s+(gqk_\w+)\s*\(", hdr, re.M))
    assert declared == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(_lib.lib, name)
    assert _lib.lib.gqk_version() >= 100


@pytest.mark.parametrize("wt", G.ALL_TYPES)
def test_type_tables(wt):
    from gguf_hip import ops

    bw, bb, rec, nplanes = ops.type_info(wt)
    _, obw, obb = G.TYPES[wt]
    assert (bw, bb) == (obw, obb)
    assert rec == bb * 256 // bw
    planes = ops.type_planes(wt)
    assert len(planes) == nplanes
    covered = []
    for size, nseg, off, seglen, stride, width in planes:
        assert size == nseg * seglen and size % width == 0 and width in (2, 4, 8, 16)
        for s in range(nseg):
            covered += list(range(off + s * stride, off + s * stride + seglen))
    assert sorted(covered) == list(range(rec))          # every raw byte of the record exactly once
    # 16-byte planes come first in every layout except for the short trailing fields
    offs = np.cumsum([0] + [p[0] for p in planes])[:-1]
    for (size, *_), o in zip(planes, offs):
        if size % 16 == 0:
            assert (64 * o) % 16 == 0


def test_unsupported_type_and_bad_shapes():
    from gguf_hip import _lib, ops

    with pytest.raises(NotImplementedError):
        ops.type_info(16)                                  # IQ2_XXS: no kernel
    assert _lib.lib.gqk_dequantize(None, 0, 99, 1, 32, None, 32, 0, None) == _lib.GQK_ERR_TYPE
    assert _lib.lib.gqk_dequantize(None, 0, 12, 1, 100, None, 100, 0, None) == _lib.GQK_ERR_SHAPE
    assert "multiple" in _lib.lib.gqk_last_error().decode()
    assert _lib.lib.gqk_tiles_bytes(12, 10, 300) == _lib.GQK_ERR_SHAPE
    assert _lib.lib.gqk_tiles_bytes(12, 70, 512) == 128 * 2 * 144
    with pytest.raises(ValueError):
        ops.plan([(12, 64, 0), (21, 64, 12345)], 512, 1)  # shards not back to back
    with pytest.raises(ValueError):
        ops.plan([(12, 64, 0)], 500, 1)                  # K not a multiple of 256
    with pytest.raises(NotImplementedError):
        ops.plan([(12, 64, 0), (16, 64, 64 * 2 * 144)], 512, 1)
    with pytest.raises(ValueError):
        ops.quant_shape(12, 4, 145)


def _rows(desc):
    return desc.numpy().reshape(-1, 16)


def test_plan_gemv_balanced_split_partition():
    from gguf_hip import ops

    for target in (1, 16, 97, 1024, 4096, 0):
        info, desc = ops.plan([(21, 6144, 0)], 20 * 256, 1, target)
        d = _rows(desc)
        S, nw = info.split, info.nw
        assert info.form == 1 and info.g == 1 and info.m_max == 4
        assert 1 <= nw <= 4 and S * nw <= 20                # every wave keeps >= 1 super-block
        if S > 1:
            assert nw == 4                                  # K splits across workgroups only past a full one
        assert d.shape[0] == info.n_desc == 96 * S          # one workgroup per (64-row tile, split)
        first = d[d[:, 3] == 0]                             # the workgroups of tile 0
        assert first[:, 5].tolist() == [s * 20 // S for s in range(S)]
        assert first[:, 6].tolist() == [(s + 1) * 20 // S for s in range(S)]
        assert first[:, 7].tolist() == list(range(S)) and (first[:, 11] == 0).all()
        assert sorted(set(d[:, 11].tolist())) == list(range(96))   # one arrival counter per tile
        # the counter region: one int per tile, at least the GEMM's 1024 workgroups, 256-byte rounded
        assert info.ctr_bytes == 4096
        assert info.workspace_bytes == (4096 + S * 4 * 6144 * 4 if S > 1 else 0)
    assert ops.plan([(21, 6144, 0)], 20 * 256, 1, 1)[0].nw == 1
    info = ops.plan([(21, 6144, 0)], 20 * 256, 1, 4096)[0]
    assert (info.nw, info.split) == (4, 5)                  # 43 waves per tile wanted: 4 x min(11, 20 // 4)
    info = ops.plan([(21, 6144, 0)], 20 * 256, 8, 0)[0]
    assert (info.nw, info.split) == (4, 5)                  # default target 2048 waves: 22 per tile


def test_plan_descriptor_rows_mixed_layer():
    from gguf_hip import ops

    K = 3 * 256
    off2 = ops.tiles_bytes(21, 70, K)
    info, desc = ops.plan([(21, 70, 0), (12, 300, off2)], K, 8, 4)
    d = _rows(desc)
    assert info.types_mask == 0 and info.n_total == 370 and info.g == 2
    assert info.split == 1 and info.workspace_bytes == 0
    # one counter region for every plan of a layer, so one workspace serves every M
    for shards, k in (([(21, 70, 0), (12, 300, off2)], K), ([(12, 70000, 0)], 512)):
        regions = {ops.plan(shards, k, m, t)[0].ctr_bytes for m in (1, 8, 16, 17, 100, 2048) for t in (0, 1, 4096)}
        assert regions == {max(4096, ((sum((n + 63) // 64 for _, n, _ in shards) * 4 + 255) // 256) * 256)}
    # one workgroup per tile: IQ3_S 2 tiles (64 + 6 rows), Q4_K 5 tiles (4 x 64 + 44)
    assert d[:, 0].tolist() == [21, 21, 12, 12, 12, 12, 12]
    assert d[:, 3].tolist() == [0, 1, 0, 1, 2, 3, 4] and d[:, 4].tolist() == [1] * 7
    assert d[:, 8].tolist() == [0, 64, 70, 134, 198, 262, 326] and d[:, 9].tolist() == [64, 6, 64, 64, 64, 64, 44]
    assert d[2, 1] == off2 and d[:, 10].tolist() == [3] * 7 and d[:, 11].tolist() == list(range(7))
    assert info.nw == 1                                     # a target of 4 waves for 7 tiles: one each
    gi, gd = ops.plan([(21, 70, 0), (12, 300, off2)], K, 100)
    g = _rows(gd)
    assert gi.form == 2 and gi.bm == 128 and g.shape[0] == 1 + 3          # two tiles per row
    assert g[:, 4].tolist() == [2, 2, 2, 1] and g[:, 6].tolist() == [3] * 4
    gi, gd = ops.plan([(21, 70, 0), (12, 300, off2)], K, 2048)
    g = _rows(gd)
    assert gi.form == 2 and gi.bm == 256 and g.shape[0] == 1 + 2          # four tiles per row
    assert g[:, 4].tolist() == [2, 4, 1] and g[:, 9].tolist() == [70, 256, 44]
    assert g[:, 8].tolist() == [0, 70, 326]
    assert ops.plan([(21, 70, 0), (12, 300, off2)], K, 40)[0].bm == 64
    assert ops.plan([(21, 70, 0), (12, 300, off2)], K, 20)[0].bm == 32


def test_plan_buckets():
    from gguf_hip import ops

    for M, g in ((1, 1), (4, 1), (5, 2), (8, 2), (9, 4), (16, 4)):
        info, _ = ops.plan([(12, 512, 0)], 512, M)
        assert info.form == 1 and info.g == g and info.m_max == 4 * g
    assert ops._pick_plan([], 1) == 0 and ops._pick_plan([], 16) == 2
    assert ops._pick_plan([], 17) == 3 and ops._pick_plan([], 32) == 3 and ops._pick_plan([], 33) == 4
    assert ops._pick_plan([], 64) == 4 and ops._pick_plan([], 65) == 5 and ops._pick_plan([], 128) == 5
    assert ops._pick_plan([], 129) == 6 and ops._pick_plan([], 8192) == 6
    # a layer with a table type (IQ4_NL / IQ4_XS / IQ3_S) leaves the GEMV above 8 rows
    for wt in (20, 23, 21):
        assert ops.plan([(wt, 512, 0)], 512, 8)[0].form == 1
        i9, i16 = ops.plan([(wt, 512, 0)], 512, 9)[0], ops.plan([(wt, 512, 0)], 512, 16)[0]
        assert (i9.form, i9.bm, i16.form, i16.bm) == (2, 32, 2, 32)
    off = ops.tiles_bytes(12, 512, 512)
    assert ops.plan([(12, 512, 0), (23, 64, off)], 512, 12)[0].form == 2
    for M, bm in ((17, 32), (32, 32), (33, 64), (64, 64), (65, 128), (128, 128), (129, 256), (2048, 256)):
        assert ops.plan([(12, 512, 0)], 512, M)[0].bm == bm
