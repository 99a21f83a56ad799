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


def _plan(*args, **kw):
    """ops.plan on a pinned 256-CU device (MI355X), so the CPU tests do not depend on a visible GPU."""
    from gguf_hip import ops

    return ops.plan(*args, cus=kw.pop("cus", 256), **kw)


def test_plan_takes_the_cu_count():
    """The CU count is a plan input: the default wave target is eight per CU, and the 128 x 128
    GEMM form's choice compares a layer's 256-row groups against it; a negative count is refused."""
    from gguf_hip import _lib

    # gate_up at M = 8 (544 tiles of 20 records): 256 CUs -> 2048 waves, 4 per tile, 512 slots:
    # 512 whole tiles and the last 32 split min(20 / 4, 512 / 2 / 32) = 5 ways; 128 CUs -> 1024
    # waves, 2 per tile, 512 slots of 2-wave workgroups: the last 32 split min(20 / 2, 8) = 8 ways
    info = _plan([(12, 34816, 0)], 5120, 8)[0]
    assert (info.nw, info.n_desc) == (4, 512 + 32 * 5)
    info = _plan([(12, 34816, 0)], 5120, 8, cus=128)[0]
    assert (info.nw, info.n_desc) == (2, 512 + 32 * 8)
    # o_proj 5120 x 5120 at M = 200: 20 groups of 256 rows * 4 < 256 CUs -> 128 x 128 tiles; not on 64 CUs
    assert _plan([(12, 5120, 0)], 5120, 200)[0].bm == 128
    assert _plan([(12, 5120, 0)], 5120, 200, cus=64)[0].bm == 256
    with pytest.raises(ValueError):
        _plan([(12, 5120, 0)], 5120, 8, cus=-1)


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
        _plan([(12, 64, 0), (21, 64, 12345)], 512, 1)  # shards not back to back
    with pytest.raises(ValueError):
        _plan([(12, 64, 0)], 500, 1)                  # K not a multiple of 256
    with pytest.raises(NotImplementedError):
        _plan([(12, 64, 0), (16, 64, 64 * 2 * 144)], 512, 1)
    with pytest.raises(ValueError):
        ops.quant_shape(12, 4, 145)


def _rows(desc):
    return desc.numpy().reshape(-1, 16)


def _check_gemv_rows(shards, K, info, desc):
    """The GEMV plan's per-row contract: every 64-row tile covered by nc rows (D_NC) whose k-ranges
    split [0, nb) evenly in split order (D_SPLIT = 0..nc-1); a split tile (nc > 1) has its own
    arrival counter and nc consecutive partial slots from D_SLOT0; the workspace holds the counter
    region and every slot.  Returns {tile: nc}."""
    nb = K // 256
    d = _rows(desc)
    assert info.form == 1 and d.shape[0] == info.n_desc
    if info.bm == 2:
        return _check_slab_rows(shards, K, info, d)
    by_tile = {}
    for row in d:
        assert row[4] == 1 and row[10] == nb
        by_tile.setdefault((int(row[1]) | int(row[2]) << 32, int(row[3])), []).append(row)
    assert len(by_tile) == sum((n + 63) // 64 for _, n, _ in shards)
    ctrs, slots, ncs = [], [], {}
    for key, rows in by_tile.items():
        nc = len(rows)
        ncs[key] = nc
        assert [int(r[12]) for r in rows] == [nc] * nc and [int(r[7]) for r in rows] == list(range(nc))
        assert [(int(r[5]), int(r[6])) for r in rows] == [(j * nb // nc, (j + 1) * nb // nc) for j in range(nc)]
        if nc > 1:
            assert len({int(r[11]) for r in rows}) == 1 and len({int(r[13]) for r in rows}) == 1
            ctrs.append(int(rows[0][11]))
            slots.append((int(rows[0][13]), nc))
    assert sorted(ctrs) == list(range(len(ctrs)))
    slots.sort()
    assert all(a + n == b for (a, n), (b, _) in zip(slots, slots[1:])) and (not slots or slots[0][0] == 0)
    n_slots = sum(n for _, n in slots)
    assert info.workspace_bytes == (info.ctr_bytes + n_slots * 64 * info.m_max * 4 if n_slots else 0)
    assert info.split == max(ncs.values())
    return ncs


def _check_slab_rows(shards, K, info, d):
    """The slab plan's rows: one per 32-row half of each 64-row tile that holds rows (D_SPLIT = the
    half), each over the whole k-range with no split (D_NC = 1), one wave per pair of super-blocks,
    no workspace.  Returns {tile: 1}."""
    nb = K // 256
    assert info.split == 1 and info.workspace_bytes == 0 and info.nw == (nb + 1) // 2 and info.g in (1, 2, 8)
    halves = {}
    col0 = 0
    cols = {}
    for wt, n, off in shards:
        for t in range((n + 63) // 64):
            cols[(off, t)] = (col0 + 64 * t, min(64, n - 64 * t))
        col0 += n
    for row in d:
        key = (int(row[1]) | int(row[2]) << 32, int(row[3]))
        assert row[4] == 1 and row[10] == nb and (row[5], row[6]) == (0, nb) and row[12] == 1
        assert (int(row[8]), int(row[9])) == cols[key]
        halves.setdefault(key, []).append(int(row[7]))
    assert set(halves) == set(cols)
    for key, hs in halves.items():
        assert hs == ([0, 1] if cols[key][1] > 32 else [0]), key
    return {k: 1 for k in halves}


def test_plan_gemv_slab_form():
    """The slab form (bm = 2) up to 8 rows and at 17 to 32 (the mid form's slab): a workgroup per
    32-row half tile over the whole k-range when the slabs fill one round of the CUs, at least half
    of them, with K <= 6144 (one wave per pair of super-blocks); at 9 to 16 rows the mid form's
    slab (g = 8) only when the slabs fill 7/8 of the CUs and no shard is IQ3_S, or every shard is
    of a light-decode type (Q8_0, Q2_K, Q4_K, Q5_K)."""
    from gguf_hip import ops

    qkv, o_proj = [(12, 7168, 0)], [(12, 5120, 0)]
    for M in (1, 4, 5, 8, 17, 32):                             # qkv: 224 slabs on 256 CUs
        info, desc = _plan(qkv, 5120, M)
        assert info.bm == 2 and info.n_desc == 224 and info.nw == 10, M
        _check_gemv_rows(qkv, 5120, info, desc)
    for M in (1, 4, 5, 8, 24):                                 # o_proj: 160 slabs
        assert _plan(o_proj, 5120, M)[0].bm == 2, M
    assert _plan([(12, 3968, 0)], 5120, 8)[0].bm != 2          # 124 slabs: under half the CUs
    assert _plan([(12, 3968, 0)], 5120, 32)[0].bm != 2
    for M in (9, 16):                                          # 9..16 rows: 224 slabs >= 7/8 of 256
        info, desc = _plan(qkv, 5120, M)
        assert info.bm == 2 and info.g == 8 and info.m_max == 32, M
        _check_gemv_rows(qkv, 5120, info, desc)
        assert _plan(o_proj, 5120, M)[0].bm == 2               # 160 slabs: Q4_K's light decode
        assert _plan([(14, 5120, 0)], 5120, M)[0].bm != 2      # Q6_K there: split-K
        assert _plan([(21, 7168, 0)], 5120, M)[0].bm != 2      # IQ3_S: split-K
        assert _plan([(21, 7168, 0)], 5120, M + 16)[0].bm == 2
    assert _plan(qkv, 5120, 33)[0].form == 2                   # above 32 rows: the GEMM
    assert _plan([(12, 9216, 0)], 5120, 1)[0].bm != 2          # 288 slabs: more than one round
    assert _plan([(12, 2048, 0)], 5120, 1)[0].bm != 2          # 64 slabs: too few CUs busy
    assert _plan([(12, 7168, 0)], 25 * 256, 8)[0].bm != 2      # 25 super-blocks: above 12 waves
    info, desc = _plan([(14, 7168, 0)], 24 * 256, 8)           # 24 super-blocks: 12 waves
    assert info.bm == 2 and info.nw == 12
    assert _plan(qkv, 5120, 8, 40)[0].bm != 2                  # an explicit wave target keeps split-K
    # ragged shards and a mixed layer on a pinned CU count: a last tile of <= 32 rows has one slab
    off = ops.tiles_bytes(12, 200, 5 * 256)
    mixed = [(12, 200, 0), (23, 232, off)]                    # 7 + 8 slabs, 5 super-blocks (odd)
    info, desc = _plan(mixed, 5 * 256, 8, cus=16)
    assert info.bm == 2 and info.n_desc == 15 and info.types_mask == 0 and info.nw == 3
    _check_gemv_rows(mixed, 5 * 256, info, desc)


def test_read_floor_argument_checks():
    """The measurement-only plain read refuses null buffers, sizes that are not whole KiB (or
    beyond 2 GiB) and grids outside 1..16 waves before any launch."""
    from gguf_hip import _lib

    f = _lib.lib.gqk_read_floor
    assert f(None, 1024, 1, 1, None, None) == _lib.GQK_ERR_ARG
    p = ctypes.c_void_p(4096)                      # never dereferenced: the checks come first
    assert f(p, 1000, 1, 1, p, None) == _lib.GQK_ERR_SHAPE
    assert f(p, (1 << 31) + 1024, 1, 1, p, None) == _lib.GQK_ERR_SHAPE
    assert f(p, 1024, 0, 1, p, None) == _lib.GQK_ERR_SHAPE
    assert f(p, 1024, 1, 17, p, None) == _lib.GQK_ERR_SHAPE
    assert "read_floor" in _lib.lib.gqk_last_error().decode()


def test_plan_gemv_balanced_split_partition():
    from gguf_hip import _lib, ops

    assert _plan([(21, 6144, 0)], 20 * 256, 1, 0)[0].bm == 2   # the default plan: 192 slabs (slab form)
    for target in (1, 16, 97, 1024, 4096):
        info, desc = _plan([(21, 6144, 0)], 20 * 256, 1, target)
        ncs = _check_gemv_rows([(21, 6144, 0)], 20 * 256, info, desc)
        S, nw = info.split, info.nw
        assert info.form == 1 and info.g == 1 and info.m_max == 4
        assert 1 <= nw <= 4 and S * nw <= 20                # every wave keeps >= 1 super-block
        if S > 1:
            assert nw == 4                                  # K splits across workgroups only past a full one
        assert set(ncs.values()) == {S}                     # 96 tiles: one round or whole rounds, no tail
        # the counter region: the fixed GQK_CTR_BYTES of every plan
        assert info.ctr_bytes == _lib.GQK_CTR_BYTES
    assert _plan([(21, 6144, 0)], 20 * 256, 1, 1)[0].nw == 1
    info = _plan([(21, 6144, 0)], 20 * 256, 1, 4096)[0]
    assert (info.nw, info.split) == (4, 5)                  # 43 waves per tile wanted: 4 x min(11, 20 // 4)
    info = _plan([(21, 6144, 0)], 20 * 256, 8, 2048)[0]
    assert (info.nw, info.split) == (4, 5)                  # the default wave target, 2048: 22 per tile


def test_plan_gemv_tail_tiles_split():
    """Whole tiles beyond full rounds of resident workgroups: a short last round (<= half the
    slots) splits K instead of putting a third whole tile on a few CUs."""
    from gguf_hip import ops

    # gate_up 34816 x 5120 at the default target: 544 tiles, 512 slots of 4 waves -> 512 whole
    # tiles, the last 32 split 5 ways (>= one record per wave; up to 8 would fit half the slots)
    info, desc = _plan([(12, 34816, 0)], 5120, 8, 0)
    ncs = _check_gemv_rows([(12, 34816, 0)], 5120, info, desc)
    order = [ncs[k] for k in sorted(ncs, key=lambda k: k[1])]
    assert order == [1] * 512 + [5] * 32 and info.n_desc == 512 + 160 and info.nw == 4
    # a full last round (no remainder) and a long one (> half the slots) stay whole
    info, desc = _plan([(12, 32768, 0)], 5120, 8, 0)
    assert set(_check_gemv_rows([(12, 32768, 0)], 5120, info, desc).values()) == {1} and info.workspace_bytes == 0
    info, desc = _plan([(12, 64 * 13, 0)], 16 * 256, 1, 16)     # 13 tiles, 8 slots of 2 waves
    assert info.nw == 2 and set(_check_gemv_rows([(12, 64 * 13, 0)], 16 * 256, info, desc).values()) == {1}
    # 800 tiles at the default target: 3 waves each, 682 slots, the last 118 tiles split 2 ways
    info, desc = _plan([(12, 64 * 800, 0)], 5120, 8, 0)
    ncs = _check_gemv_rows([(12, 64 * 800, 0)], 5120, info, desc)
    assert info.nw == 3 and sorted(ncs.values()) == [1] * 682 + [2] * 118
    # the tail spans shards: 34816 rows after a 1024-row shard of the same type (560 tiles, 48 split)
    offq = ops.tiles_bytes(14, 1024, 5120)
    info, desc = _plan([(14, 1024, 0), (14, 34816, offq)], 5120, 8, 0)
    ncs = _check_gemv_rows([(14, 1024, 0), (14, 34816, offq)], 5120, info, desc)
    assert sum(1 for v in ncs.values() if v > 1) == 48 and info.split == min(5, 256 // 48)
    off = ops.tiles_bytes(12, 1024, 5120)
    # up to four rows the same layer takes one record per wave: every tile split 5 ways x 4 waves
    info, desc = _plan([(12, 1024, 0), (14, 34816, off)], 5120, 1, 0)
    ncs = _check_gemv_rows([(12, 1024, 0), (14, 34816, off)], 5120, info, desc)
    assert set(ncs.values()) == {5} and info.n_desc == 560 * 5 and info.nw == 4 and info.bm == 1
    # ... unless the k-range does not split into single records (down: 68 super-blocks)
    assert _plan([(12, 5120, 0)], 17408, 1, 0)[0].bm == 0
    # a mixed-type layer keeps one record per wave up to eight rows (its streaming kernel is bound
    # by its costliest format's registers); a single type streams at eight, and nothing does at 16
    mixed = [(12, 7168, 0), (14, 5120, ops.tiles_bytes(12, 7168, 5120))]
    for M, bm in ((1, 1), (8, 1), (16, 0)):
        info, desc = _plan(mixed, 5120, M, 0)
        assert info.bm == bm and info.types_mask == 0, M
        if bm:
            assert set(_check_gemv_rows(mixed, 5120, info, desc).values()) == {5} and info.n_desc == 192 * 5
    assert _plan([(12, 3072, 0)], 5120, 8, 0)[0].bm == 1 and _plan([(12, 34816, 0)], 5120, 8, 0)[0].bm == 0
    # one round of split tiles with >= 2 records a wave fills the 512 slots exactly: down 5120 x
    # 17408 (80 tiles, 68 records) as 32 tiles x 7 + 48 x 6; o_proj (1 record a wave) keeps 5 each
    info, desc = _plan([(12, 5120, 0)], 17408, 8, 0)
    ncs = _check_gemv_rows([(12, 5120, 0)], 17408, info, desc)
    assert info.n_desc == 512 and sorted(ncs.values()) == [6] * 48 + [7] * 32 and info.split == 7
    info, desc = _plan([(12, 3072, 0)], 5120, 8, 0)
    assert set(_check_gemv_rows([(12, 3072, 0)], 5120, info, desc).values()) == {5} and info.n_desc == 240
    # the GEMV's bm field flags plans whose waves all stream exactly one record (3072 x 5120:
    # 20 records = 5 workgroups x 4 waves); the pipeline-free kernel serves them
    assert info.bm == 1 and _plan([(12, 9216, 0)], 5120, 1, 0)[0].bm == 1
    assert _plan([(12, 34816, 0)], 5120, 8, 0)[0].bm == 0 and _plan([(12, 5120, 0)], 17408, 8, 0)[0].bm == 0
    # small targets: 10 tiles on 8 slots of 2 waves... (target 16) -> the last 2 tiles split
    info, desc = _plan([(12, 64 * 9 + 17, 0)], 16 * 256, 1, 16)
    ncs = _check_gemv_rows([(12, 64 * 9 + 17, 0)], 16 * 256, info, desc)
    assert info.nw == 2 and sorted(ncs.values()) == [1] * 8 + [2, 2]


def test_plan_all_split_rows_interleaved_by_xcd():
    """A GEMV plan whose tiles are all split deals them eight at a time with their splits
    interleaved, so every contributor of a tile sits at workgroup indices of one residue mod 8
    (the dispatcher deals workgroups to the eight XCDs in turn) and the residues get equal work;
    a plan with whole tiles keeps the tile order."""
    from gguf_hip import ops

    for shards, K, M in (([(12, 3072, 0)], 5120, 8), ([(14, 5120, 0)], 17408, 8), ([(12, 9216, 0)], 5120, 1),
                         ([(12, 7168, 0), (14, 5120, ops.tiles_bytes(12, 7168, 5120))], 5120, 8)):
        info, desc = _plan(shards, K, M)
        d = _rows(desc)
        assert all(r[12] > 1 for r in d), (shards, K, M)
        _check_gemv_rows([(wt, n, o) for wt, n, o in shards], K, info, desc)
        residues, work = {}, [0] * 8
        for i, r in enumerate(d):
            residues.setdefault((int(r[1]) | int(r[2]) << 32, int(r[3])), set()).add(i % 8)
            work[i % 8] += int(r[6]) - int(r[5])
        assert all(len(v) == 1 for v in residues.values()), (shards, K, M)
        assert max(work) - min(work) <= K // 256, (shards, K, M, work)
    info, desc = _plan([(12, 34816, 0)], 5120, 8)            # 512 whole tiles + a split tail
    tiles = [int(r[3]) for r in _rows(desc)]
    assert tiles[:512] == list(range(512)) and tiles == sorted(tiles)


def test_plan_random_layers_stay_in_bounds():
    """Seeded random layers (1-4 shards of random types and row counts, K up to 80 super-blocks,
    M 1-600, default / tiny / odd wave targets): every descriptor row addresses a tile of its own
    shard and valid output columns, GEMV rows partition each tile's k-range with counters and
    partial slots inside the workspace (the split-K checker above), a one-record plan (bm = 1,
    the kernel without a pipeline) gives every wave exactly one record, and GEMM rows cover each
    tile exactly once over the whole k-range.  These are the bounds the kernels rely on."""
    from gguf_hip import ops

    rng = np.random.default_rng(2024)
    for case in range(300):
        K = 256 * int(rng.integers(1, 81))
        shards, off = [], 0
        for _ in range(int(rng.integers(1, 5))):
            wt = int(rng.choice(G.ALL_TYPES))
            n = int(rng.choice([rng.integers(1, 200), rng.integers(1, 40000)]))
            shards.append((wt, n, off))
            off += ops.tiles_bytes(wt, n, K)
        M = int(rng.choice([rng.integers(1, 17), rng.integers(17, 601)]))
        target = int(rng.choice([0, 0, 1, 16, int(rng.integers(2, 5000))]))
        info, desc = _plan(shards, K, M, target)
        d = _rows(desc)
        nb, n_total = K // 256, sum(n for _, n, _ in shards)
        tiles_of = {o: ((n + 63) // 64, n, wt) for wt, n, o in shards}
        col_of, c = {}, 0
        for wt, n, o in shards:
            col_of[o] = c
            c += n
        assert d.shape[0] == info.n_desc and info.n_total == n_total and info.nb == nb, case
        for row in d:
            o = int(row[1]) | int(row[2]) << 32
            ntile, n, wt = tiles_of[o]
            t0, nt = int(row[3]), int(row[4])
            assert row[0] == wt and 0 <= t0 and nt >= 1 and t0 + nt <= ntile, case
            assert int(row[8]) == col_of[o] + 64 * t0, case
            assert 1 <= int(row[9]) <= min(64 * nt, n - 64 * t0), case
            assert 0 <= int(row[5]) < int(row[6]) <= nb, case
        if info.form == 1:
            assert M <= info.m_max and 1 <= info.nw <= 8, case
            _check_gemv_rows(shards, K, info, desc)
            assert all(int(r[11]) * 4 < info.ctr_bytes for r in d if r[12] > 1), case
            if info.bm == 1:
                assert all(int(r[6]) - int(r[5]) == info.nw for r in d), case
            else:
                assert all(int(r[6]) - int(r[5]) >= info.nw for r in d), case
        else:
            groups = sum(((n + 63) // 64 + 3) // 4 for _, n, _ in shards)
            short = M <= 384 or (M <= 768 and K <= 32 * 256)
            big = 256 if not short or groups * ((M + 255) // 256) * 4 >= 256 else 128
            assert info.form == 2 and M > 32 and info.bm == (64 if M <= 64 else 128 if M <= 128 else big)
            per = 4 if info.bm == 256 else 2
            seen = {}
            for row in d:
                o, t0, nt = int(row[1]) | int(row[2]) << 32, int(row[3]), int(row[4])
                assert nt <= per and (int(row[5]), int(row[6])) == (0, nb), case
                for t in range(t0, t0 + nt):
                    seen[(o, t)] = seen.get((o, t), 0) + 1
            assert sorted(seen.values()) == [1] * sum(nt for nt, _, _ in tiles_of.values()), case


def test_plan_descriptor_rows_mixed_layer():
    from gguf_hip import _lib, ops

    K = 3 * 256
    off2 = ops.tiles_bytes(21, 70, K)
    info, desc = _plan([(21, 70, 0), (12, 300, off2)], K, 8, 4)
    d = _rows(desc)
    assert info.types_mask == 0 and info.n_total == 370 and info.g == 2
    assert info.split == 1 and info.workspace_bytes == 0
    # one counter region for every plan of every layer, so one workspace serves every layer and M
    for shards, k in (([(21, 70, 0), (12, 300, off2)], K), ([(12, 70000, 0)], 512), ([(12, 64 * 65536, 0)], 256)):
        regions = {_plan(shards, k, m, t)[0].ctr_bytes for m in (1, 8, 16, 17, 100, 2048) for t in (0, 1, 4096)}
        assert regions == {_lib.GQK_CTR_BYTES}
    # a layer with more tiles than the region has counters is refused, not silently overrun
    with pytest.raises(ValueError, match="counter region"):
        _plan([(12, 64 * 65536 + 1, 0)], 256, 8)
    # one workgroup per tile: IQ3_S 2 tiles (64 + 6 rows), Q4_K 5 tiles (4 x 64 + 44)
    assert d[:, 0].tolist() == [21, 21, 12, 12, 12, 12, 12]
    assert d[:, 3].tolist() == [0, 1, 0, 1, 2, 3, 4] and d[:, 4].tolist() == [1] * 7
    assert d[:, 8].tolist() == [0, 64, 70, 134, 198, 262, 326] and d[:, 9].tolist() == [64, 6, 64, 64, 64, 64, 44]
    assert d[2, 1] == off2 and d[:, 10].tolist() == [3] * 7 and d[:, 12].tolist() == [1] * 7   # whole tiles
    _check_gemv_rows([(21, 70, 0), (12, 300, off2)], K, info, desc)
    assert info.nw == 1                                     # a target of 4 waves for 7 tiles: one each
    gi, gd = _plan([(21, 70, 0), (12, 300, off2)], K, 100)
    g = _rows(gd)
    assert gi.form == 2 and gi.bm == 128 and g.shape[0] == 1 + 3          # two tiles per row
    assert g[:, 4].tolist() == [2, 2, 2, 1] and g[:, 6].tolist() == [3] * 4
    gi, gd = _plan([(21, 70, 0), (12, 300, off2)], K, 2048)
    g = _rows(gd)
    assert gi.form == 2 and gi.bm == 256 and g.shape[0] == 1 + 2          # four tiles per row
    assert g[:, 4].tolist() == [2, 4, 1] and g[:, 9].tolist() == [70, 256, 44]
    assert g[:, 8].tolist() == [0, 70, 326]
    assert _plan([(21, 70, 0), (12, 300, off2)], K, 40)[0].bm == 64
    info = _plan([(21, 70, 0), (12, 300, off2)], K, 20)[0]             # 17..32 rows: the mid form
    assert (info.form, info.g, info.m_max, info.bm) == (1, 8, 32, 0)


def test_plan_buckets():
    from gguf_hip import ops

    for M, g in ((1, 1), (4, 1), (5, 2), (8, 2), (9, 4), (16, 4), (17, 8), (32, 8)):
        info, _ = _plan([(12, 512, 0)], 512, M)
        assert info.form == 1 and info.g == g and info.m_max == 4 * g
    assert ops._pick_plan([], 1) == 0 and ops._pick_plan([], 16) == 2
    assert ops._pick_plan([], 17) == 3 and ops._pick_plan([], 32) == 3 and ops._pick_plan([], 33) == 4
    assert ops._pick_plan([], 64) == 4 and ops._pick_plan([], 65) == 5 and ops._pick_plan([], 128) == 5
    assert ops._pick_plan([], 129) == 6 and ops._pick_plan([], 384) == 6
    assert ops._pick_plan([], 385) == 7 and ops._pick_plan([], 512) == 7
    assert ops._pick_plan([], 513) == 8 and ops._pick_plan([], 768) == 8
    assert ops._pick_plan([], 769) == 9 and ops._pick_plan([], 8192) == 9
    # every type, the table types (IQ4_NL / IQ4_XS / IQ3_S) included, stays on the GEMV up to 16 rows,
    # then on the mid form up to 32
    for wt in (20, 23, 21):
        i9, i16, i17, i33 = (_plan([(wt, 512, 0)], 512, m)[0] for m in (9, 16, 17, 33))
        assert (i9.form, i9.g, i16.form, i16.g, i17.form, i17.g, i33.form, i33.bm) == (1, 4, 1, 4, 1, 8, 2, 64)
    off = ops.tiles_bytes(12, 512, 512)
    assert _plan([(12, 512, 0), (23, 64, off)], 512, 12)[0].form == 1
    assert _plan([(12, 512, 0), (23, 64, off)], 512, 30)[0].form == 1
    for M, bm in ((33, 64), (64, 64), (65, 128), (128, 128), (129, 128), (384, 128),
                  (512, 128), (768, 128), (769, 256), (2048, 256)):
        assert _plan([(12, 512, 0)], 512, M)[0].bm == bm
    # 129..384 rows: 256 x 256 tiles once the 256-row groups times the token blocks reach a quarter
    # of the CUs (256 assumed without a GPU): 34816 rows = 136 groups, 16384 = 64, 16000 = 63,
    # 7168 = 28, 5120 = 20
    for n, M, bm in ((34816, 129, 256), (34816, 384, 256), (7168, 256, 128), (7168, 384, 128),
                     (5120, 384, 128), (16000, 256, 128), (16000, 257, 256), (16384, 129, 256)):
        assert _plan([(12, n, 0)], 512, M)[0].bm == bm, (n, M)
    # 385..768 rows only for K up to 8192 (32 super-blocks)
    for K, M, bm in ((5120, 512, 128), (8192, 512, 128), (8448, 512, 256), (17408, 448, 256), (17408, 384, 128),
                     (5120, 768, 128), (5120, 769, 256)):
        assert _plan([(12, 5120, 0)], K, M)[0].bm == bm, (K, M)
    assert _plan([(12, 7168, 0)], 5120, 640)[0].bm == 256       # 28 groups x 3 blocks: above the quarter


def test_ggml_dequantize_rejects_rows_narrower_than_n():
    """A column-offset view whose rows hold fewer bytes than n weights need is a ValueError before
    any launch (the C side sees only the row stride, so it would read past the last row)."""
    import torch

    from gguf_hip import ops

    W = torch.zeros((4, 2 * 144), dtype=torch.uint8)            # two Q4_K blocks per row
    with pytest.raises(ValueError, match="do not hold"):
        ops.ggml_dequantize(W[:, 16:16 + 144], 12, 4, 512)      # 144 bytes for 512 weights
    with pytest.raises(ValueError, match="do not hold"):
        ops.ggml_dequantize(W, 12, 4, 300)                      # not whole blocks
    with pytest.raises(ValueError, match="rows"):
        ops.ggml_dequantize(W, 12, 5, 512)
    with pytest.raises(NotImplementedError):
        ops.ggml_dequantize(W, 16, 4, 256)                      # IQ2_XXS: no kernel
    with pytest.raises(ValueError, match="GPU"):
        ops.ggml_dequantize(W, 12, 4, 512)                      # the shape is fine: CPU tensors have no path


def test_interface_names_resolve_for_the_plugin():
    """The plugin's import lines (gguf-plugin/patches/gguf-gluon-dispatch.patch:13 and the later
    patches' additions) resolve against gguf_hip.interface, with the reference's meanings."""
    from gguf_hip import interface as I
    from gguf_hip import ops

    ns = {}
    exec("from gguf_hip.interface import GLUON_MAX_ROWS, GLUON_TYPES, gluon_mul_mat", ns)
    exec("from gguf_hip.interface import (GLUON_MAX_ROWS, GLUON_TYPES, GLUON_TILE_TYPES, gluon_mul_mat, "
         "gluon_mul_mat_iq3s_tiles, gluon_mul_mat_tiles, gluon_mul_mat_tiles_grouped, prepare_grouped_layer, "
         "repack_iq3s_tiles, repack_tiles, dequantize_tiles, dequantize_iq3s_tiles)", ns)
    assert ns["GLUON_MAX_ROWS"] == 16
    assert ns["GLUON_TYPES"] == frozenset(ops.GGUF_TYPES) == I.GLUON_TILE_TYPES
    assert {I.GGML_TYPE_Q2_K, I.GGML_TYPE_Q4_K, I.GGML_TYPE_IQ3_S, I.GGML_TYPE_IQ4_XS} == {10, 12, 21, 23}
    import torch
    with pytest.raises(NotImplementedError):
        I.gluon_mul_mat(torch.zeros((1, 256), dtype=torch.bfloat16), torch.zeros((1, 66), dtype=torch.uint8), 16, 1)
