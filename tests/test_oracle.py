"""Pins the CPU oracle (oracle/ggml_ref.py) before it is trusted as the checker.

* Golden vectors: gguf-plugin/gluon/kq_ref.py's own dequantization of random rows (Q8_0, Q3_K,
  Q5_K, Q6_K; the reference holds it bit-exact against gguf-py), tests/golden/kq_ref_*.npz.
* Tables: the IQ3_S grid and IQ4 kvalues as the reference writes them (tests/golden/*.npy).
* Closed form: every product is exact in fp32, so fp32 == float32(fp64) for every type.
* Reductions to pinned formats: Q4_K == Q5_K with zero high bits; Q2_K == Q3_K with all high
  bits set and matching scales; IQ4_NL == kvalues[Q4_0 index]; IQ4_XS == IQ4_NL per sub-block.
* Known-answer blocks for the bits no reduction reaches (Q4_0 / Q5_0 nibble and qh order,
  the Q2_K min term, the IQ3_S grid index / sign / scale arithmetic, encoded independently).
"""
import os

import numpy as np
import pytest

from oracle import ggml_ref as G
from oracle.tables import IQ3S_GRID, IQ3S_GRID_BYTES, IQ4_KVALUES

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f16b(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


@pytest.mark.parametrize("wt", [G.Q8_0, G.Q3_K, G.Q5_K, G.Q6_K])
def test_golden_kq_ref(wt):
    d = np.load(os.path.join(GOLD, f"kq_ref_{wt}.npz"))
    got = G.dequantize(d["raw"], wt, 512)
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), d["w"].view(np.uint32))


def test_tables_match_reference_text():
    grid_x4 = np.load(os.path.join(GOLD, "iq3s_grid_x4.npy"))
    assert np.array_equal(IQ3S_GRID * 4, grid_x4)
    assert np.array_equal(np.load(os.path.join(GOLD, "iq4_kvalues.npy")), IQ4_KVALUES)
    assert len(set(IQ3S_GRID.tolist())) == 512
    assert set(np.unique(IQ3S_GRID_BYTES).tolist()) == {1, 3, 5, 7, 9, 11, 13, 15}
    assert np.all(np.diff(IQ3S_GRID.astype(np.int64)) > 0)          # the table is sorted ascending
    assert IQ3S_GRID_BYTES[0, 0] == 1                                  # byte 0 (test_gguf_rco_cpu.py:373-376)


@pytest.mark.parametrize("wt", G.ALL_TYPES)
def test_fp32_equals_rounded_fp64(wt):
    rng = np.random.default_rng(wt)
    raw = G.random_blocks(rng, 9, 512, wt)
    w32 = G.dequantize(raw, wt)
    w64 = G.dequantize(raw, wt, f64=True)
    assert np.array_equal(w32, w64.astype(np.float32))
    assert np.isfinite(w32).all()


def test_q4k_is_q5k_without_high_bits():
    rng = np.random.default_rng(1)
    q4 = G.random_blocks(rng, 5, 768, G.Q4_K).reshape(5, 3, 144)
    q5 = np.zeros((5, 3, 176), np.uint8)
    q5[..., 0:16] = q4[..., 0:16]          # d, dmin, scales
    q5[..., 48:176] = q4[..., 16:144]      # qs (qh = 0)
    assert np.array_equal(G.dequantize(q4.reshape(5, -1), G.Q4_K), G.dequantize(q5.reshape(5, -1), G.Q5_K))


def _q3k_scales_bytes(u16):
    """Encode 16 six-bit values (sc + 32) into Q3_K's 12 scale bytes (inverse of the kq_ref
    decode, written as a scatter)."""
    s = np.zeros(12, np.int32)
    for i, u in enumerate(u16):
        s[i % 8] |= (u & 0xF) << (4 * (i // 8))
        s[8 + i % 4] |= ((u >> 4) & 3) << (2 * (i // 4))
    return s.astype(np.uint8)


def test_q2k_is_q3k_with_all_high_bits():
    rng = np.random.default_rng(2)
    for _ in range(20):
        q2 = G.random_blocks(rng, 1, 256, G.Q2_K)[0]
        q2[82:84] = f16b(0.0)                              # dmin = 0: no min term
        q3 = np.zeros(110, np.uint8)
        q3[0:32] = 0xFF                                    # every high bit set: q = the 2-bit value
        q3[32:96] = q2[16:80]                              # same 2-bit quant layout
        q3[96:108] = _q3k_scales_bytes([(q2[i] & 0xF) + 32 for i in range(16)])
        q3[108:110] = q2[80:82]                            # d
        assert np.array_equal(G.dequantize(q2[None], G.Q2_K), G.dequantize(q3[None], G.Q3_K))


def test_q2k_min_term_index():
    blk = np.zeros(84, np.uint8)
    blk[0:16] = (np.arange(16) << 4).astype(np.uint8)    # min nibble = group index, scale nibble 0
    blk[80:82] = f16b(1.0)
    blk[82:84] = f16b(0.5)
    w = G.dequantize(blk[None], G.Q2_K)[0]
    assert np.array_equal(w, (-0.5 * (np.arange(256) // 16)).astype(np.float32))


def test_q4_0_known_blocks():
    blk = np.zeros(18, np.uint8)
    blk[0:2] = f16b(0.25)
    blk[2:18] = (np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8)
    w = G.dequantize(blk[None], G.Q4_0)[0]
    expect = 0.25 * (np.concatenate([np.arange(16), 15 - np.arange(16)]) - 8)
    assert np.array_equal(w, expect.astype(np.float32))


def test_q5_0_high_bits():
    for j in (0, 5, 15, 16, 23, 31):
        blk = np.zeros(22, np.uint8)
        blk[0:2] = f16b(2.0)
        blk[2:6] = np.array([1 << j], np.uint32).view(np.uint8)
        w = G.dequantize(blk[None], G.Q5_0)[0]
        expect = np.full(32, -32.0, np.float32)
        expect[j] = 0.0
        assert np.array_equal(w, expect), j
    rng = np.random.default_rng(5)
    q4 = G.random_blocks(rng, 4, 256, G.Q4_0).reshape(4, 8, 18)
    q5 = np.zeros((4, 8, 22), np.uint8)
    q5[..., 0:2] = q4[..., 0:2]
    q5[..., 2:6] = 0xFF
    q5[..., 6:22] = q4[..., 2:18]
    d = G.fields(q4.reshape(4, -1), G.Q4_0, 256)["d"].astype(np.float32)
    assert np.array_equal(G.dequantize(q5.reshape(4, -1), G.Q5_0),
                          G.dequantize(q4.reshape(4, -1), G.Q4_0) + np.repeat(8 * d, 32, axis=1))


def test_iq4nl_is_kvalue_of_q4_0_index():
    rng = np.random.default_rng(6)
    raw = G.random_blocks(rng, 3, 256, G.Q4_0)
    d = np.repeat(G.fields(raw, G.Q4_0, 256)["d"], 32, axis=1).astype(np.float32)
    idx = np.rint(G.dequantize(raw, G.Q4_0) / d).astype(np.int64) + 8
    assert np.array_equal(G.dequantize(raw, G.IQ4_NL), d * IQ4_KVALUES[idx].astype(np.float32))


def test_iq4xs_is_iq4nl_per_subblock():
    rng = np.random.default_rng(7)
    for ls in (33, 32 + 5, 32 - 7, 63, 0):
        xs = G.random_blocks(rng, 1, 256, G.IQ4_XS)[0]
        xs[2:4] = np.array([sum(((ls >> 4) & 3) << (2 * ib) for ib in range(8))], np.uint16).view(np.uint8)
        xs[4:8] = (ls & 0xF) | ((ls & 0xF) << 4)
        nl = np.zeros((8, 18), np.uint8)
        nl[:, 0:2] = xs[0:2]
        nl[:, 2:18] = xs[8:136].reshape(8, 16)
        d = float(xs[0:2].view(np.float16)[0])
        expect = G.dequantize(nl.reshape(1, -1), G.IQ4_NL)[0] / np.float32(d) * np.float32(d * (ls - 32))
        assert np.array_equal(G.dequantize(xs[None], G.IQ4_XS)[0], expect.astype(np.float32)), ls


def _iq4xs_encode(d, ls8, nib256):
    """IQ4_XS block from chosen fields, written from the prose of gguf-plugin/gluon/iq4xs.py:5-11
    (not from the oracle's decode): d f16 | scales_h u16 | scales_l u8[4] | qs u8[128].  The
    6-bit scale of sub-block ib: its low 4 bits are nibble ib of scales_l (byte ib // 2, low nibble
    for even ib), its high 2 bits are bits 2 ib, 2 ib + 1 of scales_h.  Weight j < 16 of
    sub-block ib is the low nibble of qs byte 16 ib + j, weight 16 + j the high nibble."""
    blk = np.zeros(136, np.uint8)
    blk[0:2] = f16b(d)
    sh = 0
    for ib in range(8):
        ls = int(ls8[ib])
        blk[4 + ib // 2] |= (ls & 0xF) << (4 * (ib % 2))
        sh |= (ls >> 4) << (2 * ib)
        for j in range(16):
            blk[8 + 16 * ib + j] = int(nib256[32 * ib + j]) | (int(nib256[32 * ib + 16 + j]) << 4)
    blk[2:4] = np.array([sh], np.uint16).view(np.uint8)
    return blk


def test_iq4xs_known_block_distinct_subscales():
    """Eight different 6-bit sub-scales, so a decode that takes a sub-block's scale from another
    sub-block's nibble (e.g. scales_l[ib % 4] >> 4 * (ib // 4)) or bit pair fails."""
    ls = np.array([1, 62, 17, 40, 5, 33, 48, 26])
    rng = np.random.default_rng(12)
    for d in (1.0, float(np.float16(3.0517578e-4)), float(np.float16(-0.0123))):
        nib = rng.integers(0, 16, 256)
        w = G.dequantize(_iq4xs_encode(d, ls, nib)[None], G.IQ4_XS)[0]
        expect = np.repeat(np.float64(d) * (ls - 32), 32) * IQ4_KVALUES[nib].astype(np.float64)
        assert np.array_equal(w, expect.astype(np.float32))
    # one non-zero nibble field at a time: each sub-block's scale is found in its own fields only
    for ib in range(8):
        one = np.zeros(8, np.int64)
        one[ib] = ls[ib]
        nib = np.full(256, 9)                                   # kvalue 13 everywhere
        w = G.dequantize(_iq4xs_encode(1.0, one, nib)[None], G.IQ4_XS)[0].reshape(8, 32)
        for jb in range(8):
            assert np.all(w[jb] == np.float32((one[jb] - 32) * 13)), (ib, jb)


def _iq3s_encode(d, scales8, idx32, signs256):
    """IQ3_S block from chosen fields: 8 sub-block scales (4 bit), 32 grid indices (9 bit, one
    per 4 weights in order), 256 sign bits.  Scatter encoder of the GGML layout: index i of
    sub-block ib's 8 indices -> low byte qs[8 ib + i], high bit qh[ib] bit i; sign of weight
    32 ib + 8 l + j -> bit j of signs[4 ib + l]; scale of ib -> nibble ib % 2 of scales[ib // 2]."""
    blk = np.zeros(110, np.uint8)
    blk[0:2] = f16b(d)
    for ib in range(8):
        for i in range(8):
            v = idx32[8 * ib + i]
            blk[2 + 8 * ib + i] = v & 0xFF
            blk[66 + ib] |= ((v >> 8) & 1) << i
        for l in range(4):
            blk[74 + 4 * ib + l] = sum(int(signs256[32 * ib + 8 * l + j]) << j for j in range(8))
        blk[106 + ib // 2] |= scales8[ib] << (4 * (ib % 2))
    return blk


def test_iq3s_known_blocks():
    rng = np.random.default_rng(8)
    for _ in range(10):
        d = float(np.float16(rng.uniform(1e-3, 1e-2)))
        sc = rng.integers(0, 16, 8)
        idx = rng.integers(0, 512, 64)
        sg = rng.integers(0, 2, 256)
        blk = _iq3s_encode(d, sc, idx, sg)
        w = G.dequantize(blk[None], G.IQ3_S)[0]
        mags = IQ3S_GRID_BYTES[idx].reshape(-1).astype(np.float64)              # 4 magnitudes per index
        dl = np.repeat(np.float64(d) * (1 + 2 * sc), 32)
        expect = dl * mags * np.where(sg == 1, -1.0, 1.0)
        assert np.array_equal(w, expect.astype(np.float32))


def test_q8_0_quantizer_follows_baseline_rule():
    rng = np.random.default_rng(9)
    W = rng.normal(0, 0.02, size=(4, 256)).astype(np.float32)
    raw = G.quantize(W, G.Q8_0).reshape(4, 8, 34)
    amax = np.abs(W.reshape(4, 8, 32)).max(-1)
    assert np.array_equal(raw[..., 0:2].copy().view(np.float16)[..., 0], (amax / 127).astype(np.float16))
    q = raw[..., 2:].view(np.int8)
    assert np.all(np.abs(q).max(-1) == 127)


@pytest.mark.parametrize("wt", [t for t in G.ALL_TYPES if t != G.IQ3_S])
def test_quantizers_roundtrip_close(wt):
    rng = np.random.default_rng(10 + wt)
    W = rng.normal(0, 0.02, size=(6, 512)).astype(np.float32)
    w = G.dequantize(G.quantize(W, wt), wt)
    err = np.sqrt(((w - W) ** 2).mean() / (W ** 2).mean())
    assert err < 0.4, (G.NAMES[wt], err)
