"""GPU parity of the dequantizer and the tile repack (through the C ABI), bit-exact against the
oracle: fp32 equal bits, bf16 / fp16 the round-to-nearest-even of the oracle's fp32."""
import numpy as np
import pytest
import torch

from oracle import ggml_ref as G

pytestmark = pytest.mark.gpu


def _to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_dequantize_bit_exact(dev, wt):
    import gguf_hip

    rng = np.random.default_rng(100 + wt)
    n, K = 70, 768
    raw = G.random_blocks(rng, n, K, wt)
    ref = G.dequantize(raw, wt)
    W = _to_dev(raw, dev)
    got = gguf_hip.dequantize(W, wt, (n, K), torch.float32).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    ref_t = torch.from_numpy(ref)
    for dt in (torch.bfloat16, torch.float16):
        g = gguf_hip.dequantize(W, wt, (n, K), dt).cpu()
        assert torch.equal(g.view(torch.int16), ref_t.to(dt).view(torch.int16)), dt
    # the plugin's spelling (m rows, n columns, fp16 default)
    g16 = gguf_hip.ggml_dequantize(W, wt, n, K)
    assert g16.dtype == torch.float16 and torch.equal(g16.cpu(), ref_t.to(torch.float16))


@pytest.mark.parametrize("wt", [G.Q8_0, G.Q3_K, G.Q5_K, G.Q6_K], ids=lambda t: G.NAMES[t])
def test_dequantize_golden_kq_ref_rows(dev, wt):
    """The reference's own dequantization vectors (gguf-plugin/gluon/kq_ref.py, written to
    tests/golden/kq_ref_*.npz) straight through gqk_dequantize: no oracle in between."""
    import os

    import gguf_hip

    d = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", f"kq_ref_{wt}.npz"))
    raw, w = d["raw"], d["w"]
    n, K = w.shape
    got = gguf_hip.dequantize(_to_dev(raw, dev), wt, (n, K), torch.float32).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), w.view(np.uint32))
    # and through the tiles: repack, then the one-pass tile dequantizer
    tiles = gguf_hip.repack_tiles(_to_dev(raw, dev), n, wt)
    got_t = gguf_hip.dequantize_tiles(tiles, n, K, wt, torch.float32).cpu().numpy()
    assert np.array_equal(got_t.view(np.uint32), w.view(np.uint32))


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_dequantize_strided_rows_and_quantized_weights(dev, wt):
    import gguf_hip

    rng = np.random.default_rng(200 + wt)
    n, K = 33, 512
    raw = G.make_weights(rng, n, K, wt)
    rb = raw.shape[1]
    big = np.zeros((n, rb + 40), np.uint8)
    big[:, 7:7 + rb] = raw                                   # a shard view inside wider rows
    Wv = _to_dev(big, dev)[:, 7:7 + rb]
    assert Wv.stride(0) == rb + 40
    got = gguf_hip.dequantize(Wv, wt, (n, K)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), G.dequantize(raw, wt).view(np.uint32))


@pytest.mark.parametrize("wt", [G.Q4_K, G.Q8_0, G.IQ3_S], ids=lambda t: G.NAMES[t])
def test_dequantize_unaligned_output_rows(dev, wt):
    """Output rows that are not 16-byte aligned (ld_out = K + 3) take the element-wise store
    path; rows of a 16-byte aligned ld_out the vector path: both bit-exact."""
    import ctypes

    import gguf_hip
    from gguf_hip._lib import lib

    rng = np.random.default_rng(350 + wt)
    n, K = 37, 512
    raw = G.random_blocks(rng, n, K, wt)
    ref = torch.from_numpy(G.dequantize(raw, wt))
    W = _to_dev(raw, dev)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    for dt, code in ((torch.float32, 0), (torch.bfloat16, 1), (torch.float16, 2)):
        for ld in (K + 3, K + 8):
            out = torch.full((n, ld), 7, dtype=dt, device=dev)
            rc = lib.gqk_dequantize(ctypes.c_void_p(W.data_ptr()), W.stride(0), wt, n, K, ctypes.c_void_p(out.data_ptr()),
                                    ld, code, st)
            assert rc == 0
            o = out.cpu()
            assert torch.equal(o[:, :K], ref.to(dt)), (dt, ld)
            assert bool((o[:, K:] == 7).all()), (dt, ld)


@pytest.mark.parametrize("wt", [G.Q4_0, G.Q5_0, G.Q8_0, G.IQ4_NL], ids=lambda t: G.NAMES[t])
def test_dequantize_32_block_types_any_k(dev, wt):
    import gguf_hip

    rng = np.random.default_rng(300 + wt)
    raw = G.random_blocks(rng, 5, 96, wt)
    got = gguf_hip.dequantize(_to_dev(raw, dev), wt, (5, 96)).cpu().numpy()
    assert np.array_equal(got, G.dequantize(raw, wt))


def _q6_pack(rec):
    """Q6_K's first tile plane: the 256 six-bit values q = lo | hi << 4 of GGUF's ql[128] / qh[64]
    (kq_ref.py:69-79) re-packed per 16-weight group g as three dwords P_m, byte i of P_m = low six
    bits of q[16 g + 4 m + i] | bits 2m, 2m + 1 of q[16 g + 12 + i] << 6, at byte
    16 (3 (g // 4) + m) + 4 (g % 4) + i of the 192."""
    ql, qh = rec[..., :128].astype(np.uint32), rec[..., 128:192].astype(np.uint32)
    k = np.arange(256)
    q = ((ql[..., 64 * (k >> 7) + (k & 63)] >> (4 * ((k & 127) >> 6))) & 0xF) | \
        (((qh[..., 32 * (k >> 7) + (k & 31)] >> (2 * ((k & 127) >> 5))) & 3) << 4)
    out = np.zeros(rec.shape[:-1] + (192,), np.uint8)
    for g in range(16):
        for m in range(3):
            for i in range(4):
                v = (q[..., 16 * g + 4 * m + i] & 63) | (((q[..., 16 * g + 12 + i] >> (2 * m)) & 3) << 6)
                out[..., 16 * (3 * (g // 4) + m) + 4 * (g % 4) + i] = v
    return out


def _np_repack(raw, wt, n, K, planes, rec):
    nb = K // 256
    ntiles = -(-n // 64)
    rows = np.zeros((ntiles * 64, nb, rec), np.uint8)
    rows[:n] = raw.reshape(n, nb, rec)
    if wt == G.Q6_K:
        rows[:, :, :192] = _q6_pack(rows)
    out = np.zeros((ntiles, nb, 64 * rec), np.uint8)
    poff = 0
    for size, nseg, off, seglen, stride, width in planes:
        idx = np.concatenate([np.arange(off + s * stride, off + s * stride + seglen) for s in range(nseg)])
        block = rows[:, :, idx].reshape(ntiles, 64, nb, size // width, width)   # tile, row, kb, column, byte
        block = block.transpose(0, 2, 3, 1, 4).reshape(ntiles, nb, 64 * size)    # column-major: column, row, byte
        out[:, :, 64 * poff:64 * (poff + size)] = block
        poff += size
    return out.reshape(-1)


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_repack_layout_and_roundtrip(dev, wt):
    import gguf_hip

    rng = np.random.default_rng(400 + wt)
    n, K = 70, 768
    raw = G.random_blocks(rng, n, K, wt)
    W = _to_dev(raw, dev)
    tiles = gguf_hip.repack_tiles(W, n, wt)
    _, _, rec, _ = gguf_hip.type_info(wt)
    expect = _np_repack(raw, wt, n, K, gguf_hip.type_planes(wt), rec)
    assert tiles.numel() == expect.size == gguf_hip.tiles_bytes(wt, n, K)
    assert np.array_equal(tiles.cpu().numpy(), expect)
    back = gguf_hip.unrepack_tiles(tiles, n, K, wt)
    assert torch.equal(back.cpu(), torch.from_numpy(raw))
    w = gguf_hip.dequantize_tiles(tiles, n, K, wt, torch.float32).cpu().numpy()
    assert np.array_equal(w, G.dequantize(raw, wt))


@pytest.mark.parametrize("wt", [G.Q4_0, G.Q6_K, G.IQ3_S], ids=lambda t: G.NAMES[t])
def test_repack_odd_stride_rows(dev, wt):
    """Rows at an odd byte stride inside a larger buffer (the byte-wide load path), 130 rows
    (a partial last tile), and the C ABI's unrepack into rows at that stride."""
    import ctypes

    import gguf_hip
    from gguf_hip._lib import lib

    rng = np.random.default_rng(500 + wt)
    n, K = 130, 512
    raw = G.random_blocks(rng, n, K, wt)
    rb = raw.shape[1]
    big = np.zeros((n, rb + 3), np.uint8)
    big[:, 1:1 + rb] = raw
    Wbig = _to_dev(big, dev)
    view = Wbig[:, 1:1 + rb]                                     # odd base, odd row stride
    assert view.stride(0) % 2 == 1 and view.data_ptr() % 2 == 1
    tiles = gguf_hip.repack_tiles(view, n, wt)
    _, _, rec, _ = gguf_hip.type_info(wt)
    assert np.array_equal(tiles.cpu().numpy(), _np_repack(raw, wt, n, K, gguf_hip.type_planes(wt), rec))
    out = torch.full((n, rb + 3), 0xAB, dtype=torch.uint8, device=dev)
    rc = lib.gqk_unrepack(ctypes.c_void_p(tiles.data_ptr()), wt, n, K, ctypes.c_void_p(out.data_ptr() + 1),
                          out.stride(0), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    assert rc == 0
    o = out.cpu().numpy()
    assert np.array_equal(o[:, 1:1 + rb], raw) and (o[:, 0] == 0xAB).all() and (o[:, 1 + rb:] == 0xAB).all()


def test_repack_rejects_bad_k(dev):
    import gguf_hip

    W = torch.zeros((4, 18 * 3), dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        gguf_hip.repack_tiles(W, 4, G.Q4_0)                  # 96 weights: not whole super-blocks
    with pytest.raises(NotImplementedError):
        gguf_hip.dequantize(torch.zeros((4, 66), dtype=torch.uint8, device=dev), 16, (4, 256))
