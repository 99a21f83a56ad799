"""GPU parity of the plugin-import drop-in (gguf_hip.interface) and of the shared per-device
workspace: the raw-row op on strided shard views inside a captured HIP graph, the grouped op
through the reference's prepare / call pair, and one workspace serving many layers and every M
(against the oracle: tolerance 1e-2 of each output row's max |y|, gguf-plugin/test_gluon_kq_gpu.py:81-86)."""
import numpy as np
import pytest
import torch

from oracle import ggml_ref as G

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _x(M, K, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)


def _ref(x, wf):
    return G.matmul_ref(x.float().cpu().numpy(), wf)


def _capture(fn):
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        fn()
    torch.cuda.current_stream().wait_stream(st)
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def test_gluon_mul_mat_strided_shards_in_graph(dev):
    """A merged layer's weight with three shards of different types side by side in wider rows
    (the plugin's weight[start:end, :size] views, gguf-plugin/patches/gguf-gluon-dispatch.patch:57-70):
    the first call prepares each view, then a captured graph of the calls replays bit-identically
    to the eager calls, with eager work between the replays, and matches the oracle."""
    from gguf_hip import interface as I

    rng = np.random.default_rng(31)
    K = 1536
    shards = [(G.Q4_K, 130), (G.IQ3_S, 64), (G.Q6_K, 200)]
    raws = [G.make_weights(rng, n, K, wt) for wt, n in shards]
    width = max(r.shape[1] for r in raws) + 48
    big = np.zeros((sum(n for _, n in shards), width), np.uint8)
    r0 = 0
    for (wt, n), raw in zip(shards, raws):
        big[r0:r0 + n, 16:16 + raw.shape[1]] = raw
        r0 += n
    W = torch.from_numpy(big).to(dev)
    views, r0 = [], 0
    for (wt, n), raw in zip(shards, raws):
        views.append(W[r0:r0 + n, 16:16 + raw.shape[1]])
        r0 += n
    assert all(not v.is_contiguous() for v in views)
    for M in (1, 8, 16, 40):
        x = _x(M, K, 300 + M, dev)
        eager = [I.gluon_mul_mat(x, v, wt, n) for v, (wt, n) in zip(views, shards)]   # prepares each view
        torch.cuda.synchronize()
        for y, raw, (wt, n) in zip(eager, raws, shards):
            assert y.shape == (M, n) and y.dtype == x.dtype
            assert G.rel_err(y.float().cpu().numpy(), _ref(x, G.dequantize(raw, wt))) < TOL, (G.NAMES[wt], M)
        xs = x.clone()
        g, outs = _capture(lambda: [I.gluon_mul_mat(xs, v, wt, n) for v, (wt, n) in zip(views, shards)])
        for rep in range(3):
            g.replay()
            torch.cuda.synchronize()
            for y, e in zip(outs, eager):
                assert torch.equal(y, e), (M, rep)
            # eager work between replays (another M on the same weights and workspace)
            I.gluon_mul_mat(_x(3, K, 9, dev), views[0], shards[0][0], shards[0][1])
        del g
    # the cache lives on the base tensor: one entry per view, reused
    assert len(W._gguf_hip_layers) == 3
    with pytest.raises(NotImplementedError):
        I.gluon_mul_mat(_x(1, K, 0, dev), views[0], 16, 130)          # IQ2_XXS: no kernel here


def test_gluon_mul_mat_first_call_under_capture_raises(dev):
    """The raw-row op keeps a tile copy of the weight (made on its first call: device allocations
    and a plan upload).  A first call inside a HIP graph capture raises a clear error instead of
    recording them; after one eager call the same capture works, and drop_cached_layers frees the
    copy (the allocator's count falls back by at least the tiles' bytes)."""
    from gguf_hip import interface as I
    from gguf_hip import ops

    rng = np.random.default_rng(33)
    K, n = 2048, 512
    raw = G.make_weights(rng, n, K, G.Q4_K)
    W = torch.from_numpy(raw).to(dev)
    x = _x(4, K, 7, dev)
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with pytest.raises(RuntimeError, match="capture"):
        with torch.cuda.graph(g):
            I.gluon_mul_mat(x, W, G.Q4_K, n)
    del g
    torch.cuda.synchronize()
    assert not getattr(W, "_gguf_hip_layers", None)                   # nothing was cached
    before = torch.cuda.memory_allocated(dev)
    eager = I.gluon_mul_mat(x, W, G.Q4_K, n)                          # prepares the tile copy
    torch.cuda.synchronize()
    grown = torch.cuda.memory_allocated(dev) - before
    assert grown >= ops.tiles_bytes(G.Q4_K, n, K)                     # the second copy of the weight
    g, out = _capture(lambda: I.gluon_mul_mat(x, W, G.Q4_K, n))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    del g, out
    assert ops.drop_cached_layers(W) == 1
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(dev) - before <= grown - ops.tiles_bytes(G.Q4_K, n, K)


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_gluon_mul_mat_every_type_strided(dev, wt):
    """gluon_mul_mat on a shard view with a row stride wider than its rows and a column offset
    (the plugin's weight[start:end, :size], gguf-plugin/gluon/interface.py:74-80), every type, at
    GEMV and GEMM row counts: oracle within 1e-2, one cache entry on the base, repeat bit-identity."""
    from gguf_hip import interface as I

    rng = np.random.default_rng(900 + wt)
    n, K = 150, 1024
    raw = G.random_blocks(rng, n, K, wt)
    big = np.zeros((n + 30, raw.shape[1] + 48), np.uint8)
    big[10:10 + n, 32:32 + raw.shape[1]] = raw
    W = torch.from_numpy(big).to(dev)
    view = W[10:10 + n, 32:32 + raw.shape[1]]
    wf = G.dequantize(raw, wt)
    for M in (1, 7, 16, 40):
        x = _x(M, K, 950 + M, dev)
        y = I.gluon_mul_mat(x, view, wt, n)
        assert y.shape == (M, n) and G.rel_err(y.float().cpu().numpy(), _ref(x, wf)) < TOL, (G.NAMES[wt], M)
        assert torch.equal(I.gluon_mul_mat(x, view, wt, n), y), (G.NAMES[wt], M)
    assert len(W._gguf_hip_layers) == 1


def test_prepare_and_grouped_call_like_the_plugin(dev):
    """prepare_grouped_layer / gluon_mul_mat_tiles_grouped with the reference's argument tuple
    (gguf-plugin/patches/gguf-tiles-grouped.patch:106-115,130-136), and the tile views'
    one-pass dequantizer against the oracle bit for bit."""
    from gguf_hip import interface as I

    rng = np.random.default_rng(32)
    K = 2048
    shards = [(G.Q5_K, 96), (G.IQ4_XS, 70), (G.Q8_0, 128)]
    raws = [G.make_weights(rng, n, K, wt) for wt, n in shards]
    tiles = [I.repack_tiles(torch.from_numpy(r).to(dev), n, wt) for r, (wt, n) in zip(raws, shards)]
    assert tiles[0].shape == (2, K // 256, 64, 176)
    packed, views, descs, splits, nb, block_bytes = I.prepare_grouped_layer(
        tiles, [n for _, n in shards], [wt for wt, _ in shards])
    assert nb == K // 256 and [v.shape for v in views] == [t.shape for t in tiles]
    wf = np.concatenate([G.dequantize(r, wt) for r, (wt, _) in zip(raws, shards)])
    for M in (1, 5, 16, 17, 64, 200):
        x = _x(M, K, 400 + M, dev)
        y = I.gluon_mul_mat_tiles_grouped(x, packed, descs, splits, views, [n for _, n in shards],
                                          [wt for wt, _ in shards], nb, block_bytes)
        assert y.shape == (M, sum(n for _, n in shards))
        assert G.rel_err(y.float().cpu().numpy(), _ref(x, wf)) < TOL, M
    for v, raw, (wt, n) in zip(views, raws, shards):
        got = I.dequantize_tiles(v, n, K, wt, torch.float32).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), G.dequantize(raw, wt).view(np.uint32)), G.NAMES[wt]
        y = I.gluon_mul_mat_tiles(_x(4, K, 5, dev), v, n, wt)
        assert G.rel_err(y.float().cpu().numpy(), _ref(_x(4, K, 5, dev), G.dequantize(raw, wt))) < TOL


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_dequantize_tiles_one_pass(dev, wt):
    """gqk_dequantize_tiles straight from the tiles: fp32 bits of the oracle, bf16 / fp16 its
    round-to-nearest-even, a partial last tile, and output rows at an unaligned stride."""
    import ctypes

    import gguf_hip
    from gguf_hip._lib import lib

    rng = np.random.default_rng(700 + wt)
    n, K = 100, 768
    raw = G.random_blocks(rng, n, K, wt)
    ref = G.dequantize(raw, wt)
    tiles = gguf_hip.repack_tiles(torch.from_numpy(raw).to(dev), n, wt)
    got = gguf_hip.dequantize_tiles(tiles, n, K, wt, torch.float32).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    for dt in (torch.bfloat16, torch.float16):
        g = gguf_hip.dequantize_tiles(tiles, n, K, wt, dt).cpu()
        assert torch.equal(g.view(torch.int16), torch.from_numpy(ref).to(dt).view(torch.int16)), dt
    out = torch.full((n, K + 3), -1.0, dtype=torch.float32, device=dev)
    rc = lib.gqk_dequantize_tiles(ctypes.c_void_p(tiles.data_ptr()), wt, n, K, ctypes.c_void_p(out.data_ptr()),
                                  K + 3, 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    o = out.cpu().numpy()
    assert np.array_equal(o[:, :K].view(np.uint32), ref.view(np.uint32)) and np.all(o[:, K:] == -1.0)


def test_shared_workspace_many_layers(dev):
    """One workspace per device serves every layer: 100 mixed-type layers share it, each checked
    at a GEMV M (split-K), a 17-row and a stream-K GEMM M, twice for bit identity, with the
    counters back at zero at the end."""
    import gguf_hip
    from gguf_hip import ops

    rng = np.random.default_rng(33)
    K = 1024
    types = [G.Q4_K, G.Q6_K, G.IQ4_XS, G.Q8_0, G.Q3_K, G.IQ3_S, G.Q5_0]
    layers = []
    for i in range(100):
        sh = [(types[(i + j) % len(types)], int(rng.integers(1, 5)) * 64 - int(rng.integers(0, 40))) for j in range(2)]
        raws = [G.random_blocks(rng, n, K, wt) for wt, n in sh]
        gl = gguf_hip.pack_layer([torch.from_numpy(r).to(dev) for r in raws], [n for _, n in sh], [wt for wt, _ in sh],
                                 target_wgs=64 if i % 2 else 0)
        layers.append((gl, np.concatenate([G.dequantize(r, wt) for r, (wt, _) in zip(raws, sh)])))
    ws = layers[0][0].workspace
    assert all(gl.workspace is ws for gl, _ in layers)
    print(f"shared workspace: {ws.numel() * 4 / 2**20:.1f} MiB for {len(layers)} layers")
    before = torch.cuda.memory_allocated(dev)
    for M in (6, 17, 300):
        x = _x(M, K, 500 + M, dev)
        for i, (gl, wf) in enumerate(layers):
            y1 = gguf_hip.mul_mat_grouped(x, gl)
            y2 = gguf_hip.mul_mat_grouped(x, gl)
            assert torch.equal(y1, y2), (i, M)
            if i % 9 == 0:
                assert G.rel_err(y1.float().cpu().numpy(), _ref(x, wf)) < TOL, (i, M)
        del y1, y2, x
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(dev) == before   # nothing but the outputs, freed again
    assert int(ws[:ops._lib.GQK_CTR_BYTES // 4].abs().sum()) == 0


def test_graph_then_larger_eager_call_then_replay(dev):
    """A graph captured at a GEMV M, then eager calls at a large GEMM M on the same and another
    layer (the stream-K partials fill the shared workspace), then the graph replayed: the
    workspace never moved, so the replay still matches its eager result."""
    import gguf_hip

    rng = np.random.default_rng(34)
    K = 2560
    raw_a = G.random_blocks(rng, 700, K, G.Q4_K)
    raw_b = G.random_blocks(rng, 900, K, G.Q6_K)
    gla = gguf_hip.pack_layer([torch.from_numpy(raw_a).to(dev)], [700], [G.Q4_K], target_wgs=4096)
    glb = gguf_hip.pack_layer([torch.from_numpy(raw_b).to(dev)], [900], [G.Q6_K])
    ws_ptr = gla.workspace.data_ptr()
    x8 = _x(8, K, 8, dev)
    eager = gguf_hip.mul_mat_grouped(x8, gla)
    g, y = _capture(lambda: gguf_hip.mul_mat_grouped(x8, gla))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, eager)
    for M in (2048, 1000):
        xb = _x(M, K, M, dev)
        for gl, raw, wt in ((gla, raw_a, G.Q4_K), (glb, raw_b, G.Q6_K)):
            yb = gguf_hip.mul_mat_grouped(xb, gl)
            if M == 1000:
                assert G.rel_err(yb[:64].float().cpu().numpy(), _ref(xb[:64], G.dequantize(raw, wt))) < TOL
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), M
    assert gla.workspace.data_ptr() == ws_ptr and glb.workspace is gla.workspace
    assert G.rel_err(y.float().cpu().numpy(), _ref(x8, G.dequantize(raw_a, G.Q4_K))) < TOL


def test_read_floor_reads_every_byte(dev):
    """bench.py's memory floor reads each byte of the buffer once: every wave's folded word is the
    XOR of all 32-bit words of its contiguous share of 1 KiB units (a ragged split: 1,000 units
    over 7 x 3 waves, and one wave over everything)."""
    import ctypes

    from gguf_hip import _lib

    n_units = 1000
    g = torch.Generator().manual_seed(7)
    words = torch.randint(-2**31, 2**31 - 1, (n_units * 256,), generator=g, dtype=torch.int64).to(torch.int32)
    buf = words.to(dev)
    unit_xor = np.bitwise_xor.reduce(words.numpy().view(np.uint32).reshape(n_units, 256), axis=1)
    for grid, waves in ((7, 3), (1, 1)):
        W = grid * waves
        sink = torch.zeros(W, dtype=torch.int32, device=dev)
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert _lib.lib.gqk_read_floor(buf.data_ptr(), n_units * 1024, grid, waves, sink.data_ptr(), st) == 0
        torch.cuda.synchronize()
        got = sink.cpu().numpy().view(np.uint32)
        want = np.array([np.bitwise_xor.reduce(unit_xor[w * n_units // W:(w + 1) * n_units // W]) for w in range(W)],
                        dtype=np.uint32)
        assert np.array_equal(got, want)
