"""GPU parity of the grouped linear op (GEMV form M <= 16, GEMM form M > 16) against the
oracle: y = x @ dequant(W)^T in fp64 on the oracle's weights, tolerance 1e-2 relative to each
output row's max |y| (metric of gguf-plugin/test_gluon_kq_gpu.py:81-86).
Also: determinism, mixed-type layers, the GGUFLinearMethod surface, BASELINE config 1."""
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


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_gemv_and_gemm_all_types(dev, wt):
    import gguf_hip

    rng = np.random.default_rng(500 + wt)
    n, K = 200, 1024
    raw = G.make_weights(rng, n, K, wt)
    wf = G.dequantize(raw, wt)
    gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [wt])
    worst = 0.0
    for M in (1, 2, 3, 4, 5, 6, 8, 9, 12, 13, 16, 17, 32, 33, 64, 65, 130, 300):
        x = _x(M, K, 1000 + M, dev)
        y = gguf_hip.mul_mat_grouped(x, gl)
        torch.cuda.synchronize()
        assert y.shape == (M, n) and y.dtype == torch.bfloat16
        yy = y.float().cpu().numpy()
        assert np.isfinite(yy).all(), (G.NAMES[wt], M)
        e = G.rel_err(yy, _ref(x, wf))
        worst = max(worst, e)
        assert e < TOL, (G.NAMES[wt], M, e)
        if M in (1, 8, 33):
            y2 = gguf_hip.mul_mat_grouped(x, gl)
            assert torch.equal(y, y2), "not deterministic"
    print(f"{G.NAMES[wt]}: worst rel err {worst:.2e}")


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_gemv_split_k_ragged(dev, wt):
    """Many k-blocks with several split factors and a ragged row count: every split's partial
    slice is written (the reference's 0044 bug class, tiles_grouped.py:283-287)."""
    import gguf_hip

    rng = np.random.default_rng(600 + wt)
    n, K = 70, 20 * 256
    raw = G.random_blocks(rng, n, K, wt)
    wf = G.dequantize(raw, wt)
    W = torch.from_numpy(raw).to(dev)
    for target in (1, 3, 7, 40):
        gl = gguf_hip.pack_layer([W], [n], [wt], target_wgs=target)
        for M in (1, 7, 12, 32):
            x = _x(M, K, 2000 + M, dev)
            e = G.rel_err(gguf_hip.mul_mat_grouped(x, gl).float().cpu().numpy(), _ref(x, wf))
            assert e < TOL, (G.NAMES[wt], target, M, e)


def test_split_k_repeat_is_bit_identical(dev):
    """The in-kernel split-K exchange (partials, arrival counters) under repetition: every
    launch of one plan gives the same bits, and the counters return to zero."""
    import gguf_hip

    rng = np.random.default_rng(11)
    n, K = 1000, 40 * 256
    raw = G.random_blocks(rng, n, K, G.Q4_K)
    gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [G.Q4_K], target_wgs=4096)
    info = gguf_hip.ops.GqkPlanInfo.from_tuple(gl.plans[:gguf_hip.ops._NPLAN])
    assert info.split > 1, "the plan must split K"
    wf = G.dequantize(raw, G.Q4_K)
    for M in (1, 8):
        x = _x(M, K, 7000 + M, dev)
        y0 = gguf_hip.mul_mat_grouped(x, gl)
        assert G.rel_err(y0.float().cpu().numpy(), _ref(x, wf)) < TOL
        for _ in range(30):
            assert torch.equal(gguf_hip.mul_mat_grouped(x, gl), y0)
    torch.cuda.synchronize()
    assert int(gl.workspace[:info.ctr_bytes // 4].abs().sum()) == 0


@pytest.mark.parametrize("wt", [G.Q4_K, G.Q6_K, G.IQ3_S, G.Q8_0], ids=lambda t: G.NAMES[t])
def test_gemv_tail_tiles_split(dev, wt):
    """A plan with whole tiles and a split tail (10 tiles on 8 resident slots at target 16: the
    last two tiles split K over two workgroups each, the rest written directly): matches the
    oracle, repeats bit-identically, and leaves the counters at zero."""
    import gguf_hip

    rng = np.random.default_rng(40 + wt)
    n, K = 64 * 9 + 17, 16 * 256
    raw = G.random_blocks(rng, n, K, wt)
    wf = G.dequantize(raw, wt)
    gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [wt], target_wgs=16)
    for M in (1, 5, 8):
        i = gguf_hip.ops._pick_plan(gl.plans, M)
        info = gguf_hip.ops.GqkPlanInfo.from_tuple(gl.plans[i * gguf_hip.ops._NPLAN:][:gguf_hip.ops._NPLAN])
        assert info.form == 1 and info.split == 2 and info.n_desc == 8 + 2 * 2
        x = _x(M, K, 4100 + M, dev)
        y = gguf_hip.mul_mat_grouped(x, gl)
        assert G.rel_err(y.float().cpu().numpy(), _ref(x, wf)) < TOL, M
        for _ in range(5):
            assert torch.equal(gguf_hip.mul_mat_grouped(x, gl), y)
    torch.cuda.synchronize()
    assert int(gl.workspace[:info.ctr_bytes // 4].abs().sum()) == 0


def test_graph_replay_matches_eager(dev):
    """The grouped op captured in one HIP graph, as a serving loop (and bench.py) runs it: the
    GEMV with split-K partials and in-kernel counters, the GEMV with a split tail, with a fused
    bias, the mid form (17..32 rows) with split K, and the stream-K GEMM in its 64-row and 256-row
    forms.  Five replays, each after new x
    is copied into the captured inputs, followed by eager launches of the same layers (sharing
    the layers' workspaces) and a host synchronisation: every replay is bit-identical to the
    eager result on the same x, which matches the oracle, and the counters end at zero (they are
    reset by the kernels themselves, so the graph holds no memset)."""
    import gguf_hip
    from gguf_hip.synth import random_shard

    cases = [  # (type, n, K, M, target_wgs, bias)
        (G.Q4_K, 900, 12 * 256, 8, 0, False),        # GEMV, split K
        (G.Q6_K, 900, 12 * 256, 1, 0, True),         # GEMV, split K, fused bf16 bias
        (G.IQ4_XS, 64 * 9 + 17, 16 * 256, 5, 16, False),   # GEMV, whole tiles + split tail
        (G.Q5_K, 1000, 2048, 20, 0, False),          # mid form, split K
        (G.Q6_K, 1000, 2048, 40, 0, False),          # GEMM 64 x 128, stream-K only
        (G.Q4_K, 1000, 2048, 300, 0, True),          # GEMM 256 x 256, stream-K, bias
    ]
    layers, xs, biases, wfs = [], [], [], []
    for i, (wt, n, K, M, tw, has_bias) in enumerate(cases):
        W = random_shard(n, K, wt, dev, seed=700 + i)
        wfs.append(gguf_hip.dequantize(W, wt, (n, K), torch.float32))
        layers.append(gguf_hip.pack_layer([W], [n], [wt], target_wgs=tw))
        xs.append(_x(M, K, 7000 + i, dev))
        biases.append(torch.randn(n, device=dev).to(torch.bfloat16) if has_bias else None)
    for gl, (wt, n, K, M, tw, _) in zip(layers, cases):
        info = gguf_hip.ops.GqkPlanInfo.from_tuple(
            gl.plans[gguf_hip.ops._pick_plan(gl.plans, M) * gguf_hip.ops._NPLAN:][:gguf_hip.ops._NPLAN])
        assert info.form == (1 if M <= 32 else 2) and (M > 32 or info.split > 1), (G.NAMES[wt], M)

    def run():
        return [gguf_hip.mul_mat_grouped(x, gl, b) for x, gl, b in zip(xs, layers, biases)]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):      # eager warm-up: workspaces and device tables exist before capture
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ys = run()
    gen = torch.Generator(device=dev).manual_seed(99)
    for rep in range(5):
        for x in xs:
            x.copy_(torch.randn(x.shape, device=dev, generator=gen).to(torch.bfloat16))
        graph.replay()
        eager = run()
        torch.cuda.synchronize()
        for i, (y, e) in enumerate(zip(ys, eager)):
            assert torch.equal(y, e), (rep, i)
        if rep == 0:
            for y, x, wf, b in zip(ys, xs, wfs, biases):
                ref = x.float() @ wf.T + (b.float() if b is not None else 0.0)
                scale = ref.abs().amax(dim=1, keepdim=True).clamp(min=1e-30)
                assert float(((y.float() - ref).abs() / scale).amax()) < TOL
    for gl in layers:
        info = gguf_hip.ops.GqkPlanInfo.from_tuple(gl.plans[:gguf_hip.ops._NPLAN])
        assert int(gl.workspace[:info.ctr_bytes // 4].abs().sum()) == 0


def test_random_layers_match_reference(dev):
    """Seeded random layers through every form: 1-3 shards of random types (mixed layers
    included) and row counts, K of 1-24 super-blocks, M across the GEMV buckets and the four
    GEMM forms, default / tiny / large wave targets.  Each result is within 1e-2 of an fp32
    matmul of the GPU-dequantized weights (pinned bit-exact by the dequant tests)."""
    import gguf_hip
    from gguf_hip.synth import random_shard

    rng = np.random.default_rng(31)
    for case in range(24):
        K = 256 * int(rng.integers(1, 25))
        shards = [(int(rng.choice(G.ALL_TYPES)), int(rng.integers(1, 1500))) for _ in range(int(rng.integers(1, 4)))]
        M = int(rng.choice([1, 3, 5, 8, 12, 16, 20, 33, 64, 100, 129, 300]))
        target = int(rng.choice([0, 1, 16, 4096]))
        Ws = [random_shard(n, K, wt, dev, seed=100 * case + i) for i, (wt, n) in enumerate(shards)]
        wf = torch.cat([gguf_hip.dequantize(W, wt, (n, K), torch.float32) for W, (wt, n) in zip(Ws, shards)])
        gl = gguf_hip.pack_layer(Ws, [n for _, n in shards], [wt for wt, _ in shards], target_wgs=target)
        x = _x(M, K, 5000 + case, dev)
        y = gguf_hip.mul_mat_grouped(x, gl)
        ref = x.float() @ wf.T
        scale = ref.abs().amax(dim=1, keepdim=True).clamp(min=1e-30)
        err = float(((y.float() - ref).abs() / scale).amax())
        assert err < TOL, (case, [(G.NAMES[wt], n) for wt, n in shards], K, M, target, err)


def test_one_workspace_serves_every_form(dev):
    """One layer workspace across the GEMV and mid form (split tiles) and the GEMM forms (stream-K
    partials) in an order where each form's partials would land on another form's counters if
    the counter regions differed: every call matches the oracle and repeats bit-identically,
    and the counters end at zero."""
    import gguf_hip

    rng = np.random.default_rng(12)
    n, K = 900, 12 * 256
    raw = G.random_blocks(rng, n, K, G.Q4_K)
    gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [G.Q4_K], target_wgs=2048)
    wf = G.dequantize(raw, G.Q4_K)
    first = {}
    for M in (300, 1, 40, 24, 100, 300, 8, 24, 40, 1, 100):
        x = _x(M, K, 9000 + M, dev)
        y = gguf_hip.mul_mat_grouped(x, gl)
        if M not in first:
            assert G.rel_err(y.float().cpu().numpy(), _ref(x, wf)) < TOL, M
            first[M] = y
        else:
            assert torch.equal(y, first[M]), M
    torch.cuda.synchronize()
    info = gguf_hip.ops.GqkPlanInfo.from_tuple(gl.plans[:gguf_hip.ops._NPLAN])
    assert info.split > 1 and int(gl.workspace[:info.ctr_bytes // 4].abs().sum()) == 0


def test_mixed_layer_one_launch(dev):
    """A merged layer of five types in one grouped launch.  GEMV (split 1): every shard's columns
    are bit-identical to its own launch (the reference's mixed-layer identity at a fixed split,
    gguf-plugin/test_gluon_kq_gpu.py:172-195).  GEMM: the stream-K k-ranges of a tile depend on
    the launch's whole tile count, so a shard's fp32 partial sums may associate differently
    alone: its columns match the oracle and stay within bf16 rounding of its own launch."""
    import gguf_hip

    rng = np.random.default_rng(7)
    K = 1536
    shards = [(G.IQ3_S, 70), (G.Q4_K, 128), (G.Q6_K, 100), (G.Q8_0, 64), (G.IQ4_XS, 30)]
    raws = [G.make_weights(rng, n, K, wt) for wt, n in shards]
    Ws = [torch.from_numpy(r).to(dev) for r in raws]
    wf = np.concatenate([G.dequantize(r, wt) for r, (wt, _) in zip(raws, shards)])
    gl = gguf_hip.pack_layer(Ws, [n for _, n in shards], [wt for wt, _ in shards], target_wgs=1)
    singles = [gguf_hip.pack_layer([W], [n], [wt], target_wgs=1) for W, (wt, n) in zip(Ws, shards)]
    for M in (1, 6, 12, 20, 40, 200):   # 12: IQ3_S / Q8_0 / IQ4_XS in the 16 x 16 x 32 form; 20: the mid form
        x = _x(M, K, 3000 + M, dev)
        y = gguf_hip.mul_mat_grouped(x, gl)
        assert G.rel_err(y.float().cpu().numpy(), _ref(x, wf)) < TOL, M
        col = 0
        for s, (wt, n) in zip(singles, shards):
            ys = gguf_hip.mul_mat_grouped(x, s)
            if M <= 32:                     # the streaming forms (GEMV, mid): the same split per tile
                assert torch.equal(y[:, col:col + n], ys), (M, G.NAMES[wt])
            else:
                a, b = y[:, col:col + n].float(), ys.float()
                # the two fp32 sums differ by reassociation only (~1e-6 of the row's scale), so the
                # bf16 results are at most one rounding step apart
                rowmax = b.abs().amax(dim=1, keepdim=True)
                bound = torch.maximum(a.abs(), b.abs()) * 2.0 ** -7 + 1e-4 * rowmax
                assert ((a - b).abs() <= bound).all(), (M, G.NAMES[wt])
            col += n


def test_mixed_layer_default_plan_one_record(dev):
    """All eleven types in one mixed launch at the default plan: up to eight rows one record per
    wave (the mixed one-record kernels, K split five ways through the in-kernel exchange), at 16
    rows the G = 4 kernel; it matches the oracle, repeats bit-identically and leaves the counters
    at zero.  (For 22 tiles the streaming heuristic lands on the one-record plan by itself; the
    config-5 layers exercise the mixed-layer rule at 736 tiles.)"""
    import gguf_hip

    rng = np.random.default_rng(71)
    K = 20 * 256
    shards = [(wt, 64 * (1 + i % 3) - 7 * (i % 2)) for i, wt in enumerate(G.ALL_TYPES)]
    raws = [G.random_blocks(rng, n, K, wt) for wt, n in shards]
    wf = np.concatenate([G.dequantize(r, wt) for r, (wt, _) in zip(raws, shards)])
    gl = gguf_hip.pack_layer([torch.from_numpy(r).to(dev) for r in raws], [n for _, n in shards],
                             [wt for wt, _ in shards])
    for M in (1, 5, 8, 16):
        i = gguf_hip.ops._pick_plan(gl.plans, M)
        info = gguf_hip.ops.GqkPlanInfo.from_tuple(gl.plans[i * gguf_hip.ops._NPLAN:][:gguf_hip.ops._NPLAN])
        assert info.form == 1 and info.types_mask == 0, M
        if M <= 8:
            assert info.bm == 1 and info.split == 5 and info.nw == 4, M
        x = _x(M, K, 7100 + M, dev)
        y = gguf_hip.mul_mat_grouped(x, gl)
        assert G.rel_err(y.float().cpu().numpy(), _ref(x, wf)) < TOL, M
        for _ in range(3):
            assert torch.equal(gguf_hip.mul_mat_grouped(x, gl), y), M
    torch.cuda.synchronize()
    assert int(gl.workspace[:info.ctr_bytes // 4].abs().sum()) == 0


class _WT:
    def __init__(self, weight_type, shard_weight_type=None):
        self.weight_type = weight_type
        self.shard_weight_type = shard_weight_type or {}


class _Layer(torch.nn.Module):
    pass


def test_linear_method_mixed_and_single(dev):
    """GGUFLinearMethod.apply on a mixed-type merged qkv layer (gguf_shards) and on a
    single-type merged gate/up layer (one concatenated weight), with bias; M = 0 is empty."""
    import gguf_hip

    rng = np.random.default_rng(8)
    K = 1024
    # mixed qkv: shards kept as their own tensors (gguf-plugin/patches/gguf-shard-tensors.patch)
    types = {"q": G.Q5_K, "k": G.IQ4_NL, "v": G.Q6_K}
    ns = {"q": 256, "k": 64, "v": 64}
    raws = {i: G.make_weights(rng, ns[i], K, types[i]) for i in "qkv"}
    layer = _Layer()
    layer.weight = torch.nn.Parameter(torch.empty(0, dtype=torch.uint8, device=dev), requires_grad=False)
    layer.weight.shard_id = ["k", "q", "v"]
    layer.weight_type = _WT(G.Q4_K, dict(types))
    layer.gguf_shards = {i: torch.from_numpy(raws[i]).to(dev) for i in ("k", "v", "q")}
    method = gguf_hip.GGUFLinearMethod()
    method.process_weights_after_loading(layer)
    assert list(layer.gguf_groups) == ["q"] and all(layer.gguf_shards[i].numel() == 0 for i in "qkv")
    wf = np.concatenate([G.dequantize(raws[i], types[i]) for i in "qkv"])
    bias = torch.randn(384, device=dev).to(torch.bfloat16)
    for M in (1, 8, 33):
        x = _x(M, K, 4000 + M, dev)
        y = method.apply(layer, x, bias)
        ref = _ref(x, wf) + bias.float().cpu().numpy()[None]
        assert y.shape == (M, 384) and G.rel_err(y.float().cpu().numpy(), ref) < TOL
    assert method.apply(layer, torch.empty(0, K, dtype=torch.bfloat16, device=dev)).shape == (0, 384)

    # single-type merged layer: the whole weight, shard offsets as the plugin records them
    raw_g = G.make_weights(rng, 200, K, G.Q4_K)
    raw_u = G.make_weights(rng, 200, K, G.Q4_K)
    layer2 = _Layer()
    w = torch.from_numpy(np.concatenate([raw_g, raw_u])).to(dev)
    layer2.weight = torch.nn.Parameter(w, requires_grad=False)
    layer2.weight.shard_id = [0, 1]
    layer2.weight.shard_offset_map = {0: (0, 200, raw_g.shape[1]), 1: (200, 400, raw_u.shape[1])}
    layer2.weight_type = _WT(G.Q4_K, {0: G.Q4_K, 1: G.Q4_K})
    method.process_weights_after_loading(layer2)
    assert "__all__" in layer2.gguf_groups and layer2.weight.numel() == 0
    wf2 = np.concatenate([G.dequantize(raw_g, G.Q4_K), G.dequantize(raw_u, G.Q4_K)])
    for M in (3, 100):
        x = _x(M, K, 5000 + M, dev)
        assert G.rel_err(method.apply(layer2, x).float().cpu().numpy(), _ref(x, wf2)) < TOL


def test_linear_method_unquantized_shard_splits_runs(dev):
    """A merged qkv layer whose k shard is unquantized (F16): the runs are [q] and [v] (as the
    reference's _create_groups), every piece lands in its own output columns in q, k, v order,
    for bf16 x (column slices of one output) and fp32 x (concatenation)."""
    import gguf_hip

    rng = np.random.default_rng(13)
    K = 512
    rq, rv = G.make_weights(rng, 128, K, G.Q4_K), G.make_weights(rng, 64, K, G.Q6_K)
    wk = (rng.normal(size=(64, K)) * 0.02).astype(np.float16)
    layer = _Layer()
    layer.weight = torch.nn.Parameter(torch.empty(0, dtype=torch.uint8, device=dev), requires_grad=False)
    layer.weight.shard_id = ["q", "k", "v"]
    layer.weight_type = _WT(G.Q4_K, {"q": G.Q4_K, "k": 1, "v": G.Q6_K})
    layer.gguf_shards = {"q": torch.from_numpy(rq).to(dev), "k": torch.from_numpy(wk).to(dev),
                         "v": torch.from_numpy(rv).to(dev)}
    method = gguf_hip.GGUFLinearMethod()
    method.process_weights_after_loading(layer)
    assert {k: v[1] for k, v in layer.gguf_groups.items()} == {"q": ["q"], "v": ["v"]}
    wf = np.concatenate([G.dequantize(rq, G.Q4_K), wk.astype(np.float32), G.dequantize(rv, G.Q6_K)])
    bias = torch.randn(256, device=dev).to(torch.bfloat16)
    for M in (1, 8, 40):
        x = _x(M, K, 7000 + M, dev)
        y = method.apply(layer, x, bias)
        ref = _ref(x, wf) + bias.float().cpu().numpy()[None]
        assert y.shape == (M, 256) and G.rel_err(y.float().cpu().numpy(), ref) < TOL, M
        y32 = method.apply(layer, x.float())
        assert y32.dtype == torch.float32 and G.rel_err(y32.cpu().numpy(), _ref(x, wf)) < TOL, M
    # the out= form writes exactly its column slice
    gl = layer.gguf_groups["v"][0]
    x = _x(5, K, 1, dev)
    big = torch.full((5, 100), 7.0, dtype=torch.bfloat16, device=dev)
    gguf_hip.mul_mat_grouped(x, gl, out=big[:, 20:84])
    assert torch.equal(big[:, 20:84], gguf_hip.mul_mat_grouped(x, gl))
    assert bool((big[:, :20] == 7).all()) and bool((big[:, 84:] == 7).all())


def _plan_of(gl, M):
    from gguf_hip import ops

    return ops.GqkPlanInfo.from_tuple(gl.plans[ops._pick_plan(gl.plans, M) * ops._NPLAN:][:ops._NPLAN])


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_gemv_slab_form(dev, wt):
    """The slab form (a workgroup per 32-row half tile over the whole k-range, each wave's x in
    LDS, the waves combined in LDS in a fixed order; up to 8 rows and, as the mid form's slab, 9
    to 32 but for IQ3_S at 9 to 16), planned on a pinned CU count so that small shards take it: a
    last tile of <= 32 and of
    > 32 rows, an odd super-block count (a half wave without a super-block, or a wave of one
    super-block), the largest k-range (24 super-blocks, 12 waves), a fused bias, bit-identical
    repeats; against the oracle."""
    import gguf_hip

    rng = np.random.default_rng(900 + wt)
    for n, nbk, cus in ((200, 5, 8), (232, 4, 8), (100, 24, 4)):
        K = nbk * 256
        raw = G.random_blocks(rng, n, K, wt)
        wf = G.dequantize(raw, wt)
        gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [wt], cus=cus)
        bias = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 4).to(torch.bfloat16).to(dev)
        for M in (1, 3, 4, 5, 8, 12, 17, 24, 32):
            assert (_plan_of(gl, M).bm == 2) == (wt != G.IQ3_S or not 9 <= M <= 16), (n, nbk, M)
            x = _x(M, K, 3000 + M, dev)
            y = gguf_hip.mul_mat_grouped(x, gl, bias)
            e = G.rel_err(y.float().cpu().numpy(), _ref(x, wf) + bias.float().cpu().numpy()[None])
            assert e < TOL, (G.NAMES[wt], n, nbk, M, e)
            assert torch.equal(y, gguf_hip.mul_mat_grouped(x, gl, bias)), "not deterministic"
        # the same layer planned for the device: same results within the tolerance
        gd = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [wt])
        x = _x(8, K, 3100, dev)
        assert G.rel_err(gguf_hip.mul_mat_grouped(x, gd).float().cpu().numpy(), _ref(x, wf)) < TOL


def test_mid_slab_light_types_below_seven_eighths(dev):
    """At 9..16 rows the mid form's slab also serves shards whose slabs fill less than 7/8 of the
    CUs when every shard is of a light-decode type (Q4_K, Q5_K here: 7 slabs planned for 9 CUs),
    and not a Q6_K shard of the same shape; both against the oracle."""
    import gguf_hip

    rng = np.random.default_rng(913)
    n, K = 200, 5 * 256
    for wt, slab in ((G.Q4_K, True), (G.Q5_K, True), (G.Q6_K, False)):
        raw = G.random_blocks(rng, n, K, wt)
        wf = G.dequantize(raw, wt)
        gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [wt], cus=9)
        for M in (9, 12, 16):
            info = _plan_of(gl, M)
            assert (info.bm == 2 and info.g == 8) == slab, (G.NAMES[wt], M)
            x = _x(M, K, 5000 + M, dev)
            y = gguf_hip.mul_mat_grouped(x, gl)
            e = G.rel_err(y.float().cpu().numpy(), _ref(x, wf))
            assert e < TOL, (G.NAMES[wt], M, e)


def test_gemv_slab_form_mixed_layer(dev):
    """A mixed-type layer (Q4_K, IQ4_XS with its LDS tables, Q6_K) in the slab form, written into a
    column slice of a wider output."""
    import gguf_hip

    rng = np.random.default_rng(77)
    K = 5 * 256
    shards = [(G.Q4_K, 200), (G.IQ4_XS, 232), (G.Q6_K, 96)]
    raws = [G.random_blocks(rng, n, K, wt) for wt, n in shards]
    wf = np.concatenate([G.dequantize(r, wt) for r, (wt, _) in zip(raws, shards)])
    gl = gguf_hip.pack_layer([torch.from_numpy(r).to(dev) for r in raws], [n for _, n in shards],
                             [wt for wt, _ in shards], cus=20)
    n_total = sum(n for _, n in shards)
    for M in (2, 8, 20):
        info = _plan_of(gl, M)
        assert info.bm == 2 and info.types_mask == 0, M
        x = _x(M, K, 4000 + M, dev)
        out = torch.full((M, n_total + 40), 7.0, dtype=torch.bfloat16, device=dev)
        gguf_hip.mul_mat_grouped(x, gl, out=out[:, 20:20 + n_total])
        o = out.float().cpu().numpy()
        assert (o[:, :20] == 7).all() and (o[:, 20 + n_total:] == 7).all()
        assert G.rel_err(o[:, 20:20 + n_total], _ref(x, wf)) < TOL, M


def test_fused_bias(dev):
    """A bf16 bias is added in the kernels' epilogue (direct GEMV store, split-K fixup, GEMM and
    stream-K fixup): a zero bias changes no bit, a random one matches oracle + bias; an fp32 bias
    is added afterwards."""
    import gguf_hip

    rng = np.random.default_rng(12)
    n, K = 1000, 2048
    raw = G.make_weights(rng, n, K, G.Q4_K)
    wf = G.dequantize(raw, G.Q4_K)
    gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [G.Q4_K])
    zero = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    bias = (torch.randn(n, device=dev) * 4).to(torch.bfloat16)
    for M in (1, 8, 16, 24, 40, 100, 300):
        x = _x(M, K, 6000 + M, dev)
        y0 = gguf_hip.mul_mat_grouped(x, gl)
        assert torch.equal(gguf_hip.mul_mat_grouped(x, gl, zero), y0), M
        yb = gguf_hip.mul_mat_grouped(x, gl, bias).float().cpu().numpy()
        ref = _ref(x, wf) + bias.float().cpu().numpy()[None]
        assert G.rel_err(yb, ref) < TOL, M
        y32 = gguf_hip.mul_mat_grouped(x, gl, bias.float())
        assert torch.equal(y32, y0.add_(bias.float())), M
    with pytest.raises(ValueError):
        gguf_hip.mul_mat_grouped(_x(2, K, 1, dev), gl, bias[:10])


def test_raw_rows_op_and_errors(dev):
    import gguf_hip

    rng = np.random.default_rng(9)
    raw = G.make_weights(rng, 96, 512, G.Q3_K)
    x = _x(4, 512, 9, dev)
    y = gguf_hip.fused_mul_mat_gguf(x, torch.from_numpy(raw).to(dev), G.Q3_K)
    assert G.rel_err(y.float().cpu().numpy(), _ref(x, G.dequantize(raw, G.Q3_K))) < TOL
    with pytest.raises(NotImplementedError):
        gguf_hip.fused_mul_mat_gguf(x, torch.zeros((4, 66 * 2), dtype=torch.uint8, device=dev), 16)
    gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [96], [G.Q3_K])
    with pytest.raises(ValueError):
        gguf_hip.mul_mat_grouped(_x(2, 768, 1, dev), gl)       # K mismatch


def test_baseline_config1_q8_0(dev):
    """W[4096, 4096] ~ N(0, 0.02) -> Q8_0 (d = absmax / 127), x[1, 4096] bf16
    ~ N(0, 1); dequant bit-exact, y within 1e-2."""
    import gguf_hip

    rng = np.random.default_rng(1)
    N = K = 4096
    W = rng.normal(0.0, 0.02, size=(N, K)).astype(np.float32)
    raw = G.quantize(W, G.Q8_0)
    wf = G.dequantize(raw, G.Q8_0)
    Wd = torch.from_numpy(raw).to(dev)
    got = gguf_hip.dequantize(Wd, G.Q8_0, (N, K)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), wf.view(np.uint32))
    x = torch.from_numpy(rng.normal(0, 1, size=(1, K)).astype(np.float32)).to(torch.bfloat16).to(dev)
    gl = gguf_hip.pack_layer([Wd], [N], [G.Q8_0])
    e = G.rel_err(gguf_hip.mul_mat_grouped(x, gl).float().cpu().numpy(), _ref(x, wf))
    assert e < TOL, e


@pytest.mark.parametrize("n,K,M", [(1000, 2048, 300), (1000, 2048, 2148), (16384, 512, 1100),
                                   (1000, 2048, 40), (16384, 512, 100), (70000, 256, 64), (70000, 256, 120),
                                   (1000, 2048, 33), (5120, 5120, 48), (200000, 256, 40)],
                         ids=str)
@pytest.mark.parametrize("wt", [G.Q5_K, G.Q4_K, G.Q8_0], ids=lambda t: G.NAMES[t])
def test_gemm_stream_k_schedule(dev, n, K, M, wt):
    """The GEMM forms' persistent schedule (256 x 256 tiles above 128 rows, except 129..384 rows of a
    layer with few 256-row groups, which keep 128 x 128 (1000 rows at M = 300 here); 128 x 128 and
    64 x 128 at 65..128 and 33..64): whole tiles dealt to the workgroups, the remainder
    tiles' k-steps split over up to all of them (stream-K, >= 16 steps each, <= 6 per tile) and
    combined in k order by the last contributor.  Small grids are all remainder; the 16384-row
    case at M=1100 and the 70000- and 200000-row cases mix both phases.  The 256 x 256 tile runs
    with its waves 2 x 4 for Q5_K, 4 x 2 with x staged by direct-to-LDS loads for Q4_K and 4 x 2
    with x through registers for Q8_0; the 128 x 128 form stages x by direct loads.  Checked
    against an fp32 matmul of the GPU-dequantized weights (pinned bit-exact by the dequant
    tests), repeated launches bit-identical, counters back at zero."""
    import gguf_hip
    from gguf_hip.synth import random_shard

    W = random_shard(n, K, wt, dev, seed=n + M)
    wf = gguf_hip.dequantize(W, wt, (n, K), torch.float32)
    gl = gguf_hip.pack_layer([W], [n], [wt])
    x = torch.randn(M, K, device=dev, generator=torch.Generator(device=dev).manual_seed(M)).to(torch.bfloat16)
    y = gguf_hip.mul_mat_grouped(x, gl)
    ref = x.float() @ wf.T
    scale = ref.abs().amax(dim=1, keepdim=True).clamp(min=1e-30)
    assert float(((y.float() - ref).abs() / scale).amax()) < TOL
    for _ in range(3):
        assert torch.equal(gguf_hip.mul_mat_grouped(x, gl), y)
    torch.cuda.synchronize()
    info = gguf_hip.ops.GqkPlanInfo.from_tuple(gl.plans[:gguf_hip.ops._NPLAN])
    assert int(gl.workspace[:info.ctr_bytes // 4].abs().sum()) == 0    # the arrival counters


@pytest.mark.parametrize("wt", [G.Q4_K, G.Q6_K, G.Q8_0, G.IQ4_XS], ids=lambda t: G.NAMES[t])
def test_strided_activations_every_form(dev, wt):
    """x as a column slice of a wider buffer (row stride K + 24, 16-byte aligned start) goes to the
    kernels as is, in every form: GEMV (M <= 16; at 9-16 rows Q8_0 / IQ4_XS read it straight from
    global memory in the 16 x 16 x 32 form), the mid form (17..32 rows, x read straight from global
    memory) and the three GEMM tiles, with x staged through
    registers (Q6_K, Q8_0 in the 256 x 256 form) or by direct-to-LDS loads (the 128 x 128 form,
    Q4_K in the 256 x 256 form), full and partial token blocks.  Each result is bit-identical to
    the one from a contiguous copy of x."""
    import gguf_hip
    from gguf_hip.synth import random_shard

    n, K = 300, 2048
    W = random_shard(n, K, wt, dev, seed=77 + wt)
    gl = gguf_hip.pack_layer([W], [n], [wt])
    wf = gguf_hip.dequantize(W, wt, (n, K), torch.float32)
    for M in (8, 12, 20, 48, 100, 256, 300):
        big = torch.randn(M, K + 24, device=dev, generator=torch.Generator(device=dev).manual_seed(M)).to(torch.bfloat16)
        xs = big[:, 8:8 + K]
        assert xs.stride(0) == K + 24 and xs.data_ptr() % 16 == 0
        y = gguf_hip.mul_mat_grouped(xs, gl)
        assert torch.equal(y, gguf_hip.mul_mat_grouped(xs.contiguous(), gl)), (G.NAMES[wt], M)
        ref = xs.float() @ wf.T
        e = float(((y.float() - ref).abs() / ref.abs().amax(dim=1, keepdim=True).clamp(min=1e-30)).amax())
        assert e < TOL, (G.NAMES[wt], M, e)


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_mid_form_17_to_32_rows(dev, wt):
    """The mid form (17..32 rows: the GEMV's descriptor rows and split-K exchange, weights decoded
    to bf16 in registers, MFMA 32x32x16): every type on a ragged shard at several split factors
    (the wave target) against the oracle (tolerance 1e-2 of each row's max |y|), bit-identical
    repeats, a fused bias, a column slice of a wider output, and the counters back at zero."""
    import gguf_hip

    rng = np.random.default_rng(800 + wt)
    n, K = 197, 24 * 256
    raw = G.random_blocks(rng, n, K, wt)
    wf = G.dequantize(raw, wt)
    W = torch.from_numpy(raw).to(dev)
    bias = (torch.randn(n, device=dev) * 2).to(torch.bfloat16)
    for target in (0, 1, 13, 64):
        gl = gguf_hip.pack_layer([W], [n], [wt], target_wgs=target)
        for M in (17, 23, 32):
            i = gguf_hip.ops._pick_plan(gl.plans, M)
            info = gguf_hip.ops.GqkPlanInfo.from_tuple(gl.plans[i * gguf_hip.ops._NPLAN:][:gguf_hip.ops._NPLAN])
            assert info.form == 1 and info.g == 8 and info.m_max == 32, (target, M)
            x = _x(M, K, 8100 + M, dev)
            y = gguf_hip.mul_mat_grouped(x, gl)
            e = G.rel_err(y.float().cpu().numpy(), _ref(x, wf))
            assert e < TOL, (G.NAMES[wt], target, M, e)
            assert torch.equal(gguf_hip.mul_mat_grouped(x, gl), y), (target, M)
            yb = gguf_hip.mul_mat_grouped(x, gl, bias).float().cpu().numpy()
            assert G.rel_err(yb, _ref(x, wf) + bias.float().cpu().numpy()[None]) < TOL, (target, M)
            wide = torch.full((M, n + 40), 7.0, dtype=torch.bfloat16, device=dev)
            gguf_hip.mul_mat_grouped(x, gl, out=wide[:, 24:24 + n])
            assert torch.equal(wide[:, 24:24 + n], y) and bool((wide[:, :24] == 7).all())
            assert bool((wide[:, 24 + n:] == 7).all()), (target, M)
        torch.cuda.synchronize()
        assert int(gl.workspace[:info.ctr_bytes // 4].abs().sum()) == 0


def test_dequant_regime_large_m(dev, monkeypatch):
    """From DEQUANT_MIN_M rows mul_mat_grouped takes the reference's dequant regime (each shard's
    tiles dequantized, the vendor bf16 GEMM in row chunks): a mixed layer, with a bias and into a
    column slice of a wider output, matches the oracle on both sides of the threshold and at a
    chunk remainder; and at the default threshold a small layer at 4096 rows does too."""
    import gguf_hip
    from gguf_hip import ops

    rng = np.random.default_rng(21)
    K = 1536
    shards = [(G.Q4_K, 128), (G.Q6_K, 100), (G.IQ3_S, 70)]
    raws = [G.make_weights(rng, n, K, wt) for wt, n in shards]
    wf = np.concatenate([G.dequantize(r, wt) for r, (wt, _) in zip(raws, shards)])
    gl = gguf_hip.pack_layer([torch.from_numpy(r).to(dev) for r in raws], [n for _, n in shards],
                             [wt for wt, _ in shards])
    n_total = sum(n for _, n in shards)
    bias = (torch.randn(n_total, device=dev) * 4).to(torch.bfloat16)
    monkeypatch.setattr(ops, "DEQUANT_MIN_M", 48)
    monkeypatch.setattr(ops, "DEQUANT_CHUNK_M", 40)
    monkeypatch.setattr(ops, "DEQUANT_CHUNK_M_LONG_K", 40)
    for M in (47, 48, 100):
        x = _x(M, K, 8000 + M, dev)
        ref = _ref(x, wf)
        assert G.rel_err(gguf_hip.mul_mat_grouped(x, gl).float().cpu().numpy(), ref) < TOL, M
        yb = gguf_hip.mul_mat_grouped(x, gl, bias).float().cpu().numpy()
        assert G.rel_err(yb, ref + bias.float().cpu().numpy()[None]) < TOL, M
        wide = torch.full((M, n_total + 24), 7.0, dtype=torch.bfloat16, device=dev)
        gguf_hip.mul_mat_grouped(x, gl, out=wide[:, 8:8 + n_total])
        assert G.rel_err(wide[:, 8:8 + n_total].float().cpu().numpy(), ref) < TOL, M
        assert bool((wide[:, :8] == 7).all()) and bool((wide[:, 8 + n_total:] == 7).all()), M
    monkeypatch.undo()
    assert ops.DEQUANT_MIN_M == 4096
    raw = G.make_weights(rng, 96, 512, G.Q4_K)
    gl1 = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [96], [G.Q4_K])
    x = _x(4096, 512, 8100, dev)
    assert G.rel_err(gguf_hip.mul_mat_grouped(x, gl1).float().cpu().numpy(), _ref(x, G.dequantize(raw, G.Q4_K))) < TOL
