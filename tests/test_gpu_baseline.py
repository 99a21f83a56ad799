"""BASELINE shapes at full size (configs 2-5).  The oracle cannot dequantize 178 M weights in a
test's time, so these use size-independent properties: (1) a random subset of rows dequantized
on the GPU equals the oracle bit for bit; (2) the grouped op equals an fp32 GPU matmul of the
GPU-dequantized weights (pinned by (1) and by the small-shape parity tests) within 1e-2 per
output row; (3) linearity in x."""
import numpy as np
import pytest
import torch

from oracle import ggml_ref as G

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _rel(y, ref):
    y = y.double()
    ref = ref.double()
    scale = ref.abs().amax(dim=1, keepdim=True).clamp(min=1e-30)
    return float(((y - ref).abs() / scale).amax())


def _pinned_dequant(W, wt, n, K, seed):
    """fp32 weights of a full-size shard dequantized on the GPU, pinned by a random subset of
    min(48, n) rows that equals the oracle bit for bit."""
    import gguf_hip

    k = min(48, n)
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(seed))[:k].sort().values.to(W.device)
    wsub = gguf_hip.dequantize(W[rows], wt, (k, K)).cpu().numpy()
    assert np.array_equal(wsub.view(np.uint32), G.dequantize(W[rows].cpu().numpy(), wt).view(np.uint32))
    return gguf_hip.dequantize(W, wt, (n, K), torch.float32)


def _check_shard(dev, wt, n, K, Ms, seed):
    import gguf_hip
    from gguf_hip.synth import random_shard

    W = random_shard(n, K, wt, dev, seed=seed)
    wf = _pinned_dequant(W, wt, n, K, seed)
    gl = gguf_hip.pack_layer([W], [n], [wt])
    del W
    g = torch.Generator(device=dev).manual_seed(seed)
    for M in Ms:
        x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        y = gguf_hip.mul_mat_grouped(x, gl)
        ref = x.float() @ wf.T
        e = _rel(y, ref)
        assert e < TOL, (G.NAMES[wt], n, K, M, e)
        if M <= 8:
            x2 = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
            y2 = gguf_hip.mul_mat_grouped(x2, gl)
            y12 = gguf_hip.mul_mat_grouped((x.float() + x2.float()).to(torch.bfloat16), gl)
            assert _rel(y12, (x.float() + x2.float()).to(torch.bfloat16).float() @ wf.T) < TOL
            assert _rel(y.float() + y2.float(), y12.float()) < 2 * TOL     # linearity
    del wf, gl
    torch.cuda.empty_cache()


@pytest.mark.parametrize("wt", [G.Q4_K, G.Q6_K], ids=lambda t: G.NAMES[t])
@pytest.mark.parametrize("shape", [(7168, 5120), (5120, 5120), (34816, 5120), (5120, 17408)], ids=str)
def test_config2_decode_shapes(dev, wt, shape):
    _check_shard(dev, wt, *shape, Ms=(1, 2, 4, 8), seed=shape[0] + wt)


@pytest.mark.parametrize("wt", G.ALL_TYPES, ids=lambda t: G.NAMES[t])
def test_config3_all_types_big_shards(dev, wt):
    _check_shard(dev, wt, 34816, 5120, Ms=(1, 4, 8, 16, 32), seed=wt)
    _check_shard(dev, wt, 5120, 17408, Ms=(1, 4, 8, 16, 32), seed=100 + wt)


@pytest.mark.parametrize("wt", [G.Q4_K, G.Q5_K, G.IQ4_XS], ids=lambda t: G.NAMES[t])
def test_config4_prefill_gemm(dev, wt):
    _check_shard(dev, wt, 34816, 5120, Ms=(512, 2048, 8192), seed=200 + wt)
    _check_shard(dev, wt, 5120, 17408, Ms=(512, 2048, 8192), seed=300 + wt)


@pytest.mark.parametrize("wt", [G.IQ4_XS, G.IQ3_S, G.Q4_K, G.Q3_K, G.Q6_K, G.Q8_0], ids=lambda t: G.NAMES[t])
def test_reference_wide_form_edges(dev, wt):
    """The reference's wide-form edge list (gguf-plugin/test_gluon_wide_gpu.py:37-39): ffn_gate,
    attn_k / attn_v, a k / v row count with ffn_down's K, and a 48-row shard (a partial tile), at
    the row counts around every GEMM tile form's boundary."""
    for i, (n, K) in enumerate([(17408, 5120), (1024, 5120), (1024, 17408), (48, 5120)]):
        _check_shard(dev, wt, n, K, Ms=(33, 64, 65, 128, 129, 2048), seed=400 + 10 * wt + i)


@pytest.mark.parametrize("layer", [0, 1])
def test_config5_mixed_type_layers(dev, layer):
    """BASELINE config 5 at its layer shapes: decoder layers of the seeded 64-layer type draw
    (the one bench_configs.py times), each as one mixed-type grouped launch over qkv 7168 / o_proj
    5120 / gate_up 34816 rows at K = 5120 plus down 5120 x 17408, at M = 1, 8, 12, 32, 64, 100 (the
    mixed-type GEMV, with the 16 x 16 x 32 form's types at 12, and every small GEMM form, x staged
    by direct-to-LDS loads at 100): every
    shard's rows pinned bit-exact against the oracle on a subset, and the launches against an fp32
    matmul of the dequantized weights within 1e-2."""
    import gguf_hip
    from gguf_hip.synth import random_shard

    from bench_configs import LAYER_SHAPES, draw_stack_types

    types = draw_stack_types(64)[layer]
    k5 = [(t, N) for t, (_, N, K) in zip(types, LAYER_SHAPES) if K == 5120]
    assert len({t for t, _ in k5}) > 1 or layer > 0          # layer 0 of the draw mixes types
    Ws = [random_shard(N, 5120, t, dev, seed=1000 * layer + N + t) for t, N in k5]
    wf = torch.cat([_pinned_dequant(W, t, N, 5120, seed=N + t) for W, (t, N) in zip(Ws, k5)])
    gl = gguf_hip.pack_layer(Ws, [N for _, N in k5], [t for t, _ in k5])
    del Ws
    t_d = types[3]
    Wd = random_shard(5120, 17408, t_d, dev, seed=1000 * layer + 17408 + t_d)
    wd = _pinned_dequant(Wd, t_d, 5120, 17408, seed=17408 + t_d)
    gld = gguf_hip.pack_layer([Wd], [5120], [t_d])
    del Wd
    g = torch.Generator(device=dev).manual_seed(layer)
    for M in (1, 8, 12, 32, 64, 100):
        x = torch.randn(M, 5120, device=dev, generator=g).to(torch.bfloat16)
        y = gguf_hip.mul_mat_grouped(x, gl)
        assert y.shape == (M, wf.shape[0])
        e = _rel(y, x.float() @ wf.T)
        assert e < TOL, (types, M, e)
        xd = torch.randn(M, 17408, device=dev, generator=g).to(torch.bfloat16)
        e = _rel(gguf_hip.mul_mat_grouped(xd, gld), xd.float() @ wd.T)
        assert e < TOL, (types, "down", M, e)
    del wf, wd, gl, gld
    torch.cuda.empty_cache()
