"""BASELINE shapes at full size (configs 2-4).  The oracle cannot dequantize 178 M weights in a
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


def _check_shard(dev, wt, n, K, Ms, seed):
    import gguf_hip
    from gguf_hip.synth import random_shard

    W = random_shard(n, K, wt, dev, seed=seed)
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(seed))[:48].sort().values
    sub = W[rows.to(dev)].cpu().numpy()
    wsub = gguf_hip.dequantize(W[rows.to(dev)], wt, (48, K)).cpu().numpy()
    assert np.array_equal(wsub.view(np.uint32), G.dequantize(sub, wt).view(np.uint32))
    wf = gguf_hip.dequantize(W, wt, (n, K), torch.float32)
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
    _check_shard(dev, wt, 34816, 5120, Ms=(1, 8, 32), seed=wt)
    _check_shard(dev, wt, 5120, 17408, Ms=(4, 16), seed=100 + wt)


@pytest.mark.parametrize("wt", [G.Q4_K, G.Q5_K, G.IQ4_XS], ids=lambda t: G.NAMES[t])
def test_config4_prefill_gemm(dev, wt):
    _check_shard(dev, wt, 34816, 5120, Ms=(512, 2048), seed=200 + wt)
    _check_shard(dev, wt, 5120, 17408, Ms=(2048,), seed=300 + wt)
