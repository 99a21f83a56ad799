"""Seeded random layers through the planner and every launch form, against the oracle: one to three
shards of random types and row counts, k-ranges of 1 to 30 super-blocks, the device's CU count or
a pinned one (so that small shards take the slab forms), 1 to 40 batch rows, with and without a
bias; each output within 1e-2 of the row's max |y| and bit-identical on a repeat.  The seeds are
fixed and the test asserts that the draw reached every form: the GEMV at G = 1 / 2 / 4 (streaming,
one-record and slab), the mid form and its slab, and the GEMM."""
import numpy as np
import pytest
import torch

from oracle import ggml_ref as G

pytestmark = pytest.mark.gpu

NBS = (1, 2, 3, 4, 5, 7, 12, 19, 20, 24, 25, 30)
CUS = (0, 0, 4, 8, 9, 16, 32, 64)


def test_random_layers_every_form(dev):
    import gguf_hip
    from gguf_hip import ops

    rng = np.random.default_rng(20251)
    seen = set()
    for case in range(60):
        nsh = 1 if rng.random() < 0.7 else int(rng.integers(2, 4))
        nb = int(rng.choice(NBS))
        K = 256 * nb
        shards = [(int(rng.choice(G.ALL_TYPES)), int(rng.integers(1, 700))) for _ in range(nsh)]
        cus = int(rng.choice(CUS))
        raws = [G.random_blocks(rng, n, K, wt) for wt, n in shards]
        wf = np.concatenate([G.dequantize(r, wt) for r, (wt, _) in zip(raws, shards)])
        gl = gguf_hip.pack_layer([torch.from_numpy(r).to(dev) for r in raws], [n for _, n in shards],
                                 [wt for wt, _ in shards], cus=cus)
        ntot = sum(n for _, n in shards)
        for M in sorted({int(m) for m in rng.integers(1, 41, size=3)}):
            info = ops.GqkPlanInfo.from_tuple(gl.plans[ops._pick_plan(gl.plans, M) * ops._NPLAN:][:ops._NPLAN])
            seen.add((info.form, info.g, info.bm) if info.form == 1 else (info.form, 0, 0))
            g = torch.Generator().manual_seed(case * 100 + M)
            x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
            bias = (torch.randn(ntot, generator=g) * 2).to(torch.bfloat16).to(dev) if rng.random() < 0.3 else None
            y = gguf_hip.mul_mat_grouped(x, gl, bias)
            ref = G.matmul_ref(x.float().cpu().numpy(), wf)
            if bias is not None:
                ref = ref + bias.float().cpu().numpy()[None]
            e = G.rel_err(y.float().cpu().numpy(), ref)
            assert e < 1e-2, (case, shards, nb, cus, M, e)
            assert torch.equal(gguf_hip.mul_mat_grouped(x, gl, bias), y), (case, shards, nb, cus, M)
    # GEMV G = 1 / 2 / 4 (bm 0 streaming, 1 one-record), the slab (bm 2) at G = 1 / 2, the mid
    # form (g 8) and its slab, the GEMM
    want = {(1, 1, 0), (1, 1, 1), (1, 1, 2), (1, 2, 0), (1, 2, 2), (1, 4, 0), (1, 4, 1), (1, 8, 0), (1, 8, 2),
            (2, 0, 0)}
    assert want <= seen, sorted(want - seen)
