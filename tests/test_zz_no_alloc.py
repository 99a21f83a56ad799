"""gqk_linear_noalloc (the entry point that allocates nothing: its workspace is a per-GPU device
array) against gqk_linear with a caller workspace, through the C ABI: bit-identical outputs on
two calls in a row, the second with fewer rows, for a split-K GEMV plan, a slab-form GEMV plan (no
workspace at all), the mid form (17..32 rows) in its slab and with its split-K exchange, a
stream-K GEMM plan and a mixed-type layer; a plan whose workspace exceeds the array is refused
with an error."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import ggml_ref as G

pytestmark = pytest.mark.gpu


def _x(M, K, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)


def _call(fn, gl, x, alloc_ws):
    from gguf_hip import ops
    from gguf_hip._lib import lib

    M = int(x.shape[0])
    i = ops._pick_plan(gl.plans, M)
    info = ops.GqkPlanInfo.from_tuple(gl.plans[i * ops._NPLAN:(i + 1) * ops._NPLAN])
    y = torch.full((M, gl.n_total), float("nan"), dtype=torch.bfloat16, device=x.device)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [ctypes.c_void_p(gl.packed.data_ptr()), ctypes.c_void_p(gl.descs[i].data_ptr()), ctypes.byref(info),
            ctypes.c_void_p(x.data_ptr()), x.stride(0), M, ctypes.c_void_p(y.data_ptr()), y.stride(0), None]
    if alloc_ws:
        ws = gl.workspace
        rc = lib.gqk_linear(*args, ctypes.c_void_p(ws.data_ptr()), ws.numel() * 4, st)
    else:
        rc = lib.gqk_linear_noalloc(*args, st)
    return rc, y, info


def test_noalloc_matches_linear_twice_then_smaller(dev):
    import gguf_hip
    from gguf_hip._lib import lib

    rng = np.random.default_rng(41)
    K = 3072
    cases = [
        ("split-K GEMV", [(G.Q4_K, 900)], 4096, 0, (8, 3)),
        ("slab GEMV", [(G.Q6_K, 200)], 0, 8, (8, 3)),             # planned for 8 CUs: 7 slabs
        ("mid slab", [(G.Q4_K, 200)], 0, 8, (30, 17)),            # the mid form's slab, 7 slabs
        ("mid split-K", [(G.Q5_K, 900)], 4096, 0, (32, 20)),      # the mid form's exchange
        ("stream-K GEMM", [(G.Q6_K, 1000)], 0, 0, (60, 20)),
        ("mixed layer", [(G.IQ4_XS, 130), (G.Q5_K, 300), (G.Q8_0, 64)], 2048, 0, (5, 2)),
        ("mixed layer GEMM", [(G.IQ4_XS, 130), (G.Q5_K, 300), (G.Q8_0, 64)], 0, 0, (100, 33)),
    ]
    for name, shards, target, cus, Ms in cases:
        raws = [G.random_blocks(rng, n, K, wt) for wt, n in shards]
        gl = gguf_hip.pack_layer([torch.from_numpy(r).to(dev) for r in raws], [n for _, n in shards],
                                 [wt for wt, _ in shards], target_wgs=target, cus=cus)
        for M in Ms:                                          # two calls in a row, the second smaller
            x = _x(M, K, 17 + M, dev)
            rc, y_ref, info = _call(None, gl, x, True)
            assert rc == 0, lib.gqk_last_error()
            rc, y, _ = _call(None, gl, x, False)
            assert rc == 0, lib.gqk_last_error()
            torch.cuda.synchronize()
            assert torch.equal(y, y_ref), (name, M)
            wf = np.concatenate([G.dequantize(r, wt) for r, (wt, _) in zip(raws, shards)])
            assert G.rel_err(y.float().cpu().numpy(), G.matmul_ref(x.float().cpu().numpy(), wf)) < 1e-2, (name, M)
        if name == "split-K GEMV":
            assert info.split > 1
        if name in ("slab GEMV", "mid slab"):
            assert info.bm == 2 and info.workspace_bytes == 0
        if name.startswith("mid"):
            assert info.g == 8 and (info.split > 1) == (name == "mid split-K")


def test_noalloc_refuses_a_plan_beyond_its_array(dev):
    import gguf_hip
    from gguf_hip import _lib

    rng = np.random.default_rng(42)
    n, K = 34816, 256
    raw = G.random_blocks(rng, n, K, G.Q4_0)
    gl = gguf_hip.pack_layer([torch.from_numpy(raw).to(dev)], [n], [G.Q4_0])
    # the first M (in steps of 256) whose plan needs more workspace than the array on this device
    # (the stream-K partials depend on the tile count modulo the device's persistent workgroups)
    from gguf_hip import ops

    M = None
    for m in range(256, 16385, 256):
        i = ops._pick_plan(gl.plans, m)
        info = ops.GqkPlanInfo.from_tuple(gl.plans[i * ops._NPLAN:(i + 1) * ops._NPLAN])
        if _lib.lib.gqk_linear_workspace_bytes(ctypes.byref(info), m) > _lib.GQK_NOALLOC_SCRATCH_BYTES:
            M = m
            break
    assert M is not None, "no M up to 16384 needs more than the array"
    x = _x(M, K, 5, dev)
    rc, _, info = _call(None, gl, x, False)
    need = _lib.lib.gqk_linear_workspace_bytes(ctypes.byref(info), M)
    assert need > _lib.GQK_NOALLOC_SCRATCH_BYTES, (M, need)
    assert rc == _lib.GQK_ERR_SHAPE and b"no-allocation" in _lib.lib.gqk_last_error()
    # and the same layer at a decode M runs
    rc, y, _ = _call(None, gl, _x(8, K, 6, dev), False)
    assert rc == 0 and bool(torch.isfinite(y.float()).all())
