"""CPU tests of the custom ops under tracing: the fake (meta) implementations give the real op's
output shape, dtype and device without touching data, and ``mul_mat_grouped`` traces with
``make_fx`` to the one custom op call (plus the dtype casts of non-bf16 activations), so a
torch.compile'd caller sees no host-side allocation, no data access and no graph break in it
(the reference registers its grouped op with a fake for the same purpose,
gguf-plugin/patches/gguf-tiles-grouped.patch:28-72).  No kernel runs here."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from oracle import ggml_ref as G


def _fake_layer(shards, K, mode):
    """A GroupedLayer whose tensors are fake CUDA tensors of mode and whose plans are the real ones
    (planned on the host before entering the mode)."""
    from gguf_hip import ops

    off, specs = 0, []
    for wt, n in shards:
        specs.append((wt, n, off))
        off += ops.tiles_bytes(wt, n, K)
    plans = [ops.plan(specs, K, m, cus=256) for m in ops.GEMV_BUCKETS + ops.GEMM_PLAN_M]
    with mode:
        gl = ops.GroupedLayer(torch.empty(off, dtype=torch.uint8, device="cuda"), [], [n for _, n in shards],
                              [wt for wt, _ in shards], K)
        for info, desc in plans:
            gl.descs.append(torch.empty(desc.shape, dtype=desc.dtype, device="cuda"))
            gl.plans.extend(info.as_tuple())
        gl.workspace = torch.empty(1 << 16, dtype=torch.int32, device="cuda")
    return gl


@pytest.mark.parametrize("M", [1, 8, 17, 300, 2048])
def test_fake_impls_shapes(M):
    from gguf_hip import ops

    mode = FakeTensorMode()
    gl = _fake_layer([(G.Q4_K, 200), (G.Q6_K, 70)], 1024, mode)
    with mode:
        for dt in (torch.bfloat16, torch.float16, torch.float32):
            x = torch.empty(M, 1024, dtype=dt, device="cuda")
            y = ops.mul_mat_grouped(x, gl)
            assert y.shape == (M, 270) and y.dtype == dt and y.device.type == "cuda"
            yb = ops.mul_mat_grouped(x, gl, bias=torch.empty(270, dtype=torch.bfloat16, device="cuda"))
            assert yb.shape == (M, 270) and yb.dtype == dt
        wide = torch.empty(M, 300, dtype=torch.bfloat16, device="cuda")
        x = torch.empty(M, 1024, dtype=torch.bfloat16, device="cuda")
        assert ops.mul_mat_grouped(x, gl, out=wide[:, 10:280]).shape == (M, 270)
        y = torch.ops.gguf_hip.fused_mul_mat_gguf_grouped(x, gl.packed, gl.descs, gl.plans, gl.n_total, gl.workspace)
        assert y.shape == (M, 270) and y.dtype == torch.bfloat16


def test_make_fx_traces_one_op():
    from gguf_hip import ops

    mode = FakeTensorMode()
    gl = _fake_layer([(G.IQ4_XS, 128), (G.Q8_0, 64)], 512, mode)
    with mode:
        x16 = torch.empty(8, 512, dtype=torch.bfloat16, device="cuda")
        x32 = torch.empty(8, 512, dtype=torch.float32, device="cuda")
        bias = torch.empty(192, dtype=torch.bfloat16, device="cuda")
        g16 = make_fx(lambda x, b: ops.mul_mat_grouped(x, gl, bias=b))(x16, bias)
        g32 = make_fx(lambda x: ops.mul_mat_grouped(x, gl))(x32)
    calls16 = [n.target for n in g16.graph.nodes if n.op == "call_function"]
    calls32 = [n.target for n in g32.graph.nodes if n.op == "call_function"]
    op = torch.ops.gguf_hip.fused_mul_mat_gguf_grouped.default
    assert calls16 == [op], calls16          # bf16 x, bf16 bias: the op alone, bias fused
    assert calls32.count(op) == 1 and all(c in (op, torch.ops.aten._to_copy.default) for c in calls32), calls32
