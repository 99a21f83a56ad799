"""The GGUF v3 load path: the C++ reader (CPU: headers, metadata, tensor bytes, malformed files),
layer runs over the published model's tensor table (tests/golden/qwen35_iq3s_tensors.json, from
gguf-plugin/iq3s-tensor-names.json), and on the GPU a file's tensors uploaded into grouped layers
checked against the oracle."""
import json
import os
import struct

import numpy as np
import pytest

import gguf_writer as W
from oracle import ggml_ref as G

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

KVS = [
    ("general.architecture", W.STRING, "llama"),
    ("general.alignment", W.UINT32, 64),
    ("llama.block_count", W.UINT32, 2),
    ("test.u8", W.UINT8, 200), ("test.i8", W.INT8, -7), ("test.u16", W.UINT16, 65000), ("test.i16", W.INT16, -30000),
    ("test.i32", W.INT32, -123456), ("test.f32", W.FLOAT32, 0.25), ("test.bool", W.BOOL, True),
    ("test.u64", W.UINT64, 2**63 + 5), ("test.i64", W.INT64, -2**40), ("test.f64", W.FLOAT64, -1.5),
    ("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, ["<s>", "</s>", "héllo", ""])),
    ("tokenizer.ggml.scores", W.ARRAY, (W.FLOAT32, [0.0, -1.0, 2.5, 3.0])),
    ("test.empty", W.ARRAY, (W.INT32, [])),
]


def _small_model(rng, K=512):
    """Two llama blocks: q/k/v and gate/up of mixed types, o_proj/down, a norm vector, an
    unsupported type and an F16 matrix."""
    ts = []
    spec = [("blk.0.attn_q.weight", G.Q4_K, 192), ("blk.0.attn_k.weight", G.Q6_K, 64), ("blk.0.attn_v.weight", G.IQ4_XS, 64),
            ("blk.0.attn_output.weight", G.Q8_0, 96), ("blk.0.ffn_gate.weight", G.Q5_K, 128),
            ("blk.0.ffn_up.weight", G.IQ3_S, 128), ("blk.1.attn_q.weight", G.Q4_0, 64), ("blk.1.attn_k.weight", G.Q5_0, 64),
            ("blk.1.attn_v.weight", G.IQ4_NL, 64), ("blk.1.ffn_up.weight", G.Q2_K, 80), ("blk.1.ffn_gate.weight", G.Q3_K, 80)]
    for name, wt, n in spec:
        raw = G.make_weights(rng, n, K, wt)
        ts.append((name, (K, n), wt, raw.tobytes(), raw))
    norm = rng.normal(size=K).astype(np.float32)
    ts.append(("blk.0.attn_norm.weight", (K,), 0, norm.tobytes(), None))
    iq2 = rng.integers(0, 256, size=(32, K // 256 * 66), dtype=np.uint8)
    ts.append(("blk.0.ffn_down.weight", (K, 32), 16, iq2.tobytes(), None))        # IQ2_XXS: no kernel here
    f16 = rng.normal(size=(16, K)).astype(np.float16)
    ts.append(("output.weight", (K, 16), 1, f16.tobytes(), None))
    return ts


def _write(path, ts, **kw):
    return W.write_gguf(path, KVS, [(n, d, t, b) for n, d, t, b, _ in ts], **kw)


def test_reader_metadata_and_tensors(tmp_path):
    import gguf_hip

    rng = np.random.default_rng(7)
    ts = _small_model(rng)
    path = tmp_path / "m.gguf"
    offs = _write(path, ts, alignment=64)
    with gguf_hip.GGUFFile(path) as f:
        assert f.version == 3 and f.alignment == 64 and f.data_offset % 64 == 0
        fl = f.fields
        assert fl["general.architecture"] == "llama" and fl["llama.block_count"] == 2
        assert (fl["test.u8"], fl["test.i8"], fl["test.u16"], fl["test.i16"]) == (200, -7, 65000, -30000)
        assert fl["test.i32"] == -123456 and fl["test.f32"] == 0.25 and fl["test.bool"] is True
        assert fl["test.u64"] == 2**63 + 5 and fl["test.i64"] == -2**40 and fl["test.f64"] == -1.5
        assert fl["tokenizer.ggml.tokens"] == ["<s>", "</s>", "héllo", ""]
        assert fl["tokenizer.ggml.scores"].dtype == np.float32 and fl["tokenizer.ggml.scores"].tolist() == [0, -1, 2.5, 3]
        assert fl["test.empty"].size == 0
        assert [t.name for t in f.tensors] == [t[0] for t in ts]
        for t, (name, dims, wt, data, _), off in zip(f.tensors, ts, offs):
            assert t.dims == dims and t.ggml_type == wt and t.offset == off and t.nbytes == len(data)
            assert t.offset % 64 == 0
            assert f.raw(name).tobytes() == data
        assert f.tensor("blk.0.attn_k.weight").shape == (64, 512)
        assert gguf_hip.ggml_type_size(G.Q6_K) == (256, 210) and gguf_hip.ggml_type_size(16) == (256, 66)
        with pytest.raises(KeyError):
            f.tensor("nope")
    with pytest.raises(ValueError):
        f.raw("blk.0.attn_q.weight")          # closed


def test_reader_default_alignment(tmp_path):
    import gguf_hip

    rng = np.random.default_rng(8)
    raw = G.make_weights(rng, 8, 256, G.Q4_K)
    path = tmp_path / "a.gguf"
    offs = W.write_gguf(path, [("general.architecture", W.STRING, "x")],
                        [("a.weight", (256, 8), G.Q4_K, raw.tobytes()), ("b.weight", (256, 8), G.Q4_K, raw.tobytes())])
    with gguf_hip.GGUFFile(path) as f:
        assert f.alignment == 32 and [t.offset for t in f.tensors] == offs and offs[1] - offs[0] == 1152
        assert np.array_equal(f.raw("b.weight"), raw)


def _expect_error(path, match):
    import gguf_hip

    with pytest.raises(ValueError, match=match):
        gguf_hip.GGUFFile(path)


def test_reader_rejects_malformed_files(tmp_path):
    rng = np.random.default_rng(9)
    raw = G.make_weights(rng, 8, 256, G.Q4_K).tobytes()
    good = tmp_path / "g.gguf"
    W.write_gguf(good, KVS[:1], [("a.weight", (256, 8), G.Q4_K, raw)])
    blob = good.read_bytes()
    cases = {
        "magic": (b"GGUX" + blob[4:], "not a GGUF file"),
        "version": (blob[:4] + struct.pack("<I", 2) + blob[8:], "version 2"),
        "truncated": (blob[:40], "truncated|corrupt|bad"),
        "short": (blob[:10], "too short"),
        "past_end": (blob[:-100], "past the end"),
        "counts": (blob[:8] + struct.pack("<Q", 2**40) + blob[16:], "corrupt header"),
    }
    for name, (data, match) in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        _expect_error(p, match)
    _expect_error(tmp_path / "missing.gguf", "cannot open")
    # an offset that is not a multiple of the alignment, and a repeated name
    bad = tmp_path / "unaligned.gguf"
    W.write_gguf(bad, KVS[:1], [("a.weight", (256, 8), G.Q4_K, raw)])
    b = bytearray(bad.read_bytes())
    i = b.index(b"a.weight") + len(b"a.weight") + 4 + 16 + 4     # name, n_dims, dims, type -> offset
    b[i:i + 8] = struct.pack("<Q", 8)
    bad.write_bytes(bytes(b))
    _expect_error(bad, "unaligned")
    dup = tmp_path / "dup.gguf"
    W.write_gguf(dup, KVS[:1], [("a.weight", (256, 8), G.Q4_K, raw), ("a.weight", (256, 8), G.Q4_K, raw)])
    _expect_error(dup, "duplicate")
    ali = tmp_path / "ali.gguf"
    W.write_gguf(ali, [("general.alignment", W.UINT32, 48)], [("a.weight", (256, 8), G.Q4_K, raw)], alignment=48)
    _expect_error(ali, "power-of-two")


def test_layer_runs_merge_qkv_and_gate_up(tmp_path):
    import gguf_hip

    rng = np.random.default_rng(10)
    path = tmp_path / "m.gguf"
    _write(path, _small_model(rng))
    with gguf_hip.GGUFFile(path) as f:
        runs = [(n, [t.name for t in ms]) for n, ms in gguf_hip.layer_runs(f.tensors)]
    assert runs == [
        ("blk.0.attn_qkv", ["blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.0.attn_v.weight"]),
        ("blk.0.attn_output", ["blk.0.attn_output.weight"]),
        ("blk.0.ffn_gate_up", ["blk.0.ffn_gate.weight", "blk.0.ffn_up.weight"]),
        ("blk.1.attn_qkv", ["blk.1.attn_q.weight", "blk.1.attn_k.weight", "blk.1.attn_v.weight"]),
        # ffn_up comes first in the file: the run sits there, in vLLM's shard order (gate, up)
        ("blk.1.ffn_gate_up", ["blk.1.ffn_gate.weight", "blk.1.ffn_up.weight"]),
        ("blk.0.ffn_down", ["blk.0.ffn_down.weight"]),
        ("output", ["output.weight"]),
    ]


def test_published_model_tensor_table(tmp_path):
    """The published IQ3_S model's 1185-tensor table written as a header-only file (data a
    file-system hole): every tensor parses with its GGML byte size, and the layer runs are the
    64 blocks' gate/up pairs plus single calls."""
    import gguf_hip

    doc = json.load(open(os.path.join(GOLDEN, "qwen35_iq3s_tensors.json"), encoding="utf-8"))
    table = [(t["name"], tuple(t["dims"]), W.TYPE_IDS[t["type"]], None) for t in doc["tensors"]]
    path = tmp_path / "qwen35.gguf"
    W.write_gguf(path, [("general.architecture", W.STRING, doc["architecture"])], table, sparse=True)
    with gguf_hip.GGUFFile(path) as f:
        assert f.fields["general.architecture"] == "qwen35" and len(f.tensors) == 1185
        for t, (name, dims, gt, _) in zip(f.tensors, table):
            assert (t.name, t.dims, t.ggml_type, t.nbytes) == (name, dims, gt, W.nbytes(gt, dims))
        assert f.tensor("blk.0.ffn_down.weight").shape == (5120, 17408)
        total = sum(t.nbytes for t in f.tensors)
        assert os.path.getsize(path) >= total and 8e9 < total < 20e9
        runs = gguf_hip.layer_runs(f.tensors)
    names = [n for n, _ in runs]
    gate_up = [n for n in names if n.endswith("ffn_gate_up")]
    assert len(gate_up) == 64 and "token_embd" not in names and "output" in names
    assert all(len(ms) == 2 and ms[0].name.endswith("ffn_gate.weight") for n, ms in runs if n.endswith("gate_up"))
    # 48 linear-attention blocks store attn_qkv as one tensor; the 16 full-attention blocks
    # (index % 4 == 3) store q, k, v, merged here into one run
    qkv = {n: ms for n, ms in runs if n.startswith("blk.") and n.endswith("attn_qkv")}   # not the vision tower's v.blk.*
    assert len(qkv) == 64
    for n, ms in qkv.items():
        blk = int(n.split(".")[1])
        assert [m.name.split(".")[2] for m in ms] == (["attn_q", "attn_k", "attn_v"] if blk % 4 == 3 else ["attn_qkv"])
    assert len(names) == len(set(names))
    kinds = {t.ggml_type for _, ms in runs for t in ms} - set(gguf_hip.GGUF_TYPES)
    # F32 / BF16 matrices go to torch; IQ2_XXS, IQ2_XS, IQ3_XXS, IQ2_S, IQ1_M have no kernel here
    assert kinds == {0, 30, 16, 17, 18, 22, 29}


@pytest.mark.gpu
def test_load_grouped_layers_matches_oracle(dev, tmp_path):
    import torch

    import gguf_hip

    rng = np.random.default_rng(11)
    ts = _small_model(rng)
    path = tmp_path / "m.gguf"
    _write(path, ts, alignment=64)
    raws = {n: r for n, _, _, _, r in ts}
    with gguf_hip.GGUFFile(path) as f:
        layers, skipped = gguf_hip.load_grouped_layers(f, dev)
    assert set(skipped) == {"blk.0.ffn_down", "output"}
    assert set(layers) == {"blk.0.attn_qkv", "blk.0.attn_output", "blk.0.ffn_gate_up", "blk.1.attn_qkv",
                           "blk.1.ffn_gate_up"}
    names = {"blk.0.attn_qkv": ["blk.0.attn_q", "blk.0.attn_k", "blk.0.attn_v"],
             "blk.0.attn_output": ["blk.0.attn_output"], "blk.0.ffn_gate_up": ["blk.0.ffn_gate", "blk.0.ffn_up"],
             "blk.1.attn_qkv": ["blk.1.attn_q", "blk.1.attn_k", "blk.1.attn_v"],
             "blk.1.ffn_gate_up": ["blk.1.ffn_gate", "blk.1.ffn_up"]}
    for run, gl in layers.items():
        wf = []
        for view, n, wt, tn in zip(gl.views, gl.n_outs, gl.weight_types, names[run]):
            raw = raws[tn + ".weight"]
            ref = G.dequantize(raw, wt)
            got = gguf_hip.dequantize_tiles(view, n, gl.K, wt, torch.float32).cpu().numpy()
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (run, tn)
            wf.append(ref)
        wf = np.concatenate(wf)
        for M in (1, 8, 40):
            x = torch.from_numpy(rng.normal(size=(M, gl.K)).astype(np.float32)).to(torch.bfloat16).to(dev)
            y = gguf_hip.mul_mat_grouped(x, gl).float().cpu().numpy()
            e = G.rel_err(y, G.matmul_ref(x.float().cpu().numpy(), wf))
            assert e < 1e-2, (run, M, e)
