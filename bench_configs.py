#!/usr/bin/env python3
"""The other measurement configurations of the GGUF linear path on one MI355X, one JSON line per
case (bench.py keeps the single headline line of config 2).

    python bench_configs.py --config 3    # all eleven types standalone: gate_up / down, M 1..32
    python bench_configs.py --config 4    # prefill dequant-GEMM: Q4_K / Q5_K / IQ4_XS, M 512..8192
    python bench_configs.py --config 5    # the 64-layer mixed-type stack: weight-stream time per step

Timing as in bench.py: random valid GGUF blocks generated on the GPU, rotating copies whose
packed bytes exceed the 256 MB Infinity Cache (config 3: > 1 GB per case), launches captured in a
HIP graph and timed with events; the median of five replays of the graph.  GB/s counts packed
GGUF block bytes (the reference's convention, gguf-plugin/README.md:134-137); TFLOP/s counts
2*M*N*K.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "hyperqwen-rtx4080s32_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

from bench import BF16_PEAK_TFLOPS, HBM_PEAK_GBS, _capture, _time_graph  # noqa: E402

ALL_TYPES = (2, 6, 8, 10, 11, 12, 13, 14, 20, 21, 23)
CONFIG3_SHAPES = (("gate_up", 34816, 5120), ("down", 5120, 17408))
LAYER_SHAPES = (("qkv", 7168, 5120), ("o_proj", 5120, 5120), ("gate_up", 34816, 5120), ("down", 5120, 17408))


def _emit(rec: dict) -> None:
    print(json.dumps(rec), flush=True)


def _median_ms(g, torch, launches: int, reps: int = 3) -> float:
    g.replay()
    return statistics.median(_time_graph(g, reps, torch) for _ in range(5)) / launches


def _copies(nbytes: int, floor_bytes: float, cap: int = 24) -> int:
    return max(2, min(cap, math.ceil(floor_bytes / nbytes)))


def config3(torch, gguf_hip, random_shard, dev, ms: list[int], types=ALL_TYPES, shapes=CONFIG3_SHAPES) -> None:
    """every type alone as the (34816, 5120) and (5120, 17408) shards."""
    for wt in types:
        for name, N, K in shapes:
            nbytes = random_shard(64, K, wt, dev).numel() // 64 * N
            gls = []
            for c in range(_copies(nbytes, 1.1e9)):
                W = random_shard(N, K, wt, dev, seed=7919 * c + wt)
                gls.append(gguf_hip.pack_layer([W], [N], [wt]))
                del W
            torch.cuda.empty_cache()
            for M in ms:
                x = torch.randn(M, K, device=dev).to(torch.bfloat16)

                def f(x=x, gls=gls):
                    for gl in gls:
                        gguf_hip.mul_mat_grouped(x, gl)
                g = _capture(f, torch)
                t = _median_ms(g, torch, len(gls))
                del g
                gbs = nbytes / (t * 1e-3) / 1e9
                i = gguf_hip.ops._pick_plan(gls[0].plans, M)
                info = gguf_hip.ops.GqkPlanInfo.from_tuple(gls[0].plans[i * gguf_hip.ops._NPLAN:][:gguf_hip.ops._NPLAN])
                form = (("slab_g%d" % info.g if info.bm == 2 else f"gemv_g{info.g}") if info.g <= 4 else "mid") \
                    if info.form == 1 else f"gemm{info.bm}"
                _emit({"config": 3, "type": gguf_hip.TYPE_NAMES[wt], "shard": name, "N": N, "K": K, "M": M,
                       "form": form, "us": round(t * 1e3, 2), "packed_bytes": nbytes,
                       "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "copies": len(gls)})
            del gls
            torch.cuda.empty_cache()


def config4(torch, gguf_hip, random_shard, dev, ms: list[int]) -> None:
    """the prefill dequant-GEMM, Q4_K / Q5_K / IQ4_XS at both shapes."""
    for wt in (12, 13, 23):
        for name, N, K in CONFIG3_SHAPES:
            gls = []
            for c in range(3):
                W = random_shard(N, K, wt, dev, seed=104729 * c + wt)
                gls.append(gguf_hip.pack_layer([W], [N], [wt]))
                del W
            torch.cuda.empty_cache()
            for M in ms:
                x = torch.randn(M, K, device=dev).to(torch.bfloat16)

                def f(x=x, gls=gls):
                    for gl in gls:
                        gguf_hip.mul_mat_grouped(x, gl)
                g = _capture(f, torch)
                t = _median_ms(g, torch, len(gls), reps=2)
                del g
                tf = 2.0 * M * N * K / (t * 1e-3) / 1e12
                path = "dequant_vendor_gemm" if M >= gguf_hip.ops.DEQUANT_MIN_M else "fused_gemm"
                _emit({"config": 4, "type": gguf_hip.TYPE_NAMES[wt], "shard": name, "N": N, "K": K, "M": M,
                       "path": path, "ms": round(t, 4), "TFLOPs": round(tf, 1),
                       "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)})
                del x
            del gls
            torch.cuda.empty_cache()


def draw_stack_types(layers: int, seed: int = 5) -> list[list[int]]:
    """Per layer, a GGML type for each of qkv, o_proj, gate_up, down: a seeded draw over the
    eleven types weighted toward Q4_K / Q5_K / IQ4_XS (0.3 / 0.2 / 0.2, the other eight share 0.3)."""
    import numpy as np

    p = np.full(len(ALL_TYPES), 0.3 / 8)
    for t, w in ((12, 0.3), (13, 0.2), (23, 0.2)):
        p[ALL_TYPES.index(t)] = w
    rng = np.random.default_rng(seed)
    return [[int(ALL_TYPES[i]) for i in rng.choice(len(ALL_TYPES), size=len(LAYER_SHAPES), p=p)]
            for _ in range(layers)]


def build_stack(torch, gguf_hip, random_shard, dev, layers: int):
    """The config-5 stack resident in HBM: per layer one mixed-type grouped layer over its three
    K = 5120 matrices (qkv, o_proj, gate_up) and down alone ('grouped': 2 launches per layer), and
    the same packed bytes as one layer per matrix ('per_linear': 4 launches, as vLLM's four
    linear layers call it).  Returns (grouped, per_linear, packed GGUF bytes, types per layer)."""
    types = draw_stack_types(layers)
    grouped, per_linear = [], []
    packed_bytes = 0
    for li, tl in enumerate(types):
        k5 = [(t, s) for t, s in zip(tl, LAYER_SHAPES) if s[2] == 5120]
        sizes = [gguf_hip.tiles_bytes(t, N, K) for t, (_, N, K) in k5]
        packed = torch.empty(sum(sizes), dtype=torch.uint8, device=dev)
        off = 0
        for (t, (_, N, K)), size in zip(k5, sizes):
            W = random_shard(N, K, t, dev, seed=1000 * li + N + t)
            packed_bytes += W.numel()
            packed[off:off + size].copy_(gguf_hip.repack_tiles(W, N, t))
            del W
            off += size
        ns, ts = [N for _, (_, N, _) in k5], [t for t, _ in k5]
        grouped.append((5120, gguf_hip.grouped_layer_from_packed(packed, ns, ts, 5120)))
        off = 0
        for n, t, size in zip(ns, ts, sizes):
            per_linear.append((5120, gguf_hip.grouped_layer_from_packed(packed[off:off + size], [n], [t], 5120)))
            off += size
        t_d = tl[3]
        W = random_shard(5120, 17408, t_d, dev, seed=1000 * li + 17408 + t_d)
        packed_bytes += W.numel()
        down = gguf_hip.pack_layer([W], [5120], [t_d])
        del W
        grouped.append((17408, down))
        per_linear.append((17408, down))
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return grouped, per_linear, packed_bytes, types


def time_stack(torch, gguf_hip, dev, lst, M: int) -> float:
    """ms per step of one pass over the stack's launches at M rows (graph replays, median).  Every
    launch reads an input of its own, as a decoder's linear calls do."""
    xs = [torch.randn(M, K, device=dev).to(torch.bfloat16) for K, _ in lst]

    def f():
        for x, (_, gl) in zip(xs, lst):
            gguf_hip.mul_mat_grouped(x, gl)
    g = _capture(f, torch)
    t = _median_ms(g, torch, 1, reps=2)
    del g
    return t


def config5(torch, gguf_hip, random_shard, dev, ms: list[int], layers: int) -> None:
    """`layers` decoder layers, each with qkv / o_proj / gate_up / down of a
    drawn type, resident in HBM (one copy: the stack itself is far beyond the Infinity Cache).
    Two launch schedules stream the same bytes: 'grouped' = one mixed-type launch per layer over
    its three K = 5120 matrices plus one for down (a launch needs one K), 'per_linear' = one
    launch per matrix, as vLLM's four linear layers call it."""
    t0 = time.perf_counter()
    grouped, per_linear, packed_bytes, types = build_stack(torch, gguf_hip, random_shard, dev, layers)
    counts = {gguf_hip.TYPE_NAMES[t]: sum(tl.count(t) for tl in types) for t in ALL_TYPES}
    weights = layers * sum(N * K for _, N, K in LAYER_SHAPES)
    _emit({"config": 5, "layers": layers, "packed_bytes": packed_bytes, "weights": weights,
           "bpw": round(8 * packed_bytes / weights, 3), "type_counts": counts,
           "load_s": round(time.perf_counter() - t0, 2)})
    for M in ms:
        for sched, lst in (("grouped", grouped), ("per_linear", per_linear)):
            t = time_stack(torch, gguf_hip, dev, lst, M)
            gbs = packed_bytes / (t * 1e-3) / 1e9
            _emit({"config": 5, "schedule": sched, "M": M, "launches_per_step": len(lst), "ms_per_step": round(t, 4),
                   "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, required=True, choices=(3, 4, 5))
    ap.add_argument("--m", default="", help="comma-separated batch rows (default: the config's own list)")
    ap.add_argument("--layers", type=int, default=64, help="config 5: decoder layers")
    ap.add_argument("--types", default="", help="config 3: comma-separated type names (default: all eleven)")
    ap.add_argument("--shards", default="", help="config 3: comma-separated shard names, gate_up / down (default: both)")
    args = ap.parse_args()

    import torch

    import gguf_hip
    from gguf_hip.synth import random_shard

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    default_ms = {3: "1,4,8,16,32", 4: "512,2048,8192", 5: "1,8,32,64"}[args.config]
    ms = [int(v) for v in (args.m or default_ms).split(",")]
    if args.config == 3:
        names = {v: k for k, v in gguf_hip.TYPE_NAMES.items()}
        types = [names[t] for t in args.types.split(",")] if args.types else ALL_TYPES
        shapes = [s for s in CONFIG3_SHAPES if not args.shards or s[0] in args.shards.split(",")]
        config3(torch, gguf_hip, random_shard, dev, ms, types, shapes)
    elif args.config == 4:
        config4(torch, gguf_hip, random_shard, dev, ms)
    else:
        config5(torch, gguf_hip, random_shard, dev, ms, args.layers)
    return 0


if __name__ == "__main__":
    sys.exit(main())
