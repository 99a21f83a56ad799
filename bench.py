#!/usr/bin/env python3
"""Benchmark of the GGUF quantized linear path on one MI355X (BASELINE.json's metric).

Workload (the configuration the metric is quoted on): the Q4_K and Q6_K
decode GEMV at the 27B-class dense shapes (N, K) in {(7168, 5120) qkv, (5120, 5120) o_proj,
(34816, 5120) gate_up, (5120, 17408) down}, batch rows M = 8 (default), bf16 activations.
One step = one grouped launch per (type, shape) shard over one batch, i.e. every shard's
packed weights streamed once.  Weights are random valid GGUF blocks generated on the GPU
(kernel time does not depend on the values) in `--copies` rotating copies (> 1 GB in total) so
the 256 MB Infinity Cache cannot serve a repeat; launches are captured in HIP graphs and timed
with events on the launch stream.

value = packed GGUF bytes per step / time per step (GB/s; inputs resident in HBM).
roofline = the dominant kernel (the shard with the largest launch time): packed bytes per
launch / its average launch duration vs 8 TB/s.  The M = 2048 dequant-GEMM (config 4, Q4_K
gate_up) is reported beside it as TFLOP/s vs 2.5 PFLOP/s bf16.
cpu_baseline = the reference CPU path (gguf-py's dequantizer, as restated by oracle/, plus
torch.matmul in fp32) on a bounded row sample of the Q4_K / Q6_K gate_up shards.
"""
from __future__ import annotations

import argparse
import ctypes
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

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0        # MI355X dense bf16 MFMA
Q4_K, Q6_K = 12, 14
SHAPES = [("qkv", 7168, 5120), ("o_proj", 5120, 5120), ("gate_up", 34816, 5120), ("down", 5120, 17408)]
METRIC = "packed-weight GB/s (% HBM peak) at M=1-32; bf16 TFLOP/s (% MFMA) at M=2048"


def _time_graph(graph, reps, torch):
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        graph.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def _capture(fn, torch):
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        fn()                                  # warm the allocator outside the capture
    torch.cuda.current_stream().wait_stream(st)
    with torch.cuda.graph(g):
        fn()
    return g


def _form(info) -> str:
    """The launch form of a plan: the GEMV (token groups g), its slab form, the mid form, the GEMM tile."""
    if info.form != 1:
        return f"gemm{info.bm}"
    return f"slab_g{info.g}" if info.bm == 2 else f"gemv_g{info.g}" if info.g <= 4 else "mid"


def _source_sha16(rel: str) -> str:
    import hashlib

    with open(os.path.join(REPO, rel), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def _traffic(symbol: str, dom: dict, M: int) -> tuple[int | None, str]:
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter's reading on a plain copy of
    known size; PMC counters are not read in this run), and where the figure comes from.  A
    summary counts only for the same kernel symbol and workload, taken from the same kernel
    source (its recorded sha256 prefix equals the current file's): a kernel changed since the
    profile gives None, with the reason."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None, "no profiles/traffic.json"
    with open(path, encoding="utf-8") as f:
        rec = json.load(f)
    for r in rec.get("kernels", []):
        if r.get("symbol") == symbol and r.get("N") == dom["N"] and r.get("K") == dom["K"] and r.get("M") == M:
            src = r.get("source")
            if not src or r.get("source_sha16") != _source_sha16(src):
                return None, (f"profiles/traffic.json holds {symbol} at this shape, but from another version of "
                              f"{src or 'its source'}: stale, not used")
            return r["hbm_bytes_per_launch"], ("profiles/traffic.json: rocprofv3 FETCH_SIZE / WRITE_SIZE of the "
                                               f"same kernel source ({src} sha256 {r['source_sha16']}), "
                                               "not measured in this run")
    return None, f"no PMC summary of {symbol} at this shape in profiles/traffic.json"


def cpu_baseline(seconds: float = 15.0) -> dict:
    """The reference CPU path on a bounded sample: oracle dequant (numpy, row chunks on a thread
    pool) + fp32 torch.matmul over the whole Q4_K and Q6_K gate_up shards at M = 8, passes
    repeated for about `seconds` (at least 3), median pass reported."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    from oracle import ggml_ref as G

    cores = max(1, min(16, os.cpu_count() or 1))
    torch.set_num_threads(cores)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            cpu_model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    pool = ThreadPoolExecutor(cores)
    rng = np.random.default_rng(0)
    K, M = 5120, 8
    x = torch.randn(M, K)

    def deq(raw, wt):
        chunks = np.array_split(raw, cores)
        return np.concatenate(list(pool.map(lambda c: G.dequantize(c, wt), chunks)))

    rows = 34816                                              # the whole gate_up shard of each type
    raws = {wt: G.random_blocks(rng, rows, K, wt) for wt in (Q4_K, Q6_K)}
    nbytes = sum(r.nbytes for r in raws.values())

    def one():
        t_deq = t_mm = 0.0
        for wt, raw in raws.items():
            t0 = time.perf_counter()
            w = torch.from_numpy(deq(raw, wt))
            t1 = time.perf_counter()
            y = x @ w.T
            t2 = time.perf_counter()
            assert y.shape == (M, rows)
            t_deq += t1 - t0
            t_mm += t2 - t1
        return t_deq, t_mm

    runs = []
    t_start = time.perf_counter()
    while len(runs) < 3 or (time.perf_counter() - t_start < seconds and len(runs) < 50):
        runs.append(one())
    td = statistics.median(r[0] for r in runs)
    tm = statistics.median(r[1] for r in runs)
    pool.shutdown()
    return {"value": round(nbytes / (td + tm) / 1e9, 4), "unit": "GB/s", "cores": cores,
            "kind": "port", "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "cpu_model": cpu_model,
            "sample": f"whole Q4_K + Q6_K gate_up shards (34816 x 5120 each, {nbytes} packed bytes), M={M}: "
                      f"oracle dequant {td * 1e3:.1f} ms + torch fp32 matmul {tm * 1e3:.1f} ms per pass on "
                      f"{cores} threads, median of {len(runs)} passes",
            "dequant_ms": round(td * 1e3, 2), "matmul_ms": round(tm * 1e3, 2)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--m", type=int, default=8, help="batch rows of the decode GEMV (1..32)")
    ap.add_argument("--copies", type=int, default=3, help="rotating weight copies of the step (> 1 GB in total)")
    ap.add_argument("--shard-bytes", type=float, default=320e6,
                    help="per-shard timings rotate at least this many bytes of copies (> the 256 MB Infinity Cache)")
    ap.add_argument("--extra-m", default="16,32",
                    help="also time every shard alone at these batch rows (comma-separated; empty: skip)")
    ap.add_argument("--stack-m", default="1,8,32,64", help="config 5 lines: batch rows (comma-separated)")
    ap.add_argument("--stack-layers", type=int, default=64, help="config 5 lines: decoder layers (0: skip)")
    ap.add_argument("--gemm-m", type=int, default=2048, help="batch rows of the prefill GEMM line (0: skip)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-floor", dest="floor", action="store_false",
                    help="skip the per-shard memory floor (plain streaming read of the same bytes)")
    ap.add_argument("--detail", action="store_true", help="print the per-shard table to stderr")
    ap.add_argument("--only", default="", help="TYPE:SHARD (e.g. Q6_K:gate_up): run that shard alone, "
                    "so a profiler's per-kernel statistics cover exactly one launch shape")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB 3 times (the byte-counter calibration "
                         "for rocprofv3 FETCH_SIZE / WRITE_SIZE runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the GGUF linear path has no collective; "
              "sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import gguf_hip
    from gguf_hip.synth import random_shard

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calib_copy:
        src = torch.ones(args.calib_copy << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    M = args.m
    shards = []                     # (type, name, N, K, [GroupedLayer per copy], bytes)
    only = tuple(args.only.split(":")) if args.only else None
    for wt in (Q4_K, Q6_K):
        for name, N, K in SHAPES:
            if only and (gguf_hip.TYPE_NAMES[wt], name) != only:
                continue
            nbytes = gguf_hip.tiles_bytes(wt, N, K) // ((N + 63) // 64 * 64) * N   # packed GGUF bytes
            gls = []
            for c in range(max(args.copies, math.ceil(args.shard_bytes / nbytes))):
                W = random_shard(N, K, wt, dev, seed=1000 * c + N + wt)
                assert W.numel() == nbytes
                gls.append(gguf_hip.pack_layer([W], [N], [wt]))
                del W
            shards.append((wt, name, N, K, gls, nbytes))
    torch.cuda.empty_cache()
    xs = {K: torch.randn(M, K, device=dev).to(torch.bfloat16) for K in {s[3] for s in shards}}
    step_bytes = sum(s[5] for s in shards)

    # one graph per copy: every shard once (one step)
    def step_fn(c):
        def f():
            for wt, name, N, K, gls, nb in shards:
                gguf_hip.mul_mat_grouped(xs[K], gls[c % len(gls)])
        return f

    graphs = [_capture(step_fn(c), torch) for c in range(args.copies)]
    for i in range(args.warmup):
        graphs[i % args.copies].replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    s.record()
    for i in range(args.steps):
        graphs[i % args.copies].replay()
    e.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = s.elapsed_time(e) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # per-shard launch time (graph of every copy, > 256 MB of them, twice; average per launch)
    def shard_us(gls, x):
        reps = max(1, 8 // len(gls))

        def f():
            for _ in range(reps):
                for gl in gls:
                    gguf_hip.mul_mat_grouped(x, gl)
        g = _capture(f, torch)
        g.replay()
        t = statistics.median(_time_graph(g, 5, torch) for _ in range(5)) / (reps * len(gls))
        del g
        return t * 1e3

    # the shard's memory floor: a plain streaming read of the same packed bytes on the shard's own
    # grid (gqk_read_floor), timed the same way (the same rotating copies, graph replays, events)
    def floor_us(gls, grid, waves):
        sink = torch.empty(grid * waves, dtype=torch.int32, device=dev)
        reps = max(1, 8 // len(gls))

        def f():
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for _ in range(reps):
                for gl in gls:
                    gguf_hip._lib.check(gguf_hip._lib.lib.gqk_read_floor(
                        gl.packed.data_ptr(), gl.packed.numel() // 1024 * 1024, grid, waves, sink.data_ptr(), st),
                        "bench floor")
        g = _capture(f, torch)
        g.replay()
        t = statistics.median(_time_graph(g, 5, torch) for _ in range(5)) / (reps * len(gls))
        del g
        return t * 1e3

    def plan_of(gl, m):
        return gguf_hip.ops.GqkPlanInfo.from_tuple(
            gl.plans[gguf_hip.ops._pick_plan(gl.plans, m) * gguf_hip.ops._NPLAN:][:gguf_hip.ops._NPLAN])

    rows = []
    for wt, name, N, K, gls, nb in shards:
        us = shard_us(gls, xs[K])
        info = plan_of(gls[0], M)
        fl = floor_us(gls, info.n_desc, info.nw) if args.floor else None
        rows.append({"type": gguf_hip.TYPE_NAMES[wt], "shard": name, "N": N, "K": K, "us": round(us, 2),
                     "copies": len(gls),
                     "GBps": round(nb / (us * 1e-6) / 1e9, 1), "g": info.g, "split": info.split, "wgs": info.n_desc,
                     "waves_per_wg": info.nw, "one_record": info.bm == 1, "form": _form(info),
                     "floor_us": round(fl, 2) if fl else None})
    # the rest of the metric's range (M = 9..32: speculative rows of several streams)
    extra = []
    for Me in [int(v) for v in args.extra_m.split(",") if v]:
        xe = {K: torch.randn(Me, K, device=dev).to(torch.bfloat16) for K in xs}
        for wt, name, N, K, gls, nb in shards:
            us = shard_us(gls, xe[K])
            info = plan_of(gls[0], Me)
            gbs = nb / (us * 1e-6) / 1e9
            extra.append({"M": Me, "type": gguf_hip.TYPE_NAMES[wt], "shard": name, "N": N, "K": K, "us": round(us, 2),
                          "form": _form(info), "GBps": round(gbs, 1),
                          "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
        del xe
    dom = max(rows, key=lambda r: r["us"])
    dom_wt = next(s[0] for s in shards if gguf_hip.TYPE_NAMES[s[0]] == dom["type"] and s[1] == dom["shard"])
    dom_w = next(s[5] for s in shards if gguf_hip.TYPE_NAMES[s[0]] == dom["type"] and s[1] == dom["shard"])
    # algorithmic bytes of one launch: packed weights + x (bf16) read once + y (bf16) written once
    dom_bytes = dom_w + 2 * M * dom["K"] + 2 * M * dom["N"]
    achieved = dom_bytes / (dom["us"] * 1e-6) / 1e9
    # the kernel's template arguments: token groups, type, and whether it is the build without the
    # register pipeline (plans whose waves all stream one record)
    dom_symbol = f"gqk::gemv_kernel<{dom['g']}, {dom_wt}, {'true' if dom['one_record'] else 'false'}>"
    traffic, traffic_source = _traffic(dom_symbol, dom, M)
    if args.detail:
        for r in rows:
            print(json.dumps(r), file=sys.stderr)

    gemm = None
    if args.gemm_m:
        del graphs
        Mg = args.gemm_m
        wt, name, N, K, gls, nb = next((s for s in shards if s[0] == Q4_K and s[1] == "gate_up"), shards[0])
        xg = torch.randn(Mg, K, device=dev).to(torch.bfloat16)

        def fg():
            for gl in gls:
                gguf_hip.mul_mat_grouped(xg, gl)
        g = _capture(fg, torch)
        g.replay()
        t = statistics.median(_time_graph(g, 3, torch) for _ in range(3)) / len(gls)
        tflops = 2.0 * Mg * N * K / (t * 1e-3) / 1e12
        gemm = {"type": gguf_hip.TYPE_NAMES[wt], "shard": name, "N": N, "K": K, "M": Mg, "ms": round(t, 4),
                "TFLOPs": round(tflops, 1), "frac": round(tflops / BF16_PEAK_TFLOPS, 4)}

    stack = None
    if args.stack_layers > 0 and not only:
        # the mixed-type stack, the north star's "M=1..8 mixed-type GEMV"
        from bench_configs import build_stack, time_stack
        del shards, xs
        torch.cuda.empty_cache()
        grouped, per_linear, stack_bytes, _ = build_stack(torch, gguf_hip, random_shard, dev, args.stack_layers)
        stack = {"workload": f"BASELINE config 5: {args.stack_layers} decoder layers (seeded type draw over the eleven "
                             "types weighted toward Q4_K / Q5_K / IQ4_XS), the weight stream of one decode step",
                 "packed_bytes": stack_bytes,
                 "bpw": round(8 * stack_bytes / (args.stack_layers * sum(N * K for _, N, K in SHAPES)), 3),
                 "schedules": {
                     "per_linear": "the reference's schedule: one grouped launch per linear module (qkv, o_proj, "
                                   "gate_up, down: 4 per decoder layer, as the plugin's _create_groups groups "
                                   "each module's shards), each on its own input",
                     "grouped": "one mixed-type launch per layer over qkv + o_proj + gate_up (K = 5120) plus one "
                                "for down, on a single x: a weight-stream bound that a decoder cannot issue "
                                "(o_proj reads the attention output and gate_up the post-attention norm)"},
                 "lines": []}
        for Ms in [int(v) for v in args.stack_m.split(",") if v]:
            for sched, lst in (("per_linear", per_linear), ("grouped", grouped)):
                t = time_stack(torch, gguf_hip, dev, lst, Ms)
                gbs = stack_bytes / (t * 1e-3) / 1e9
                stack["lines"].append({"schedule": sched, "M": Ms, "launches_per_step": len(lst),
                                       "ms_per_step": round(t, 4), "GBps": round(gbs, 1),
                                       "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                                    "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}})
        del grouped, per_linear

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic: random valid GGUF blocks generated on the GPU",
        "config": {"workload": f"BASELINE config 2: Q4_K + Q6_K decode GEMV, M={M}, shapes "
                               "qkv 7168x5120, o_proj 5120x5120, gate_up 34816x5120, down 5120x17408",
                   "M": M, "copies": args.copies, "bytes_per_step": step_bytes,
                   "hbm_frac": round(value / HBM_PEAK_GBS, 4), "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_source,
                     "kernel": f"{dom['type']} {dom['shard']} {dom['N']}x{dom['K']} M={M}", "symbol": dom_symbol,
                     "launch_us": dom["us"], "bytes_per_launch": dom_bytes},
        "shards": rows,
        "memory_floor": None if not args.floor else {
            "what": "gqk_read_floor: a plain streaming read of each shard's packed bytes on the shard's own grid "
                    "(same rotating copies, graph replays and events as the shard lines); the sum over the "
                    "step's shards against the sum of their launch times",
            "floor_us": round(sum(r["floor_us"] for r in rows), 2),
            "launch_us": round(sum(r["us"] for r in rows), 2),
            "floor_GBps": round(step_bytes / (sum(r["floor_us"] for r in rows) * 1e-6) / 1e9, 1),
            "frac_of_floor": round(sum(r["floor_us"] for r in rows) / sum(r["us"] for r in rows), 4)},
        "shards_extra_m": extra,
        "gemm": gemm,
        "stack": stack,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
