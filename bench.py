"""Benchmark of the MI355X attention hot path (decode + causal prefill), one JSON line.

A step is one decode-attention pass over all 28 layers of a Llama-3.2-3B-shaped f16 KV cache
at KV length 4096: 28 launches, each reading a different layer slice,
as the reference's `abench` iterates every layer (src/metal_backend.mm:613-615, GB/s formula
src/main.cpp:446-447). The 28 slices (470 MB) exceed the 256 MB last-level cache, so the reads
come from HBM. `value` is decode-attention HBM GB/s over the timed steps.

The same line carries the prefill figures (C2, C4, C5-prefill: TFLOPS and the f16-MFMA
fraction), the decode sweep (C1, C5 lengths), the roofline of the dominant (decode) kernel and
the CPU baseline (the oracle on the host cores).

Launches go through the C ABI on torch's current stream and are captured once into a HIP graph
per step (28 launches), then replayed; HIP events on that stream bracket the timed region.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "inference-agent_amd"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, 8 TB/s
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense f16 MFMA, 2.5 PFLOP/s
METRIC = "decode-attn HBM GB/s + prefill-attn TFLOPS, Llama-3.2-3B GQA, 1 MI355X"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", choices=["all", "decode", "prefill"], default="all",
                    help="restrict the GPU work (for profiling runs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


class DecodeBench:
    """28-layer f16 cache at n_ctx = n_keys; one call per layer per step."""

    def __init__(self, torch, ia, W, n_keys, kv_scale, seed, n_layer=28):
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        kv = W.KV_DIM
        self.n_layer, self.n_keys = n_layer, n_keys
        self.k = (torch.randn(n_layer * n_keys, kv, generator=g, device=dev) * kv_scale).half()
        self.v = (torch.randn(n_layer * n_keys, kv, generator=g, device=dev) * kv_scale).half()
        self.q = torch.randn(W.N_HEAD * W.HEAD_DIM, generator=g, device=dev)
        self.out = torch.empty_like(self.q)
        self.descs = [ia.decode_desc(W.N_HEAD, W.N_HEAD_KV, W.HEAD_DIM, n_keys, kv_offset=l * n_keys * kv)
                      for l in range(n_layer)]
        self.ws = ia.Workspace(dev)
        self.ia = ia
        self.splits = ia.decode_splits(self.descs[0])

    def step(self):
        for d in self.descs:
            self.ia.attn_decode(self.q, self.k, self.v, self.out, d, workspace=self.ws)


class PrefillBench:
    def __init__(self, torch, ia, W, w, seed):
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        kv = W.KV_DIM
        self.k = torch.randn(w.n_keys, kv, generator=g, device=dev).half()
        self.v = torch.randn(w.n_keys, kv, generator=g, device=dev).half()
        self.q = torch.randn(w.n_tok, W.N_HEAD * W.HEAD_DIM, generator=g, device=dev)
        self.out = torch.empty_like(self.q)
        self.desc = ia.prefill_desc(W.N_HEAD, W.N_HEAD_KV, W.HEAD_DIM, w.pos, w.n_tok)
        self.ws = ia.Workspace(dev)
        self.ia = ia
        self.splits = ia.prefill_splits(self.desc)

    def step(self):
        self.ia.attn_prefill(self.q, self.k, self.v, self.out, self.desc, workspace=self.ws)


def time_steps(torch, fn, steps, warmup, use_graph, calls_per_step):
    """Returns seconds per step over `steps` timed steps (after `warmup`)."""
    stream = torch.cuda.current_stream()
    graph = None
    if use_graph:
        fn()  # allocate workspaces outside capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        run = graph.replay
    else:
        run = fn
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        run()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


def cpu_baseline(W, seconds):
    """The CPU oracle (C++ restatement of src/cpu_backend.cpp:51-69) on the host cores."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_lib

    threads = min(24, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)), os.cpu_count() or 1)
    w = W.C3
    q, kb, vb = W.make_inputs(w)
    oracle_lib.attn_decode(q, kb, vb, W.N_HEAD, W.N_HEAD_KV, W.HEAD_DIM, w.n_keys, threads=threads)
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle_lib.attn_decode(q, kb, vb, W.N_HEAD, W.N_HEAD_KV, W.HEAD_DIM, w.n_keys, threads=threads)
        calls += 1
    dt = (time.perf_counter() - t0) / calls
    return {"value": round(w.decode_bytes() / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{calls} oracle decode calls at KV 4096 (C3, one layer slice), "
                      f"{dt * 1e3:.2f} ms/call, {threads} threads over the 24 heads"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the attention hot path runs on one "
              "MI355X; see DESIGN.md for how it would shard). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import ingot_attn as ia
    import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU", file=sys.stderr)
        sys.exit(1)
    ia.load_library()
    use_graph = not args.no_graph
    res = {}

    # ---- decode: headline (C3, 28-layer rotation) and sweep
    head = None
    if args.only in ("all", "decode"):
        sweep = {}
        for name, n_keys, kv_scale, seed in [("C3-decode-4096", 4096, 0.5, 3),
                                             ("C1-decode-512", 512, 1.0, 1),
                                             ("C5-decode-1024", 1024, 1.0, 50),
                                             ("C5-decode-2048", 2048, 1.0, 51),
                                             ("C5-decode-8192", 8192, 1.0, 53)]:
            b = DecodeBench(torch, ia, W, n_keys, kv_scale, seed)
            steps = args.steps if name.startswith("C3") else max(5, args.steps // 2)
            sps = time_steps(torch, b.step, steps, args.warmup, use_graph, b.n_layer)
            us = sps / b.n_layer * 1e6
            nbytes = W.Workload(name, "decode", n_keys).decode_bytes()
            gbs = nbytes / (us * 1e-6) / 1e9
            sweep[name] = {"us_per_call": round(us, 3), "GB/s": round(gbs, 1),
                           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "splits": b.splits}
            if name.startswith("C3"):
                head = (sps, us, nbytes, gbs, steps)
            del b
            torch.cuda.empty_cache()
        res["decode"] = sweep

    # ---- prefill
    if args.only in ("all", "prefill"):
        pre = {}
        for w in (W.C4, W.C2, W.C5_PREFILL):
            b = PrefillBench(torch, ia, W, w, w.seed)
            steps = max(5, args.steps // 2)
            sps = time_steps(torch, b.step, steps, args.warmup, use_graph, 1)
            tfs = w.prefill_flops() / sps / 1e12
            gbs = w.prefill_bytes() / sps / 1e9
            pre[w.name] = {"us_per_call": round(sps * 1e6, 2), "TFLOPS": round(tfs, 1),
                           "mfma_frac": round(tfs / MFMA_F16_PEAK_TFS, 4),
                           "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                           "splits": b.splits}
            del b
            torch.cuda.empty_cache()
        res["prefill"] = pre

    cpu = None if args.no_cpu else cpu_baseline(W, args.cpu_seconds)

    if head is not None:
        sps, us, nbytes, gbs, steps = head
        value, unit, ms = gbs, "GB/s", sps * 1e3
        roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                    "kernel": "attn_decode_kernel<3>", "bytes_per_launch": nbytes,
                    "us_per_launch": round(us, 3)}
        workload = "C3 decode attention, KV 4096, 24Q/8KV heads, hd 128, 28-layer f16 cache rotation"
    else:
        c4 = res["prefill"]["C4-prefill-512@3584"]
        value, unit, ms, steps = c4["TFLOPS"], "TFLOPS", c4["us_per_call"] / 1e3, max(5, args.steps // 2)
        roofline = {"bound": "mfma", "achieved": c4["TFLOPS"], "peak": MFMA_F16_PEAK_TFS,
                    "unit": "TFLOP/s", "frac": c4["mfma_frac"], "traffic": None,
                    "kernel": "attn_prefill_kernel<3,1>"}
        workload = "C4 causal prefill 512 queries at 3584 over KV 4096"
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": unit, "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": workload, "n_head": 24, "n_head_kv": 8, "head_dim": 128,
                   "n_layer": 28, "graph": use_graph},
        "roofline": roofline, "cpu_baseline": cpu, "results": res,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
