"""Benchmark of the MI355X attention hot path (decode + causal prefill), one JSON line.

A step is one decode-attention pass over all 28 layers of a Llama-3.2-3B-shaped f16 KV cache
at KV length 4096 (K,V ~ N(0,1)*0.5): 28 launches, each reading a
different layer slice, as the reference's `abench` iterates every layer
(src/metal_backend.mm:613-615; GB/s formula src/main.cpp:446-447). The 28 slices (470 MB)
exceed the 256 MB last-level cache, so the reads come from HBM. `value` is decode-attention
HBM GB/s over the timed steps (whole-job throughput: 28 x 16.8 MB per step / step time).

The steps are captured once into a HIP graph (28 launches through the C ABI on torch's current
stream) and replayed; HIP events on that stream bracket the timed region. `roofline.achieved`
divides the algorithmic bytes of one launch by the average launch duration over that timed
region (28 x steps launches back to back); the rocprofv3 kernel-trace summary of
`python bench.py --only c3 --no-cpu` (profiles/attn_decode_C3_kernel_trace.md) gives the same
kernel's average duration. `roofline.traffic` is the HBM bytes per launch measured with
rocprofv3 FETCH_SIZE / WRITE_SIZE on that kernel, calibrated on a copy kernel of known size
(`python bench.py --only copy-probe`, profiles/attn_decode_C3_traffic.md); the line names the
profile and kernel it came from (`traffic_source`).

The same line carries the prefill figures (C4, C5-prefill, C2: TFLOPS and fractions of the
f16-MFMA and HBM peaks), the decode sweep (C1, C5 lengths), the fused RoPE + KV-cache store
that precedes attention (GB/s for a 512-token chunk and one decode token), the attention output
projection wo with its residual add (GB/s for one token, TFLOPS for a 512-token chunk, four
GGUF weight types), the whole Llama-3.2-3B forward pass with Q4_0 weights (decode tok/s at
position 128, 512-token prefill tok/s; llama-bench's tg/pp measures) and the CPU baseline
(the oracle, a C++ restatement of Ingot's CPU attention, on the host cores).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import statistics
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "inference-agent_amd"))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, 8 TB/s
# HBM bytes per C3 decode launch: (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0) KiB from rocprofv3, the
# factors from the copy probe (profiles/attn_decode_C3_traffic.md).
C3_TRAFFIC_BYTES = int((8461.0 * 2.0 + 444.75) * 1024)
C3_TRAFFIC_SOURCE = ("profiles/attn_decode_C3_traffic.md: rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0 "
                     "of attn_decode_kernel<3,4,false,false> (inference-agent_amd/csrc/attn_decode.hip)")
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense f16 MFMA, 2.5 PFLOP/s
WARMUP_SECONDS = 0.3
METRIC = "decode-attn HBM GB/s + prefill-attn TFLOPS, Llama-3.2-3B GQA, 1 MI355X"

# name -> (kind, n_keys, pos, n_tok, kv_scale, seed)
DECODE = {"c3": ("C3-decode-4096", 4096, 0.5, 3), "c1": ("C1-decode-512", 512, 1.0, 1),
          "c5d1k": ("C5-decode-1024", 1024, 1.0, 50), "c5d2k": ("C5-decode-2048", 2048, 1.0, 51),
          "c5d8k": ("C5-decode-8192", 8192, 1.0, 53)}
PREFILL = {"c4": "C4-prefill-512@3584", "c5p": "C5-prefill-2048@6144", "c2": "C2-prefill-512@0"}
# name -> (weight type, n_tok): the attention output projection wo (3072 x 3072) with the residual
# add, for one decode token and a 512-token prefill chunk
LINEAR = {"wo1-f16": ("F16", 1), "wo1-q8": ("Q8_0", 1), "wo1-q4": ("Q4_0", 1), "wo1-q6k": ("Q6_K", 1),
          "wo512-f16": ("F16", 512), "wo512-q8": ("Q8_0", 512), "wo512-q4": ("Q4_0", 512),
          "wo512-q6k": ("Q6_K", 512)}
# name -> weight type: the whole Llama-3.2-3B forward pass (28 layers, tied embeddings) with
# random-byte weights, one decode token at position 128 and a 512-token prefill chunk at 0
MODEL = {"model-q4": "Q4_0"}
MODEL_PHASES = {"model-q4": (("decode", 1, 128), ("prefill", 512, 0)),
                "model-q4-decode": (("decode", 1, 128),), "model-q4-prefill": (("prefill", 512, 0),)}
# name -> (pos, n_tok): the KV-store step before attention, for a prefill chunk and a decode token
KVSTORE = {"kv512": ("kv-store-512@3584", 3584, 512), "kv1": ("kv-store-1@4095", 4095, 1)}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="all",
                    help="all | decode | prefill | kvstore | linear | model | envelope | probes | copy-probe | one of "
                    + ", ".join(list(DECODE) + list(PREFILL) + list(KVSTORE) + list(LINEAR)))
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
        self.nbytes = W.Workload("d", "decode", n_keys).decode_bytes()

    def launch(self, layer):
        self.ia.attn_decode(self.q, self.k, self.v, self.out, self.descs[layer], workspace=self.ws)

    def step(self):
        for l in range(self.n_layer):
            self.launch(l)


class PrefillBench:
    """28-layer f16 cache at n_ctx = pos + n_tok; one prefill call per layer per step (the
    layers' K/V differ, q and out are reused)."""

    def __init__(self, torch, ia, W, w, seed, n_layer=28):
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        kv = W.KV_DIM
        self.w, self.n_layer = w, n_layer
        self.k = torch.randn(n_layer * w.n_keys, kv, generator=g, device=dev).half()
        self.v = torch.randn(n_layer * w.n_keys, kv, generator=g, device=dev).half()
        self.q = torch.randn(w.n_tok, W.N_HEAD * W.HEAD_DIM, generator=g, device=dev)
        self.out = torch.empty_like(self.q)
        self.descs = [ia.prefill_desc(W.N_HEAD, W.N_HEAD_KV, W.HEAD_DIM, w.pos, w.n_tok,
                                      kv_offset=l * w.n_keys * kv) for l in range(n_layer)]
        self.ws = ia.Workspace(dev)
        self.ia = ia
        self.splits = ia.prefill_splits(self.descs[0])

    def step(self):
        for d in self.descs:
            self.ia.attn_prefill(self.q, self.k, self.v, self.out, d, workspace=self.ws)


class KvStoreBench:
    """ingot_rope_kv_store on n_tok tokens at `pos` for each of 28 layers per step (q rotated in
    place, K/V into the layer's slice of a 28-layer cache); algorithmic bytes per token: q read
    and written (f32), k and v read (f32), K and V written (f16) = 36,864 B for 24 Q / 8 KV
    heads."""

    def __init__(self, torch, ia, W, pos, n_tok, seed, n_layer=28):
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        kv = W.KV_DIM
        n_ctx = pos + n_tok
        self.n_layer = n_layer
        self.q = torch.randn(n_tok, W.N_HEAD * W.HEAD_DIM, generator=g, device=dev)
        self.k = torch.randn(n_tok, kv, generator=g, device=dev)
        self.v = torch.randn(n_tok, kv, generator=g, device=dev)
        self.kc = torch.zeros(n_layer * n_ctx, kv, dtype=torch.float16, device=dev)
        self.vc = torch.zeros_like(self.kc)
        i = torch.arange(W.HEAD_DIM // 2, device=dev, dtype=torch.float32)
        self.inv = torch.pow(torch.tensor(500000.0, device=dev), -2.0 * i / W.HEAD_DIM)
        self.descs = [ia.rope_kv_desc(W.N_HEAD, W.N_HEAD_KV, W.HEAD_DIM, pos, n_tok,
                                      dst_offset=(l * n_ctx + pos) * kv) for l in range(n_layer)]
        self.ia = ia
        self.nbytes = n_tok * (2 * 4 * W.N_HEAD * W.HEAD_DIM + 2 * 4 * kv + 2 * 2 * kv)

    def step(self):
        for d in self.descs:
            self.ia.rope_kv_store(self.q, self.k, self.v, self.kc, self.vc, self.inv, d)


class LinearBench:
    """ingot_linear for wo (n_in = n_out = 3072) with accumulate, one call per weight copy per
    step. The weight bytes are replicated into enough copies (>= 28, >= 1 GiB together) that
    the reads come from HBM rather than the 256 MB last-level cache. Algorithmic bytes per call:
    the weights, x (f32) and out read and written (f32); flops: 2 * n_tok * n_in * n_out."""

    def __init__(self, torch, ia, gb, t, n_tok, seed, n_in=3072, n_out=3072):
        dev = torch.device("cuda:0")
        raw = gb.random_weights(t, n_out, n_in, seed=seed).reshape(-1)
        wb = raw.size
        pitch = (wb + 255) // 256 * 256
        self.n_copies = max(28, -(-(1 << 30) // pitch))
        one = torch.from_numpy(raw).to(dev)
        self.w = torch.empty(self.n_copies, pitch, dtype=torch.uint8, device=dev)
        self.w[:, :wb] = one
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.x = torch.randn(n_tok, n_in, generator=g, device=dev)
        self.out = torch.randn(n_tok, n_out, generator=g, device=dev)
        self.desc = ia.linear_desc(t, n_in, n_out, n_tok, accumulate=True)
        self.ia = ia
        self.nbytes = wb + 4 * n_tok * (n_in + 2 * n_out)
        self.flops = 2 * n_tok * n_in * n_out

    def step(self):
        for i in range(self.n_copies):
            self.ia.linear(self.w[i], self.x, self.out, self.desc)


class ModelBench:
    """ingot_forward.HipForward (every step a libingot_attn.so call) over a full-size synthetic
    Llama-3.2-3B; a step is one forward_batch (n tokens at `pos`), tokens already on the device."""

    def __init__(self, torch, t, n_tok, pos, n_ctx=1024):
        import llama_synth as ls
        from ingot_forward import HipForward

        self.model = ls.make_bench_model(ls.LLAMA32_3B, t, seed=5)
        self.weight_bytes = ls.weight_bytes(self.model)
        self.fw = HipForward(self.model, n_ctx=n_ctx, n_batch=max(n_tok, 1))
        self.n_tok, self.pos = n_tok, pos
        self.toks = list(range(1, n_tok + 1))
        self.dev_toks = torch.tensor(self.toks, dtype=torch.int32, device=self.fw.dev)

    def step(self):
        self.fw.forward_batch(self.toks, self.pos, tokens_on_device=self.dev_toks)


def time_steps(torch, fn, steps, warmup, use_graph):
    """Seconds per step over `steps` timed steps (after `warmup`), graph-replayed by default."""
    stream = torch.cuda.current_stream()
    run = fn
    if use_graph:
        fn()  # allocate workspaces outside capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        run = graph.replay
    # Warm up for at least `warmup` replays and at least WARMUP_SECONDS of GPU work: the first
    # tenths of a second after a burst starts run measurably slower (clock ramp, first-touch
    # translation misses), by up to 15% for the longest prefill.
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < WARMUP_SECONDS:
        for _ in range(max(1, warmup)):
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
    """The CPU oracle (C++ restatement of src/cpu_backend.cpp:51-69) on the host cores: the
    median of the per-call times over `seconds` of calls on every thread used, and the median of
    5 calls on one thread."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_lib

    threads = max(1, min(24, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)), os.cpu_count() or 1))
    try:
        import psutil

        physical, logical = psutil.cpu_count(logical=False), psutil.cpu_count()
    except ImportError:
        physical, logical = None, os.cpu_count()
    w = W.C3
    q, kb, vb = W.make_inputs(w)

    def call(nt):
        t = time.perf_counter()
        oracle_lib.attn_decode(q, kb, vb, W.N_HEAD, W.N_HEAD_KV, W.HEAD_DIM, w.n_keys, threads=nt)
        return time.perf_counter() - t

    call(threads)
    times, t0 = [], time.perf_counter()
    while time.perf_counter() - t0 < seconds or len(times) < 5:
        times.append(call(threads))
    dt = statistics.median(times)
    dt1 = statistics.median([call(1) for _ in range(5)])
    gbs = lambda t: round(w.decode_bytes() / t / 1e9, 3)
    return {"value": gbs(dt), "unit": "GB/s", "cores": threads, "kind": "port",
            "host": {"threads_used": threads, "physical_cores": physical, "logical_cpus": logical,
                     "note": "threads = the box's CPU share for this job (OMP_NUM_THREADS), on a host "
                             "with the physical cores listed"},
            "single_thread": {"value": gbs(dt1), "ms_per_call": round(dt1 * 1e3, 2)},
            "sample": f"median of {len(times)} oracle decode calls at KV 4096 (C3 shape, one layer slice), "
                      f"{dt * 1e3:.2f} ms/call, {threads} threads over the 24 heads; one thread: median of "
                      f"5 calls, {dt1 * 1e3:.1f} ms/call"}


# Shapes outside the Llama-3.2-3B headline (the a10 envelope and other group sizes), one size
# each: (name, n_head, n_head_kv, head_dim, n_keys) for decode, (..., pos, n_tok) for prefill.
ENVELOPE_DECODE = (("decode-64/8-hd128-4096", 64, 8, 128, 4096),
                   ("decode-32/8-hd64-4096", 32, 8, 64, 4096),
                   ("decode-16/8-hd256-4096", 16, 8, 256, 4096),
                   ("decode-24/8-hd96-4096", 24, 8, 96, 4096))  # the fallback kernel (attn_naive.hip)
ENVELOPE_PREFILL = (("prefill-32/8-hd128-512@3584", 32, 8, 128, 3584, 512),
                    ("prefill-32/8-hd64-512@3584", 32, 8, 64, 3584, 512),
                    ("prefill-16/8-hd256-512@3584", 16, 8, 256, 3584, 512),
                    ("prefill-24/8-hd96-128@0", 24, 8, 96, 0, 128))  # the fallback kernel


def envelope(torch, ia, steps, warmup, use_graph):
    """Decode and prefill at other head sizes and group sizes: 16 rotated layer slices of a
    random f16 cache (K/V from HBM), per-call time, algorithmic bytes or FLOPs."""
    dev = torch.device("cuda:0")
    ws = ia.Workspace(dev)
    n_layer = 16
    out = {}
    for name, nh, nkv, hd, L in ENVELOPE_DECODE:
        kvd = nkv * hd
        k = torch.randn(n_layer * L, kvd, device=dev).half()
        v = torch.randn_like(k)
        q = torch.randn(nh * hd, device=dev)
        o = torch.empty_like(q)
        ds = [ia.decode_desc(nh, nkv, hd, L, kv_offset=i * L * kvd) for i in range(n_layer)]
        sps = time_steps(torch, lambda: [ia.attn_decode(q, k, v, o, d, workspace=ws) for d in ds],
                         steps, warmup, use_graph) / n_layer
        nbytes = 2 * L * kvd * 2 + 2 * nh * hd * 4
        out[name] = {"us_per_call": round(sps * 1e6, 3), "GB/s": round(nbytes / sps / 1e9, 1),
                     "hbm_frac": round(nbytes / sps / 1e9 / HBM_PEAK_GBS, 4)}
        del k, v
        torch.cuda.empty_cache()
    for name, nh, nkv, hd, pos, nt in ENVELOPE_PREFILL:
        kvd, nk = nkv * hd, pos + nt
        k = torch.randn(n_layer * nk, kvd, device=dev).half()
        v = torch.randn_like(k)
        q = torch.randn(nt, nh * hd, device=dev)
        o = torch.empty_like(q)
        ds = [ia.prefill_desc(nh, nkv, hd, pos, nt, kv_offset=i * nk * kvd) for i in range(n_layer)]
        sps = time_steps(torch, lambda: [ia.attn_prefill(q, k, v, o, d, workspace=ws) for d in ds],
                         max(5, steps // 5), warmup, use_graph) / n_layer
        flops = 4 * hd * nh * (nt * pos + nt * (nt + 1) // 2)
        out[name] = {"us_per_call": round(sps * 1e6, 2), "TFLOPS": round(flops / sps / 1e12, 1),
                     "mfma_frac": round(flops / sps / 1e12 / MFMA_F16_PEAK_TFS, 4)}
        del k, v
        torch.cuda.empty_cache()
    return out


def probes(torch, W):
    """Achievable peaks on this box, measured the same way as the kernels: a plain streaming
    read of the C3 decode bytes (1024 workgroups, 28 rotated copies so the data comes from HBM)
    and back-to-back f16 MFMAs with no memory traffic (both MFMA shapes the kernels use)."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "inference-agent_amd", "libingot_probe.so"))
    lib.ingot_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    lib.ingot_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    sink = torch.zeros(1 << 16, device=dev)
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    n = W.C3.decode_bytes() // 256 * 256
    buf = torch.ones(28, n // 4, device=dev)
    rd = time_steps(torch, lambda: [lib.ingot_probe_read(ctypes.c_void_p(buf[i].data_ptr()), n, 1024,
                                                         ctypes.c_void_p(sink.data_ptr()), stream())
                                    for i in range(28)], 20, 3, True) / 28
    del buf
    out = {"read_C3_bytes": {"us_per_call": round(rd * 1e6, 3), "GB/s": round(n / rd / 1e9, 1),
                             "bytes": n, "frac_of_8TBs": round(n / rd / 8e12, 4)}}
    # The asymptotic rate: one launch reading 33.6 MB (C5-8192's bytes) and one reading 1 GiB.
    for name, nbytes, copies, blocks in (("read_C5_8192_bytes", W.Workload("d", "decode", 8192).decode_bytes(), 14, 2048),
                                         ("read_1GiB", 1 << 30, 2, 8192)):
        nb = nbytes // 256 * 256
        big = torch.ones(copies, nb // 4, device=dev)
        t = time_steps(torch, lambda: [lib.ingot_probe_read(ctypes.c_void_p(big[i].data_ptr()), nb, blocks,
                                                            ctypes.c_void_p(sink.data_ptr()), stream())
                                       for i in range(copies)], 10, 2, True) / copies
        out[name] = {"us_per_call": round(t * 1e6, 2), "GB/s": round(nb / t / 1e9, 1), "bytes": nb,
                     "workgroups": blocks, "frac_of_8TBs": round(nb / t / 8e12, 4)}
        del big
        torch.cuda.empty_cache()
    blocks, iters = 1024, 1000
    for shape, name, mnk in ((0, "mfma_32x32x16_f16", 8 * 32 * 32 * 16), (1, "mfma_16x16x32_f16", 16 * 16 * 16 * 32)):
        t = time_steps(torch, lambda: lib.ingot_probe_mfma(shape, blocks, iters, ctypes.c_void_p(sink.data_ptr()),
                                                           stream()), 10, 2, True)
        flops = blocks * 4 * iters * mnk * 2
        out[name] = {"TFLOPS": round(flops / t / 1e12, 1), "frac_of_2.5PF": round(flops / t / 2.5e15, 4)}
    return out


def copy_probe(torch, mib=64):
    """The plain copy probe (probe_copy) over a buffer of known size, 5 dispatches: the run that
    calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE against bytes actually moved
    (rocprofv3 --pmc FETCH_SIZE -- python3 bench.py --only copy-probe)."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "inference-agent_amd", "libingot_probe.so"))
    lib.ingot_probe_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_void_p]
    n = mib << 20
    src = torch.ones(n // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        rc = lib.ingot_probe_copy(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), n, 2048,
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError("ingot_probe_copy failed")
    torch.cuda.synchronize()
    if not bool((dst == 1).all()):
        raise RuntimeError("copy probe: wrong result")
    return {"copy_probe": {"MiB_per_dispatch": mib, "dispatches": 5}}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the attention hot path runs on one "
              "MI355X; it shards by KV head and is not run across GPUs here). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import ingot_attn as ia
    import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU", file=sys.stderr)
        sys.exit(1)
    ia.load_library()
    use_graph = not args.no_graph
    sel = args.only
    if sel == "copy-probe":
        print(json.dumps({"metric": METRIC, "results": copy_probe(torch)}), flush=True)
        return
    want = lambda key, group: sel in ("all", group, key)
    res = {"decode": {}, "prefill": {}, "kv_store": {}, "linear": {}, "model": {}}

    head = None
    for key, (name, n_keys, kv_scale, seed) in DECODE.items():
        if not want(key, "decode"):
            continue
        b = DecodeBench(torch, ia, W, n_keys, kv_scale, seed)
        steps = args.steps if key == "c3" else max(5, args.steps // 5)
        sps = time_steps(torch, b.step, steps, args.warmup, use_graph)
        us_thru = sps / b.n_layer * 1e6
        gbs = b.nbytes / (us_thru * 1e-6) / 1e9
        res["decode"][name] = {"us_per_call": round(us_thru, 3), "GB/s": round(gbs, 1),
                               "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                               "splits": b.splits, "bytes_per_call": b.nbytes}
        if key == "c3":
            head = (sps, us_thru, b.nbytes, gbs, steps)
        del b
        torch.cuda.empty_cache()

    phead = None
    for key, name in PREFILL.items():
        if not want(key, "prefill"):
            continue
        w = W.BY_NAME[name]
        b = PrefillBench(torch, ia, W, w, w.seed)
        steps = max(5, args.steps // 5)
        sps = time_steps(torch, b.step, steps, args.warmup, use_graph) / b.n_layer
        tfs = w.prefill_flops() / sps / 1e12
        gbs = w.prefill_bytes() / sps / 1e9
        res["prefill"][name] = {"us_per_call": round(sps * 1e6, 2), "TFLOPS": round(tfs, 1),
                                "mfma_frac": round(tfs / MFMA_F16_PEAK_TFS, 4),
                                "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                                "flops_per_call": w.prefill_flops(), "splits": b.splits}
        if phead is None:
            phead = (name, sps, tfs, steps, sps * b.n_layer)
        del b
        torch.cuda.empty_cache()

    for key, (name, pos, n_tok) in KVSTORE.items():
        if not want(key, "kvstore"):
            continue
        b = KvStoreBench(torch, ia, W, pos, n_tok, 7)
        steps = max(5, args.steps // 5)
        sps = time_steps(torch, b.step, steps, args.warmup, use_graph) / b.n_layer
        gbs = b.nbytes / sps / 1e9
        res["kv_store"][name] = {"us_per_call": round(sps * 1e6, 3), "GB/s": round(gbs, 1),
                                 "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": b.nbytes}
        del b
        torch.cuda.empty_cache()

    import gguf_blocks as gb

    for key, (t, n_tok) in LINEAR.items():
        if not want(key, "linear"):
            continue
        b = LinearBench(torch, ia, gb, t, n_tok, 31)
        steps = max(5, args.steps // 5)
        sps = time_steps(torch, b.step, steps, args.warmup, use_graph) / b.n_copies
        gbs = b.nbytes / sps / 1e9
        tfs = b.flops / sps / 1e12
        res["linear"][f"wo-{t}-{n_tok}tok"] = {
            "us_per_call": round(sps * 1e6, 3), "GB/s": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "TFLOPS": round(tfs, 2),
            "mfma_frac": round(tfs / MFMA_F16_PEAK_TFS, 4), "bytes_per_call": b.nbytes,
            "flops_per_call": b.flops}
        del b
        torch.cuda.empty_cache()

    for key, phases in MODEL_PHASES.items():
        if not (sel in ("model", key) or (sel == "all" and key == "model-q4")):
            continue
        t = MODEL[key[:8]]
        entry = {}
        for phase, n_tok, pos in phases:
            b = ModelBench(torch, t, n_tok, pos)
            steps = max(5, args.steps // 5)
            sps = time_steps(torch, b.step, steps, args.warmup, use_graph)
            entry[f"{phase}_ms"] = round(sps * 1e3, 3)
            entry[f"{phase}_tok_s"] = round(n_tok / sps, 1)
            if phase == "decode":
                entry["decode_weight_GB/s"] = round(b.weight_bytes / sps / 1e9, 1)
            entry["weight_bytes"] = b.weight_bytes
            del b
            torch.cuda.empty_cache()
        res["model"][f"Llama-3.2-3B-{t}"] = entry

    if sel in ("all", "envelope"):
        res["envelope"] = envelope(torch, ia, args.steps, args.warmup, use_graph)

    if sel in ("all", "probes"):
        res["probes"] = probes(torch, W)

    cpu = None if args.no_cpu else cpu_baseline(W, args.cpu_seconds)

    if head is None and phead is None:
        print(json.dumps({"metric": METRIC, "results": res}), flush=True)
        return
    if head is not None:
        sps, us_thru, nbytes, gbs, steps = head
        value, unit, ms = gbs, "GB/s", sps * 1e3
        roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                    "traffic": C3_TRAFFIC_BYTES, "traffic_source": C3_TRAFFIC_SOURCE,
                    "kernel": "attn_decode_kernel<3,4,false,false>",
                    "bytes_per_launch": nbytes, "us_per_launch": round(us_thru, 3)}
        workload = ("C3 decode attention, KV 4096, 24 Q / 8 KV heads, hd 128, f16 cache, "
                    "28-layer slice rotation (470 MB)")
    else:
        name, sps, tfs, steps, step_s = phead
        value, unit, ms = tfs, "TFLOPS", step_s * 1e3
        roofline = {"bound": "mfma", "achieved": round(tfs, 1), "peak": MFMA_F16_PEAK_TFS,
                    "unit": "TFLOP/s", "frac": round(tfs / MFMA_F16_PEAK_TFS, 4), "traffic": None,
                    "kernel": "attn_prefill_kernel<3,4>"}
        workload = f"{name} causal prefill, 24 Q / 8 KV heads, hd 128, f16 cache, 28 layers"
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
