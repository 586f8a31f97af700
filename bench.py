#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric): Q4_K decode GEMV at 4096x12288 (Qwen3-8B down_proj,
x f32 [1x12288]) in GB/s of algorithmic bytes (quantized weight + x + y), with the
weights rotated over enough distinct copies (>= 512 MB) that every launch streams
them from HBM, not from the 256 MB Infinity Cache.  A "step" is one GEMV over one
weight copy.  Launches are captured in a HIP graph (the decode loop's production
form) and timed with HIP events on the launch stream.

Also reported (fields of the same JSON line): the other BASELINE configs where
implemented, the roofline fraction of the headline kernel and a CPU baseline (the
oracle's restatement of QLinear::forward, full dequant + f32 GEMV, 1 thread) on a
bounded sample.

Usage: python bench.py [--gpus 1] [--steps 2000] [--warmup 200]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2516.6
METRIC = "Q4_K GEMV GB/s (% HBM peak) at 4096x12288; prefill TFLOP/s at M=512"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_copies(fmt_bytes, qt, n, k, min_bytes):
    import nn_amd
    per = len(fmt_bytes)
    copies = max(2, -(-min_bytes // per))
    ws = [nn_amd.QuantizedWeight.from_quantized(fmt_bytes, qt, (n, k)) for _ in range(copies)]
    return ws


def time_graph(fn_list, steps, warmup):
    """Capture fn_list (one launch each) into a graph, replay until `steps` launches
    ran, return seconds per launch measured with events on the current stream."""
    import torch
    for i in range(warmup):
        fn_list[i % len(fn_list)]()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for fn in fn_list:
                fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    reps = max(1, steps // len(fn_list))
    g.replay()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(reps):
        g.replay()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) / 1e3 / (reps * len(fn_list)), reps * len(fn_list)


def bench_q4k_gemv(steps, warmup):
    import torch

    import nn_amd
    n, k = 4096, 12288
    w = nn_amd.synth_normal(2, 1, (n, k), 0.02)
    wb = nn_amd.quantize_q4_k(w)
    copies = make_copies(wb, nn_amd.QuantType.Q4_K, n, k, 512 << 20)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(2, 2, (1, k), 1.0)).to(dev)
    ys = [torch.empty((1, n), device=dev) for _ in copies]
    from nn_amd import _lib
    import ctypes
    L = _lib.load()

    def launcher(wi, yi):
        def f():
            st = torch.cuda.current_stream().cuda_stream
            rc = L.nnq_linear(wi.handle, ctypes.c_void_p(x.data_ptr()), 0, 1, k, None, 0,
                              ctypes.c_void_p(yi.data_ptr()), 0, ctypes.c_void_p(st))
            assert rc == 0, _lib.last_error()
        return f

    fns = [launcher(c, y) for c, y in zip(copies, ys)]
    sec, nsteps = time_graph(fns, steps, warmup)
    algo = len(wb) + k * 4 + n * 4
    # cache-resident (single copy) figure, labelled as such
    sec1, _ = time_graph(fns[:1] * 20, max(200, steps // 10), 10)
    return dict(sec=sec, steps=nsteps, algo_bytes=algo, copies=len(copies), sec_single=sec1, wbytes=wb, x=x,
                n=n, k=k)


def bench_q4k_gemm(m, n, k, steps, warmup, min_bytes=256 << 20):
    """Prefill GEMM: X [m, k] bf16 (N(0,1)) x Q4_K W [n, k]^T -> Y [m, n] bf16, f32 accumulate.
    A call is the activation staging kernel plus the GEMM kernel."""
    import torch

    import nn_amd
    w = nn_amd.synth_normal(4, k, (n, k), 0.02)
    wb = nn_amd.quantize_q4_k(w)
    copies = make_copies(wb, nn_amd.QuantType.Q4_K, n, k, min_bytes)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(4, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    ys = [torch.empty((m, n), device=dev, dtype=torch.bfloat16) for _ in copies]
    from nn_amd import _lib
    import ctypes
    L = _lib.load()

    def launcher(wi, yi):
        def f():
            st = torch.cuda.current_stream().cuda_stream
            rc = L.nnq_linear(wi.handle, ctypes.c_void_p(x.data_ptr()), 2, m, k, None, 0,
                              ctypes.c_void_p(yi.data_ptr()), 2, ctypes.c_void_p(st))
            assert rc == 0, _lib.last_error()
        return f

    fns = [launcher(c, y) for c, y in zip(copies, ys)]
    sec, nsteps = time_graph(fns, steps, warmup)
    flops = 2.0 * m * n * k
    return dict(sec=sec, steps=nsteps, tflops=flops / sec / 1e12, m=m, n=n, k=k, copies=len(copies))


def cpu_baseline_q4k(wb, xnp, n, k, budget_s=10.0):
    from oracle import oracle as O
    t0 = time.perf_counter()
    calls = 0
    while True:
        O.q4k_linear(xnp, wb, n)
        calls += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = (time.perf_counter() - t0) / calls
    return dt, calls


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the quantized-linear kernels run on one device's share "
              "(multi-GPU sharding is design-only, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch

    import nn_amd
    nn_amd.init(0)
    log("bench: Q4_K GEMV 4096x12288 (rotating copies)")
    r = bench_q4k_gemv(args.steps, args.warmup)
    gbs = r["algo_bytes"] / r["sec"] / 1e9
    gbs1 = r["algo_bytes"] / r["sec_single"] / 1e9
    log(f"  {r['sec'] * 1e6:.2f} us/step  {gbs:.1f} GB/s  (cache-resident single copy: {gbs1:.1f} GB/s)")

    prefill = {}
    if not args.no_prefill:
        for (m, n, k) in [(512, 12288, 4096), (512, 4096, 12288)]:
            log(f"bench: Q4_K prefill GEMM M={m} N={n} K={k} (bf16 in/out)")
            g = bench_q4k_gemm(m, n, k, max(50, args.steps // 10), 20)
            log(f"  {g['sec'] * 1e6:.2f} us/call  {g['tflops']:.1f} TFLOP/s "
                f"({100 * g['tflops'] / FP16_PEAK_TFLOPS:.1f}% of fp16 dense peak)")
            prefill[f"{m}x{n}x{k}"] = {"us_per_call": round(g["sec"] * 1e6, 3), "tflops": round(g["tflops"], 2),
                                       "frac_fp16_peak": round(g["tflops"] / FP16_PEAK_TFLOPS, 4),
                                       "tokens_per_s": round(m / g["sec"], 1)}

    cpu = None
    if not args.no_cpu:
        log("bench: CPU baseline (oracle QLinear::forward restatement, 1 thread)")
        xnp = r["x"].cpu().numpy()
        dt, calls = cpu_baseline_q4k(r["wbytes"], xnp, r["n"], r["k"], args.cpu_budget)
        cpu = {"value": round(r["algo_bytes"] / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{calls} full Q4_K 4096x12288 GEMV calls (dequant whole matrix + f32 x@W^T, "
                         f"as QLinear::forward), {dt:.3f} s/call"}
        log(f"  cpu {cpu['value']} GB/s")

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(r["sec"] * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, f32 activations, f32 accumulate",
        "data": "synthetic (seeded splitmix64 N(0,0.02) weights quantized by BlockQ4K::quantize, N(0,1) x)",
        "config": {"workload": "Q4_K decode GEMV 4096x12288 (Qwen3-8B down_proj), x f32 [1x12288], y f32",
                   "n": r["n"], "k": r["k"], "weight_copies": r["copies"],
                   "algorithmic_bytes_per_step": r["algo_bytes"], "timing": "HIP graph of launches, HIP events",
                   "cache_resident_single_copy_GBps": round(gbs1, 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
        "prefill_q4k_gemm": prefill or None,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
