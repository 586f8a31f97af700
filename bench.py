#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric): Q4_K decode GEMV at 4096x12288 (Qwen3-8B down_proj,
x f32 [1x12288]) in GB/s of algorithmic bytes (quantized weight + x + y), with the
weight rotated over enough distinct copies (>= 512 MB) that every launch streams it
from HBM, not from the 256 MB Infinity Cache.  A "step" is one GEMV over one weight
copy.  Launches are captured in a HIP graph and replayed on torch's current stream;
HIP events recorded on that same stream bracket exactly `--steps` launches.

The same JSON line also carries the other BASELINE configs (fields under "configs"):
Q8_0 GEMV 4096x4096, Q4_K gate+up GEMV 24576x4096, the Q6_K LM head 151936x4096
with its fused argmax, the Q4_K prefill GEMMs at M=512 and the GPT-OSS MXFP4 MoE
layer; the roofline of the headline kernel; and a CPU baseline (the oracle's
restatement of QLinear::forward, whole-matrix dequant + f32 GEMV, 1 thread) on a
bounded sample.

Usage: python bench.py [--gpus 1] [--steps 2000] [--warmup 200]
       python bench.py --only-headline ...   (the headline GEMV alone, for profiling)
       python bench.py --copy-calibration    (a 256 MiB device copy, the yardstick for
                                              rocprofv3 FETCH_SIZE / WRITE_SIZE)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 MFMA
METRIC = "Q4_K GEMV GB/s (% HBM peak) at 4096x12288; prefill TFLOP/s at M=512"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gemv_4096x12288_traffic.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def lib():
    from nn_amd import _lib
    return _lib.load()


def vp(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def cur_stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def check(rc):
    if rc != 0:
        from nn_amd import _lib
        raise RuntimeError(f"nnq call failed ({rc}): {_lib.last_error()}")


def make_copies(fmt_bytes, qt, n, k, min_bytes, layout=0):
    import nn_amd
    copies = max(1, -(-min_bytes // len(fmt_bytes)))
    return [nn_amd.QuantizedWeight.from_quantized(fmt_bytes, qt, (n, k), layout=layout) for _ in range(copies)]


def time_graph(fn_list, steps, warmup, min_graph_calls=200):
    """Capture rounds of fn_list (one call each per round, at least `min_graph_calls`
    calls) into one HIP graph, replay it until about `steps` calls ran, and return
    seconds per call from events on the replay stream.  Long graphs keep the
    per-replay launch cost out of the per-call figure, as in a decode loop."""
    import torch
    for i in range(warmup):
        fn_list[i % len(fn_list)]()
    torch.cuda.synchronize()
    rounds = max(1, -(-min_graph_calls // len(fn_list)))
    per_graph = rounds * len(fn_list)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(rounds):
                for fn in fn_list:
                    fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    g.replay()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(reps):
        g.replay()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) / 1e3 / (reps * per_graph), reps * per_graph


# ---------------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------------

def bench_gemv(fmt, n, k, steps, warmup, seed, min_bytes=512 << 20, single=False):
    """Decode GEMV y[1, n] = x[1, k] W^T, x f32 ~ N(0,1), W ~ N(0,0.02) quantized."""
    import torch

    import nn_amd
    qt, layout, quant = {"q4_k": (nn_amd.QuantType.Q4_K, 0, nn_amd.quantize_q4_k),
                         "q8_0": (nn_amd.QuantType.Q8_0, 0, nn_amd.quantize_q8_0)}[fmt]
    wb = quant(nn_amd.synth_normal(seed, 1, (n, k), 0.02))
    copies = make_copies(wb, qt, n, k, min_bytes, layout)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(seed, 2, (1, k), 1.0)).to(dev)
    ys = [torch.empty((1, n), device=dev) for _ in copies]
    L = lib()

    def launcher(wi, yi):
        def f():
            check(L.nnq_linear(wi.handle, vp(x), 0, 1, k, None, 0, vp(yi), 0, cur_stream()))
        return f

    fns = [launcher(c, y) for c, y in zip(copies, ys)]
    sec, nsteps = time_graph(fns, steps, warmup)
    algo = len(wb) + k * 4 + n * 4
    out = dict(sec=sec, steps=nsteps, algo_bytes=algo, copies=len(copies), gbs=algo / sec / 1e9, wbytes=wb, x=x,
               n=n, k=k)
    if single:  # cache-resident figure (one copy replayed), labelled as such
        sec1, _ = time_graph(fns[:1] * 20, max(200, steps // 10), 10)
        out["gbs_single"] = algo / sec1 / 1e9
    return out


def bench_lm_head(steps, warmup, seed=3):
    """Config 3: Q6_K LM head 151936x4096 (nn-gguf layout) with the fused first-index argmax."""
    import torch

    import nn_amd
    n, k = 151936, 4096
    wb = nn_amd.quantize_q6_k(nn_amd.synth_normal(seed, 1, (n, k), 0.02))
    copies = make_copies(wb, nn_amd.QuantType.Q6_K, n, k, 512 << 20, layout=1)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(seed, 2, (k,), 1.0)).to(dev)
    logits = [torch.empty(n, device=dev) for _ in copies]
    idx = torch.empty(len(copies), dtype=torch.int32, device=dev)
    st = torch.zeros(len(copies), dtype=torch.int32, device=dev)
    L = lib()

    def launcher(i):
        def f():
            check(L.nnq_linear_argmax(copies[i].handle, vp(x), k, None, 0, vp(logits[i]),
                                      ctypes.c_void_p(idx.data_ptr() + 4 * i), ctypes.c_void_p(st.data_ptr() + 4 * i),
                                      cur_stream()))
        return f

    sec, nsteps = time_graph([launcher(i) for i in range(len(copies))], steps, warmup)
    # the same LM head followed by sampling (temperature 0.7, top-k 50, top-p 0.9, the
    # SamplingConfig defaults) over the 151936 logits, on the device
    from nn_amd import _lib as NL
    cfg = NL.Sampling(0.7, 50, 1, 0.9, 1.0, 0.0, 12345)

    def sampler(i):
        def f():
            check(L.nnq_linear_sample(copies[i].handle, vp(x), k, None, 0, vp(logits[i]), None, 0, ctypes.byref(cfg),
                                      ctypes.c_void_p(idx.data_ptr() + 4 * i), cur_stream()))
        return f

    sec_s, _ = time_graph([sampler(i) for i in range(len(copies))], steps, warmup)
    algo = len(wb) + k * 4 + n * 4 + 4
    return dict(sec=sec, steps=nsteps, gbs=algo / sec / 1e9, algo_bytes=algo, copies=len(copies), sec_sample=sec_s)


def bench_gemm(m, n, k, steps, warmup, min_bytes=256 << 20):
    """Config 4: X [m, k] bf16 ~ N(0,1) times Q4_K W [n, k]^T -> Y [m, n] bf16, f32 accumulate.
    A call is the activation-staging kernel plus the GEMM kernel."""
    import torch

    import nn_amd
    wb = nn_amd.quantize_q4_k(nn_amd.synth_normal(4, k, (n, k), 0.02))
    copies = make_copies(wb, nn_amd.QuantType.Q4_K, n, k, min_bytes)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(4, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    ys = [torch.empty((m, n), device=dev, dtype=torch.bfloat16) for _ in copies]
    L = lib()

    def launcher(wi, yi):
        def f():
            check(L.nnq_linear(wi.handle, vp(x), 2, m, k, None, 0, vp(yi), 2, cur_stream()))
        return f

    sec, nsteps = time_graph([launcher(c, y) for c, y in zip(copies, ys)], steps, warmup, min_graph_calls=20)
    flops = 2.0 * m * n * k
    return dict(sec=sec, steps=nsteps, tflops=flops / sec / 1e12, copies=len(copies))


def bench_mlp(steps, warmup, m=1, seed=8, min_bytes=512 << 20):
    """Qwen3-8B SwiGLU MLP decode (hidden 4096, intermediate 12288, Q4_K gate / up /
    down, bf16 x [m, 4096] -> f32 y): nnq_mlp_forward, rotating copies of the layer."""
    import torch

    import nn_amd
    H, I = 4096, 12288
    bg = nn_amd.quantize_q4_k(nn_amd.synth_normal(seed, 1, (I, H), 0.02))
    bu = nn_amd.quantize_q4_k(nn_amd.synth_normal(seed, 2, (I, H), 0.02))
    bd = nn_amd.quantize_q4_k(nn_amd.synth_normal(seed, 3, (H, I), 0.02))
    per = len(bg) + len(bu) + len(bd)
    copies = [nn_amd.QuantizedMLP(bg, bu, bd, nn_amd.QuantType.Q4_K, H, I) for _ in range(max(1, -(-min_bytes // per)))]
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(seed, 4, (m, H), 1.0)).to(dev).to(torch.bfloat16)
    ys = [torch.empty((m, H), device=dev) for _ in copies]
    st = torch.zeros(1, dtype=torch.int32, device=dev)
    L = lib()

    def launcher(c, y):
        def f():
            check(L.nnq_mlp_forward(c._h, vp(x), 2, m, H, vp(y), 0, vp(st), cur_stream()))
        return f

    sec, nsteps = time_graph([launcher(c, y) for c, y in zip(copies, ys)], steps, warmup, min_graph_calls=40)
    algo = per + m * H * 2 + m * H * 4 + 2 * (m * 2 * I * 4)  # weights, x, y, gate | up written and read
    return dict(sec=sec, steps=nsteps, gbs=algo / sec / 1e9, tokens_per_s=m / sec, copies=len(copies))


def bench_moe(steps, warmup, seed=20):
    """Config 5: GPT-OSS-20B-style MXFP4 MoE, 32 experts, top-4, hidden = intermediate
    = 2880, 256 bf16 tokens, router logits ~ N(0,1).  One copy of the 423 MB expert
    weights already exceeds the Infinity Cache."""
    import torch

    import nn_amd
    E, H, I, T, K = 32, 2880, 2880, 256, 4
    gp, gs = nn_amd.quantize_mxfp4(nn_amd.synth_normal(seed, 1, (E, H, 2 * I), 0.02))
    dp, ds = nn_amd.quantize_mxfp4(nn_amd.synth_normal(seed, 2, (E, I, H), 0.02))
    gb = nn_amd.synth_normal(seed, 3, (E, 2 * I), 0.02)
    db = nn_amd.synth_normal(seed, 4, (E, H), 0.02)
    moe = nn_amd.QuantizedMoE(E, H, I, gp, gs, gb, dp, ds, db)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(seed, 5, (T, H), 1.0)).to(dev).to(torch.bfloat16)
    logits = torch.from_numpy(nn_amd.synth_normal(seed, 6, (T, E), 1.0)).to(dev)
    y = torch.empty((T, H), device=dev)
    L = lib()

    def f():
        check(L.nnq_moe_forward(moe._h, vp(x), 2, T, vp(logits), K, ctypes.c_float(7.0), vp(y), None, None,
                                cur_stream()))

    sec, nsteps = time_graph([f], steps, warmup, min_graph_calls=20)
    # the whole block: router Linear on the device, then the same layer
    rmoe = nn_amd.QuantizedMoE(E, H, I, gp, gs, gb, dp, ds, db, router_weight=nn_amd.synth_normal(seed, 7, (E, H), 0.02),
                               router_bias=nn_amd.synth_normal(seed, 8, (E,), 0.1))
    st = torch.zeros(1, dtype=torch.int32, device=dev)

    def fb():
        check(L.nnq_moe_block_forward(rmoe._h, rmoe._router, vp(x), 2, T, K, ctypes.c_float(7.0), vp(y), None, None,
                                      vp(st), cur_stream()))

    sec_block, _ = time_graph([fb], steps, warmup, min_graph_calls=20)
    del rmoe
    _, ti, _ = moe.forward(x, logits, top_k=K, return_routing=True)
    used = len(np.unique(ti.cpu().numpy()))
    per_expert = (H * 2 * I + I * H) * 17 // 32 + (2 * I + H) * 4  # MXFP4 codes + scales + biases
    algo = used * per_expert + T * H * 2 + T * E * 4 + T * H * 4
    flops = 2.0 * T * K * (H * 2 * I + I * H)
    return dict(sec=sec, steps=nsteps, gbs=algo / sec / 1e9, tflops=flops / sec / 1e12, tokens_per_s=T / sec,
                experts_used=used, algo_bytes=algo, sec_block=sec_block)


def cpu_baseline_q4k(wb, xnp, n, k, budget_s=10.0):
    """The oracle's restatement of QLinear::forward (whole-matrix dequant then f32
    x @ W^T), single-threaded, timed on this host for about `budget_s` seconds."""
    from oracle import oracle as O
    t0 = time.perf_counter()
    calls = 0
    while True:
        O.q4k_linear(xnp, wb, n)
        calls += 1
        if time.perf_counter() - t0 > budget_s:
            break
    return (time.perf_counter() - t0) / calls, calls


def copy_calibration():
    """A plain 256 MiB device-to-device copy (read 256 MiB, write 256 MiB) repeated: the
    reference point that scales rocprofv3's FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch
    n = 256 << 20
    a = torch.ones(n // 4, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(20):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"copy calibration: 20 x copy of {n} bytes")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--only-gemm", action="store_true", help="only the two M=512 prefill GEMMs (for PMC runs)")
    ap.add_argument("--only-moe", action="store_true", help="only the MXFP4 MoE layer (for PMC runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: every box in this run has one MI355X, and the quantized-linear "
              "kernels run on one device's share (the multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(2)
    import nn_amd
    nn_amd.init(0)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.only_gemm:
        for (m, n, k) in [(512, 12288, 4096), (512, 4096, 12288)]:
            g = bench_gemm(m, n, k, args.steps, args.warmup)
            log(f"prefill GEMM {m}x{n}x{k}: {g['sec'] * 1e6:.2f} us/call  {g['tflops']:.1f} TFLOP/s")
        return
    if args.only_moe:
        g = bench_moe(args.steps, args.warmup)
        log(f"MXFP4 MoE: {g['sec'] * 1e6:.2f} us/call  {g['gbs']:.1f} GB/s")
        return

    log("bench: Q4_K GEMV 4096x12288 (rotating copies)")
    r = bench_gemv("q4_k", 4096, 12288, args.steps, args.warmup, seed=2, single=True)
    log(f"  {r['sec'] * 1e6:.2f} us/step  {r['gbs']:.1f} GB/s  (cache-resident single copy: {r['gbs_single']:.1f} GB/s)")

    configs = {}
    if not args.only_headline:
        few = max(100, args.steps // 10)
        log("bench: Q8_0 GEMV 4096x4096")
        g = bench_gemv("q8_0", 4096, 4096, few, 20, seed=1)
        configs["q8_0_gemv_4096x4096"] = {"us": round(g["sec"] * 1e6, 3), "GBps": round(g["gbs"], 1),
                                          "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4)}
        log("bench: Q4_K GEMV 24576x4096 (fused gate+up)")
        g = bench_gemv("q4_k", 24576, 4096, few, 20, seed=5)
        configs["q4_k_gemv_24576x4096"] = {"us": round(g["sec"] * 1e6, 3), "GBps": round(g["gbs"], 1),
                                           "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4)}
        log("bench: Qwen3-8B MLP decode (Q4_K gate | up GEMV + SwiGLU-staging down GEMV)")
        g = bench_mlp(few, 20)
        configs["q4_k_qwen3_8b_mlp_decode_m1"] = {"us": round(g["sec"] * 1e6, 3), "GBps": round(g["gbs"], 1),
                                                  "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4),
                                                  "tokens_per_s": round(g["tokens_per_s"], 1)}
        log("bench: Q6_K LM head 151936x4096 + argmax")
        g = bench_lm_head(max(40, args.steps // 40), 10)
        configs["q6_k_lm_head_151936x4096_argmax"] = {"us": round(g["sec"] * 1e6, 3), "GBps": round(g["gbs"], 1),
                                                      "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4),
                                                      "tokens_per_s": round(1.0 / g["sec"], 1),
                                                      "with_sampling_us": round(g["sec_sample"] * 1e6, 3)}
        for (m, n, k) in [(512, 12288, 4096), (512, 4096, 12288)]:
            log(f"bench: Q4_K prefill GEMM M={m} N={n} K={k} (bf16 in/out)")
            g = bench_gemm(m, n, k, max(50, args.steps // 20), 10)
            configs[f"q4_k_prefill_gemm_{m}x{n}x{k}"] = {
                "us": round(g["sec"] * 1e6, 3), "TFLOPs": round(g["tflops"], 2),
                "frac_mfma16": round(g["tflops"] / MFMA16_PEAK_TFLOPS, 4), "tokens_per_s": round(m / g["sec"], 1)}
            log(f"  {g['sec'] * 1e6:.2f} us/call  {g['tflops']:.1f} TFLOP/s")
        log("bench: MXFP4 MoE (32 experts, top-4, 2880/2880, 256 tokens)")
        g = bench_moe(max(20, args.steps // 100), 5)
        configs["mxfp4_moe_e32_k4_h2880_t256"] = {
            "us": round(g["sec"] * 1e6, 3), "GBps": round(g["gbs"], 1), "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4),
            "TFLOPs": round(g["tflops"], 2), "tokens_per_s": round(g["tokens_per_s"], 1),
            "experts_used": g["experts_used"], "with_router_us": round(g["sec_block"] * 1e6, 3)}
        for name, c in configs.items():
            log(f"  {name}: {c}")

    cpu = None
    if not args.no_cpu and not args.only_headline:
        log("bench: CPU baseline (oracle QLinear::forward restatement, 1 thread)")
        dt, calls = cpu_baseline_q4k(r["wbytes"], r["x"].cpu().numpy(), r["n"], r["k"], args.cpu_budget)
        cpu = {"value": round(r["algo_bytes"] / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{calls} full Q4_K 4096x12288 GEMV calls (whole-matrix dequant + f32 x@W^T, as "
                         f"QLinear::forward), {dt * 1e3:.1f} ms/call, on this host"}
        log(f"  cpu {cpu['value']} GB/s")

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as fh:
            traffic = json.load(fh).get("traffic_bytes_per_launch")
    line = {
        "metric": METRIC,
        "value": round(r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(r["sec"] * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k",
        "data": "synthetic (seeded splitmix64 N(0,0.02) weights quantized by BlockQ4K::quantize, N(0,1) x)",
        "config": {"workload": "Q4_K decode GEMV 4096x12288 (Qwen3-8B down_proj), x f32 [1x12288], y f32",
                   "n": r["n"], "k": r["k"], "weight_copies": r["copies"],
                   "algorithmic_bytes_per_step": r["algo_bytes"],
                   "timing": "HIP graph of launches replayed on one stream, HIP events on that stream",
                   "cache_resident_single_copy_GBps": round(r["gbs_single"], 1)},
        "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "configs": configs or None,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
