#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric): Q4_K decode GEMV at 4096x12288 (Qwen3-8B down_proj,
x f32 [1x12288]) in GB/s of algorithmic bytes (quantized weight + x + y).  A "step" is
one GEMV launch over one weight copy; the weight rotates over enough distinct copies
(>= 512 MB, twice the Infinity Cache) that every launch streams it from HBM.

Timing: one timed window is exactly `--steps` calls on torch's current stream,
bracketed by HIP events recorded on the same stream, with a device-side sleep queued
ahead of it.  Short windows (up to 256 calls and about 0.3 ms of device time, as the
headline at the driver's --steps 20) are eager launches, with a sleep long enough that
all of them are queued before the start event fires (checked per window); longer ones
are one HIP graph of exactly `--steps` calls, replayed once per window (a graph replay
carries a fixed start-up cost of several microseconds, which a short window would spread
over few calls; eager launches carry dispatch gaps per kernel).  Windows are repeated and the JSON carries the
median window (p10 / p90 beside it).  Inputs are resident in HBM before timing starts.

The same JSON line carries the roofline of the headline kernel (achieved, peak, its
measured traffic, and `floor_frac`: a pure 16-byte streaming read of the same bytes at
the same launch cadence against the kernel), measured achievable peaks (device copy,
torch's f16 GEMM at the prefill shapes), the other benchmark configs (Q8_0 GEMV with its
own streaming-read floor, Q4_K
gate+up GEMV, MLP decode, the Q6_K LM head with argmax and sampling, the Q4_K prefill
GEMMs at M = 16, 64, 128, 512, the MXFP4 MoE), and the CPU baseline: the reference's
flow (the oracle's block decoders and blocked f32 products, OpenMP) on this host, one
thread and all threads, with the host's core count.

Usage: python bench.py [--gpus 1] [--steps 2000] [--warmup 200] [--windows 25]
       python bench.py --only headline --no-single    (one kernel population, for rocprofv3)
       python bench.py --only q8_0|gateup|mlp|lm_head|gemm|moe|floor ...
       python bench.py --copy-calibration             (a 256 MiB device copy, the yardstick
                                                       for rocprofv3 FETCH_SIZE / WRITE_SIZE)
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

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 MFMA
METRIC = "Q4_K GEMV GB/s (% HBM peak) at 4096x12288; prefill TFLOP/s at M=512"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
TRAFFIC_FILE_REL = "profiles/traffic.json"
PROBE_LIB = os.path.join(ROOT, "nn_amd", "libnnq_probe.so")


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


def stats(per_step):
    a = np.sort(np.asarray(per_step, np.float64))
    return {"median": float(np.median(a)), "p10": float(np.percentile(a, 10)), "p90": float(np.percentile(a, 90)),
            "mean": float(a.mean()), "windows": int(a.size)}


EAGER_MAX_STEPS = 256  # short windows (calls, estimated device time) are timed as eager launches
EAGER_MAX_WINDOW_S = 3e-4


def _sleep_rate():
    """Device seconds per cycle of torch.cuda._sleep, measured once."""
    import torch
    global _SLEEP_S_PER_CYCLE
    if _SLEEP_S_PER_CYCLE is None:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(100_000)
        a.record()
        torch.cuda._sleep(2_000_000)
        b.record()
        torch.cuda.synchronize()
        _SLEEP_S_PER_CYCLE = a.elapsed_time(b) / 1e3 / 2_000_000
    return _SLEEP_S_PER_CYCLE


_SLEEP_S_PER_CYCLE = None


def time_windows(fn_list, steps, warmup, windows, per_call_s=None):
    """Time `windows` windows of exactly `steps` calls (cycling through fn_list), each
    bracketed by HIP events on the current stream; returns the per-call time statistics
    over the windows, in seconds.

    Short windows (at most EAGER_MAX_STEPS calls and EAGER_MAX_WINDOW_S of estimated
    device time, from `per_call_s`): eager launches, enqueued behind a device-side sleep
    long enough that every launch of the window is queued before the start event fires
    (checked on the host for each window: a window whose enqueue outlasted its sleep is
    timed again with a longer one), so the window times the device's back-to-back
    execution, not the host's launch rate.  Otherwise: one HIP graph of exactly `steps`
    calls, replayed once per window after a device-side sleep.  A graph replay carries a
    fixed start-up cost of several microseconds, which a short window would spread over
    few calls; eager launches carry dispatch gaps per kernel, which add up over long
    windows of multi-kernel calls."""
    import time

    import torch
    for i in range(warmup):
        fn_list[i % len(fn_list)]()
    torch.cuda.synchronize()
    if per_call_s is not None and steps <= EAGER_MAX_STEPS and steps * per_call_s <= EAGER_MAX_WINDOW_S:
        spc = _sleep_rate()
        t0 = time.perf_counter()
        for i in range(steps):
            fn_list[i % len(fn_list)]()
        enq = time.perf_counter() - t0
        torch.cuda.synchronize()
        per = []
        for w in range(windows):
            sleep_s = max(1e-4, 4 * enq)
            for _attempt in range(4):
                st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda._sleep(int(sleep_s / spc))
                t0 = time.perf_counter()
                st.record()
                for i in range(steps):
                    fn_list[i % len(fn_list)]()
                en.record()
                enq_w = time.perf_counter() - t0
                torch.cuda.synchronize()
                if enq_w < 0.8 * sleep_s:
                    per.append(st.elapsed_time(en) / 1e3 / steps)
                    break
                sleep_s *= 4
            else:
                raise RuntimeError("could not enqueue a window ahead of the device")
        return {**stats(per), "method": "eager"}
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                fn_list[i % len(fn_list)]()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(windows)]
    for st, en in ev:
        torch.cuda._sleep(200_000)  # ~100 us of device time ahead of the window
        st.record()
        g.replay()
        en.record()
    torch.cuda.synchronize()
    per = [st.elapsed_time(en) / 1e3 / steps for st, en in ev]
    del g
    return {**stats(per), "method": "graph"}


WINDOWS = None  # --windows: a fixed window count (profiler runs), else sized to a time budget


def windows_for(steps, per_call_s, budget_s=0.5, lo=5, hi=40):
    if WINDOWS:
        return WINDOWS
    return int(max(lo, min(hi, budget_s / max(steps * per_call_s, 1e-9))))


def trace_fields(tr, algo_bytes, st):
    """The roofline's profile-derived figures for a config of profiles/traffic.json: the
    fraction from the rocprofv3 kernel trace taken at the bench's own cadence (the same
    launches, eager windows of --steps 20), the traced empty kernel of the same run, and
    where the traffic figure comes from."""
    if not tr:
        return {}
    out = {"traffic_source": f"{TRAFFIC_FILE_REL} configs.{tr['name']}: FETCH_SIZE and WRITE_SIZE per dispatch "
                             f"(the table of {tr['source']}, one counter per rocprofv3 run) scaled by a 256 MiB "
                             f"device copy under the same counters"}
    t = tr.get("trace")
    if t:
        out["frac_trace"] = round(algo_bytes / (t["avg_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        out["trace"] = {"kernel_avg_us": t["avg_us"], "kernel_median_us": t["median_us"],
                        "kernel_p10_us": t["p10_us"], "kernel_p90_us": t["p90_us"], "dispatches": t["dispatches"],
                        "empty_kernel_avg_us": t["empty_avg_us"],
                        "event_us_per_step_p10_p90": [round(st["p10"] * 1e6, 3), round(st["p90"] * 1e6, 3)],
                        "source": f"{t['source']} ({t['command']})",
                        "note": "traced kernel durations run from each dispatch's start to its end, so they "
                                "leave out the gaps between launches that the event-timed value includes; the "
                                "empty kernel of the same traced run shows what a dispatch that does nothing "
                                "takes under the tracer"}
    return out


def traffic_record(name):
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as fh:
        rec = json.load(fh).get("configs", {}).get(name)
    return dict(rec, name=name) if rec else None


# ---------------------------------------------------------------------------------
# floors and achievable peaks
# ---------------------------------------------------------------------------------

def probe_lib():
    if not os.path.exists(PROBE_LIB):
        raise RuntimeError(f"{PROBE_LIB} is missing: run python -m nn_amd.build")
    L = ctypes.CDLL(PROBE_LIB)
    L.probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    L.probe_empty.argtypes = [ctypes.c_void_p]
    return L


def bench_floor(nbytes, steps, warmup, min_bytes=512 << 20):
    """A pure streaming read of `nbytes` (16-byte non-temporal loads, no compute) over
    rotating buffers, at several grid sizes, and an empty kernel, both replayed in
    graphs of `steps` launches: the per-launch floors of an HBM-streaming decode
    kernel of that size."""
    import torch
    P = probe_lib()
    chunk = 65536
    nb = -(-nbytes // chunk) * chunk
    copies = max(1, -(-min_bytes // nb))
    bufs = [torch.empty(nb, dtype=torch.uint8, device="cuda:0").fill_(i + 1) for i in range(copies)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    best = None
    for wg in (256, 512, 1024, 2048):
        def rd(b, wg=wg):
            def f():
                check(P.probe_stream_read(ctypes.c_void_p(b.data_ptr()), nb, wg, vp(sink), cur_stream()))
            return f
        st = time_windows([rd(b) for b in bufs], steps, warmup, windows_for(steps, 7e-6), per_call_s=7e-6)
        if best is None or st["median"] < best[1]["median"]:
            best = (wg, st)

    def emp():
        check(P.probe_empty(cur_stream()))
    est = time_windows([emp], steps, warmup, windows_for(steps, 2e-6), per_call_s=2e-6)
    del bufs
    return {"bytes": nb, "workgroups": best[0], "read": best[1], "empty": est}


def achievable_copy():
    """Device-to-device copy of 1 GiB (read + write bytes per second)."""
    import torch
    n = 1 << 30
    a = torch.ones(n // 4, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(10):
        b.copy_(a)
    en.record()
    torch.cuda.synchronize()
    sec = st.elapsed_time(en) / 1e3 / 10
    del a, b
    return 2.0 * n / sec / 1e9


def achievable_f16_gemm(m, n, k):
    """torch's f16 GEMM (hipBLASLt / rocBLAS, no dequantization) at the same shape, TFLOP/s."""
    import torch
    x = torch.randn(m, k, device="cuda:0", dtype=torch.float16)
    w = torch.randn(n, k, device="cuda:0", dtype=torch.float16)
    wt = w.t().contiguous()
    for _ in range(5):
        torch.matmul(x, wt)
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(50):
        torch.matmul(x, wt)
    en.record()
    torch.cuda.synchronize()
    return 2.0 * m * n * k / (st.elapsed_time(en) / 1e3 / 50) / 1e12


# ---------------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------------

def bench_gemv(fmt, n, k, steps, warmup, seed, min_bytes=512 << 20, single=False, long_steps=0):
    """Decode GEMV y[1, n] = x[1, k] W^T, x f32 ~ N(0,1), W ~ N(0,0.02) quantized.
    long_steps > steps: also the same launches timed in graphs of long_steps launches (a
    graph replay's fixed start-up cost, ~8-9 us, spread over more launches)."""
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
    st = time_windows(fns, steps, warmup, windows_for(steps, 8e-6), per_call_s=8e-6)
    algo = len(wb) + k * 4 + n * 4
    out = dict(st=st, steps=steps, algo_bytes=algo, copies=len(copies), gbs=algo / st["median"] / 1e9, wbytes=wb,
               x=x, n=n, k=k)
    if single:  # cache-resident figure (one copy replayed), labelled as such
        st1 = time_windows(fns[:1], steps, warmup, windows_for(steps, 6e-6), per_call_s=6e-6)
        out["gbs_single"] = algo / st1["median"] / 1e9
    if long_steps > steps:
        out["st_long"] = time_windows(fns, long_steps, 0, 5)
        out["long_steps"] = long_steps
    return out


def bench_lm_head(steps, warmup, seed=3):
    """Config 3: Q6_K LM head 151936x4096 (nn-gguf layout) with the fused first-index argmax,
    and the same head followed by sampling."""
    import torch

    import nn_amd
    n, k = 151936, 4096
    wb = nn_amd.quantize_q6_k(nn_amd.synth_normal(seed, 1, (n, k), 0.02))
    copies = make_copies(wb, nn_amd.QuantType.Q6_K, n, k, 512 << 20, layout=1)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(seed, 2, (k,), 1.0)).to(dev)
    logits = [torch.empty(n, device=dev) for _ in copies]
    idx = torch.empty(len(copies), dtype=torch.int32, device=dev)
    stv = torch.zeros(len(copies), dtype=torch.int32, device=dev)
    L = lib()

    def launcher(i):
        def f():
            check(L.nnq_linear_argmax(copies[i].handle, vp(x), k, None, 0, vp(logits[i]),
                                      ctypes.c_void_p(idx.data_ptr() + 4 * i),
                                      ctypes.c_void_p(stv.data_ptr() + 4 * i), cur_stream()))
        return f

    st = time_windows([launcher(i) for i in range(len(copies))], steps, warmup, windows_for(steps, 9e-5), per_call_s=9e-5)
    # the same LM head followed by sampling (temperature 0.7, top-k 50, top-p 0.9, the
    # SamplingConfig defaults) over the 151936 logits, on the device
    from nn_amd import _lib as NL
    cfg = NL.Sampling(0.7, 50, 1, 0.9, 1.0, 0.0, 12345)

    def sampler(i):
        def f():
            check(L.nnq_linear_sample(copies[i].handle, vp(x), k, None, 0, vp(logits[i]), None, 0, ctypes.byref(cfg),
                                      ctypes.c_void_p(idx.data_ptr() + 4 * i), cur_stream()))
        return f

    st_s = time_windows([sampler(i) for i in range(len(copies))], steps, warmup, windows_for(steps, 1.1e-4), per_call_s=1.1e-4)
    algo = len(wb) + k * 4 + n * 4 + 4
    return dict(st=st, steps=steps, gbs=algo / st["median"] / 1e9, algo_bytes=algo, copies=len(copies), st_sample=st_s,
                wbytes=wb, x=x)


def bench_gemm(m, n, k, steps, warmup, min_bytes=512 << 20, fmt="q4_k"):
    """Config 4: X [m, k] bf16 ~ N(0,1) times Q4_K W [n, k]^T -> Y [m, n] bf16, f32 accumulate
    (fmt q8_0 / q6_k: the same product over those formats' prefill GEMM)."""
    import torch

    import nn_amd
    w = nn_amd.synth_normal(4, k, (n, k), 0.02)
    if fmt == "q8_0":
        wb, qt, lay = nn_amd.quantize_q8_0(w), nn_amd.QuantType.Q8_0, nn_amd.Layout.GGUF
    elif fmt == "q6_k":
        wb, qt, lay = nn_amd.quantize_q6_k(w), nn_amd.QuantType.Q6_K, nn_amd.Layout.NN_GGUF
    else:
        wb, qt, lay = nn_amd.quantize_q4_k(w), nn_amd.QuantType.Q4_K, nn_amd.Layout.GGUF
    copies = make_copies(wb, qt, n, k, min_bytes, layout=lay)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(nn_amd.synth_normal(4, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    ys = [torch.empty((m, n), device=dev, dtype=torch.bfloat16) for _ in copies]
    L = lib()

    def launcher(wi, yi):
        def f():
            check(L.nnq_linear(wi.handle, vp(x), 2, m, k, None, 0, vp(yi), 2, cur_stream()))
        return f

    st = time_windows([launcher(c, y) for c, y in zip(copies, ys)], steps, warmup, windows_for(steps, 1e-4), per_call_s=1e-4)
    flops = 2.0 * m * n * k
    algo = len(wb) + m * k * 2 + m * n * 2
    return dict(st=st, steps=steps, tflops=flops / st["median"] / 1e12, gbs=algo / st["median"] / 1e9,
                copies=len(copies), wbytes=wb, x=x)


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
    stv = torch.zeros(1, dtype=torch.int32, device=dev)
    L = lib()

    def launcher(c, y):
        def f():
            check(L.nnq_mlp_forward(c._h, vp(x), 2, m, H, vp(y), 0, vp(stv), cur_stream()))
        return f

    st = time_windows([launcher(c, y) for c, y in zip(copies, ys)], steps, warmup, windows_for(steps, 2e-5), per_call_s=2e-5)
    algo = per + m * H * 2 + m * H * 4 + 2 * (m * I * 4)  # weights, x, y, h written and read
    return dict(st=st, steps=steps, gbs=algo / st["median"] / 1e9, tokens_per_s=m / st["median"], copies=len(copies))


def moe_inputs(seed=20):
    import nn_amd
    E, H, I, T = 32, 2880, 2880, 256
    gp, gs = nn_amd.quantize_mxfp4(nn_amd.synth_normal(seed, 1, (E, H, 2 * I), 0.02))
    dp, ds = nn_amd.quantize_mxfp4(nn_amd.synth_normal(seed, 2, (E, I, H), 0.02))
    gb = nn_amd.synth_normal(seed, 3, (E, 2 * I), 0.02)
    db = nn_amd.synth_normal(seed, 4, (E, H), 0.02)
    x = nn_amd.synth_normal(seed, 5, (T, H), 1.0)
    lg = nn_amd.synth_normal(seed, 6, (T, E), 1.0)
    return dict(E=E, H=H, I=I, T=T, K=4, gp=gp, gs=gs, gb=gb, dp=dp, ds=ds, db=db, x=x, lg=lg,
                rw=nn_amd.synth_normal(seed, 7, (E, H), 0.02), rb=nn_amd.synth_normal(seed, 8, (E,), 0.1))


def bench_moe(steps, warmup, mi):
    """Config 5: GPT-OSS-20B-style MXFP4 MoE, 32 experts, top-4, hidden = intermediate
    = 2880, 256 bf16 tokens, router logits ~ N(0,1).  One copy of the 423 MB expert
    weights already exceeds the Infinity Cache."""
    import torch

    import nn_amd
    E, H, I, T, K = mi["E"], mi["H"], mi["I"], mi["T"], mi["K"]
    moe = nn_amd.QuantizedMoE(E, H, I, mi["gp"], mi["gs"], mi["gb"], mi["dp"], mi["ds"], mi["db"])
    dev = torch.device("cuda:0")
    x = torch.from_numpy(mi["x"]).to(dev).to(torch.bfloat16)
    logits = torch.from_numpy(mi["lg"]).to(dev)
    y = torch.empty((T, H), device=dev)
    L = lib()

    def f():
        check(L.nnq_moe_forward(moe._h, vp(x), 2, T, vp(logits), K, ctypes.c_float(7.0), vp(y), None, None,
                                cur_stream()))

    st = time_windows([f], steps, warmup, windows_for(steps, 2e-4), per_call_s=2e-4)
    # the whole block: router Linear on the device, then the same layer
    rmoe = nn_amd.QuantizedMoE(E, H, I, mi["gp"], mi["gs"], mi["gb"], mi["dp"], mi["ds"], mi["db"],
                               router_weight=mi["rw"], router_bias=mi["rb"])
    stv = torch.zeros(1, dtype=torch.int32, device=dev)

    def fb():
        check(L.nnq_moe_block_forward(rmoe._h, rmoe._router, vp(x), 2, T, K, ctypes.c_float(7.0), vp(y), None, None,
                                      vp(stv), cur_stream()))

    st_b = time_windows([fb], steps, warmup, windows_for(steps, 2e-4), per_call_s=2e-4)
    del rmoe
    _, ti, _ = moe.forward(x, logits, top_k=K, return_routing=True)
    used = len(np.unique(ti.cpu().numpy()))
    per_expert = (H * 2 * I + I * H) * 17 // 32 + (2 * I + H) * 4  # MXFP4 codes + scales + biases
    algo = used * per_expert + T * H * 2 + T * E * 4 + T * H * 4
    flops = 2.0 * T * K * (H * 2 * I + I * H)
    return dict(st=st, steps=steps, gbs=algo / st["median"] / 1e9, tflops=flops / st["median"] / 1e12,
                tokens_per_s=T / st["median"], experts_used=used, algo_bytes=algo, st_block=st_b)


# ---------------------------------------------------------------------------------
# CPU baseline: the reference's flow on this host (oracle decoders + f32 products)
# ---------------------------------------------------------------------------------

def timed_calls(fn, budget_s, max_calls=1000):
    fn()  # warm (page faults, BLAS thread start)
    t0 = time.perf_counter()
    calls = 0
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el > budget_s or calls >= max_calls:
            return el / calls, calls


def cpu_baselines(head, lm, gemms, mi, budget):
    """Each workload on one thread (as the reference runs: no rayon, no BLAS threads) and on
    all of this process's cores (OpenMP); per-call seconds on bounded samples.  Buffers are
    allocated once, outside the timed calls."""
    from oracle import cpu_baseline as CB
    host = CB.host_info()
    allt = CB.all_threads()
    out = {"host": host, "threads_all": allt}

    def both(name, make_fn, budget_s):
        r = {}
        for th in (1, allt):
            with CB.blas_threads(th):
                fn = make_fn(th)
                fn()  # first touch of the output buffers, outside the timing
                dt, calls = timed_calls(fn, budget_s)
            r[f"t{th}"] = {"sec": dt, "calls": calls}
            log(f"  cpu {name} threads={th}: {dt * 1e3:.2f} ms/call over {calls} calls")
        out[name] = r
        return r

    # headline Q4_K GEMV 4096x12288: QLinear::forward (decode the whole matrix per call,
    # crates/nn-core/src/layers/quantized/linear.rs:366-400) and the load-time form
    # (nn-gguf decodes at load, crates/nn-gguf/src/reader.rs:280; an f32 GEMV per call)
    n, k = head["n"], head["k"]
    xh = np.ascontiguousarray(head["x"].cpu().numpy().astype(np.float32).reshape(1, k))
    wf = np.empty(n * k, np.float32)
    yh = np.empty((1, n), np.float32)
    wb = np.ascontiguousarray(head["wbytes"], np.uint8)
    both("q4k_gemv_qlinear_forward", lambda th: (lambda: CB.q4k_qlinear(wb, n, k, xh, wf, yh, th)), budget)
    CB.dequant_q4k(wb, n * k, allt, wf)
    wmat = wf.reshape(n, k)
    both("q4k_gemv_loadtime_dequant", lambda th: (lambda: CB.matmul_xwt(xh, wmat, th, yh)), budget / 2)
    del wf, wmat
    # Q6_K LM head: decoded at load (the reference's only Q6_K path), f32 GEMV + argmax per call
    if lm is not None:
        ln, lk = 151936, 4096
        lw = CB.dequant_q6k(lm["wbytes"], ln * lk, allt).reshape(ln, lk)
        xl = np.ascontiguousarray(lm["x"].cpu().numpy().astype(np.float32).reshape(1, lk))
        yl = np.empty((1, ln), np.float32)
        both("q6k_lm_head_argmax", lambda th: (lambda: CB.argmax(CB.matmul_xwt(xl, lw, th, yl))), budget / 2)
        del lw
    # prefill M=512: QLinear::forward per call (decode + f32 GEMM)
    for key, g in gemms.items():
        gm, gn, gk = g["shape"]
        xg = np.ascontiguousarray(g["x"].float().cpu().numpy())
        gw = np.empty(gn * gk, np.float32)
        yg = np.empty((gm, gn), np.float32)
        gb = np.ascontiguousarray(g["wbytes"], np.uint8)
        both(f"q4k_prefill_{gm}x{gn}x{gk}",
             lambda th, gb=gb, gn=gn, gk=gk, xg=xg, gw=gw, yg=yg: (lambda: CB.q4k_qlinear(gb, gn, gk, xg, gw, yg, th)),
             budget / 2)
        del gw, yg
    # MoE config 5: decode each used expert once per call; the faithful form decodes all
    # 32 experts on every expert call, sampled over 2 expert calls and scaled
    if mi is not None:
        args = (mi["x"], mi["lg"], mi["K"], mi["gp"], mi["gs"], mi["gb"], mi["dp"], mi["ds"], mi["db"], mi["I"])
        E, H = mi["lg"].shape[1], mi["x"].shape[1]
        once = CB.moe_buffers(E, H, mi["I"])
        both("mxfp4_moe_decode_once", lambda th: (lambda: CB.moe_forward(*args, threads=th, bufs=once)), budget / 2)
        del once
        used = mi.get("experts_used", 32)
        r = {}
        every = CB.moe_buffers(E, H, mi["I"], faithful=True)
        for th in (1, allt):
            with CB.blas_threads(th):
                CB.moe_forward(*args, faithful=True, expert_limit=1, threads=th, bufs=every)  # first touch
                t0 = time.perf_counter()
                _, ran = CB.moe_forward(*args, faithful=True, expert_limit=2, threads=th, bufs=every)
                dt = (time.perf_counter() - t0) / ran * used
            r[f"t{th}"] = {"sec": dt, "calls": 1, "sample": f"{ran} of {used} expert calls, scaled by {used}/{ran}"}
            log(f"  cpu mxfp4_moe_faithful threads={th}: {dt * 1e3:.1f} ms/call (sampled)")
        out["mxfp4_moe_faithful"] = r
    return out


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


def ms3(st):
    return {"us": round(st["median"] * 1e6, 3), "us_p10": round(st["p10"] * 1e6, 3),
            "us_p90": round(st["p90"] * 1e6, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-budget", type=float, default=3.0, help="seconds per CPU baseline measurement")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-single", action="store_true", help="skip the cache-resident single-copy headline timing")
    ap.add_argument("--only", default="", help="comma list: headline,q8_0,gateup,mlp,lm_head,gemm,moe,floor")
    ap.add_argument("--only-headline", action="store_true", help="same as --only headline --no-single")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--windows", type=int, default=0,
                    help="timed replays per config (default: as many as fit 0.5 s, 5 to 40)")
    args = ap.parse_args()
    global WINDOWS
    WINDOWS = args.windows if args.windows > 0 else None
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: every box in this run has one MI355X, and the quantized-linear "
              "kernels run on one device's share (the multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(2)
    if args.only_headline:
        args.only, args.no_single = "headline", True
    only = set(filter(None, args.only.split(",")))
    full = not only

    def want(name):
        return full or name in only

    import nn_amd
    nn_amd.init(0)
    if args.copy_calibration:
        copy_calibration()
        return
    K, W = args.steps, args.warmup
    few = max(20, K // 10)
    configs, results = {}, {}

    r = None
    if want("headline"):
        log(f"bench: Q4_K GEMV 4096x12288 (rotating copies), {K} steps per window")
        r = bench_gemv("q4_k", 4096, 12288, K, W, seed=2, single=not args.no_single,
                       long_steps=0 if args.no_single else 2000)
        log(f"  {r['st']['median'] * 1e6:.3f} us/step (p10 {r['st']['p10'] * 1e6:.3f}, p90 {r['st']['p90'] * 1e6:.3f})"
            f"  {r['gbs']:.1f} GB/s")
        if "st_long" in r:
            log(f"  {r['st_long']['median'] * 1e6:.3f} us/step in graphs of {r['long_steps']} launches")
    floor = None
    if want("floor") or (full and r is not None):
        log("bench: floors (28 MB streaming read, empty launch)")
        floor = bench_floor(28377088, K, W)
        log(f"  read {floor['read']['median'] * 1e6:.3f} us @ {floor['workgroups']} WGs, "
            f"empty {floor['empty']['median'] * 1e6:.3f} us")
    if want("q8_0"):
        log("bench: Q8_0 GEMV 4096x4096")
        g = bench_gemv("q8_0", 4096, 4096, few, 20, seed=1)
        configs["q8_0_gemv_4096x4096"] = {**ms3(g["st"]), "GBps": round(g["gbs"], 1),
                                          "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4)}
        if full:
            # the same streaming-read floor as the headline's, for this launch's bytes
            fq = bench_floor(g["algo_bytes"], few, 20)["read"]["median"]
            configs["q8_0_gemv_4096x4096"].update(floor_us=round(fq * 1e6, 3), floor_frac=round(fq / g["st"]["median"], 4))
    if want("gateup"):
        log("bench: Q4_K GEMV 24576x4096 (fused gate+up)")
        g = bench_gemv("q4_k", 24576, 4096, few, 20, seed=5)
        configs["q4_k_gemv_24576x4096"] = {**ms3(g["st"]), "GBps": round(g["gbs"], 1),
                                           "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4)}
    if want("mlp"):
        log("bench: Qwen3-8B MLP decode (Q4_K gate | up GEMV + down GEMV)")
        g = bench_mlp(few, 20)
        configs["q4_k_qwen3_8b_mlp_decode_m1"] = {**ms3(g["st"]), "GBps": round(g["gbs"], 1),
                                                  "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4),
                                                  "tokens_per_s": round(g["tokens_per_s"], 1)}
    lm = None
    if want("lm_head"):
        log("bench: Q6_K LM head 151936x4096 + argmax")
        lm = bench_lm_head(max(10, K // 40), 5)
        configs["q6_k_lm_head_151936x4096_argmax"] = {
            **ms3(lm["st"]), "GBps": round(lm["gbs"], 1), "frac_hbm": round(lm["gbs"] / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(1.0 / lm["st"]["median"], 1), "with_sampling": ms3(lm["st_sample"])}
    gemms = {}
    if want("gemm"):
        blas = {}
        for (m, n, k) in [(512, 12288, 4096), (512, 4096, 12288), (128, 12288, 4096), (128, 4096, 12288),
                          (64, 12288, 4096), (64, 4096, 12288), (16, 12288, 4096), (16, 4096, 12288)]:
            log(f"bench: Q4_K prefill GEMM M={m} N={n} K={k} (bf16 in/out)")
            g = bench_gemm(m, n, k, max(20, K // 20), 10)
            name = f"q4_k_prefill_gemm_{m}x{n}x{k}"
            c = {**ms3(g["st"]), "TFLOPs": round(g["tflops"], 2), "frac_mfma16": round(g["tflops"] / MFMA16_PEAK_TFLOPS, 4),
                 "GBps": round(g["gbs"], 1), "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4),
                 "tokens_per_s": round(m / g["st"]["median"], 1)}
            if m == 512:
                blas[(n, k)] = achievable_f16_gemm(m, n, k)
                c["torch_f16_gemm_TFLOPs"] = round(blas[(n, k)], 1)
                c["frac_of_torch_f16_gemm"] = round(g["tflops"] / blas[(n, k)], 4)
                gemms[name] = dict(shape=(m, n, k), wbytes=g["wbytes"], x=g["x"])
            configs[name] = c
            log(f"  {c}")
        for fmt, (m, n, k) in [("q8_0", (512, 4096, 4096)), ("q6_k", (512, 4096, 12288))]:
            log(f"bench: {fmt} prefill GEMM M={m} N={n} K={k} (bf16 in/out)")
            g = bench_gemm(m, n, k, max(20, K // 20), 10, fmt=fmt)
            c = {**ms3(g["st"]), "TFLOPs": round(g["tflops"], 2), "frac_mfma16": round(g["tflops"] / MFMA16_PEAK_TFLOPS, 4),
                 "tokens_per_s": round(m / g["st"]["median"], 1)}
            configs[f"{fmt}_prefill_gemm_{m}x{n}x{k}"] = c
            log(f"  {c}")
    mi = None
    if want("moe"):
        log("bench: MXFP4 MoE (32 experts, top-4, 2880/2880, 256 tokens)")
        mi = moe_inputs()
        g = bench_moe(max(10, K // 100), 5, mi)
        mi["experts_used"] = g["experts_used"]
        configs["mxfp4_moe_e32_k4_h2880_t256"] = {
            **ms3(g["st"]), "GBps": round(g["gbs"], 1), "frac_hbm": round(g["gbs"] / HBM_PEAK_GBS, 4),
            "TFLOPs": round(g["tflops"], 2), "tokens_per_s": round(g["tokens_per_s"], 1),
            "experts_used": g["experts_used"], "with_router": ms3(g["st_block"])}
    for name, c in configs.items():
        tr = traffic_record(name)
        if tr:
            c["traffic_bytes"] = tr["traffic_bytes_per_launch"]
        log(f"  {name}: {c}")
    if r is None:
        return

    achievable = {}
    if full:
        achievable["d2d_copy_GBps"] = round(achievable_copy(), 1)

    cpu = None
    if not args.no_cpu and full:
        log("bench: CPU baseline (reference flow: oracle decoders and f32 products, OpenMP)")
        cb = cpu_baselines(r, lm, gemms, mi, args.cpu_budget)
        hb = r["algo_bytes"]
        ta = cb["threads_all"]
        q1, qa = cb["q4k_gemv_qlinear_forward"]["t1"], cb["q4k_gemv_qlinear_forward"][f"t{ta}"]
        # the all-core figure is the value only when it beats one core
        use_all = ta > 1 and qa["sec"] < q1["sec"]
        qv, cores = (qa, ta) if use_all else (q1, 1)
        cpu = {"value": round(hb / qv["sec"] / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
               "sample": f"{qv['calls']} calls of the whole Q4_K 4096x12288 GEMV as QLinear::forward runs it "
                         f"(the oracle's decoders to an f32 buffer allocated once, then x @ W^T; OpenMP, "
                         f"-O3), {qv['sec'] * 1e3:.2f} ms/call on {cores} thread(s)",
               "single_thread_value": round(hb / q1["sec"] / 1e9, 4),
               "all_threads_value": round(hb / qa["sec"] / 1e9, 4), "threads_all": ta,
               "host": cb["host"]}
        variants = {}
        for name, v in cb.items():
            if name in ("host", "threads_all"):
                continue
            variants[name] = {f"ms_{t}": round(x["sec"] * 1e3, 3) for t, x in v.items()}
        cpu["variants_ms_per_call"] = variants

    tr = traffic_record("q4_k_gemv_4096x12288")
    line = {
        "metric": METRIC,
        "value": round(r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(r["st"]["median"] * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k",
        "data": "synthetic (seeded splitmix64 N(0,0.02) weights quantized by BlockQ4K::quantize, N(0,1) x)",
        "config": {"workload": "Q4_K decode GEMV 4096x12288 (Qwen3-8B down_proj), x f32 [1x12288], y f32",
                   "n": r["n"], "k": r["k"], "weight_copies": r["copies"],
                   "algorithmic_bytes_per_step": r["algo_bytes"],
                   "timing": (f"exactly {K} launches per window, " +
                              ("eager, all queued behind a device-side sleep before the start event"
                               if r["st"]["method"] == "eager" else "one HIP graph replay") +
                              f"; HIP events on the launch stream; median of {r['st']['windows']} windows"),
                   "us_per_step_p10": round(r["st"]["p10"] * 1e6, 3),
                   "us_per_step_p90": round(r["st"]["p90"] * 1e6, 3),
                   **({"cache_resident_single_copy_GBps": round(r["gbs_single"], 1)} if "gbs_single" in r else {}),
                   **({"long_graph": {"steps_per_window": r["long_steps"], **ms3(r["st_long"]),
                                      "GBps": round(r["algo_bytes"] / r["st_long"]["median"] / 1e9, 1),
                                      "frac_hbm": round(r["algo_bytes"] / r["st_long"]["median"] / 1e9 / HBM_PEAK_GBS, 4),
                                      "note": "the same launches in graphs of this many launches: the fixed start-up "
                                              "cost of each graph replay spread over more launches"}}
                      if "st_long" in r else {})},
        "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": tr["traffic_bytes_per_launch"] if tr else None,
                     **trace_fields(tr, r["algo_bytes"], r["st"])},
        "cpu_baseline": cpu,
        "configs": configs or None,
    }
    if floor is not None:
        fr = floor["read"]["median"]
        line["roofline"].update({
            "floor_us": round(fr * 1e6, 3), "floor_GBps": round(r["algo_bytes"] / fr / 1e9, 1),
            "floor_frac": round(fr / r["st"]["median"], 4),
            "floor": f"pure 16-byte streaming read of {floor['bytes']} B per launch ({floor['workgroups']} workgroups, "
                     f"rotating buffers), timed as the headline; empty-kernel launch "
                     f"{floor['empty']['median'] * 1e6:.3f} us"})
    if achievable:
        line["achievable"] = achievable
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
