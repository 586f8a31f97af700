"""CPU baseline of the quantized-linear path, as the reference runs it: block decode
to f32, then an f32 sgemm (crates/nn-core/src/dyn_tensor/ops/matmul.rs:18-52).

Benchmark infrastructure: bench.py's cpu_baseline leg and the tests that check it
load this module; no product code does.  The decoders are the oracle's own, built at
-O3 (libcpu_baseline.so), run over block ranges on a pool of threads (ctypes releases
the GIL, identical values); the f32 GEMM is numpy's BLAS (OpenBLAS), a faster stand-in
for the reference's matrixmultiply, with its thread count set through threadpoolctl.
Results agree with the oracle to f32 rounding only, so this is a speed baseline, never
a parity reference.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from contextlib import contextmanager

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(HERE, "libcpu_baseline.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_sz = ctypes.c_size_t


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            subprocess.run(["make", "-s", "-C", HERE], check=True)
        L = ctypes.CDLL(_LIB)
        for name in ("orc_dequant_q4_k_gguf", "orc_dequant_q6_k_legacy"):
            getattr(L, name).argtypes = [_u8p, _sz, _sz, _f32p]
            getattr(L, name).restype = _sz
        L.orc_mxfp4_dequantize.argtypes = [_u8p, _u8p, _sz, _sz, _f32p]
        _lib = L
    return _lib


_pools = {}


def _parallel(nblocks, threads, fn):
    """fn(b0, b1) over [0, nblocks) split into `threads` contiguous ranges."""
    if threads <= 1 or nblocks < 2 * threads:
        fn(0, nblocks)
        return
    from concurrent.futures import ThreadPoolExecutor
    pool = _pools.get(threads)
    if pool is None:
        pool = _pools[threads] = ThreadPoolExecutor(max_workers=threads)
    per = -(-nblocks // threads)
    list(pool.map(lambda b0: fn(b0, min(nblocks, b0 + per)), range(0, nblocks, per)))


def _p(a, t):
    return a.ctypes.data_as(t)


def host_info() -> dict:
    """The host's CPU: logical CPUs, the ones this process may use, OMP_NUM_THREADS (the
    GPU boxes set it to the host's share of cores) and the model name."""
    model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or aff
    return {"nproc": os.cpu_count(), "affinity": aff, "omp_num_threads": omp, "model": model}


def all_threads() -> int:
    """Threads for an all-core run: OMP_NUM_THREADS (on a GPU box, the host's share of
    cores) capped by the CPUs this process may run on."""
    h = host_info()
    return max(1, min(h["omp_num_threads"], h["affinity"]))


@contextmanager
def blas_threads(n: int):
    """numpy's BLAS limited to n threads inside the block."""
    from threadpoolctl import threadpool_limits
    with threadpool_limits(limits=n, user_api="blas"):
        yield


def dequant_q4k(wb, count, threads=1, out=None):
    wb = np.ascontiguousarray(wb, np.uint8)
    out = np.empty(count, np.float32) if out is None else out
    L = lib()
    _parallel(count // 256, threads, lambda b0, b1: L.orc_dequant_q4_k_gguf(
        _p(wb[b0 * 144:], _u8p), (b1 - b0) * 144, (b1 - b0) * 256, _p(out[b0 * 256:], _f32p)))
    return out


def dequant_q6k(wb, count, threads=1, out=None):
    wb = np.ascontiguousarray(wb, np.uint8)
    out = np.empty(count, np.float32) if out is None else out
    L = lib()
    _parallel(count // 256, threads, lambda b0, b1: L.orc_dequant_q6_k_legacy(
        _p(wb[b0 * 210:], _u8p), (b1 - b0) * 210, (b1 - b0) * 256, _p(out[b0 * 256:], _f32p)))
    return out


def dequant_mxfp4(packed, scales, count, threads=1, out=None):
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint8)
    out = np.empty(count, np.float32) if out is None else out
    L = lib()
    _parallel(count // 32, threads, lambda b0, b1: L.orc_mxfp4_dequantize(
        _p(packed[b0 * 16:], _u8p), _p(scales[b0:], _u8p), b1 - b0, (b1 - b0) * 32, _p(out[b0 * 32:], _f32p)))
    return out


def argmax(v) -> int:
    """First index of the maximum (argreduce.rs:105-118; the inputs here are finite)."""
    return int(np.argmax(v))


def moe_forward(x, logits, top_k, gp, gs, gb, dp, ds, db, inter, limit=7.0, faithful=False, expert_limit=0,
                threads=1):
    """QuantizedDecoderLayer::moe_forward with router logits given
    (crates/nn-gptoss/src/quantized_model.rs:132-194): softmax, top-k, renormalise, then per
    expert in ascending order over its tokens: x @ Wgu + b, clamp(silu(gate)) * up,
    @ Wd + b, weighted index_add.  faithful: every expert call decodes all experts'
    weights (expert_forward, :107, :123), as the reference does; otherwise only the expert
    in use.  expert_limit > 0 runs only that many experts that have tokens (a bounded
    sample).  Returns (y, experts run).  Call inside blas_threads(threads)."""
    x = np.asarray(x, np.float32)
    logits = np.asarray(logits, np.float32)
    T, H = x.shape
    E = logits.shape[1]
    I = inter
    gu_per, dn_per = H * 2 * I, I * H
    z = logits - logits.max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    ti = np.argsort(-p, axis=1, kind="stable")[:, :top_k]
    tw = np.take_along_axis(p, ti, axis=1)
    tw = tw / tw.sum(axis=1, keepdims=True)
    y = np.zeros((T, H), np.float32)
    wgu = np.empty((E if faithful else 1) * gu_per, np.float32)
    wdn = np.empty((E if faithful else 1) * dn_per, np.float32)
    ran = 0
    for e in range(E):
        rows, slots = np.nonzero(ti == e)
        if rows.size == 0:
            continue
        if expert_limit and ran >= expert_limit:
            break
        ran += 1
        if faithful:
            dequant_mxfp4(gp, gs, E * gu_per, threads, wgu)
            dequant_mxfp4(dp, ds, E * dn_per, threads, wdn)
            Wg = wgu[e * gu_per:(e + 1) * gu_per].reshape(H, 2 * I)
            Wd = wdn[e * dn_per:(e + 1) * dn_per].reshape(I, H)
        else:
            dequant_mxfp4(gp[e * gu_per // 2:(e + 1) * gu_per // 2], gs[e * gu_per // 32:(e + 1) * gu_per // 32],
                          gu_per, threads, wgu)
            dequant_mxfp4(dp[e * dn_per // 2:(e + 1) * dn_per // 2], ds[e * dn_per // 32:(e + 1) * dn_per // 32],
                          dn_per, threads, wdn)
            Wg = wgu.reshape(H, 2 * I)
            Wd = wdn.reshape(I, H)
        gu = x[rows] @ Wg + gb[e]
        g, u = gu[:, :I], gu[:, I:]
        h = np.clip(g / (1.0 + np.exp(-g)), -limit, limit) * u
        yo = h @ Wd + db[e]
        y[rows] += yo * tw[rows, slots][:, None]  # a token meets an expert at most once
    return y, ran
