"""CPU baseline of the quantized-linear path, as the reference runs it: block decode
to f32, then an f32 product (crates/nn-core/src/layers/quantized/linear.rs:366-400 ->
crates/nn-core/src/dyn_tensor/ops/matmul.rs:18-52).

Benchmark infrastructure: bench.py's cpu_baseline leg and the tests that check it
load this module; no product code does.  libcpu_baseline.so (cpu_baseline.c) holds the
oracle's own decoders built at -O3 and run over block ranges under OpenMP, and a
cache-blocked f32 product (x . W^T) with the columns split over OpenMP threads, and its
x . W form for the MoE's experts (W stored [in, out]).  Every product runs on the same
OpenMP threads as the decoders: with numpy's BLAS beside them, the decoders' idle OpenMP
threads spun through the BLAS calls and all-thread runs were slower than one thread.
Decoded values are bit-identical to the oracle's; products agree with it to f32 rounding
only, so this is a speed baseline, never a parity reference.
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
_i64 = ctypes.c_int64
_int = ctypes.c_int


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            subprocess.run(["make", "-s", "-C", HERE], check=True)
        L = ctypes.CDLL(_LIB)
        for name in ("cb_dequant_q4k", "cb_dequant_q6k"):
            getattr(L, name).argtypes = [_u8p, _sz, _f32p, _int]
        L.cb_dequant_mxfp4.argtypes = [_u8p, _u8p, _sz, _f32p, _int]
        L.cb_matmul_xwt.argtypes = [_f32p, _i64, _f32p, _i64, _i64, _f32p, _int]
        L.cb_matmul_xw.argtypes = [_f32p, _i64, _f32p, _i64, _i64, _f32p, _int]
        L.cb_q4k_qlinear.argtypes = [_u8p, _i64, _i64, _f32p, _i64, _f32p, _f32p, _int]
        L.cb_argmax.argtypes = [_f32p, _i64]
        L.cb_argmax.restype = _i64
        L.cb_max_threads.restype = _int
        _lib = L
    return _lib


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
    lib().cb_dequant_q4k(_p(wb, _u8p), count // 256, _p(out, _f32p), threads)
    return out


def dequant_q6k(wb, count, threads=1, out=None):
    wb = np.ascontiguousarray(wb, np.uint8)
    out = np.empty(count, np.float32) if out is None else out
    lib().cb_dequant_q6k(_p(wb, _u8p), count // 256, _p(out, _f32p), threads)
    return out


def dequant_mxfp4(packed, scales, count, threads=1, out=None):
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint8)
    out = np.empty(count, np.float32) if out is None else out
    lib().cb_dequant_mxfp4(_p(packed, _u8p), _p(scales, _u8p), count // 32, _p(out, _f32p), threads)
    return out


def matmul_xwt(x, w, threads=1, out=None):
    """y = x . w^T in f32 (x [m, k], w [n, k], both C-contiguous f32)."""
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32) if out is None else out
    lib().cb_matmul_xwt(_p(x, _f32p), m, _p(w, _f32p), n, k, _p(out, _f32p), threads)
    return out


def matmul_xw(x, w, threads=1, out=None):
    """y = x . w for w [k, n] row-major (f32; OpenMP over column blocks)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = x.shape
    n = w.shape[1]
    out = np.empty((m, n), np.float32) if out is None else out
    lib().cb_matmul_xw(_p(x, _f32p), m, _p(w, _f32p), k, n, _p(out, _f32p), threads)
    return out


def q4k_qlinear(wb, n, k, x, wbuf, out, threads=1):
    """QLinear::forward with a Q4_K weight: decode all of W into wbuf (allocated once by
    the caller), then out = x . W^T."""
    lib().cb_q4k_qlinear(_p(wb, _u8p), n, k, _p(x, _f32p), x.shape[0], _p(wbuf, _f32p), _p(out, _f32p), threads)
    return out


def argmax(v) -> int:
    """First index of the maximum (argreduce.rs:105-118; the inputs here are finite)."""
    v = np.ascontiguousarray(v, np.float32).ravel()
    return int(lib().cb_argmax(_p(v, _f32p), v.size))


def moe_buffers(E, H, inter, faithful=False):
    """moe_forward's decode buffers (gate_up, down), allocated once by the caller so that
    no timed call pays first-touch page faults"""
    n = E if faithful else 1
    return np.empty(n * H * 2 * inter, np.float32), np.empty(n * inter * H, np.float32)


def moe_forward(x, logits, top_k, gp, gs, gb, dp, ds, db, inter, limit=7.0, faithful=False, expert_limit=0,
                threads=1, bufs=None):
    """QuantizedDecoderLayer::moe_forward with router logits given
    (crates/nn-gptoss/src/quantized_model.rs:132-194): softmax, top-k, renormalise, then per
    expert in ascending order over its tokens: x @ Wgu + b, clamp(silu(gate)) * up,
    @ Wd + b, weighted index_add.  faithful: every expert call decodes all experts'
    weights (expert_forward, :107, :123), as the reference does; otherwise only the expert
    in use.  expert_limit > 0 runs only that many experts that have tokens (a bounded
    sample).  bufs: moe_buffers(...) of the same form, else allocated here.  Returns (y,
    experts run).  Decoders and products run on `threads` OpenMP threads."""
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
    wgu, wdn = bufs if bufs is not None else moe_buffers(E, H, I, faithful)
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
        gu = matmul_xw(x[rows], Wg, threads) + gb[e]
        g, u = gu[:, :I], gu[:, I:]
        h = np.clip(g / (1.0 + np.exp(-g)), -limit, limit) * u
        yo = matmul_xw(h, Wd, threads) + db[e]
        y[rows] += yo * tw[rows, slots][:, None]  # a token meets an expert at most once
    return y, ran
