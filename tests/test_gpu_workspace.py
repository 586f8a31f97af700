"""Workspace sharing across host threads and capture-workspace release (GPU).

Eager calls on one stream share that stream's workspace.  Two host threads that call on
the same stream must not interleave their copies and kernels on it, nor free the buffer
the other's call holds when the workspace grows: each call holds the stream from its
first scratch request until its last enqueue.  Every result is compared with the same
call made alone (bit-equal: the kernels are deterministic).
"""
import ctypes
import threading

import pytest
import torch

from test_gpu_linear import make_weight

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def dev():
    import nn_amd
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nn_amd.init(0)
    return torch.device("cuda:0")


def q4k_bytes(n, k, seed):
    import nn_amd
    return nn_amd.quantize_q4_k(nn_amd.synth_normal(seed, 1, (n, k), 0.02))


def misaligned(x):
    """a contiguous copy of x that starts 4 bytes past an aligned address (the call stages
    it through the workspace with a device copy)"""
    flat = torch.empty(x.numel() + 1, dtype=x.dtype, device=x.device)
    v = flat[1:].view(x.shape)
    v.copy_(x)
    return v


def test_two_threads_one_stream(dev):
    """Thread A and thread B call nnq_linear on one stream at the same time: A with prefill
    batches whose inputs are staged through the workspace, B with growing batches (each
    growth frees the old buffer stream-ordered) and a release of the workspace between
    rounds.  Every output equals the single-threaded result."""
    import nn_amd
    from nn_amd import _lib
    n, k = 1024, 4096
    w = make_weight("q4_k", q4k_bytes(n, k, seed=5), n, k)
    ms_a = [300, 129, 512]
    ms_b = [40, 200, 400, 700, 1000]
    xa = {m: torch.from_numpy(nn_amd.synth_normal(100 + m, 2, (m, k), 1.0)).to(dev) for m in ms_a}
    xb = {m: torch.from_numpy(nn_amd.synth_normal(200 + m, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16) for m in ms_b}
    ref_a = {m: nn_amd.quantized_linear(x, w) for m, x in xa.items()}
    ref_b = {m: nn_amd.quantized_linear(x, w) for m, x in xb.items()}
    torch.cuda.synchronize()
    xa_mis = {m: misaligned(x) for m, x in xa.items()}
    torch.cuda.synchronize()

    S = torch.cuda.Stream()
    lib = _lib.load()
    rounds = 6
    # outputs allocated up front, so the threads only call the library
    ya = [[torch.empty(m, n, device=dev) for m in ms_a] for _ in range(rounds)]
    yb = [[torch.empty(m, n, device=dev) for m in ms_b] for _ in range(rounds)]
    torch.cuda.synchronize()
    errors = []
    start = threading.Barrier(2)

    def call(x, y, dt):
        rc = lib.nnq_linear(w.handle, ctypes.c_void_p(x.data_ptr()), dt, x.shape[0], k, None, 0,
                            ctypes.c_void_p(y.data_ptr()), 0, ctypes.c_void_p(S.cuda_stream))
        if rc:
            errors.append(lib.nnq_last_error().decode())

    def thread_a():
        start.wait()
        for r in range(rounds):
            for i, m in enumerate(ms_a):
                call(xa_mis[m], ya[r][i], 0)

    def thread_b():
        start.wait()
        for r in range(rounds):
            for i, m in enumerate(ms_b):
                call(xb[m], yb[r][i], 2)
            if lib.nnq_release_workspace(ctypes.c_void_p(S.cuda_stream)):
                errors.append(lib.nnq_last_error().decode())

    ts = [threading.Thread(target=thread_a), threading.Thread(target=thread_b)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for r in range(rounds):
        for i, m in enumerate(ms_a):
            assert torch.equal(ya[r][i], ref_a[m]), f"thread A round {r} m={m}"
        for i, m in enumerate(ms_b):
            assert torch.equal(yb[r][i], ref_b[m]), f"thread B round {r} m={m}"


def test_release_capture_workspaces(dev):
    """A capture's workspace lives until nnq_release_capture_workspaces: graphs replay
    correctly before it, the call returns the memory to the device, and a graph captured
    afterwards allocates again and replays correctly."""
    import nn_amd
    from nn_amd import _lib
    lib = _lib.load()
    m, n, k = 512, 4096, 12288
    w = make_weight("q4_k", q4k_bytes(n, k, seed=9), n, k)
    x = torch.from_numpy(nn_amd.synth_normal(9, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    ref = nn_amd.quantized_linear(x, w)
    torch.cuda.synchronize()

    def capture_and_check():
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                y = nn_amd.quantized_linear(x, w)
        torch.cuda.current_stream().wait_stream(s)
        for i in range(3):
            y.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, ref), f"replay {i}"
        g.reset()
        del g, y

    capture_and_check()
    capture_and_check()
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    assert lib.nnq_release_capture_workspaces() == 0, lib.nnq_last_error()
    free1, _ = torch.cuda.mem_get_info()
    # each capture held at least its GEMM's activation staging (m * k * 2 bytes)
    print(f"released {(free1 - free0) / 2**20:.1f} MiB")
    assert free1 - free0 >= 2 * m * k * 2
    capture_and_check()
    assert lib.nnq_release_capture_workspaces() == 0, lib.nnq_last_error()
