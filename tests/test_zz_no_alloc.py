"""GPU check of nnq_linear_sample_noalloc (LM head + sampling with the fixed device
scratch, no allocation) through the C ABI, against nnq_linear_sample on the same
inputs: logits bit-identical (the same GEMV kernels) and the same token, on two calls
in a row, the second with a smaller vocabulary and other sampling settings; then the
call inside a captured HIP graph, replayed with eager calls between the replays (each
leaves its own contents in the shared array); then the capacity error."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def dev():
    import nn_amd
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nn_amd.init(0)
    return torch.device("cuda:0")


def _vp(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _weight(n, k, seed):
    import nn_amd
    wb = nn_amd.quantize_q6_k(nn_amd.synth_normal(seed, 1, (n, k), 0.02))
    return nn_amd.QuantizedWeight.from_quantized(wb, nn_amd.QuantType.Q6_K, (n, k), layout=nn_amd.Layout.NN_GGUF)


def _call(fn_name, w, x, bias, past, cfg, dev):
    from nn_amd import _lib
    L = _lib.load()
    n, k = w.shape
    logits = torch.empty(n, dtype=torch.float32, device=dev)
    tok = torch.full((1,), -1, dtype=torch.int32, device=dev)
    rc = getattr(L, fn_name)(w.handle, _vp(x), k, _vp(bias), n if bias is not None else 0, _vp(logits), _vp(past),
                             0 if past is None else past.numel(), ctypes.byref(cfg), _vp(tok), _stream())
    assert rc == 0, _lib.last_error()
    return logits, tok


def test_noalloc_matches_linear_sample_twice(O, dev):
    import nn_amd
    from nn_amd import _lib
    cases = [
        # the Qwen3 LM head, then a smaller vocabulary with a bias, penalties and top_k None
        (151936, 4096, 50, 0.9, None, [], 1234),
        (5000, 1024, None, 0.8, 0.3, [7, 7, 4000, 12], 987),
    ]
    for n, k, top_k, top_p, bias_sigma, past, seed in cases:
        w = _weight(n, k, seed)
        x = torch.from_numpy(nn_amd.synth_normal(seed, 2, (k,), 1.0)).to(dev)
        bias = None if bias_sigma is None else torch.from_numpy(nn_amd.synth_normal(seed, 3, (n,), bias_sigma)).to(dev)
        pt = torch.tensor(past, dtype=torch.int32, device=dev) if past else None
        cfg = _lib.Sampling(0.7, -1 if top_k is None else top_k, 0 if top_p is None else 1,
                            0.0 if top_p is None else top_p, 1.2 if past else 1.0, 0.1 if past else 0.0, seed)
        lg_a, tok_a = _call("nnq_linear_sample_noalloc", w, x, bias, pt, cfg, dev)
        lg_b, tok_b = _call("nnq_linear_sample", w, x, bias, pt, cfg, dev)
        torch.cuda.synchronize()
        assert torch.equal(lg_a, lg_b), (n, k)
        assert int(tok_a.item()) == int(tok_b.item()), (n, k)
        ref = O.sample_token(lg_a.cpu().numpy(), temperature=0.7, top_k=top_k, top_p=top_p,
                             repetition_penalty=1.2 if past else 1.0, frequency_penalty=0.1 if past else 0.0,
                             past_tokens=past, seed=seed)
        assert int(tok_a.item()) == ref, (n, k)


def test_noalloc_in_captured_graph(dev):
    import nn_amd
    from nn_amd import _lib
    n, k = 32000, 2048
    w = _weight(n, k, 55)
    x = torch.from_numpy(nn_amd.synth_normal(55, 2, (k,), 1.0)).to(dev)
    cfg = _lib.Sampling(1.0, 40, 1, 0.95, 1.0, 0.0, 4242)
    ref_lg, ref_tok = _call("nnq_linear_sample", w, x, None, None, cfg, dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            lg, tok = _call("nnq_linear_sample_noalloc", w, x, None, None, cfg, dev)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(lg, ref_lg), f"replay {i}"
        assert int(tok.item()) == int(ref_tok.item()), f"replay {i}"
        # an eager call in between, with other inputs, leaves its own contents in the array
        other = torch.from_numpy(nn_amd.synth_normal(56 + i, 2, (k,), 1.0)).to(dev)
        _call("nnq_linear_sample_noalloc", w, other, None, None, cfg, dev)
        torch.cuda.synchronize()


def test_noalloc_capacity_error(dev):
    from nn_amd import _lib
    w = _weight(40000, 256, 9)
    x = torch.zeros(256, dtype=torch.float32, device=dev)
    logits = torch.empty(40000, dtype=torch.float32, device=dev)
    tok = torch.empty(1, dtype=torch.int32, device=dev)
    cfg = _lib.Sampling(1.0, 1000, 0, 0.0, 1.0, 0.0, 1)  # 20 blocks x 1000 > 16384 candidates
    rc = _lib.load().nnq_linear_sample_noalloc(w.handle, _vp(x), 256, None, 0, _vp(logits), None, 0,
                                               ctypes.byref(cfg), _vp(tok), _stream())
    assert rc == 13 and "top-k" in _lib.last_error()
