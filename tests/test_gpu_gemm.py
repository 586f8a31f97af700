"""GPU parity for the Q4_K prefill GEMM (m > 8 tokens).

The HIP GEMM runs through the C ABI (nn_amd -> libnnq.so) and is compared with the
CPU oracle on the same bytes and activations (tolerances as in test_gpu_linear):
normwise and elementwise max relative error <= 1e-3 (near-zero skip at 1% of the
peak), per-row cosine >= 0.99999.  Small shapes use the oracle's own f32 path
(QLinear::forward restated: full dequant + x @ W^T); the benchmark shapes use the
oracle's bit-exact dequant followed by an f64 matmul (numpy), which is the exact
product the f32 reference approximates.
"""
import numpy as np
import pytest
import torch

from test_gpu_linear import check_close, make_weight, rand_bytes

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


def ref_f64(O, wb, n, k, x, legacy=False):
    w = (O.dequant_q4_k_legacy if legacy else O.dequant_q4_k)(wb, n * k).reshape(n, k)
    return (np.asarray(x, np.float64) @ w.astype(np.float64).T).astype(np.float32)


@pytest.mark.parametrize("m", [9, 33, 100])
@pytest.mark.parametrize("n,k", [(48, 256), (200, 1024), (64, 2048)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_gemm_small_vs_oracle(O, dev, m, n, k, xdt):
    import nn_amd
    wb = q4k_bytes(n, k, seed=31 + n + k)
    w = make_weight("q4_k", wb, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(5 + m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    ref = O.q4k_linear(x.float().cpu().numpy(), wb, n)
    check_close(ref, y, f"gemm m={m} n={n} k={k} x={xdt}")


@pytest.mark.parametrize("m,n,k", [
    (16, 9216, 4096),  # three tiles per workgroup, sixteen waves, one super-block each
    (11, 9216, 6144),  # three tiles, eight waves over 24 super-blocks: three per wave
    (5, 4096, 12288),  # one tile, sixteen waves over 48 super-blocks
    (13, 256, 512),    # one tile, two super-blocks: fourteen waves without one
    (7, 100, 768),     # N not a multiple of 16 (the last tile's extra columns unwritten)
])
def test_gemm_thin_configs(O, dev, m, n, k):
    """The one-launch kernel for 5..16 bf16 token rows (nnq_gemm_thin.hip) in each of its
    launch configurations, on random block bytes (arbitrary finite d, dmin, scales), with
    a bias, f32 and bf16 outputs (bf16: the f32 result rounded once)."""
    import nn_amd
    b = rand_bytes("q4_k", n, k, seed=1000 + m + n)
    w = make_weight("q4_k", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(m, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    bias = torch.from_numpy(nn_amd.synth_normal(m + 1, 3, (n,), 0.5)).to(dev)
    y32 = nn_amd.quantized_linear(x, w, bias)
    yb = nn_amd.quantized_linear(x, w, bias, out_dtype=torch.bfloat16)
    ref = ref_f64(O, b, n, k, x.float().cpu().numpy()) + bias.cpu().numpy()
    check_close(ref, y32.cpu().numpy(), f"thin m={m} n={n} k={k}")
    assert torch.equal(yb, y32.to(torch.bfloat16)), "bf16 output is the f32 result rounded once"


def test_gemm_thin_nonfinite_rows(O, dev):
    """The thin kernel (7 bf16 rows): a NaN in one token's activation and an infinity in
    another's make all of those tokens' outputs NaN (the infinity meets the offset term's
    opposite infinity), as the staged GEMMs' per-row scale does; the other rows stay
    within the bars."""
    import nn_amd
    m, n, k = 7, 96, 1024
    wb = q4k_bytes(n, k, seed=17)
    w = make_weight("q4_k", wb, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(17, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    ref = ref_f64(O, wb, n, k, x.float().cpu().numpy())
    x[2, 300] = float("nan")
    x[5, 17] = float("inf")
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    assert np.isnan(y[2]).all() and np.isnan(y[5]).all()
    keep = [0, 1, 3, 4, 6]
    check_close(ref[keep], y[keep], "thin finite rows")


def test_gemm_legacy_random_blocks(O, dev):
    """nn-gguf layout with random block bytes (arbitrary finite d / dmin / scales)."""
    import nn_amd
    m, n, k = 40, 96, 1024
    b = rand_bytes("q4_k", n, k, seed=77)
    w = make_weight("q4_k_legacy", b, n, k)
    x = nn_amd.synth_normal(77, 2, (m, k), 1.0)
    y = nn_amd.quantized_linear(torch.from_numpy(x).to(dev), w).cpu().numpy()
    check_close(ref_f64(O, b, n, k, x, legacy=True), y, "gemm legacy random")


def test_gemm_zero_d_blocks(O, dev):
    """Super-blocks with d = 0 (only the min term survives) inside a row."""
    import nn_amd
    m, n, k = 24, 32, 1024
    b = q4k_bytes(n, k, seed=3).reshape(-1, 144).copy()
    b[::3, 0:2] = 0  # d = +0.0 for every third super-block
    b = b.ravel()
    w = make_weight("q4_k", b, n, k)
    x = nn_amd.synth_normal(3, 2, (m, k), 1.0)
    y = nn_amd.quantized_linear(torch.from_numpy(x).to(dev), w).cpu().numpy()
    check_close(ref_f64(O, b, n, k, x), y, "gemm zero-d blocks")


def test_gemm_bias_bf16_out_and_nan_row(O, dev):
    import nn_amd
    m, n, k = 64, 160, 2048
    wb = q4k_bytes(n, k, seed=11)
    w = make_weight("q4_k", wb, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(11, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    bias = torch.from_numpy(nn_amd.synth_normal(11, 3, (n,), 0.5)).to(dev)
    y32 = nn_amd.quantized_linear(x, w, bias)
    yb = nn_amd.quantized_linear(x, w, bias, out_dtype=torch.bfloat16)
    ref = ref_f64(O, wb, n, k, x.float().cpu().numpy()) + bias.cpu().numpy()
    check_close(ref, y32.cpu().numpy(), "gemm bias")
    ref_b = torch.from_numpy(ref).to(torch.bfloat16).float().numpy()
    got_b = yb.float().cpu().numpy()
    assert np.all(np.abs(got_b - ref_b) <= np.abs(ref_b) * 2.0 ** -7 + 1e-30)
    x[5, 100] = float("nan")
    yn = nn_amd.quantized_linear(x, w).cpu().numpy()
    assert np.isnan(yn[5]).all() and np.isfinite(np.delete(yn, 5, axis=0)).all()


@pytest.mark.parametrize("m,xdt", [(16, "bf16"), (64, "bf16"), (128, "bf16"), (512, "bf16"), (64, "f32"), (5, "bf16"),
                                   (3, "bf16")])
@pytest.mark.parametrize("n,k", [(12288, 4096), (4096, 12288)])
def test_gemm_baseline_shapes(O, dev, m, n, k, xdt):
    """Config 4: both Qwen3-8B MLP matrices at M = 16, 64, 128 (the GEMV-to-GEMM
    crossover) and 512, bf16 activations, f32 and bf16 outputs; also f32 activations
    and 5- and 3-token batches (3: the smallest that runs the GEMM)."""
    import nn_amd
    wb = q4k_bytes(n, k, seed=4000 + k)
    w = make_weight("q4_k", wb, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(4000 + m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    ref = ref_f64(O, wb, n, k, x.float().cpu().numpy())
    check_close(ref, y, f"gemm {m}x{n}x{k} x={xdt}")
    yb = nn_amd.quantized_linear(x, w, out_dtype=torch.bfloat16).float().cpu().numpy()
    ref_b = torch.from_numpy(y).to(torch.bfloat16).float().numpy()
    assert np.array_equal(yb, ref_b), "bf16 output must be the f32 result rounded once"


@pytest.mark.parametrize("m,n,k", [(130, 256, 4096), (256, 384, 2048), (128, 192, 256), (300, 640, 1280),
                                   (384, 1024, 4096), (128, 4096, 4096), (9, 128, 256), (17, 4096, 12288),
                                   (40, 384, 4096), (64, 192, 2048), (33, 768, 8192), (100, 1152, 1024),
                                   (20, 576, 2048), (50, 576, 4096), (24, 1536, 4096)])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_gemm_ring_edges(O, dev, m, n, k, xdt):
    """The LDS-ring kernel's edges: 32-, 64- and 128-row tiles with a ragged last row
    tile, 128- and 192-wide column tiles, a single super-block, K split 1 to 16 ways,
    bf16 activations and f32 ones (staged hi and lo planes as two sets of slabs), with
    random block bytes (arbitrary finite d / dmin / scales), d = 0 super-blocks, bias,
    f32 and bf16 outputs; the split-K sum is deterministic (two calls agree bit for bit)."""
    import nn_amd
    b = rand_bytes("q4_k", n, k, seed=m + n + k).reshape(-1, 144).copy()
    b[::5, 0:2] = 0  # d = +0.0 for every fifth super-block
    b = b.ravel()
    w = make_weight("q4_k_legacy", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    bias = torch.from_numpy(nn_amd.synth_normal(m, 3, (n,), 0.5)).to(dev)
    y = nn_amd.quantized_linear(x, w, bias)
    y2 = nn_amd.quantized_linear(x, w, bias)
    assert torch.equal(y, y2), "repeated calls must agree bit for bit"
    ref = ref_f64(O, b, n, k, x.float().cpu().numpy(), legacy=True) + bias.cpu().numpy()
    check_close(ref, y.cpu().numpy(), f"gemm ring {m}x{n}x{k} x={xdt}")
    yb = nn_amd.quantized_linear(x, w, bias, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(yb, y.to(torch.bfloat16).float().cpu().numpy()), "bf16 output: the f32 result rounded once"


def test_gemm_graph_replay(O, dev):
    """The prefill GEMM (staging, ring kernel, split-K finalize) captured into a HIP graph
    replays to the eager result every time, with eager GEMMs between the replays."""
    import nn_amd
    m, n, k = 256, 4096, 4096
    wb = q4k_bytes(n, k, seed=12)
    w = make_weight("q4_k", wb, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(12, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    ref = nn_amd.quantized_linear(x, w)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            y = nn_amd.quantized_linear(x, w)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {i}"
        other = nn_amd.quantized_linear(x, w)  # eager call on another stream's workspace
        torch.cuda.synchronize()
        assert torch.equal(other, ref)


def test_graph_replay_on_other_stream_concurrent_with_eager(O, dev):
    """A graph captured on stream S keeps its own scratch: replayed on stream A while eager
    GEMMs with other inputs run on S, with no host synchronisation in between, every
    replay and every eager call gives its own eager result.  Then the stream's eager
    workspace is released and the next call allocates again."""
    import ctypes

    import nn_amd
    from nn_amd import _lib
    m, n, k = 256, 4096, 4096
    w = make_weight("q4_k", q4k_bytes(n, k, seed=21), n, k)
    x1 = torch.from_numpy(nn_amd.synth_normal(21, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    x2 = torch.from_numpy(nn_amd.synth_normal(22, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    ref1 = nn_amd.quantized_linear(x1, w)
    ref2 = nn_amd.quantized_linear(x2, w)
    S, A = torch.cuda.Stream(), torch.cuda.Stream()
    S.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(S):
        nn_amd.quantized_linear(x2, w)  # S's eager workspace exists before the capture
        with torch.cuda.graph(g, stream=S):
            yg = nn_amd.quantized_linear(x1, w)
    torch.cuda.synchronize()
    eager = []
    for _ in range(3):
        with torch.cuda.stream(A):
            g.replay()
        with torch.cuda.stream(S):
            eager.append(nn_amd.quantized_linear(x2, w))
    torch.cuda.synchronize()
    assert torch.equal(yg, ref1)
    for y in eager:
        assert torch.equal(y, ref2)
    with torch.cuda.stream(S):
        assert _lib.load().nnq_release_workspace(ctypes.c_void_p(S.cuda_stream)) == 0
        y = nn_amd.quantized_linear(x2, w)
    torch.cuda.synchronize()
    assert torch.equal(y, ref2)
