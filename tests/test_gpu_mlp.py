"""GPU parity for the Qwen3 SwiGLU MLP (Qwen3MLP::forward, crates/nn-qwen3/src/layers.rs:40-47).

nn_amd.QuantizedMLP runs through the C ABI (nnq_mlp_forward): for m <= 2 the gate | up
GEMV and a down GEMV that forms silu(gate) * up while staging its input; for larger m
the gate | up linear (GEMM for Q4_K beyond 8 tokens), a SwiGLU kernel and the down
linear.  The oracle composes the reference's steps on the same block bytes
(QLinear::forward / quantized_matmul per format, silu, product, down).  Bars as in
test_gpu_linear: normwise and elementwise max relative error <= 1e-3 (near-zero skip
at 1% of the peak), per-row cosine >= 0.99999; bf16 outputs equal the f32 result
rounded once; a NaN input raises NonFiniteData as check_output_finite does.
"""
import numpy as np
import pytest
import torch

from test_gpu_linear import check_close

pytestmark = pytest.mark.gpu

FMT = {"q8_0": (8, 0), "q4_k": (12, 0), "q6_k": (14, 1)}


@pytest.fixture(scope="module", autouse=True)
def dev():
    import nn_amd
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nn_amd.init(0)
    return torch.device("cuda:0")


def encode(O, fmt, w):
    return {"q8_0": O.quantize_q8_0, "q4_k": O.quantize_q4_k, "q6_k": O.quantize_q6_k}[fmt](w)


def make_mlp(O, H, I, gu_fmt, dn_fmt, seed):
    import nn_amd
    wg = nn_amd.synth_normal(seed, 1, (I, H), 0.03)
    wu = nn_amd.synth_normal(seed, 2, (I, H), 0.03)
    wd = nn_amd.synth_normal(seed, 3, (H, I), 0.03)
    bg, bu, bd = encode(O, gu_fmt, wg), encode(O, gu_fmt, wu), encode(O, dn_fmt, wd)
    mlp = nn_amd.QuantizedMLP(bg, bu, bd, FMT[gu_fmt][0], H, I, down_type=FMT[dn_fmt][0],
                              layout=FMT[gu_fmt][1], down_layout=FMT[dn_fmt][1])
    ref = lambda x: O.mlp_forward(x, (FMT[gu_fmt][0], bg), (FMT[gu_fmt][0], bu), (FMT[dn_fmt][0], bd), H, I)
    return mlp, ref


@pytest.mark.parametrize("m", [1, 2, 3, 12])
@pytest.mark.parametrize("gu_fmt,dn_fmt", [("q4_k", "q4_k"), ("q4_k", "q6_k"), ("q8_0", "q8_0"),
                                           ("q6_k", "q8_0")])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_mlp_small_vs_oracle(O, dev, m, gu_fmt, dn_fmt, xdt):
    import nn_amd
    H, I = 512, 768
    mlp, ref = make_mlp(O, H, I, gu_fmt, dn_fmt, seed=H + I + m)
    x = torch.from_numpy(nn_amd.synth_normal(m, 4, (m, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    y = mlp(x)
    r, bad = ref(x.float().cpu().numpy())
    assert not bad
    check_close(r, y.cpu().numpy(), f"mlp {gu_fmt}/{dn_fmt} m={m} x={xdt}")
    yb = mlp(x, out_dtype=torch.bfloat16)
    assert torch.equal(yb.float(), y.to(torch.bfloat16).float()), "bf16 output: the f32 result rounded once"


@pytest.mark.parametrize("m", [1, 2, 16])
def test_mlp_qwen3_8b_shape(O, dev, m):
    """Qwen3-8B: hidden 4096, intermediate 12288, Q4_K gate / up / down, bf16 input."""
    import nn_amd
    H, I = 4096, 12288
    mlp, ref = make_mlp(O, H, I, "q4_k", "q4_k", seed=8)
    x = torch.from_numpy(nn_amd.synth_normal(80 + m, 4, (m, H), 1.0)).to(dev).to(torch.bfloat16)
    y = mlp(x)
    r, bad = ref(x.float().cpu().numpy())
    assert not bad
    check_close(r, y.cpu().numpy(), f"mlp qwen3-8b m={m}")


@pytest.mark.parametrize("m", [1, 4])
def test_mlp_nonfinite_raises(O, dev, m):
    import nn_amd
    H, I = 256, 512
    mlp, _ = make_mlp(O, H, I, "q4_k", "q6_k", seed=5)
    x = torch.from_numpy(nn_amd.synth_normal(5, 4, (m, H), 1.0)).to(dev)
    mlp(x)  # finite: no error; the status is cleared by every call
    x[m - 1, 3] = float("nan")
    with pytest.raises(nn_amd.NonFiniteData):
        mlp(x)
    y = mlp(x, check=False)
    assert torch.isnan(y[m - 1]).all()
    x[m - 1, 3] = 0.0
    mlp(x)  # finite again: the status of the previous call does not leak


@pytest.mark.parametrize("m", [1, 12])
def test_mlp_graph_replay(O, dev, m):
    """Captured into a HIP graph (the per-stream workspace grows under capture), the
    MLP replays to the eager result every time, with eager calls on another stream
    (another workspace) between the replays."""
    import nn_amd
    H, I = 512, 768
    mlp, _ = make_mlp(O, H, I, "q4_k", "q6_k", seed=9)
    x = torch.from_numpy(nn_amd.synth_normal(9, 4, (m, H), 1.0)).to(dev).to(torch.bfloat16)
    ref = mlp(x)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            y = mlp(x, check=False)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {i}"
        other = mlp(x * 0.5)  # eager call between replays
        torch.cuda.synchronize()
        assert torch.isfinite(other).all()


def test_mlp_misaligned_x(O, dev):
    """The fused MLP on a narrowed input view (not 16-byte aligned) equals the aligned call."""
    import nn_amd
    H, I = 256, 512
    g, u, d = (nn_amd.quantize_q4_k(nn_amd.synth_normal(61, j, s, 0.02)) for j, s in ((1, (I, H)), (2, (I, H)),
                                                                                        (3, (H, I))))
    mlp = nn_amd.QuantizedMLP(g, u, d, nn_amd.QuantType.Q4_K, H, I)
    for m in (1, 2, 5, 20):
        x = torch.from_numpy(nn_amd.synth_normal(62 + m, 4, (m, H), 1.0)).to(dev)
        big = torch.zeros(m * H + 4, device=dev)
        big[1:1 + m * H] = x.reshape(-1)
        assert torch.equal(mlp(big[1:1 + m * H].view(m, H)), mlp(x))
