"""GPU parity for the Q8_0 / Q6_K prefill GEMM (m > 8 tokens, nnq_gemm_blk.hip).

QLinear::forward with a batch of tokens over these formats
(crates/nn-core/src/layers/quantized/linear.rs:366-400, quantized_matmul_core,
crates/nn-core/src/dyn_tensor/quantized_matmul.rs:232-272) against the oracle on the
same bytes and activations, with the linear bars (normwise and elementwise relative
error <= 1e-3, per-row cosine >= 0.99999):
  * random block bytes (every code, every int8 sub-scale including -128, random f16
    scales): the f16 B operands (q for Q8_0; sc * (q' & ~1) and sc * (q' & 1) for Q6_K)
    must be exact for every combination, which these cover;
  * quantized N(0, 0.02) weights at the Qwen3-8B / GPT-OSS shapes;
  * Q8_0 rows whose block count is padded to groups of 8 (K = 2880, 4128);
  * f32 (hi + lo staging) and bf16 activations, f32 and bf16 outputs, bias, row counts
    that leave partial tiles (m = 9, 33, 130, 320 and 1100: the 128-row and, with bf16
    input, 128-column tiles; n = 96 and 520 leave a partial column tile), and m = 8 /
    m = 9 consistency (GEMV vs GEMM).
"""
import numpy as np
import pytest
import torch

from test_gpu_linear import check_close, make_weight, oracle_linear, quantized_weight_bytes, rand_bytes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def dev():
    import nn_amd
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nn_amd.init(0)
    return torch.device("cuda:0")


def run(w, x, dev, xdt="f32", bias=None, out_dtype=None):
    import nn_amd
    xt = torch.from_numpy(x).to(dev)
    if xdt == "bf16":
        xt = xt.to(torch.bfloat16)
    kw = {} if out_dtype is None else dict(out_dtype=out_dtype)
    y = nn_amd.quantized_linear(xt, w, bias, **kw)
    return xt.float().cpu().numpy(), y


@pytest.mark.parametrize("fmt", ["q8_0", "q6_k"])
@pytest.mark.parametrize("n,k", [(64, 256), (100, 512), (300, 2048)])
@pytest.mark.parametrize("m", [9, 16, 33, 64, 130])
def test_gemm_blk_random_bytes(O, dev, fmt, n, k, m):
    import nn_amd
    b = rand_bytes(fmt, n, k, seed=31 * n + k + m)
    w = make_weight(fmt, b, n, k)
    x = nn_amd.synth_normal(n + m, 2, (m, k), 1.0)
    xf, y = run(w, x, dev)
    check_close(oracle_linear(O, fmt, b, n, k, xf), y.cpu().numpy(), f"{fmt} random n={n} k={k} m={m}")


@pytest.mark.parametrize("fmt", ["q8_0", "q6_k"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
@pytest.mark.parametrize("m", [12, 64, 200, 320])
def test_gemm_blk_quantized(O, dev, fmt, xdt, m):
    import nn_amd
    n, k = 520, 4096
    b = quantized_weight_bytes(fmt, n, k, seed=m + 3, O=O)
    w = make_weight(fmt, b, n, k)
    xf, y = run(w, nn_amd.synth_normal(m, 5, (m, k), 1.0), dev, xdt)
    check_close(oracle_linear(O, fmt, b, n, k, xf), y.cpu().numpy(), f"{fmt} quantized m={m} x={xdt}")


@pytest.mark.parametrize("k", [320, 2880, 4128])
@pytest.mark.parametrize("m,xdt", [(9, "f32"), (40, "bf16"), (128, "f32")])
def test_gemm_q8_0_padded_blocks(O, dev, k, m, xdt):
    """Block counts 10, 90 and 129: the device rows are padded to groups of 8 blocks,
    whose activation columns the kernel zero-fills."""
    import nn_amd
    n = 96
    b = quantized_weight_bytes("q8_0", n, k, seed=k + m, O=O)
    w = make_weight("q8_0", b, n, k)
    xf, y = run(w, nn_amd.synth_normal(k + m, 2, (m, k), 1.0), dev, xdt)
    check_close(oracle_linear(O, "q8_0", b, n, k, xf), y.cpu().numpy(), f"q8_0 padded k={k} m={m} x={xdt}")


@pytest.mark.parametrize("fmt", ["q8_0", "q6_k"])
def test_gemm_blk_bias_and_bf16_out(O, dev, fmt):
    import nn_amd
    n, k, m = 200, 1024, 24
    b = quantized_weight_bytes(fmt, n, k, seed=17, O=O)
    w = make_weight(fmt, b, n, k)
    bias = torch.from_numpy(nn_amd.synth_normal(3, 3, (n,), 0.5)).to(dev)
    x = nn_amd.synth_normal(11, 2, (m, k), 1.0)
    xf, y32 = run(w, x, dev, "bf16", bias)
    _, yb = run(w, x, dev, "bf16", bias, out_dtype=torch.bfloat16)
    ref = oracle_linear(O, fmt, b, n, k, xf) + bias.cpu().numpy()
    check_close(ref, y32.cpu().numpy(), f"{fmt} bias")
    # the bf16 store is the f32 result rounded once
    yb_f = yb.float().cpu().numpy()
    assert np.array_equal(yb_f, y32.to(torch.bfloat16).float().cpu().numpy())


@pytest.mark.parametrize("fmt", ["q8_0", "q6_k"])
def test_gemv_gemm_crossover_consistent(O, dev, fmt):
    """Rows 0..7 of a 9-token call (GEMM) agree with the same rows as an 8-token call
    (decode GEMV passes), both within the bars of the oracle."""
    import nn_amd
    n, k = 160, 2048
    b = quantized_weight_bytes(fmt, n, k, seed=23, O=O)
    w = make_weight(fmt, b, n, k)
    x = nn_amd.synth_normal(5, 2, (9, k), 1.0)
    _, y9 = run(w, x, dev)
    _, y8 = run(w, x[:8].copy(), dev)
    ref = oracle_linear(O, fmt, b, n, k, x)
    check_close(ref, y9.cpu().numpy(), f"{fmt} m=9")
    check_close(ref[:8], y8.cpu().numpy(), f"{fmt} m=8")


@pytest.mark.parametrize("fmt", ["q8_0", "q6_k"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_gemm_blk_tall_tiles(O, dev, fmt, xdt):
    """From 1024 rows on the tiles are 128 rows high (f32 input: two staged planes, the
    largest LDS footprint); 1100 rows leave a ragged last tile."""
    import nn_amd
    n, k, m = 96, 512, 1100
    b = quantized_weight_bytes(fmt, n, k, seed=29, O=O)
    w = make_weight(fmt, b, n, k)
    xf, y = run(w, nn_amd.synth_normal(m, 7, (m, k), 1.0), dev, xdt)
    check_close(oracle_linear(O, fmt, b, n, k, xf), y.cpu().numpy(), f"{fmt} m={m} x={xdt}")


@pytest.mark.parametrize("fmt,n,k,m", [("q8_0", 4096, 4096, 128), ("q6_k", 4096, 12288, 64)])
def test_gemm_blk_baseline_shapes(O, dev, fmt, n, k, m):
    """A Qwen3-8B-sized Q8_0 projection and the Q6_K ffn_down of Q4_K_M-style models."""
    import nn_amd
    b = quantized_weight_bytes(fmt, n, k, seed=n + m, O=O)
    w = make_weight(fmt, b, n, k)
    xf, y = run(w, nn_amd.synth_normal(m, 9, (m, k), 1.0), dev, "bf16")
    check_close(oracle_linear(O, fmt, b, n, k, xf), y.cpu().numpy(), f"{fmt} {n}x{k} m={m}")


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k"])
def test_gemm_row_chunks(O, dev, fmt):
    """A batch whose f32 activations pass 2^31 bytes per two planes (17000 x 32768) runs as
    launches of gemm_chunk_rows rows (16128 here) that share one scratch: rows at the
    start, across the chunk boundary and at the end match the oracle."""
    import nn_amd
    m, n, k = 17000, 64, 32768
    b = quantized_weight_bytes(fmt, n, k, seed=97, O=O)
    w = make_weight(fmt, b, n, k)
    g = torch.Generator(device=dev).manual_seed(97)
    x = torch.randn((m, k), device=dev, generator=g)
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    for r0 in (0, 16100, m - 64):
        xs = x[r0:r0 + 64].cpu().numpy()
        check_close(oracle_linear(O, fmt, b, n, k, xs), y[r0:r0 + 64], f"{fmt} rows {r0}..{r0 + 63} of {m}")
    del x
    torch.cuda.empty_cache()


# The Q8_0 wide kernel (nnq_gemm_wide8.hip: bf16 activations, more than 128 rows, K a
# multiple of 256): 2 or 4 column tiles per workgroup, the K range split in two (slab sum)
# when the workgroups alone would leave CUs idle, partial row tiles, random block bytes.
@pytest.mark.parametrize("m,n,k", [(300, 4096, 4096), (512, 4096, 4096), (700, 1024, 2048), (129, 2048, 12288),
                                   (1000, 768, 256), (260, 12288, 4096), (1100, 320, 1024)])
def test_gemm_q80_wide(O, dev, m, n, k):
    import nn_amd
    b = rand_bytes("q8_0", n, k, seed=m + n + k)
    w = make_weight("q8_0", b, n, k)
    x = nn_amd.synth_normal(m + 5, 2, (m, k), 1.0)
    bias = torch.from_numpy(nn_amd.synth_normal(m, 3, (n,), 0.5)).to(dev)
    xt = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    y = nn_amd.quantized_linear(xt, w, bias)
    assert torch.equal(y, nn_amd.quantized_linear(xt, w, bias)), "not deterministic"
    ref = oracle_linear(O, "q8_0", b, n, k, xt.float().cpu().numpy()) + bias.cpu().numpy()
    check_close(ref, y.cpu().numpy(), f"q8_0 wide {m}x{n}x{k}")
    # the bf16 output is the f32 result rounded once
    yb = nn_amd.quantized_linear(xt, w, bias, out_dtype=torch.bfloat16)
    assert torch.equal(yb, y.to(torch.bfloat16)), "bf16 output is not the f32 result rounded once"
