"""GPU parity for the quantized linear path (decode GEMV, dequant, LM-head argmax).

The HIP kernels run through the C ABI (nn_amd -> libnnq.so) and are compared with
the CPU oracle on the same bytes and activations:
  * dequantization: bit-exact (f32 bit patterns equal);
  * linear outputs: normwise max|y - ref| / max|ref| <= 1e-3, elementwise max
    relative error <= 1e-3 over outputs with |ref| >= ABS_TOL_FRAC * max|ref|
    (nn-reftest's near-zero skip, crates/nn-reftest/src/compare.rs:95-100), and
    per-row cosine >= 0.99999 (f64, compare.rs:113-124);
  * argmax: identical index.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
ABS_TOL_FRAC = 1e-2
COS_MIN = 0.99999


@pytest.fixture(scope="module", autouse=True)
def dev():
    import nn_amd
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nn_amd.init(0)
    return torch.device("cuda:0")


def rand_bytes(fmt, n, k, seed):
    """Random block bytes with finite f16 scales (all other bits random)."""
    rng = np.random.default_rng(seed)
    if fmt == "q8_0":
        b = rng.integers(0, 256, (n * k // 32, 34), dtype=np.uint8)
        b[:, 0:2] = (b[:, 0:2].copy().view(np.uint16) & 0x7BFF).view(np.uint8)
    elif fmt == "q4_k":
        b = rng.integers(0, 256, (n * k // 256, 144), dtype=np.uint8)
        b[:, 0:4] = (b[:, 0:4].copy().view(np.uint16) & 0x7BFF).view(np.uint8)
    else:
        b = rng.integers(0, 256, (n * k // 256, 210), dtype=np.uint8)
        b[:, 208:210] = (b[:, 208:210].copy().view(np.uint16) & 0x7BFF).view(np.uint8)
    return b.ravel()


def quantized_weight_bytes(fmt, n, k, seed, O):
    import nn_amd
    w = nn_amd.synth_normal(seed, 1, (n, k), 0.02)
    if fmt == "q8_0":
        return O.quantize_q8_0(w)
    if fmt in ("q4_k", "q4_k_legacy"):
        return O.quantize_q4_k(w)
    return O.quantize_q6_k(w)


QT = {"q8_0": (8, 0), "q4_k": (12, 0), "q4_k_legacy": (12, 1), "q6_k": (14, 1)}


def oracle_dequant(O, fmt, b, count):
    return {"q8_0": O.dequant_q8_0, "q4_k": O.dequant_q4_k, "q4_k_legacy": O.dequant_q4_k_legacy,
            "q6_k": O.dequant_q6_k}[fmt](b, count)


def oracle_linear(O, fmt, b, n, k, x):
    x = np.asarray(x, np.float32).reshape(-1, k)
    if fmt == "q8_0":
        return O.q8_0_matmul(x, b, n)
    wf = oracle_dequant(O, fmt, b, n * k).reshape(n, k)
    return O.matmul_xwt(x, wf)


def make_weight(fmt, b, n, k):
    import nn_amd
    qt, lay = QT[fmt]
    return nn_amd.QuantizedWeight.from_quantized(b, qt, (n, k), layout=lay)


def check_close(ref, got, what):
    import oracle.oracle as Ox
    ref = np.asarray(ref, np.float32).reshape(-1, ref.shape[-1])
    got = np.asarray(got, np.float32).reshape(ref.shape)
    peak = float(np.abs(ref).max())
    m = Ox.compare(ref, got, abs_tol=ABS_TOL_FRAC * peak)
    cos = Ox.row_cosines(ref, got)
    # the share of outputs below the elementwise bar's floor (normwise and cosine cover them)
    skipped = float((np.abs(ref) < ABS_TOL_FRAC * peak).mean())
    print(f"{what}: normwise={m['normwise']:.2e} max_rel={m['max_rel']:.2e} min_row_cos={cos.min():.8f} "
          f"elementwise-skipped={skipped:.2%}")
    assert np.isfinite(got).all(), what
    assert m["normwise"] <= REL_TOL, what
    assert m["max_rel"] <= REL_TOL, what
    assert cos.min() >= COS_MIN, what


# ---------------------------------------------------------------------------------
# dequantization: bit-exact
# ---------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt,n,k", [("q8_0", 37, 320), ("q8_0", 16, 4128), ("q4_k", 37, 512), ("q4_k", 64, 4096),
                                     ("q4_k_legacy", 33, 768), ("q6_k", 37, 512), ("q6_k", 17, 2048)])
def test_dequant_bit_exact(O, fmt, n, k):
    b = rand_bytes("q4_k" if fmt == "q4_k_legacy" else fmt, n, k, seed=n * 7 + k)
    w = make_weight(fmt, b, n, k)
    got = w.dequantize().cpu().numpy()
    ref = oracle_dequant(O, fmt, b, n * k).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_q4k_reference_known_block(O):
    # crates/nn-gguf/src/dequant.rs:764-818 block through both Q4_K layouts
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[4] = 0x02
    blk[16:32] = 0x33
    b = np.tile(blk, 2)
    leg = make_weight("q4_k_legacy", b, 1, 512).dequantize().cpu().numpy()[0]
    gg = make_weight("q4_k", b, 1, 512).dequantize().cpu().numpy()[0]
    assert np.all(leg[:32] == 6.0) and np.all(leg[32:256] == 0.0)
    assert np.all(gg[:16] == 6.0) and np.all(gg[16:256] == 0.0)


# ---------------------------------------------------------------------------------
# linear / GEMV parity
# ---------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q4_k_legacy", "q6_k"])
@pytest.mark.parametrize("n,k", [(48, 256), (37, 1024), (300, 4096)])
@pytest.mark.parametrize("m", [1, 2, 3, 8])
def test_linear_small(O, dev, fmt, n, k, m):
    import nn_amd
    b = quantized_weight_bytes(fmt, n, k, seed=1000 + n + k, O=O)
    if fmt == "q4_k_legacy":
        b = rand_bytes("q4_k", n, k, seed=n + k)  # legacy bytes: random blocks decode under the nn-gguf layout
    w = make_weight(fmt, b, n, k)
    x = nn_amd.synth_normal(7 + m, 2, (m, k), 1.0)
    y = nn_amd.quantized_linear(torch.from_numpy(x).to(dev), w).cpu().numpy()
    ref = oracle_linear(O, fmt, b, n, k, x)
    check_close(ref, y, f"{fmt} n={n} k={k} m={m}")


@pytest.mark.parametrize("k", [320, 2880, 4128])
@pytest.mark.parametrize("m", [1, 2, 3, 8, 12])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_linear_q8_0_padded_blocks(O, dev, k, m, xdt):
    """Q8_0 rows whose block count is not a multiple of 8 (10, 90 and 129 blocks): the
    device layout pads each row to whole 8-block groups, which must add nothing.  2880
    is GPT-OSS's hidden size; m = 12 runs an 8-token and a 4-token pass."""
    import nn_amd
    n = 80
    b = quantized_weight_bytes("q8_0", n, k, seed=k + m, O=O)
    w = make_weight("q8_0", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(k + m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    ref = oracle_linear(O, "q8_0", b, n, k, x.float().cpu().numpy())
    check_close(ref, y, f"q8_0 padded k={k} m={m} x={xdt}")


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("n,k,m,xdt", [(16385, 1024, 1, "f32"), (16385, 4096, 2, "f32"), (20000, 2048, 2, "bf16"),
                                       (40000, 256, 1, "bf16")])
def test_linear_streaming_many_tiles(O, dev, fmt, n, k, m, xdt):
    """Decode GEMV over at least four tiles per CU (the streaming form that stages x
    once per workgroup and prefetches the next tile): ragged last tile, m = 1 and 2,
    f32 and bf16 x, bias, and the fused argmax over the same launch."""
    import nn_amd
    b = quantized_weight_bytes(fmt, n, k, seed=31 + n + k, O=O)
    w = make_weight(fmt, b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(17 + m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    bias = nn_amd.synth_normal(5, 3, (n,), 0.5)
    y = nn_amd.quantized_linear(x, w, torch.from_numpy(bias).to(dev)).cpu().numpy()
    ref = oracle_linear(O, fmt, b, n, k, x.float().cpu().numpy()) + bias[None, :]
    check_close(ref, y, f"{fmt} streaming n={n} k={k} m={m} x={xdt}")
    if m == 1:
        logits, idx = nn_amd.linear_argmax(x[0].float(), w)
        ref0 = oracle_linear(O, fmt, b, n, k, x[0:1].float().cpu().numpy())[0]
        check_close(ref0[None], logits.cpu().numpy()[None], f"{fmt} streaming logits")
        assert int(idx) == O.argmax(ref0)


@pytest.mark.parametrize("k", [768, 1536, 2560, 6144, 16384, 20480])
@pytest.mark.parametrize("m,xdt", [(1, "f32"), (2, "f32"), (1, "bf16"), (2, "bf16"), (3, "f32"), (4, "bf16")])
def test_q4k_decode_launch_shapes(O, dev, k, m, xdt):
    """Every decode launch shape: K of 3, 6, 10, 24, 64 and 80 units (one wave with a
    partial second unit, one and several passes), a 37-row tail tile, f32 and bf16 x,
    one, two and (four token rows) three and four tokens."""
    import nn_amd
    n = 37
    b = quantized_weight_bytes("q4_k", n, k, seed=77 + k, O=O)
    w = make_weight("q4_k", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(11 + m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    ref = oracle_linear(O, "q4_k", b, n, k, x.float().cpu().numpy())
    check_close(ref, y, f"q4_k decode n={n} k={k} m={m} x={xdt}")


@pytest.mark.parametrize("fmt,m,xdt", [("q4_k", 5, "bf16"), ("q4_k", 6, "bf16"), ("q4_k", 8, "bf16"), ("q4_k", 6, "f32"),
                                       ("q4_k", 7, "f32"), ("q4_k", 9, "f32"), ("q4_k", 4, "bf16"), ("q4_k", 3, "bf16"),
                                       ("q4_k", 2, "bf16"),
                                       ("q6_k", 6, "f32"), ("q6_k", 7, "bf16"), ("q6_k", 8, "f32"), ("q8_0", 8, "bf16"),
                                       ("q8_0", 12, "f32"), ("q8_0", 16, "f32"), ("q8_0", 17, "f32"), ("q8_0", 5, "bf16"),
                                       ("q6_k", 3, "bf16"), ("q6_k", 9, "bf16"), ("q6_k", 5, "f32")])
def test_linear_gemm_crossover(O, dev, fmt, m, xdt):
    """Batches on both sides of each format's GEMV-to-GEMM crossover (Q4_K from 3 tokens
    with bf16 activations and from 9 with f32 ones, Q6_K from 9, Q8_0 from 9 with bf16
    and from 17 with f32 ones; smaller Q8_0 and Q6_K batches run the batched decode
    kernels in passes of 8 and 4 tokens), with a ragged tile."""
    import nn_amd
    n, k = 200, 1024
    b = quantized_weight_bytes(fmt, n, k, seed=300 + m, O=O)
    w = make_weight(fmt, b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(29 + m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    ref = oracle_linear(O, fmt, b, n, k, x.float().cpu().numpy())
    check_close(ref, y, f"{fmt} crossover m={m} x={xdt}")


@pytest.mark.parametrize("k", [1024, 2048, 4096, 6144, 8192, 12288, 16384])
@pytest.mark.parametrize("m,xdt", [(1, "f32"), (2, "f32"), (1, "bf16"), (2, "bf16")])
def test_q6k_decode_launch_shapes(O, dev, k, m, xdt):
    """Every Q6_K decode launch shape: K of 4, 8, 16, 24, 32, 48 and 64 units (one and
    two passes), a 37-row tail tile, f32 and bf16 x, with a bias."""
    import nn_amd
    n = 37
    b = quantized_weight_bytes("q6_k", n, k, seed=57 + k, O=O)
    w = make_weight("q6_k", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(19 + m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    bias = nn_amd.synth_normal(7, 3, (n,), 0.5)
    y = nn_amd.quantized_linear(x, w, torch.from_numpy(bias).to(dev)).cpu().numpy()
    ref = oracle_linear(O, "q6_k", b, n, k, x.float().cpu().numpy()) + bias[None, :]
    check_close(ref, y, f"q6_k decode n={n} k={k} m={m} x={xdt}")


@pytest.mark.parametrize("k", [1024, 2048, 2080, 4096, 6144, 8192, 12288, 16416])
@pytest.mark.parametrize("m,xdt", [(1, "f32"), (2, "f32"), (1, "bf16"), (2, "bf16")])
def test_q80_decode_launch_shapes(O, dev, k, m, xdt):
    """Every Q8_0 decode launch shape: K of 4, 8, 16, 24, 32 and 48 units, 2080 (9
    units, the last one padded: 65 blocks) and 16416 (65 units: two passes, the second
    partial and padded), a 37-row tail tile, f32 and bf16 x."""
    import nn_amd
    n = 37
    b = quantized_weight_bytes("q8_0", n, k, seed=91 + k, O=O)
    w = make_weight("q8_0", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(13 + m, 2, (m, k), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    ref = oracle_linear(O, "q8_0", b, n, k, x.float().cpu().numpy())
    check_close(ref, y, f"q8_0 decode n={n} k={k} m={m} x={xdt}")


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
def test_linear_bf16_in_out_bias(O, dev, fmt):
    import nn_amd
    n, k, m = 200, 2048, 2
    b = quantized_weight_bytes(fmt, n, k, seed=5, O=O)
    w = make_weight(fmt, b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(3, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    bias = torch.from_numpy(nn_amd.synth_normal(3, 3, (n,), 0.5)).to(dev)
    y32 = nn_amd.quantized_linear(x, w, bias)
    yb = nn_amd.quantized_linear(x, w, bias, out_dtype=torch.bfloat16)
    xf = x.float().cpu().numpy()
    ref = oracle_linear(O, fmt, b, n, k, xf) + bias.cpu().numpy()
    check_close(ref, y32.cpu().numpy(), f"{fmt} bf16-in")
    # the bf16 store is the f32 result rounded once (<= 1 bf16 ulp from round(ref))
    yb_f = yb.float().cpu().numpy()
    ref_b = torch.from_numpy(ref).to(torch.bfloat16).float().numpy()
    ulp = np.abs(ref_b) * 2.0 ** -7
    assert np.all(np.abs(yb_f - ref_b) <= ulp + 1e-30)


def test_linear_batched_rank_folding(O, dev):
    import nn_amd
    n, k = 64, 512
    b = quantized_weight_bytes("q8_0", n, k, seed=9, O=O)
    w = make_weight("q8_0", b, n, k)
    x = nn_amd.synth_normal(4, 4, (2, 3, 1, k), 1.0)
    y = nn_amd.quantized_matmul_q8_0(torch.from_numpy(x).to(dev), w)
    assert tuple(y.shape) == (2, 3, 1, n)
    check_close(oracle_linear(O, "q8_0", b, n, k, x), y.cpu().numpy(), "q8_0 4-D batch")


def test_linear_zero_rows_and_errors(dev):
    import nn_amd
    b = np.zeros(144 * 2, np.uint8)
    w = nn_amd.QuantizedWeight.from_quantized(b, nn_amd.QuantType.Q4_K, (2, 256))
    y = nn_amd.quantized_linear(torch.zeros((0, 256), device=dev), w)
    assert tuple(y.shape) == (0, 2)
    with pytest.raises(nn_amd.ShapeMismatch):
        nn_amd.quantized_linear(torch.zeros((1, 512), device=dev), w)
    with pytest.raises(nn_amd.BiasMismatch):
        nn_amd.quantized_linear(torch.zeros((1, 256), device=dev), w, torch.zeros(3, device=dev))
    with pytest.raises(nn_amd.RankMismatch):
        nn_amd.quantized_linear(torch.zeros(256, device=dev), w)
    with pytest.raises(nn_amd.WrongQuantType):
        nn_amd.quantized_matmul_q8_0(torch.zeros((1, 256), device=dev), w)


def test_linear_known_values_q8_0(dev):
    # quantized_matmul_tests.rs:150-163, 323-350: dequant 1.0 weights, ones input, bias
    import nn_amd
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2:] = 2
    w = nn_amd.QuantizedWeight.from_quantized(np.tile(blk, 2), nn_amd.QuantType.Q8_0, (2, 32))
    y = nn_amd.quantized_linear(torch.ones((1, 32), device=dev), w, torch.tensor([10.0, 20.0], device=dev))
    assert np.allclose(y.cpu().numpy(), [[42.0, 52.0]], atol=1e-4)


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0", "q6_k"])
@pytest.mark.parametrize("m", [1, 2])
def test_nan_input_propagates(O, dev, fmt, m):
    """A NaN in one token's x makes every output of that token NaN, the other
    token's outputs stay finite."""
    import nn_amd
    n, k = 32, 512
    b = quantized_weight_bytes(fmt, n, k, seed=3, O=O)
    w = make_weight(fmt, b, n, k)
    x = torch.ones((m, k), device=dev)
    x[0, 7] = float("nan")
    y = nn_amd.quantized_linear(x, w)
    assert torch.isnan(y[0]).all()
    if m == 2:
        assert torch.isfinite(y[1]).all()


# ---------------------------------------------------------------------------------
# benchmark shapes
# ---------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt,n,k", [("q8_0", 4096, 4096), ("q4_k", 4096, 12288), ("q4_k", 24576, 4096)])
def test_linear_baseline_shapes(O, dev, fmt, n, k):
    import nn_amd
    b = quantized_weight_bytes(fmt, n, k, seed=2024, O=O)
    w = make_weight(fmt, b, n, k)
    x = nn_amd.synth_normal(2024, 2, (1, k), 1.0)
    y = nn_amd.quantized_linear(torch.from_numpy(x).to(dev), w).cpu().numpy()
    check_close(oracle_linear(O, fmt, b, n, k, x), y, f"{fmt} {n}x{k}")
    # size-independent property: the dequant of the same device weight reproduces the oracle decode
    got = w.dequantize()
    ref = torch.from_numpy(oracle_dequant(O, fmt, b, n * k).reshape(n, k)).to(dev)
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))


def test_lm_head_q6k_argmax_full(O, dev):
    """Config 3: Q6_K LM head 151936 x 4096, logits within tolerance, argmax bit-exact."""
    import nn_amd
    n, k = 151936, 4096
    b = quantized_weight_bytes("q6_k", n, k, seed=3, O=O)
    w = make_weight("q6_k", b, n, k)
    x = nn_amd.synth_normal(3, 2, (k,), 1.0)
    logits, idx = nn_amd.linear_argmax(torch.from_numpy(x).to(dev), w)
    ref = oracle_linear(O, "q6_k", b, n, k, x)[0]
    check_close(ref[None], logits.cpu().numpy()[None], "q6_k lm head")
    top2 = np.sort(ref)[-2:]
    print(f"argmax oracle={O.argmax(ref)} gpu={int(idx)} margin={top2[1] - top2[0]:.3e}")
    assert int(idx) == O.argmax(ref)


def test_argmax_semantics(dev):
    import nn_amd
    v = torch.tensor([1.0, 3.0, 3.0, 2.0], device=dev)
    assert int(nn_amd.argmax(v)) == 1
    assert int(nn_amd.argmax(torch.full((1000,), -float("inf"), device=dev))) == 0
    v = torch.randn(100_003, device=dev)
    v[77_777] = 10.0
    v[99_999] = 10.0
    assert int(nn_amd.argmax(v)) == 77_777
    v[5] = float("nan")
    with pytest.raises(nn_amd.NonFiniteData):
        nn_amd.argmax(v)


def test_lm_head_argmax_graph_replay(O, dev):
    """The streaming LM head (one argmax key per workgroup, then argmax_final_kernel)
    captured into a HIP graph: every replay, and eager calls with another input between
    the replays, give the oracle's index."""
    import nn_amd
    n, k = 32768, 1024
    b = quantized_weight_bytes("q6_k", n, k, seed=41, O=O)
    w = make_weight("q6_k", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(41, 2, (k,), 1.0)).to(dev)
    ref = O.argmax(oracle_linear(O, "q6_k", b, n, k, x.cpu().numpy())[0])
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            logits, idx = nn_amd.linear_argmax(x, w, check=False)  # no host read under capture
    torch.cuda.current_stream().wait_stream(s)
    x2 = torch.from_numpy(nn_amd.synth_normal(42, 2, (k,), 1.0)).to(dev)
    ref2 = O.argmax(oracle_linear(O, "q6_k", b, n, k, x2.cpu().numpy())[0])
    assert ref2 != ref
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert int(idx) == ref, f"replay {i}"
        _, i2 = nn_amd.linear_argmax(x2, w)  # eager, between the replays
        torch.cuda.synchronize()
        assert int(i2) == ref2, f"eager after replay {i}"


def test_host_bias_moves_to_the_device(O, dev):
    """A bias given as a CPU tensor is copied to the input's device (never handed to a
    kernel as a host address): every entry point with a bias gives the same result as
    with the bias already on the device."""
    import nn_amd
    n, k = 300, 1024
    b = quantized_weight_bytes("q6_k", n, k, seed=91, O=O)
    w = make_weight("q6_k", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(91, 2, (1, k), 1.0)).to(dev)
    bias_h = torch.from_numpy(nn_amd.synth_normal(91, 3, (n,), 0.5))
    bias_d = bias_h.to(dev)
    assert torch.equal(nn_amd.quantized_linear(x, w, bias_h), nn_amd.quantized_linear(x, w, bias_d))
    lh, ih = nn_amd.linear_argmax(x, w, bias_h)
    ld, idd = nn_amd.linear_argmax(x, w, bias_d)
    assert torch.equal(lh, ld) and int(ih) == int(idd)
    lh, th = nn_amd.linear_sample(x, w, bias_h, seed=5)
    ld, td = nn_amd.linear_sample(x, w, bias_d, seed=5)
    assert torch.equal(lh, ld) and int(th) == int(td)
    ref = oracle_linear(O, "q6_k", b, n, k, x.cpu().numpy()) + bias_h.numpy()
    check_close(ref, ld.cpu().numpy()[None, :], "q6_k linear + host bias")


@pytest.mark.parametrize("fmt,m", [("q4_k", 1), ("q4_k", 40), ("q6_k", 3), ("q8_0", 12)])
def test_misaligned_views(O, dev, fmt, m):
    """Narrowed views whose data pointer is not 16-byte aligned (an f32 row offset by one
    element, a bf16 one by one element) are staged through the workspace: the results
    equal those of the same values at aligned addresses, bit for bit; an output pointer
    offset by 2 bytes (bf16) is computed in the workspace and copied out."""
    import ctypes

    import nn_amd
    from nn_amd import _lib
    n, k = 256, 1024
    b = quantized_weight_bytes(fmt, n, k, seed=5 + m, O=O)
    w = make_weight(fmt, b, n, k)
    for dt in (torch.float32, torch.bfloat16):
        x = torch.from_numpy(nn_amd.synth_normal(7 + m, 2, (m, k), 1.0)).to(dev).to(dt)
        big = torch.zeros(m * k + 8, dtype=dt, device=dev)
        big[1:1 + m * k] = x.reshape(-1)
        xv = big[1:1 + m * k].view(m, k)
        assert xv.data_ptr() % 16 != 0
        assert torch.equal(nn_amd.quantized_linear(xv, w), nn_amd.quantized_linear(x, w))
        ybig = torch.zeros(m * n + 8, dtype=torch.bfloat16, device=dev)
        yv = ybig[1:1 + m * n]
        rc = _lib.load().nnq_linear(w.handle, ctypes.c_void_p(xv.data_ptr()), 2 if dt == torch.bfloat16 else 0, m, k,
                                    None, 0, ctypes.c_void_p(yv.data_ptr()), 2,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, _lib.last_error()
        ref = nn_amd.quantized_linear(x, w, out_dtype=torch.bfloat16).reshape(-1)
        assert torch.equal(yv, ref)
    if m == 1:
        x = torch.from_numpy(nn_amd.synth_normal(9, 2, (k,), 1.0)).to(dev)
        big = torch.zeros(k + 4, device=dev)
        big[1:1 + k] = x
        la, ia = nn_amd.linear_argmax(big[1:1 + k], w)
        lb, ib = nn_amd.linear_argmax(x, w)
        assert torch.equal(la, lb) and int(ia) == int(ib)
        la, ta = nn_amd.linear_sample(big[1:1 + k], w, seed=3)
        lb, tb = nn_amd.linear_sample(x, w, seed=3)
        assert torch.equal(la, lb) and int(ta) == int(tb)
