"""GPU parity for the GPT-OSS MXFP4 mixture-of-experts layer.

The device pipeline (route -> permute -> gate_up + SwiGLU -> down -> combine) runs
through the C ABI and is compared with the CPU oracle's restatement of
QuantizedDecoderLayer::moe_forward (crates/nn-gptoss/src/quantized_model.rs:99-194):
  * routing: the top-k expert sets equal per token, weights within 1e-6;
  * expert decode: bit-exact with Mxfp4Tensor::dequantize;
  * outputs: normwise and elementwise max relative error <= 1e-3 (near-zero skip at
    1% of the peak) and per-row cosine >= 0.99999.
Small layers use the oracle's own f32 forward; the benchmark layer (config 5) uses
the oracle's routing and bit-exact decode with the expert math in f64.
"""
import numpy as np
import pytest
import torch

from test_gpu_linear import check_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def dev():
    import nn_amd
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nn_amd.init(0)
    return torch.device("cuda:0")


def make_layer(E, H, I, seed):
    import nn_amd
    wgu = nn_amd.synth_normal(seed, 1, (E, H, 2 * I), 0.02)
    wdn = nn_amd.synth_normal(seed, 2, (E, I, H), 0.02)
    gp, gs = nn_amd.quantize_mxfp4(wgu)
    dp, ds = nn_amd.quantize_mxfp4(wdn)
    gb = nn_amd.synth_normal(seed, 3, (E, 2 * I), 0.02)
    db = nn_amd.synth_normal(seed, 4, (E, H), 0.02)
    return dict(gp=gp, gs=gs, gb=gb, dp=dp, ds=ds, db=db)


def upload(L, E, H, I):
    import nn_amd
    return nn_amd.QuantizedMoE(E, H, I, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"])


def ref_f64(O, x, logits, k, L, E, H, I, limit=7.0):
    """moe_forward with the oracle's routing and decode, expert math in f64."""
    probs = O.softmax_rows(logits)
    tw, ti = O.topk_rows(probs, k)
    tw = (tw / tw.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    out = np.zeros((x.shape[0], H), np.float64)
    gper, dper = H * 2 * I, I * H
    for e in range(E):
        rows = [(t, s) for t in range(x.shape[0]) for s in range(k) if ti[t, s] == e]
        if not rows:
            continue
        toks = np.array([t for t, _ in rows])
        w = np.array([tw[t, s] for t, s in rows], np.float64)
        Wg = O.mxfp4_dequantize(L["gp"][e * gper // 2:(e + 1) * gper // 2], L["gs"][e * gper // 32:(e + 1) * gper // 32],
                                gper).reshape(H, 2 * I).astype(np.float64)
        Wd = O.mxfp4_dequantize(L["dp"][e * dper // 2:(e + 1) * dper // 2], L["ds"][e * dper // 32:(e + 1) * dper // 32],
                                dper).reshape(I, H).astype(np.float64)
        gu = x[toks].astype(np.float64) @ Wg + L["gb"][e].astype(np.float64)
        g, u = gu[:, :I], gu[:, I:]
        h = np.clip(g / (1.0 + np.exp(-g)), -limit, limit) * u
        y = h @ Wd + L["db"][e].astype(np.float64)
        out[toks] += w[:, None] * y
    return out.astype(np.float32), ti, tw


# Shapes cover the expert kernel's variants: chunks of 3 k-blocks (K / 32 divisible by
# 3) or 1, scales staged in LDS or (K too long for LDS: 5120-wide gate_up input,
# 9600-wide down input) loaded beside the codes, bf16 and f32 (hi + lo) activations.
@pytest.mark.parametrize("E,H,I,T,k,xdt", [(4, 64, 64, 24, 2, "f32"), (8, 256, 320, 64, 4, "bf16"),
                                          (8, 256, 320, 64, 4, "f32"), (6, 128, 96, 40, 3, "bf16"),
                                          (16, 96, 64, 150, 4, "bf16"), (3, 96, 96, 70, 2, "f32"),
                                          (2, 5120, 64, 8, 2, "bf16"), (1, 64, 9600, 4, 1, "f32")])
def test_moe_small_vs_oracle(O, dev, E, H, I, T, k, xdt):
    import nn_amd
    L = make_layer(E, H, I, seed=E * 7 + H)
    moe = upload(L, E, H, I)
    x = torch.from_numpy(nn_amd.synth_normal(9, 5, (T, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    logits = torch.from_numpy(nn_amd.synth_normal(9, 6, (T, E), 1.0)).to(dev)
    y, ti, tw = moe.forward(x, logits, top_k=k, return_routing=True)
    xf = x.float().cpu().numpy()
    ref, rti, rtw = O.moe_forward(xf, logits.cpu().numpy(), k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    gti = ti.cpu().numpy().astype(np.uint32)
    assert np.array_equal(np.sort(gti, axis=1), np.sort(rti, axis=1)), "routing expert sets differ"
    assert np.array_equal(gti, rti), "routing order differs"
    assert np.allclose(tw.cpu().numpy(), rtw, rtol=1e-6, atol=1e-7)
    check_close(ref, y.cpu().numpy(), f"moe E={E} H={H} I={I} T={T} k={k} x={xdt}")


# Uneven loads: a large logit on expert 0 sends every token there (more than 64 rows:
# several passes of the expert kernel over its token rows, the last one partial), and a
# single decode token (one row per expert used).
@pytest.mark.parametrize("E,H,I,T,k,xdt,skew", [(8, 256, 320, 200, 2, "bf16", True), (4, 96, 96, 130, 1, "f32", True),
                                               (8, 256, 320, 1, 4, "f32", False), (32, 96, 64, 1, 4, "bf16", False)])
def test_moe_uneven_loads_vs_oracle(O, dev, E, H, I, T, k, xdt, skew):
    import nn_amd
    L = make_layer(E, H, I, seed=E * 11 + T)
    moe = upload(L, E, H, I)
    x = torch.from_numpy(nn_amd.synth_normal(13, 5, (T, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    lg = nn_amd.synth_normal(13, 6, (T, E), 1.0)
    if skew:
        lg[:, 0] += 12.0
    logits = torch.from_numpy(lg).to(dev)
    y, ti, tw = moe.forward(x, logits, top_k=k, return_routing=True)
    ref, rti, rtw = O.moe_forward(x.float().cpu().numpy(), lg, k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    counts = np.bincount(rti.ravel(), minlength=E)
    if skew:
        assert counts[0] == T and T > 64, "every token routed to expert 0, more than one 64-row pass"
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), rti), "routing differs"
    assert np.allclose(tw.cpu().numpy(), rtw, rtol=1e-6, atol=1e-7)
    check_close(ref, y.cpu().numpy(), f"moe uneven E={E} H={H} I={I} T={T} k={k} x={xdt} skew={skew}")


# More than 256 experts (Kimi-K2-style 384, odd counts, a batch over two 1024-token
# permutation chunks): routing keeps the token's probabilities in LDS, the permutation
# walks the experts in groups of 256.
@pytest.mark.parametrize("E,H,I,T,k,xdt", [(384, 64, 64, 100, 8, "bf16"), (1000, 96, 64, 300, 4, "f32"),
                                          (300, 64, 64, 1100, 2, "bf16"), (257, 64, 32, 64, 6, "f32")])
def test_moe_many_experts_vs_oracle(O, dev, E, H, I, T, k, xdt):
    import nn_amd
    L = make_layer(E, H, I, seed=E + T)
    moe = upload(L, E, H, I)
    x = torch.from_numpy(nn_amd.synth_normal(17, 5, (T, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    lg = nn_amd.synth_normal(17, 6, (T, E), 1.0)
    lg[0, 5] = np.inf       # a +inf logit: uniform over the +inf entries of that token
    lg[1, : E // 2] = -np.inf  # zero probabilities for half of the experts
    lg[2, E - 1] = 40.0     # the last expert first
    logits = torch.from_numpy(lg).to(dev)
    y, ti, tw = moe.forward(x, logits, top_k=k, return_routing=True)
    ref, rti, rtw = O.moe_forward(x.float().cpu().numpy(), lg, k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), rti), "routing differs"
    assert np.allclose(tw.cpu().numpy(), rtw, rtol=1e-6, atol=1e-7)
    check_close(ref, y.cpu().numpy(), f"moe E={E} H={H} I={I} T={T} k={k} x={xdt}")


# Routing on batches across the 1024-token permutation chunk and small to medium
# expert counts, with special rows: a +inf logit, half the experts at -inf, exact ties
# that go to the lowest index, the last expert first.
@pytest.mark.parametrize("E,T,k", [(32, 512, 4), (32, 513, 4), (32, 1024, 4), (32, 1025, 4), (20, 7, 3), (33, 300, 4),
                                   (32, 1, 8), (2, 600, 2), (2, 200, 2)])
def test_moe_routing_special_rows(O, dev, E, T, k):
    import nn_amd
    H, I = 64, 32
    L = make_layer(E, H, I, seed=E * 3 + T)
    moe = upload(L, E, H, I)
    x = torch.from_numpy(nn_amd.synth_normal(19, 5, (T, H), 1.0)).to(dev).to(torch.bfloat16)
    lg = nn_amd.synth_normal(19, 6, (T, E), 2.0)
    if T > 3:
        lg[1, min(3, E - 1)] = np.inf
        lg[2, : E // 2] = -np.inf
        lg[3, :] = 0.5  # every probability equal: experts 0 .. k-1
    lg[-1, E - 1] = 40.0
    logits = torch.from_numpy(lg).to(dev)
    y, ti, tw = moe.forward(x, logits, top_k=k, return_routing=True)
    ref, rti, rtw = O.moe_forward(x.float().cpu().numpy(), lg, k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), rti), "routing differs"
    assert np.allclose(tw.cpu().numpy(), rtw, rtol=1e-6, atol=1e-7)
    if T > 3:
        assert list(rti[3]) == list(range(k))
    check_close(ref, y.cpu().numpy(), f"moe routing E={E} T={T} k={k}")


def test_moe_expert_dequant_bit_exact(O, dev):
    E, H, I = 3, 96, 64
    L = make_layer(E, H, I, seed=5)
    moe = upload(L, E, H, I)
    gper, dper = H * 2 * I, I * H
    for e in range(E):
        gu, dn = moe.dequant_expert(e)
        rg = O.mxfp4_dequantize(L["gp"][e * gper // 2:(e + 1) * gper // 2], L["gs"][e * gper // 32:(e + 1) * gper // 32],
                                gper).reshape(H, 2 * I)
        rd = O.mxfp4_dequantize(L["dp"][e * dper // 2:(e + 1) * dper // 2], L["ds"][e * dper // 32:(e + 1) * dper // 32],
                                dper).reshape(I, H)
        assert np.array_equal(gu.cpu().numpy().view(np.uint32), rg.view(np.uint32))
        assert np.array_equal(dn.cpu().numpy().view(np.uint32), rd.view(np.uint32))


def test_moe_dequant_extreme_scales(O, dev):
    """E8M0 bytes 0, 1, 127, 200 and every fp4 code decode exactly (byte 0 -> 2^-126)."""
    import nn_amd
    E, H, I = 1, 32, 32
    gp = np.arange(H * 2 * I // 2, dtype=np.uint32).astype(np.uint8)
    gs = np.array([0, 1, 127, 200] * (H * 2 * I // 32 // 4), np.uint8)
    dp = (np.arange(I * H // 2, dtype=np.uint32) * 7).astype(np.uint8)
    ds = np.array([126, 0, 128, 1] * (I * H // 32 // 4), np.uint8)
    moe = nn_amd.QuantizedMoE(E, H, I, gp, gs, np.zeros((E, 2 * I), np.float32), dp, ds,
                              np.zeros((E, H), np.float32))
    gu, dn = moe.dequant_expert(0)
    rg = O.mxfp4_dequantize(gp, gs, H * 2 * I).reshape(H, 2 * I)
    rd = O.mxfp4_dequantize(dp, ds, I * H).reshape(I, H)
    assert np.array_equal(gu.cpu().numpy().view(np.uint32), rg.view(np.uint32))
    assert np.array_equal(dn.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    assert (rg != 0).any() and (np.abs(rg[rg != 0]) < 1e-37).any(), "the case covers subnormal decodes"


def test_moe_baseline_config(O, dev):
    """Config 5: 32 experts, hidden = intermediate = 2880, top-4, 256 bf16 tokens."""
    import nn_amd
    E, H, I, T, k = 32, 2880, 2880, 256, 4
    L = make_layer(E, H, I, seed=20)
    moe = upload(L, E, H, I)
    x = torch.from_numpy(nn_amd.synth_normal(20, 5, (T, H), 1.0)).to(dev).to(torch.bfloat16)
    logits = torch.from_numpy(nn_amd.synth_normal(20, 6, (T, E), 1.0)).to(dev)
    y, ti, tw = moe.forward(x, logits, top_k=k, return_routing=True)
    ref, rti, rtw = ref_f64(O, x.float().cpu().numpy(), logits.cpu().numpy(), k, L, E, H, I)
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), rti)
    assert np.allclose(tw.cpu().numpy(), rtw, rtol=1e-6, atol=1e-7)
    counts = np.bincount(rti.ravel(), minlength=E)
    print(f"expert loads min {counts.min()} max {counts.max()}")
    check_close(ref, y.cpu().numpy(), "moe config 5")


def make_router(E, H, seed):
    import nn_amd
    return nn_amd.synth_normal(seed, 7, (E, H), 0.02), nn_amd.synth_normal(seed, 8, (E,), 0.1)


@pytest.mark.parametrize("E,H,T,xdt", [(32, 2880, 256, "bf16"), (32, 2880, 37, "f32"), (20, 96, 5, "bf16"),
                                      (384, 128, 33, "f32")])
def test_router_logits_vs_oracle(O, dev, E, H, T, xdt):
    """The router Linear on the f32 MFMA against the oracle's f32 x @ W^T + b (same
    products, another summation order): max abs difference <= 1e-5 of the peak."""
    import nn_amd
    I = 32
    L = make_layer(E, H, I, seed=E + H)
    rw, rb = make_router(E, H, seed=T)
    moe = nn_amd.QuantizedMoE(E, H, I, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"],
                              router_weight=rw, router_bias=rb)
    x = torch.from_numpy(nn_amd.synth_normal(T, 5, (T, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    got = moe.router_logits(x).cpu().numpy()
    ref = O.router_logits(x.float().cpu().numpy(), rw, rb)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), np.abs(got - ref).max()


@pytest.mark.parametrize("E,H,I,T,k,xdt", [(8, 256, 320, 64, 4, "bf16"), (16, 96, 64, 150, 4, "f32"),
                                          (32, 2880, 2880, 256, 4, "bf16"), (300, 64, 64, 40, 4, "f32")])
def test_moe_block_vs_oracle(O, dev, E, H, I, T, k, xdt):
    """moe_forward with its router: device logits, routing, experts and combine against
    the oracle's router Linear followed by its moe_forward restatement."""
    import nn_amd
    L = make_layer(E, H, I, seed=E * 3 + H)
    rw, rb = make_router(E, H, seed=E + T)
    moe = nn_amd.QuantizedMoE(E, H, I, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"],
                              router_weight=rw, router_bias=rb)
    x = torch.from_numpy(nn_amd.synth_normal(T + 1, 5, (T, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    y, ti, tw = moe.block_forward(x, top_k=k, return_routing=True)
    xf = x.float().cpu().numpy()
    logits = O.router_logits(xf, rw, rb)
    if H * I > 100000:
        ref, rti, rtw = ref_f64(O, xf, logits, k, L, E, H, I)
    else:
        ref, rti, rtw = O.moe_forward(xf, logits, k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), rti), "routing differs"
    assert np.allclose(tw.cpu().numpy(), rtw, rtol=1e-5, atol=1e-6)
    check_close(ref, y.cpu().numpy(), f"moe block E={E} H={H} I={I} T={T} k={k} x={xdt}")


# top_k above 8 (experts_per_token up to the expert count, quantized_model.rs:92,141):
# the general routing path (E <= 256 and E > 256), the general permutation (batches over
# 1024 tokens), the general combine, and k = E.
@pytest.mark.parametrize("E,H,I,T,k,xdt", [(32, 96, 64, 40, 16, "bf16"), (24, 64, 64, 1100, 12, "f32"),
                                          (300, 64, 64, 30, 20, "bf16"), (16, 64, 64, 50, 16, "f32")])
def test_moe_top_k_above_8(O, dev, E, H, I, T, k, xdt):
    import nn_amd
    L = make_layer(E, H, I, seed=E * 5 + k)
    rw, rb = make_router(E, H, seed=E + k)
    moe = nn_amd.QuantizedMoE(E, H, I, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"],
                              router_weight=rw, router_bias=rb)
    x = torch.from_numpy(nn_amd.synth_normal(k + 3, 5, (T, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    xf = x.float().cpu().numpy()
    logits = torch.from_numpy(nn_amd.synth_normal(k + 3, 6, (T, E), 1.0)).to(dev)
    y, ti, tw = moe.forward(x, logits, top_k=k, return_routing=True)
    ref, rti, rtw = O.moe_forward(xf, logits.cpu().numpy(), k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), rti), "routing differs"
    assert np.allclose(tw.cpu().numpy(), rtw, rtol=1e-6, atol=1e-7)
    check_close(ref, y.cpu().numpy(), f"moe E={E} T={T} k={k} x={xdt}")
    yb, tib, twb = moe.block_forward(x, top_k=k, return_routing=True)
    lg = O.router_logits(xf, rw, rb)
    refb, rtib, rtwb = O.moe_forward(xf, lg, k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    assert np.array_equal(tib.cpu().numpy().astype(np.uint32), rtib), "block routing differs"
    assert np.allclose(twb.cpu().numpy(), rtwb, rtol=1e-5, atol=1e-6)
    check_close(refb, yb.cpu().numpy(), f"moe block E={E} T={T} k={k} x={xdt}")


def test_moe_block_nonfinite_raises(O, dev):
    import nn_amd
    E, H, I, T = 4, 64, 64, 6
    L = make_layer(E, H, I, seed=3)
    rw, rb = make_router(E, H, seed=3)
    moe = nn_amd.QuantizedMoE(E, H, I, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"],
                              router_weight=rw, router_bias=rb)
    x = torch.from_numpy(nn_amd.synth_normal(3, 5, (T, H), 1.0)).to(dev)
    moe.block_forward(x, top_k=2)
    x[2, 5] = float("nan")
    with pytest.raises(nn_amd.NonFiniteData):
        moe.block_forward(x, top_k=2)
    x[2, 5] = 1.0
    moe.block_forward(x, top_k=2)  # the status is cleared by every call


# ---- nn-core OCP MXFP4 layout (crates/nn-core/src/layers/quantized/mxfp4.rs) -------------


def test_ocp_dequant_bit_exact(O, dev):
    """nnq_dequant_mxfp4_ocp against the oracle's dequantize_tensor, f32 bit patterns
    equal: random codes under every shared_exp 0..254 (byte 0 is 2^-127, subnormal
    results included), a length that ends inside a block; shared_exp 255 scales by +inf
    (infinities equal, NaN where the code is a zero)."""
    import nn_amd
    rng = np.random.default_rng(11)
    nb = 255 * 4
    blocks = rng.integers(0, 256, (nb, 17), dtype=np.uint8)
    blocks[:, 0] = np.arange(nb) % 255
    n = nb * 32 - 13
    got = nn_amd.dequantize_mxfp4_ocp(blocks.ravel(), n).cpu().numpy()
    ref = O.ocp_dequantize(blocks.ravel(), n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    inf_blocks = rng.integers(0, 256, (8, 17), dtype=np.uint8)
    inf_blocks[:, 0] = 255
    got = nn_amd.dequantize_mxfp4_ocp(inf_blocks.ravel(), 256).cpu().numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        ref = O.ocp_dequantize(inf_blocks.ravel(), 256)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])


def make_layer_ocp(E, H, I, seed):
    import nn_amd
    gb_ = nn_amd.quantize_mxfp4_ocp(nn_amd.synth_normal(seed, 1, (E, H, 2 * I), 0.02))
    db_ = nn_amd.quantize_mxfp4_ocp(nn_amd.synth_normal(seed, 2, (E, I, H), 0.02))
    return dict(gblk=gb_, dblk=db_, gb=nn_amd.synth_normal(seed, 3, (E, 2 * I), 0.02),
                db=nn_amd.synth_normal(seed, 4, (E, H), 0.02))


def ref_f64_ocp(O, x, logits, k, L, E, H, I, limit=7.0):
    """moe_forward with the oracle's routing and the OCP decode, expert math in f64."""
    probs = O.softmax_rows(logits)
    tw, ti = O.topk_rows(probs, k)
    tw = (tw / tw.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    out = np.zeros((x.shape[0], H), np.float64)
    gper, dper = H * 2 * I, I * H
    Wg_all = O.ocp_dequantize(L["gblk"], E * gper).reshape(E, H, 2 * I).astype(np.float64)
    Wd_all = O.ocp_dequantize(L["dblk"], E * dper).reshape(E, I, H).astype(np.float64)
    for e in range(E):
        rows = [(t, s) for t in range(x.shape[0]) for s in range(k) if ti[t, s] == e]
        if not rows:
            continue
        toks = np.array([t for t, _ in rows])
        w = np.array([tw[t, s] for t, s in rows], np.float64)
        gu = x[toks].astype(np.float64) @ Wg_all[e] + L["gb"][e].astype(np.float64)
        g, u = gu[:, :I], gu[:, I:]
        h = np.clip(g / (1.0 + np.exp(-g)), -limit, limit) * u
        out[toks] += w[:, None] * (h @ Wd_all[e] + L["db"][e].astype(np.float64))
    return out.astype(np.float32), ti, tw


@pytest.mark.parametrize("E,H,I,T,k,xdt", [(8, 256, 320, 64, 4, "bf16"), (6, 128, 96, 40, 3, "f32"),
                                          (4, 96, 64, 130, 2, "bf16")])
def test_moe_ocp_vs_oracle(O, dev, E, H, I, T, k, xdt):
    """The MoE layer on nn-core OCP MXFP4 experts (nnq_moe_create_ocp): routing equal to
    the oracle's, outputs within the linear bars of the oracle's OCP decode with the
    expert math in f64, and each expert's device decode bit-exact with dequantize_tensor,
    with some blocks forced to shared_exp 0 (2^-127)."""
    import nn_amd
    L = make_layer_ocp(E, H, I, seed=E * 5 + I)
    L["gblk"].reshape(-1, 17)[::97, 0] = 0
    moe = nn_amd.QuantizedMoE.from_ocp(E, H, I, L["gblk"], L["gb"], L["dblk"], L["db"])
    x = torch.from_numpy(nn_amd.synth_normal(13, 5, (T, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    logits = torch.from_numpy(nn_amd.synth_normal(13, 6, (T, E), 1.0)).to(dev)
    y, ti, tw = moe.forward(x, logits, top_k=k, return_routing=True)
    ref, rti, rtw = ref_f64_ocp(O, x.float().cpu().numpy(), logits.cpu().numpy(), k, L, E, H, I)
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), rti), "routing differs"
    assert np.allclose(tw.cpu().numpy(), rtw, rtol=1e-6, atol=1e-7)
    check_close(ref, y.cpu().numpy(), f"moe ocp E={E} H={H} I={I} T={T} k={k} x={xdt}")
    gper, dper = H * 2 * I, I * H
    Wg = O.ocp_dequantize(L["gblk"], E * gper).reshape(E, H, 2 * I)
    Wd = O.ocp_dequantize(L["dblk"], E * dper).reshape(E, I, H)
    for e in (0, E - 1):
        gu, dn = moe.dequant_expert(e)
        assert np.array_equal(gu.cpu().numpy().view(np.uint32), Wg[e].view(np.uint32))
        assert np.array_equal(dn.cpu().numpy().view(np.uint32), Wd[e].view(np.uint32))


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_moe_long_batch_chunks(O, dev, xdt):
    """Beyond 16384 token-expert assignments the layer runs in token chunks: 4500 tokens
    at top-4 (18000 assignments, a chunk boundary at token 4096) against the oracle, with
    the logits given and with the router on the device; a NaN in a first-chunk token still
    raises after the second chunk (the second chunk's router must not clear the status)."""
    import nn_amd
    E, H, I, T, k = 8, 96, 64, 4500, 4
    L = make_layer(E, H, I, seed=41)
    rw, rb = make_router(E, H, seed=42)
    moe = nn_amd.QuantizedMoE(E, H, I, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"],
                              router_weight=rw, router_bias=rb)
    x = torch.from_numpy(nn_amd.synth_normal(43, 5, (T, H), 1.0)).to(dev)
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    xf = x.float().cpu().numpy()
    logits = torch.from_numpy(nn_amd.synth_normal(43, 6, (T, E), 1.0)).to(dev)
    y, ti, tw = moe.forward(x, logits, top_k=k, return_routing=True)
    ref, rti, rtw = O.moe_forward(xf, logits.cpu().numpy(), k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), rti)
    check_close(ref, y.cpu().numpy(), f"moe long batch x={xdt}")
    yb, tib, _ = moe.block_forward(x, top_k=k, return_routing=True)
    lg = O.router_logits(xf, rw, rb)
    refb, rtib, _ = O.moe_forward(xf, lg, k, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"], I)
    assert np.array_equal(tib.cpu().numpy().astype(np.uint32), rtib)
    check_close(refb, yb.cpu().numpy(), f"moe block long batch x={xdt}")
    x[10, 3] = float("nan")
    with pytest.raises(nn_amd.NonFiniteData):
        moe.block_forward(x, top_k=k)


def test_moe_misaligned_x(O, dev):
    """A token batch at an address that is not 16-byte aligned (a narrowed view) gives the
    same routing and outputs as the aligned batch, through the router and the experts; so
    does an output at such an address."""
    import nn_amd
    E, H, I, T, k = 8, 96, 64, 20, 2
    L = make_layer(E, H, I, seed=51)
    rw, rb = make_router(E, H, seed=52)
    moe = nn_amd.QuantizedMoE(E, H, I, L["gp"], L["gs"], L["gb"], L["dp"], L["ds"], L["db"],
                              router_weight=rw, router_bias=rb)
    for dt in (torch.float32, torch.bfloat16):
        x = torch.from_numpy(nn_amd.synth_normal(53, 5, (T, H), 1.0)).to(dev).to(dt)
        big = torch.zeros(T * H + 8, dtype=dt, device=dev)
        big[1:1 + T * H] = x.reshape(-1)
        xv = big[1:1 + T * H].view(T, H)
        assert xv.data_ptr() % 16 != 0
        logits = torch.from_numpy(nn_amd.synth_normal(53, 6, (T, E), 1.0)).to(dev)
        assert torch.equal(moe.forward(xv, logits, top_k=k), moe.forward(x, logits, top_k=k))
        assert torch.equal(moe.block_forward(xv, top_k=k), moe.block_forward(x, top_k=k))
        assert torch.equal(moe.router_logits(xv), moe.router_logits(x))
    # an output at a 4-byte (not 16-byte) aligned address takes the combine's per-element
    # form: bit-identical to the 16-byte form the aligned output takes
    from nn_amd import _lib
    from nn_amd.quantized import _DTYPE, _ptr, _stream
    x = torch.from_numpy(nn_amd.synth_normal(54, 5, (T, H), 1.0)).to(dev)
    logits = torch.from_numpy(nn_amd.synth_normal(54, 6, (T, E), 1.0)).to(dev)
    ybig = torch.full((T * H + 4,), float("nan"), dtype=torch.float32, device=dev)
    yv = ybig[1:1 + T * H].view(T, H)
    assert yv.data_ptr() % 16 != 0
    rc = _lib.load().nnq_moe_forward(moe._h, _ptr(x), _DTYPE[x.dtype], T, _ptr(logits), k, 7.0, _ptr(yv), None, None, _stream(x))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(yv, moe.forward(x, logits, top_k=k))
