"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture exactly (decoded f32 bit patterns, f32
outputs), so a change to the oracle's arithmetic cannot go unnoticed.
GPU: the HIP path against the same fixtures: dequantization bit-exact, linear and
MoE outputs within the parity bar of test_gpu_linear (normwise and elementwise
max-rel <= 1e-3 with the near-zero skip at 1% of the peak, row cosine >= 0.99999),
MoE routing equal.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


DEC = [("q8_0", 32), ("q4_k", 256), ("q4_k_legacy", 256), ("q6_k", 256)]


def oracle_dec(O, name):
    return {"q8_0": O.dequant_q8_0, "q4_k": O.dequant_q4_k, "q4_k_legacy": O.dequant_q4_k_legacy,
            "q6_k": O.dequant_q6_k}[name]


@pytest.mark.parametrize("name,per", DEC)
@pytest.mark.parametrize("kind", ["random", "encoded"])
def test_oracle_decode_fixtures(O, name, per, kind):
    g = load("decode_blocks.npz")
    got = oracle_dec(O, name)(g[f"{name}_{kind}_bytes"], 8 * per).view(np.uint32)
    assert np.array_equal(got, g[f"{name}_{kind}_f32bits"])


def test_oracle_mxfp4_fixture(O):
    g = load("decode_blocks.npz")
    got = O.mxfp4_dequantize(g["mxfp4_packed"], g["mxfp4_scales"], g["mxfp4_scales"].size * 32).view(np.uint32)
    assert np.array_equal(got, g["mxfp4_f32bits"])


@pytest.mark.parametrize("name", ["q8_0", "q4_k", "q4_k_legacy", "q6_k"])
@pytest.mark.parametrize("m", [1, 3, 16])
def test_oracle_linear_fixtures(O, name, m):
    g = load("linear_small.npz")
    n, k = (int(v) for v in g[f"{name}_shape"])
    x, b = g[f"{name}_x_m{m}"], g[f"{name}_bytes"]
    if name == "q8_0":
        y = O.q8_0_matmul(x, b, n)
    else:
        y = O.matmul_xwt(x, oracle_dec(O, name)(b, n * k).reshape(n, k))
    assert np.array_equal(y.view(np.uint32), g[f"{name}_y_m{m}"].view(np.uint32))


def test_oracle_moe_fixture(O):
    g = load("moe_small.npz")
    E, K, T, H, I = (int(v) for v in g["dims"])
    y, ti, tw = O.moe_forward(g["x"], g["logits"], K, g["gu_packed"], g["gu_scales"], g["gu_bias"], g["dn_packed"],
                              g["dn_scales"], g["dn_bias"], I, float(g["limit"]))
    assert np.array_equal(ti, g["topk_idx"]) and np.array_equal(tw, g["topk_w"])
    # expf in the SwiGLU comes from the host libm: equal to within an ulp or two
    assert np.allclose(y, g["y"], rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------------
# the HIP path against the fixtures
# ---------------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("name,per", DEC)
@pytest.mark.parametrize("kind", ["random", "encoded"])
def test_gpu_decode_fixtures(name, per, kind):
    import nn_amd
    from test_gpu_linear import make_weight
    nn_amd.init(0)
    g = load("decode_blocks.npz")
    n = 8 * per // 256 if per == 256 else 8
    k = 8 * per // n
    w = make_weight(name, g[f"{name}_{kind}_bytes"], n, k)
    got = w.dequantize().cpu().numpy().reshape(-1).view(np.uint32)
    assert np.array_equal(got, g[f"{name}_{kind}_f32bits"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["q8_0", "q4_k", "q4_k_legacy", "q6_k"])
@pytest.mark.parametrize("m", [1, 3, 16])
def test_gpu_linear_fixtures(name, m):
    import torch

    import nn_amd
    from test_gpu_linear import check_close, make_weight
    nn_amd.init(0)
    g = load("linear_small.npz")
    n, k = (int(v) for v in g[f"{name}_shape"])
    w = make_weight(name, g[f"{name}_bytes"], n, k)
    y = nn_amd.quantized_linear(torch.from_numpy(g[f"{name}_x_m{m}"]).to("cuda:0"), w).cpu().numpy()
    check_close(g[f"{name}_y_m{m}"], y, f"golden {name} m={m}")


@pytest.mark.gpu
def test_gpu_moe_fixture():
    import torch

    import nn_amd
    from test_gpu_linear import check_close
    nn_amd.init(0)
    g = load("moe_small.npz")
    E, K, T, H, I = (int(v) for v in g["dims"])
    moe = nn_amd.QuantizedMoE(E, H, I, g["gu_packed"], g["gu_scales"], g["gu_bias"], g["dn_packed"], g["dn_scales"],
                              g["dn_bias"])
    y, ti, tw = moe.forward(torch.from_numpy(g["x"]).to("cuda:0"), torch.from_numpy(g["logits"]).to("cuda:0"),
                            top_k=K, return_routing=True)
    assert np.array_equal(ti.cpu().numpy().astype(np.uint32), g["topk_idx"])
    assert np.allclose(tw.cpu().numpy(), g["topk_w"], rtol=1e-6, atol=1e-7)
    check_close(g["y"], y.cpu().numpy(), "golden moe")
