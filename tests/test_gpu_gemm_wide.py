"""GPU parity for the Q4_K prefill GEMMs of bf16 activations at every batch size the
random-byte shapes below reach: the wide-wave-tile kernel (more than 128 rows), the
skinny kernel (17 to 32 rows over three tiles per workgroup), the one-launch thin kernel
(up to 16 rows) and the ring kernel between them, against the oracle's bit-exact decode
followed by an f64 product (tolerances as in test_gpu_linear).  Shapes cover both wide
column-tile widths (96 columns, and 64 with the K range split in two), ragged row tiles
(the last tile partly past M, a row group partly past M), random block bytes (arbitrary
finite d / dmin / scales, with d = 0 super-blocks), bias, f32 and bf16 outputs, and
repeated calls agreeing bit for bit."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import ref_f64
from test_gpu_linear import check_close, make_weight, rand_bytes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def dev():
    import nn_amd
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nn_amd.init(0)
    return torch.device("cuda:0")


@pytest.mark.parametrize("m,n,k", [(300, 12288, 1024), (512, 12288, 512), (129, 4096, 2048), (700, 4096, 1536),
                                   (257, 6144, 1024), (1000, 8192, 512), (5, 12288, 1024), (32, 12288, 512),
                                   (48, 12288, 1024), (64, 4096, 8192), (17, 3072, 12288), (63, 768, 2048), (40, 1528, 1024), (300, 1528, 512)])
@pytest.mark.parametrize("legacy", [False, True])
def test_wide_random_blocks(O, dev, m, n, k, legacy):
    import nn_amd
    b = rand_bytes("q4_k", n, k, seed=m * 7 + n + k).reshape(-1, 144).copy()
    b[::7, 0:2] = 0  # d = +0.0 for every seventh super-block
    b = b.ravel()
    w = make_weight("q4_k_legacy" if legacy else "q4_k", b, n, k)
    x = torch.from_numpy(nn_amd.synth_normal(m + 1, 2, (m, k), 1.0)).to(dev).to(torch.bfloat16)
    bias = torch.from_numpy(nn_amd.synth_normal(m + 1, 3, (n,), 0.5)).to(dev)
    y = nn_amd.quantized_linear(x, w, bias)
    y2 = nn_amd.quantized_linear(x, w, bias)
    assert torch.equal(y, y2), "repeated calls must agree bit for bit"
    ref = ref_f64(O, b, n, k, x.float().cpu().numpy(), legacy=legacy) + bias.cpu().numpy()
    check_close(ref, y.cpu().numpy(), f"gemm wide {m}x{n}x{k} legacy={legacy}")
    yb = nn_amd.quantized_linear(x, w, bias, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(yb, y.to(torch.bfloat16).float().cpu().numpy()), "bf16 output: the f32 result rounded once"


def test_wide_row_scales(O, dev):
    """Rows of very different magnitudes (1e-6 to 1e4) and a zero row: each row has its own
    power-of-two staging scale, so every row keeps its relative accuracy."""
    import nn_amd
    m, n, k = 260, 12288, 512
    wb = nn_amd.quantize_q4_k(nn_amd.synth_normal(9, 1, (n, k), 0.02))
    w = make_weight("q4_k", wb, n, k)
    xs = nn_amd.synth_normal(9, 2, (m, k), 1.0)
    xs *= (10.0 ** np.linspace(-6, 4, m)).astype(np.float32)[:, None]
    xs[17] = 0.0
    x = torch.from_numpy(xs).to(dev).to(torch.bfloat16)
    y = nn_amd.quantized_linear(x, w).cpu().numpy()
    ref = ref_f64(O, wb, n, k, x.float().cpu().numpy())
    assert np.all(y[17] == 0.0)
    keep = np.arange(m) != 17
    r, g = ref[keep], y[keep]
    # per row, normwise against that row's peak (the rows' scales differ by 10 decades)
    err = np.abs(g - r).max(axis=1) / np.abs(r).max(axis=1)
    print(f"row-scale sweep: worst per-row normwise {err.max():.2e}")
    assert err.max() <= 1e-3
