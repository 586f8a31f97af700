"""C-ABI checks that need no GPU: libnnq.so loads, exports every symbol that
include/nnq.h declares, its host encoders agree byte-for-byte with the oracle's
restatement of the reference quantizers, and argument validation reports the
reference's error kinds before any device work."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    from nn_amd import _lib
    return _lib.load()


def header_symbols():
    txt = open(os.path.join(ROOT, "include", "nnq.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(nnq_[a-z0-9_]+)\s*\(", txt)))


def test_exports_every_declared_symbol(lib):
    from nn_amd import _lib
    syms = header_symbols()
    assert len(syms) >= 19
    for s in syms:
        assert hasattr(lib, s), s
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"


def test_q4k_encoder_matches_oracle(O):
    import nn_amd
    rng = np.random.default_rng(0)
    for scale in (0.02, 1.0, 1e-3):
        v = (rng.standard_normal(256 * 37 + 100) * scale).astype(np.float32)
        assert np.array_equal(nn_amd.quantize_q4_k(v), O.quantize_q4_k(v))
    v = np.full(256, -1.0, np.float32)
    v[0] = 0.0
    assert np.array_equal(nn_amd.quantize_q4_k(v), O.quantize_q4_k(v))
    for c in (0.5, -0.5, 0.0):
        v = np.full(512, c, np.float32)
        assert np.array_equal(nn_amd.quantize_q4_k(v), O.quantize_q4_k(v))


def test_q4k_encoder_rejects_non_finite():
    import nn_amd
    v = np.full(256, 0.5, np.float32)
    v[128] = np.nan
    with pytest.raises(nn_amd.NonFiniteData):
        nn_amd.quantize_q4_k(v)


def test_other_encoders_match_oracle(O):
    import nn_amd
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(256 * 64) * 0.02).astype(np.float32)
    assert np.array_equal(nn_amd.quantize_q8_0(v), O.quantize_q8_0(v))
    assert np.array_equal(nn_amd.quantize_q6_k(v), O.quantize_q6_k(v))
    v2 = np.concatenate([v, np.float32([np.nan, np.inf, -7.0, 1e-40, 6.0])])
    a, b = nn_amd.quantize_mxfp4(v2), O.mxfp4_quantize(v2)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_synth_generator(O):
    import nn_amd
    a = nn_amd.synth_normal(42, 3, (1 << 16,), 0.02)
    b = nn_amd.synth_normal(42, 3, (1 << 16,), 0.02)
    c = nn_amd.synth_normal(42, 4, (1 << 16,), 0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 5e-4 and abs(a.std() - 0.02) < 5e-4
    # the generator's words are splitmix64 of the keyed counter (test_prng.rs:18-22)
    u = (O.splitmix64((42 + 3 * 0xD1B54A32D192ED03) % 2**64) >> 11) * 2.0 ** -53
    u2 = (O.splitmix64((42 + 3 * 0xD1B54A32D192ED03 + 0x9E3779B97F4A7C15) % 2**64) >> 11) * 2.0 ** -53
    v0 = np.float32(0.02 * np.sqrt(-2 * np.log(1 - u)) * np.cos(2 * np.pi * u2))
    assert abs(a[0] - v0) <= 1e-9


def test_weight_create_validation_without_device(lib):
    from nn_amd import _lib
    h = ctypes.c_void_p()
    buf = np.zeros(144 * 4, np.uint8)
    vp = buf.ctypes.data_as(ctypes.c_void_p)
    # k not a multiple of the block size -> InvalidShape (QuantizedStorage::new)
    assert lib.nnq_weight_create(12, 0, vp, buf.size, 4, 100, ctypes.byref(h)) == _lib.ERR_INVALID_SHAPE
    # wrong byte count -> DataLengthMismatch
    assert lib.nnq_weight_create(12, 0, vp, buf.size - 1, 4, 256, ctypes.byref(h)) == _lib.ERR_DATA_LENGTH
    assert "expected 576" in _lib.last_error()
    # not a linear block format
    assert lib.nnq_weight_create(39, 0, vp, buf.size, 4, 256, ctypes.byref(h)) == _lib.ERR_WRONG_FORMAT
    # a null weight handle is "not quantized"
    assert lib.nnq_linear(None, None, 0, 1, 256, None, 0, None, 0, None) == _lib.ERR_NOT_QUANTIZED


def test_moe_create_limits_without_device(lib):
    """The MoE upload checks its shape before any device allocation: hidden / inter
    multiples of 32 (InvalidShape), at most 4096 experts and 32768 hidden / inter
    (Unsupported: the expert kernels address activation chunks with 32-bit offsets)."""
    from nn_amd import _lib
    h = ctypes.c_void_p()
    dummy = np.zeros(64, np.uint8)
    vp = dummy.ctypes.data_as(ctypes.c_void_p)
    args = lambda E, H, I: (E, H, I, vp, vp, vp, vp, vp, vp, ctypes.byref(h))
    assert lib.nnq_moe_create(*args(4, 40, 64)) == _lib.ERR_INVALID_SHAPE
    assert lib.nnq_moe_create(*args(4097, 64, 64)) == _lib.ERR_UNSUPPORTED
    assert lib.nnq_moe_create(*args(4, 32800, 64)) == _lib.ERR_UNSUPPORTED
    assert "32768" in _lib.last_error()
    assert lib.nnq_moe_create(*args(4, 64, 32800)) == _lib.ERR_UNSUPPORTED
    assert lib.nnq_moe_create_ocp(4, 32800, 64, vp, vp, vp, vp, ctypes.byref(h)) == _lib.ERR_UNSUPPORTED
    assert not h.value


def test_python_mirror_validation_without_device():
    import nn_amd
    with pytest.raises(nn_amd.WeightRank):
        nn_amd.QuantizedWeight.from_quantized(np.zeros(144, np.uint8), nn_amd.QuantType.Q4_K, (1, 1, 256))
    with pytest.raises(nn_amd.InvalidShape):
        nn_amd.QuantizedWeight.from_quantized(np.zeros(34, np.uint8), nn_amd.QuantType.Q8_0, (1, 30))
    with pytest.raises(nn_amd.DataLengthMismatch):
        nn_amd.QuantizedWeight.from_quantized(np.zeros(33, np.uint8), nn_amd.QuantType.Q8_0, (1, 32))
    assert nn_amd.QuantType.Q4_K.expected_bytes(512) == 288 and nn_amd.QuantType.Q4_K.expected_bytes(100) is None


def test_no_device_is_reported(lib):
    import torch
    from nn_amd import _lib
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    c = ctypes.c_int(-1)
    assert lib.nnq_device_count(ctypes.byref(c)) == 0 and c.value == 0
    assert lib.nnq_init(0) == _lib.ERR_NO_DEVICE


def _fake_weight(n=16, k=256):
    """A QuantizedWeight with a null handle: enough for the host-side checks, which
    must reject the call before anything reaches the C ABI."""
    import nn_amd
    return nn_amd.QuantizedWeight(ctypes.c_void_p(), nn_amd.QuantType.Q4_K, nn_amd.Layout.GGUF, (n, k), 0)


def test_host_tensors_are_refused_before_any_launch():
    """The C ABI takes device pointers only and cannot tell a host address from a device
    one, so every wrapper refuses a CPU input with Unsupported on the host."""
    import torch

    import nn_amd
    w = _fake_weight()
    x = torch.zeros(1, 256)
    with pytest.raises(nn_amd.Unsupported):
        nn_amd.quantized_linear(x, w)
    with pytest.raises(nn_amd.Unsupported):
        nn_amd.linear_argmax(x, w)
    with pytest.raises(nn_amd.Unsupported):
        nn_amd.linear_sample(x, w)
    with pytest.raises(nn_amd.Unsupported):
        nn_amd.argmax(torch.zeros(8))
    with pytest.raises(nn_amd.Unsupported):
        nn_amd.sample_token(torch.zeros(8))
    moe = object.__new__(nn_amd.QuantizedMoE)
    moe._h = moe._router = None
    moe.num_experts, moe.hidden, moe.inter, moe.device = 4, 64, 64, 0
    with pytest.raises(nn_amd.Unsupported):
        moe.forward(torch.zeros(2, 64), torch.zeros(2, 4))


def test_ocp_mxfp4_encoder_matches_oracle(O):
    """nnq_quantize_mxfp4_ocp (nn-core quantize_tensor) byte for byte against the
    oracle, over lengths that pad the last block and values across the whole exponent
    range: zeros, tiny blocks whose shared_exp clamps to 0, large ones clamped to 254."""
    import nn_amd
    rng = np.random.default_rng(3)
    for n in (0, 1, 31, 50, 64, 1000, 32 * 257 + 5):
        v = (rng.standard_normal(n) * 10.0 ** rng.uniform(-45, 38, n)).astype(np.float32)
        v[::7] = 0.0
        assert np.array_equal(nn_amd.quantize_mxfp4_ocp(v), O.ocp_quantize(v)), n
    for scale in (1e-40, 1e-38, 3e37, 3.4e38):
        v = (rng.uniform(-1, 1, 96) * scale).astype(np.float32)
        assert np.array_equal(nn_amd.quantize_mxfp4_ocp(v), O.ocp_quantize(v)), scale
    with pytest.raises(nn_amd.NonFiniteData):
        nn_amd.quantize_mxfp4_ocp(np.array([0.0, np.inf], np.float32))
