"""Pin the CPU oracle (oracle/nnq_oracle.c) before trusting it as the checker.

Each test restates a known-answer test of the reference (cited), an invariant its
Kani harnesses prove, a closed form fixed by IEEE arithmetic, or an independent
brute-force computation (numpy / f64) on small inputs.
"""
import numpy as np
import pytest


def f16b(v):
    return int(np.float16(v).view(np.uint16))


def block_bytes(*pairs, size):
    b = np.zeros(size, np.uint8)
    for off, val in pairs:
        b[off] = val
    return b


# ---------------------------------------------------------------------------------
# half precision (the `half` crate: IEEE 754 binary16, RNE)
# ---------------------------------------------------------------------------------

def test_f16_to_f32_exhaustive_matches_numpy(O):
    bits = np.arange(65536, dtype=np.uint16)
    a = O.f16_bits_to_f32(bits)
    b = bits.view(np.float16).astype(np.float32)
    fin = ~np.isnan(b)
    assert np.array_equal(a[fin].view(np.uint32), b[fin].view(np.uint32))
    assert np.isnan(a[~fin]).all()


def test_f32_to_f16_rne_matches_numpy(O):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(200_000) * 10.0 ** rng.integers(-9, 6, 200_000)).astype(np.float32)
    edge = np.array([65504, 65519.99, 65520, 65536, 2.98e-8, 2.9802322e-08, 5.96e-8, 6.1e-5, -0.0, np.inf, -np.inf,
                     1e-45, 3.0e-5], np.float32)
    raw = rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, edge, raw[~np.isnan(raw)]])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16_bits(x), ref)


def test_bf16_round_trip(O):
    x = np.array([1.0, 1.00390625, 1.005859375, -3.5, 1e-40, 3.3e38], np.float32)
    b = O.f32_to_bf16_bits(x)
    # RNE: 1.00390625 = 1 + 2^-8 is a tie -> even (1.0); 1.005859375 rounds up
    assert list(b[:3]) == [0x3F80, 0x3F80, 0x3F81]
    assert np.array_equal(O.bf16_bits_to_f32(b)[[0, 3]], np.float32([1.0, -3.5]))


def test_splitmix64_published_vector(O):
    # SplitMix64 seeded with 0: the first output mixes 0x9E3779B97F4A7C15 (Vigna 2015)
    assert O.splitmix64(0x9E3779B97F4A7C15) == 0xE220A8397B1DCDAF
    assert O.splitmix64(2 * 0x9E3779B97F4A7C15 % 2**64) == 0x6E789E6AA1B965F4


# ---------------------------------------------------------------------------------
# Q8_0
# ---------------------------------------------------------------------------------

def test_q8_0_zero_scale(O):
    # crates/nn-gguf/src/dequant.rs:699-715
    blk = np.zeros(34, np.uint8)
    blk[2:] = 42
    assert np.all(O.dequant_q8_0(blk, 32) == 0.0)


def test_q8_0_cross_crate_block(O):
    # crates/nn-import/src/gguf_expanded_tests.rs:894-925: scale 0.25, values -10..21
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    blk[2:] = (np.arange(32) - 10).astype(np.int8).view(np.uint8)
    assert np.array_equal(O.dequant_q8_0(blk, 32), 0.25 * (np.arange(32) - 10).astype(np.float32))


def test_q8_0_decode_closed_form(O):
    rng = np.random.default_rng(1)
    raw = rng.integers(0, 256, 34 * 64, dtype=np.uint8)
    d = raw.reshape(64, 34)[:, :2].copy().view(np.uint16).ravel()
    d = d & 0x7BFF  # finite scales
    raw.reshape(64, 34)[:, :2] = d.view(np.uint8).reshape(64, 2)
    got = O.dequant_q8_0(raw, 64 * 32)
    q = raw.reshape(64, 34)[:, 2:].view(np.int8).astype(np.float64)
    exact = d.view(np.float16).astype(np.float64)[:, None] * q  # exact in binary32 (<= 19 bits)
    assert np.array_equal(got, exact.astype(np.float32).ravel())


def test_q8_0_short_buffer_clamps(O):
    # crates/nn-gguf/src/security_tests.rs:693-700
    assert O.dequant_q8_0(np.zeros(20, np.uint8), 32).size == 0


def make_q8_0_weight(n, k, scale, values):
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(scale).tobytes(), np.uint8)
    blk[2:] = np.asarray(values, np.int8).view(np.uint8)
    return np.tile(blk, n * (k // 32))


def test_q8_0_matmul_known_values(O):
    # crates/nn-core/src/dyn_tensor/quantized_matmul_tests.rs:150-163 and :166-200
    w = make_q8_0_weight(2, 32, 0.5, [2] * 32)
    assert np.all(np.abs(O.q8_0_matmul(np.ones((1, 32), np.float32), w, 2) - 32.0) < 0.5)
    w = make_q8_0_weight(1, 32, 1.0, [1] * 32)
    x = np.stack([np.ones(32, np.float32), 2 * np.ones(32, np.float32)])
    y = O.q8_0_matmul(x, w, 1)
    assert abs(y[0, 0] - 32.0) < 0.5 and abs(y[1, 0] - 64.0) < 1.0


def test_q8_0_matmul_batch_4d_and_multiblock(O):
    # quantized_matmul_tests.rs:296-318 (4-D batch) and :528-545 (two blocks)
    w = make_q8_0_weight(3, 32, 1.0, [1] * 32)
    y = O.q8_0_matmul(np.full((2, 2, 1, 32), 2.0, np.float32), w, 3)
    assert y.shape == (2, 2, 1, 3) and np.all(np.abs(y - 64.0) < 1.0)
    w = make_q8_0_weight(2, 64, 1.0, [1] * 32)
    assert np.all(np.abs(O.q8_0_matmul(np.ones((1, 64), np.float32), w, 2) - 64.0) < 1.0)


def test_q8_0_matmul_bias_values(O):
    # quantized_matmul_tests.rs:323-350 and :383-418 (bias added after the fused matmul)
    w = make_q8_0_weight(2, 32, 1.0, [1] * 32)
    y = O.q8_0_matmul(np.ones((1, 32), np.float32), w, 2) + np.float32([10, 20])
    assert np.allclose(y, [[42, 52]], atol=1.0)
    w = make_q8_0_weight(3, 32, 1.0, [1] * 32)
    y = O.q8_0_matmul(np.full((2, 1, 32), 0.5, np.float32), w, 3) + np.float32([100, 200, 300])
    assert np.allclose(y[0, 0], [116, 216, 316], atol=1.0)


def test_q8_0_fused_matches_dequant_then_matmul(O):
    # quantized_matmul_tests.rs:457-491: fused vs dequant+matmul within 1e-3
    w = make_q8_0_weight(4, 64, 0.25, [4] * 32)
    x = ((np.arange(128) % 64) * 0.1 - 3.0).astype(np.float32).reshape(2, 64)
    fused = O.q8_0_matmul(x, w, 4)
    ref = O.matmul_xwt(x, O.dequant_q8_0(w, 4 * 64).reshape(4, 64))
    assert np.max(np.abs(fused - ref)) < 1e-3


def test_q8_0_fused_against_f64_bruteforce(O):
    rng = np.random.default_rng(3)
    n, k = 37, 320
    w = O.quantize_q8_0(rng.standard_normal(n * k).astype(np.float32) * 0.02)
    x = rng.standard_normal((3, k)).astype(np.float32)
    wf = O.dequant_q8_0(w, n * k).reshape(n, k).astype(np.float64)
    exact = x.astype(np.float64) @ wf.T
    got = O.q8_0_matmul(x, w, n)
    assert np.max(np.abs(got - exact)) <= 1e-5 * np.max(np.abs(exact))


# ---------------------------------------------------------------------------------
# Q4_K, GGUF-spec layout (nn-core BlockQ4K)
# ---------------------------------------------------------------------------------

def pack_scale_min(sc, mn):
    """The packing written by BlockQ4K::quantize (linear.rs:121-133)."""
    s = np.zeros(12, np.uint8)
    for j in range(8):
        ls, lm = sc[j], mn[j]
        if j < 4:
            s[j] = ls
            s[j + 4] = lm
        else:
            s[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            s[j - 4] |= (ls >> 4) << 6
            s[j] |= (lm >> 4) << 6
    return s


def test_q4k_scale_min_pack_roundtrip_exhaustive(O):
    # Kani harnesses q4k_scale_pack_roundtrip_low/high (linear.rs:633-668): every j and 6-bit pair
    for j in range(8):
        for sc in range(64):
            for mn in range(0, 64, 3 if j % 2 else 1):
                q = np.zeros(12, np.uint8)
                if j < 4:
                    q[j], q[j + 4] = sc, mn
                else:
                    q[j + 4] = (sc & 0xF) | ((mn & 0xF) << 4)
                    q[j - 4] |= (sc >> 4) << 6
                    q[j] |= (mn >> 4) << 6
                assert O.q4k_get_scale_min(j, q) == (sc, mn)


def q4k_block(d, dmin, sc, mn, q):
    """BlockQ4K bytes from scales/mins and 256 4-bit values (GGUF element order)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    b[4:16] = pack_scale_min(sc, mn)
    q = np.asarray(q, np.uint8)
    for g in range(4):
        b[16 + 32 * g:16 + 32 * g + 32] = q[64 * g:64 * g + 32] | (q[64 * g + 32:64 * g + 64] << 4)
    return b


def test_q4k_gguf_decode_known_block(O):
    # element e of sub-block j = e // 32 decodes to d*sc_j*q_e - dmin*m_j (linear.rs:63-92)
    sc = [1, 2, 3, 4, 63, 33, 17, 0]
    mn = [0, 5, 9, 62, 1, 63, 20, 7]
    q = np.arange(256) % 16
    blk = q4k_block(0.5, 0.25, sc, mn, q)
    got = O.dequant_q4_k(blk, 256)
    exp = np.array([0.5 * sc[e // 32] * q[e] - 0.25 * mn[e // 32] for e in range(256)], np.float64)
    assert np.array_equal(got, exp.astype(np.float32))


def test_q4k_gguf_decode_closed_form_random(O):
    # F13: d*sc and dmin*m are exact, so each output is round_f32(d*sc*q - dmin*m) of the exact value
    rng = np.random.default_rng(11)
    nb = 200
    raw = rng.integers(0, 256, 144 * nb, dtype=np.uint8).reshape(nb, 144)
    dd = raw[:, :4].copy().view(np.uint16) & 0x7BFF
    raw[:, :4] = dd.view(np.uint8)
    got = O.dequant_q4_k(raw.ravel(), 256 * nb).reshape(nb, 256)
    for b in range(nb):
        d, dmin = dd[b].view(np.float16).astype(np.float64)
        for e in range(0, 256, 7):
            j = e // 32
            sc, mn = O.q4k_get_scale_min(j, raw[b, 4:16])
            g, i = e // 64, e % 64
            byte = raw[b, 16 + 32 * g + (i % 32)]
            qv = (byte & 0xF) if i < 32 else (byte >> 4)
            assert got[b, e] == np.float32(d * sc * qv - dmin * mn)


def test_q4k_quantize_round_trip_bounds(O):
    # crates/nn-core/src/layers/quantized/linear_tests.rs:33-99
    cases = [(np.zeros(256, np.float32), 0.01), (np.arange(256, dtype=np.float32) / 255.0, 0.1),
             (np.arange(256, dtype=np.float32) / 127.5 - 1.0, 0.2), (np.full(256, 0.5, np.float32), 0.1)]
    for v, tol in cases:
        r = O.dequant_q4_k(O.quantize_q4_k(v), 256)
        assert np.max(np.abs(r - v)) < tol


def test_q4k_quantize_clustered_at_min_and_nan(O):
    # linear_tests.rs:300-332
    v = np.full(256, -1.0, np.float32)
    v[0] = 0.0
    assert np.isfinite(O.dequant_q4_k(O.quantize_q4_k(v), 256)).all()
    v = np.full(256, 0.5, np.float32)
    v[128] = np.nan
    with pytest.raises(O.OracleError):
        O.quantize_q4_k(v)


def test_q4k_nearest_int_cases(O):
    # linear_tests.rs:258-298 (f32::round: half away from zero)
    assert [O.q4k_nearest_int(v) for v in (0.0, 1.5, -1.5, 0.4, -0.4, 2.5)] == [0, 2, -2, 0, 0, 3]
    for bad in (np.nan, np.inf, -np.inf):
        with pytest.raises(O.OracleError):
            O.q4k_nearest_int(bad)


def test_q4k_qlinear_round_trip_weight_tolerance(O):
    # linear_tests.rs:118-142: from_linear -> dequantize within 0.1 for small weights
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((8, 512)) * 0.1).astype(np.float32)
    r = O.dequant_q4_k(O.quantize_q4_k(w), w.size).reshape(w.shape)
    assert np.max(np.abs(r - w)) < 0.1


def test_q4k_padding_non_aligned(O):
    # QLinear::from_linear pads the flattened weight to a multiple of 256 (linear.rs:323-328)
    v = np.arange(300, dtype=np.float32) / 300.0
    b = O.quantize_q4_k(v)
    assert b.size == 2 * 144
    assert np.max(np.abs(O.dequant_q4_k(b, 512)[:300] - v)) < 0.1


# ---------------------------------------------------------------------------------
# Q4_K, nn-gguf layout
# ---------------------------------------------------------------------------------

def test_q4k_legacy_known_values_and_divergence(O):
    # crates/nn-gguf/src/dequant.rs:764-818: d=1, scales[0]=2, q=3 -> 6.0 for sub-block 0
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[4] = 0x02
    blk[16:32] = 0x33
    leg = O.dequant_q4_k_legacy(blk, 256)
    assert np.all(np.abs(leg[:32] - 6.0) < 1e-4) and np.all(np.abs(leg[32:]) < 1e-6)
    # the same bytes under the GGUF layout: elements 16..31 are 0 (the two decoders differ)
    gg = O.dequant_q4_k(blk, 256)
    assert np.all(gg[:16] == 6.0) and np.all(gg[16:32] == 0.0)


def test_q4k_legacy_with_dmin_and_zero(O):
    # dequant.rs:820-852 and :748-762
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[4] = 0x01
    blk[8] = 0x04
    assert np.all(np.abs(O.dequant_q4_k_legacy(blk, 256)[:32] + 2.0) < 1e-3)
    z = np.zeros(144, np.uint8)
    z[4:16] = 0xFF
    z[16:] = 0xAB
    assert np.all(O.dequant_q4_k_legacy(z, 256) == 0.0)
    assert O.dequant_q4_k_legacy(np.zeros(100, np.uint8), 256).size == 0  # security_tests.rs:702-709


# ---------------------------------------------------------------------------------
# Q6_K, nn-gguf layout (crates/nn-gguf/src/dequant.rs:1158-1399)
# ---------------------------------------------------------------------------------

def q6(d, scales=(), ql=(), qh=()):
    b = np.zeros(210, np.uint8)
    b[208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    for i, v in scales:
        b[192 + i] = np.uint8(np.int8(v).view(np.uint8))
    for i, v in ql:
        b[i] = v
    for i, v in qh:
        b[128 + i] = v
    return b


def test_q6k_zero_d_and_zero_scales(O):
    b = q6(0.0)
    b[:192] = 0xAB
    b[192:208] = 0x7F
    assert np.all(O.dequant_q6_k(b, 256) == 0.0)
    b = q6(1.0)
    b[:192] = 0xFF
    assert np.all(O.dequant_q6_k(b, 256) == 0.0)


def test_q6k_known_values(O):
    # centered q=32 -> 0; d=0.5 sc=2 q=35 -> 3.0; sc=-3 q=33 -> -3.0; q=63 -> 62.0; q=0 -> -64.0
    b = q6(1.0, scales=[(i, 1) for i in range(16)], qh=[(i, 0xAA) for i in range(64)])
    assert np.all(np.abs(O.dequant_q6_k(b, 256)) < 1e-4)
    b = q6(0.5, scales=[(0, 2)], ql=[(i, 0x33) for i in range(8)], qh=[(i, 0xAA) for i in range(4)])
    r = O.dequant_q6_k(b, 256)
    assert np.all(np.abs(r[:16] - 3.0) < 1e-3) and np.all(np.abs(r[16:]) < 1e-4)
    b = q6(1.0, scales=[(0, -3)], ql=[(i, 0x11) for i in range(8)], qh=[(i, 0xAA) for i in range(4)])
    assert np.all(np.abs(O.dequant_q6_k(b, 256)[:16] + 3.0) < 1e-3)
    b = q6(0.5, scales=[(0, 4)], ql=[(i, 0xFF) for i in range(8)], qh=[(i, 0xFF) for i in range(4)])
    r = O.dequant_q6_k(b, 256)
    assert np.all(np.abs(r[:16] - 62.0) < 1e-2) and np.all(np.abs(r[16:]) < 1e-4)
    b = q6(1.0, scales=[(0, 2)])
    assert np.all(np.abs(O.dequant_q6_k(b, 256)[:16] + 64.0) < 1e-2)


def test_q6k_two_blocks_length_finite_short(O):
    data = np.zeros(420, np.uint8)
    data[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    data[418:420] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    assert np.all(O.dequant_q6_k(data, 512) == 0.0)
    assert O.dequant_q6_k(np.zeros(840, np.uint8), 1024).size == 1024  # gguf_expanded_tests.rs:465-470
    pat = ((np.arange(210) * 17) % 256).astype(np.uint8)  # gguf_expanded_tests.rs:472-480
    assert np.isfinite(O.dequant_q6_k(pat, 256)).all()
    assert O.dequant_q6_k(np.zeros(100, np.uint8), 256).size == 0  # security_tests.rs:711-717


def test_q6k_element_mapping_closed_form(O):
    rng = np.random.default_rng(9)
    raw = rng.integers(0, 256, 210 * 20, dtype=np.uint8).reshape(20, 210)
    dd = raw[:, 208:210].copy().view(np.uint16) & 0x7BFF
    raw[:, 208:210] = dd.view(np.uint8)
    got = O.dequant_q6_k(raw.ravel(), 20 * 256).reshape(20, 256)
    idx = np.arange(256)
    lo = (raw[:, idx // 2] >> (4 * (idx % 2))) & 0xF
    hi = (raw[:, 128 + idx // 4] >> (2 * (idx % 4))) & 3
    q = (lo | (hi << 4)).astype(np.float64) - 32
    sc = raw[:, 192:208].view(np.int8).astype(np.float64)[:, idx // 16]
    exact = dd.view(np.float16).astype(np.float64) * sc * q  # exact (<= 23 significant bits)
    assert np.array_equal(got, exact.astype(np.float32))


# ---------------------------------------------------------------------------------
# GPT-OSS MXFP4 (crates/nn-gptoss/src/quantize.rs:270-404, tests/integration.rs:125-160)
# ---------------------------------------------------------------------------------

def test_mxfp4_lut_and_e8m0(O):
    assert [O.lib().orc_mxfp4_lut(i) for i in range(16)] == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                                                             -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    dec = O.lib().orc_mxfp4_decode_e8m0
    assert (dec(127), dec(128), dec(126)) == (1.0, 2.0, 0.5)
    assert dec(0) == 2.0 ** -126 and dec(1) == 2.0 ** -126
    enc = O.lib().orc_mxfp4_e8m0_from_max
    assert (enc(0.0), enc(float("nan")), enc(6.0), enc(1e-40)) == (0, 0, 127, 0)


def test_mxfp4_round_trips(O):
    v = np.float32([0.0, 1.0, -1.0, 2.0, -2.0, 3.0, -3.0, 4.0])
    p, s = O.mxfp4_quantize(v)
    assert np.all(np.abs(O.mxfp4_dequantize(p, s, 8) - v) < 1e-6)
    v = ((np.arange(64) - 32.0) * 0.1).astype(np.float32)
    p, s = O.mxfp4_quantize(v)
    r = O.mxfp4_dequantize(p, s, 64)
    for i in range(64):
        assert abs(v[i] - r[i]) <= O.lib().orc_mxfp4_decode_e8m0(int(s[i // 32])) + 1e-6
    p, s = O.mxfp4_quantize(np.zeros(64, np.float32))
    assert np.all(O.mxfp4_dequantize(p, s, 64) == 0.0)
    v = np.float32([0.5, -0.25, 1.0, 0.0, -1.0, 0.75, -0.5, 0.125])
    p, s = O.mxfp4_quantize(v)
    assert np.all(np.abs(O.mxfp4_dequantize(p, s, 8) - v) < 2.0)


def test_mxfp4_sizes_large_subnormal(O):
    p, s = O.mxfp4_quantize(np.arange(50, dtype=np.float32))
    assert s.size == 2 and O.mxfp4_dequantize(p, s, 50).size == 50
    p, s = O.mxfp4_quantize(np.ones(128, np.float32))
    assert s.size == 4 and p.size == 64
    p, s = O.mxfp4_quantize(np.float32([1000.0, -500.0, 250.0, -125.0]))
    assert np.isfinite(O.mxfp4_dequantize(p, s, 4)).all()
    p, s = O.mxfp4_quantize(np.full(32, np.finfo(np.float32).tiny / 100, np.float32))
    assert np.all(np.abs(O.mxfp4_dequantize(p, s, 32)) < 1e-30)


def test_mxfp4_nibble_order_and_ties(O):
    # pair p: HIGH nibble = element 2p (quantize.rs:147-155); ties keep the lower magnitude (strict <)
    v = np.zeros(32, np.float32)
    v[0], v[1] = 6.0, -0.5
    p, s = O.mxfp4_quantize(v)
    assert s[0] == 127 and p[0] == (0x7 << 4 | 0x9)
    enc = O.lib().orc_mxfp4_quantize_fp4
    assert enc(1.25, 1.0) == 2 and enc(2.5, 1.0) == 4 and enc(5.0, 1.0) == 6 and enc(0.25, 1.0) == 0
    assert enc(float("inf"), 1.0) == 0 and enc(-1.75, 1.0) == 0xB


# ---------------------------------------------------------------------------------
# argmax / softmax / topk / MoE
# ---------------------------------------------------------------------------------

def test_argmax_semantics(O):
    assert O.argmax(np.float32([1, 3, 3, 2])) == 1  # first maximum (strict >)
    assert O.argmax(np.float32([-np.inf, -np.inf])) == 0
    with pytest.raises(O.OracleError):
        O.argmax(np.float32([1, np.nan, 2]))


def test_softmax_topk_small(O):
    x = np.float32([[1.0, 2.0, 3.0, 0.5], [0.0, 0.0, -np.inf, 1.0]])
    p = O.softmax_rows(x)
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    assert np.allclose(p, e / e.sum(1, keepdims=True), rtol=1e-6, atol=0)
    v, i = O.topk_rows(p, 2)
    assert i.tolist() == [[2, 1], [3, 0]]
    assert O.softmax_rows(np.full((1, 3), -np.inf, np.float32)).tolist() == [[0.0, 0.0, 0.0]]


def moe_f64(x, logits, k, Wg, bg, Wd, bd, inter, limit):
    """Independent f64 restatement of moe_forward (quantized_model.rs:132-194)."""
    T, H = x.shape
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    out = np.zeros((T, H))
    for t in range(T):
        order = sorted(range(logits.shape[1]), key=lambda e: (-p[t, e], e))[:k]
        w = p[t, order] / p[t, order].sum()
        for e, we in sorted(zip(order, w)):
            gu = x[t] @ Wg[e] + bg[e]
            g, u = gu[:inter], gu[inter:]
            sg = np.clip(g / (1 + np.exp(-g)), -limit, limit)
            out[t] += we * ((sg * u) @ Wd[e] + bd[e])
    return out


def test_moe_matches_f64_bruteforce(O):
    rng = np.random.default_rng(21)
    E, K, T, H, I = 4, 2, 6, 64, 32
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    gu = (rng.standard_normal(E * H * 2 * I) * 0.1).astype(np.float32)
    dn = (rng.standard_normal(E * I * H) * 0.1).astype(np.float32)
    gb = (rng.standard_normal(E * 2 * I) * 0.1).astype(np.float32)
    db = (rng.standard_normal(E * H) * 0.1).astype(np.float32)
    gp, gs = O.mxfp4_quantize(gu)
    dp, ds = O.mxfp4_quantize(dn)
    y, ti, tw = O.moe_forward(x, logits, K, gp, gs, gb, dp, ds, db, I, 7.0)
    y2, _, _ = O.moe_forward(x, logits, K, gp, gs, gb, dp, ds, db, I, 7.0, faithful=True)
    assert np.array_equal(y, y2)
    Wg = O.mxfp4_dequantize(gp, gs, E * H * 2 * I).reshape(E, H, 2 * I).astype(np.float64)
    Wd = O.mxfp4_dequantize(dp, ds, E * I * H).reshape(E, I, H).astype(np.float64)
    ref = moe_f64(x.astype(np.float64), logits.astype(np.float64), K, Wg, gb.reshape(E, 2 * I), Wd,
                  db.reshape(E, H), I, 7.0)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    assert np.allclose(tw.sum(1), 1.0, atol=1e-6)


# ---------------------------------------------------------------------------------
# build-defined input generators (no reference encoder exists): round-trip bounds
# ---------------------------------------------------------------------------------

def test_q8_0_encoder_round_trip_bound(O):
    """d = f16(amax / 127), q = round(v / d): every decoded value within d / 2 (+ the f16
    rounding of d) of the input, and the block maximum maps to |q| = 127."""
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(32 * 64) * 0.02).astype(np.float32)
    b = O.quantize_q8_0(v)
    dec = O.dequant_q8_0(b, v.size)
    d = O.f16_bits_to_f32(b.reshape(-1, 34)[:, 0:2].copy().view(np.uint16).ravel())
    err = np.abs(dec - v).reshape(-1, 32)
    assert np.all(err <= d[:, None] * 0.5 + np.abs(v).reshape(-1, 32) * 2.0 ** -10 + 1e-12)
    q = b.reshape(-1, 34)[:, 2:].view(np.int8)
    assert np.all(np.abs(q).max(axis=1) >= 126)


def test_q6_k_encoder_round_trip_bound(O):
    """Decoded values within half a quantisation step (d * |sc|) of the input plus the
    rounding of the f16 / int8 scales (a few percent of the block range)."""
    rng = np.random.default_rng(12)
    v = (rng.standard_normal(256 * 16) * 0.02).astype(np.float32)
    b = O.quantize_q6_k(v)
    dec = O.dequant_q6_k(b, v.size)
    rng_blk = np.abs(v).reshape(-1, 256).max(axis=1)
    err = np.abs(dec - v).reshape(-1, 256).max(axis=1)
    assert np.all(err <= rng_blk * 0.05)
    assert np.corrcoef(dec, v)[0, 1] > 0.999


# ---- Qwen3 SwiGLU MLP glue (crates/nn-qwen3/src/layers.rs:40-47) ----------------------


def test_silu_mul_closed_form(O):
    """silu(g) * u = g / (1 + e^-g) * u (ops/math.rs:140): against f64, plus the fixed
    points silu(0) = 0, silu(-inf) = -0 and silu(+inf) = +inf."""
    rng = np.random.default_rng(7)
    g = np.concatenate([rng.normal(0, 4, 4000), [0.0, -0.0, 30.0, -30.0, 88.0, -88.0, 1e-30]]).astype(np.float32)
    u = rng.normal(0, 2, g.size).astype(np.float32)
    h = O.silu_mul(g, u)
    ref = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64))) * u.astype(np.float64)
    err = np.abs(h - ref) / np.maximum(np.abs(ref), 1e-30)
    assert err.max() < 4e-7, err.max()
    # swapping gate and up must change the result (the oracle is not symmetric)
    assert not np.allclose(O.silu_mul(u, g), h, rtol=1e-3)
    assert O.silu_mul(np.array([0.0], np.float32), np.array([5.0], np.float32))[0] == 0.0
    assert np.isinf(O.silu_mul(np.array([np.inf], np.float32), np.array([1.0], np.float32))[0])


def test_mlp_forward_matches_f64(O):
    """The composed MLP (quantized gate / up / down) against f64 math on the oracle's
    bit-exact dequantized weights; Q4_K gate / up, Q6_K down (the Q4_K_M mix)."""
    import nn_amd
    H, I, m = 256, 512, 3
    wg, wu = nn_amd.synth_normal(3, 1, (I, H), 0.05), nn_amd.synth_normal(3, 2, (I, H), 0.05)
    wd = nn_amd.synth_normal(3, 3, (H, I), 0.05)
    bg, bu, bd = O.quantize_q4_k(wg), O.quantize_q4_k(wu), O.quantize_q6_k(wd)
    x = nn_amd.synth_normal(3, 4, (m, H), 1.0)
    y, bad = O.mlp_forward(x, (12, bg), (12, bu), (14, bd), H, I)
    assert not bad
    Wg = O.dequant_q4_k(bg, I * H).reshape(I, H).astype(np.float64)
    Wu = O.dequant_q4_k(bu, I * H).reshape(I, H).astype(np.float64)
    Wd = O.dequant_q6_k(bd, H * I).reshape(H, I).astype(np.float64)
    g, u = x @ Wg.T, x @ Wu.T
    ref = (g / (1.0 + np.exp(-g)) * u) @ Wd.T
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    x[1, 7] = np.nan
    y2, bad2 = O.mlp_forward(x, (12, bg), (12, bu), (14, bd), H, I)
    assert bad2 and np.isnan(y2[1]).all() and np.isfinite(y2[[0, 2]]).all()


def test_router_logits_matches_f64(O):
    """Router Linear (core_layers.rs:118-140): x @ W^T + b against f64; the bias is added
    after the product (a missing or doubled bias fails)."""
    import nn_amd
    x = nn_amd.synth_normal(11, 1, (5, 96), 1.0)
    w = nn_amd.synth_normal(11, 2, (8, 96), 0.1)
    b = nn_amd.synth_normal(11, 3, (8,), 1.0)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b.astype(np.float64)
    got = O.router_logits(x, w, b)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    assert np.abs(O.router_logits(x, w) + b - ref).max() <= 1e-5 * np.abs(ref).max()


# ---- token sampling (crates/nn-gptoss/src/sampling.rs) ---------------------------------


def test_sample_token_reference_cases(O):
    """The reference's own sample_token tests (sampling.rs:566-606) and its step tests
    restated through the whole pipeline."""
    greedy = dict(temperature=1e-7, top_k=1, top_p=None)
    assert O.sample_token([1.0, 5.0, 3.0, 0.5], **greedy) == 1
    assert O.sample_token([3.9, 4.0, 3.8], repetition_penalty=10.0, past_tokens=[1], **greedy) == 0
    assert O.sample_token([1.01, 1.0, 1.0, 1.0, 1.0], temperature=1e-7, top_k=1, top_p=0.9) == 0
    # top_k larger than the vocabulary keeps every finite logit; top_p = 1 keeps all
    picks = {O.sample_token([1.0, 2.0, 3.0], temperature=1.0, top_k=10, top_p=1.0, seed=s) for s in range(0, 10000, 37)}
    assert picks == {0, 1, 2}
    # a very small top_p keeps only the peak (sampling.rs:494-500)
    assert {O.sample_token([0.0, 10.0, 0.0], temperature=1.0, top_k=None, top_p=0.01, seed=s)
            for s in range(0, 10000, 101)} == {1}
    # top_k = 0: no candidates, argmax of the original logits; max_by keeps the LAST maximum
    assert O.sample_token([1.0, 3.0, 3.0, 2.0], temperature=1.0, top_k=0, top_p=None) == 2
    assert O.argmax_slice([1.0, 3.0, 3.0, 2.0]) == 2


def test_sample_token_penalties_per_occurrence(O):
    """Repetition penalty divides positive / multiplies negative logits once per
    occurrence (:277-290); frequency penalty subtracts once per occurrence (:297-306)."""
    greedy = dict(temperature=1e-7, top_k=1, top_p=None)
    assert O.sample_token([3.0, 1.0], repetition_penalty=2.0, past_tokens=[0], **greedy) == 0    # 1.5 > 1
    assert O.sample_token([3.0, 1.0], repetition_penalty=2.0, past_tokens=[0, 0], **greedy) == 1  # 0.75 < 1
    assert O.sample_token([-1.0, -1.5], repetition_penalty=2.0, past_tokens=[0], **greedy) == 1   # -2 < -1.5
    assert O.sample_token([0.0, -0.5], repetition_penalty=9.0, past_tokens=[0], **greedy) == 0    # zero unchanged
    assert O.sample_token([1.0, 2.0], repetition_penalty=9.0, past_tokens=[5], **greedy) == 1     # out of range
    assert O.sample_token([5.0, 4.2], frequency_penalty=0.5, past_tokens=[0], **greedy) == 0     # 4.5
    assert O.sample_token([5.0, 4.2], frequency_penalty=0.5, past_tokens=[0, 0], **greedy) == 1  # 4.0


def test_sample_token_selection_matches_softmax(O):
    """Over all 10000 selector values (seed % 10000) the picks follow the softmax of
    logit / temperature in candidate (index) order: the count of each token equals the
    number of selectors in its cumulative interval, against an f64 closed form."""
    logits = np.array([0.3, -1.2, 2.0, 0.9, 1.4, -0.2], np.float32)
    T = 0.8
    counts = np.zeros(6, int)
    for s in range(10000):
        counts[O.sample_token(logits, temperature=T, top_k=4, top_p=None, seed=s)] += 1
    keep = np.argsort(-logits)[:4]
    z = logits[np.sort(keep)].astype(np.float64) / T
    p = np.exp(z - z.max())
    p /= p.sum()
    assert set(np.nonzero(counts)[0]) == set(keep.tolist())
    assert np.abs(counts[np.sort(keep)] / 10000.0 - p).max() <= 2e-4
    # with top_p the candidates are walked in descending order and cut at cumulative >= p
    z6 = logits.astype(np.float64) / T
    q = np.exp(z6 - z6.max())
    q /= q.sum()
    order = np.argsort(-logits)
    cut = int(np.searchsorted(np.cumsum(q[order]), 0.8) + 1)
    picks = {O.sample_token(logits, temperature=T, top_k=None, top_p=0.8, seed=s) for s in range(0, 10000, 7)}
    assert picks == set(order[:cut].tolist())


def test_sample_token_top_k_none_keeps_pos_inf(O):
    """top_k None makes every logit v > -inf a candidate, +inf included
    (sampling.rs:158-165); a +inf candidate makes softmax_candidates uniform
    (:371-391).  top_k Some(k >= n) keeps the finite logits only (apply_top_k,
    :250-256).  Checked over all 10000 selectors against the closed form: uniform
    probabilities 1/c walked in candidate order, cumulative sums in f32."""
    lg = np.array([0.0, np.inf, 1.0, 2.0, -np.inf], np.float32)

    def uniform_pick(cands, s):
        sel = np.float32(s % 10000) / np.float32(10000.0)
        cum = np.float32(0.0)
        for c in cands:
            cum = np.float32(cum + np.float32(1.0) / np.float32(len(cands)))
            if sel < cum:
                return c
        return cands[-1]

    for s in range(10000):
        # None, no top-p: candidates 0, 1 (+inf), 2, 3 in index order, uniform
        assert O.sample_token(lg, temperature=1.0, top_k=None, top_p=None, seed=s) == uniform_pick([0, 1, 2, 3], s)
    # the values the reference gives for two selectors (0.26 and 0.51)
    assert O.sample_token(lg, temperature=1.0, top_k=None, top_p=None, seed=2600) == 1
    assert O.sample_token(lg, temperature=1.0, top_k=None, top_p=None, seed=5100) == 2
    for s in range(0, 10000, 3):
        # None with top-p 0.6: descending order 1 (+inf), 3, 2, 0 at 1/4 each; the cut keeps
        # three (cumulative 0.75 >= 0.6), sampled uniformly in that order
        assert O.sample_token(lg, temperature=1.0, top_k=None, top_p=0.6, seed=s) == uniform_pick([1, 3, 2], s)
    # Some(k >= n): finite only, so the softmax of [0, 1, 2] over indices 0, 2, 3
    z = np.array([0.0, 1.0, 2.0])
    p = np.exp(z - z.max())
    p /= p.sum()
    counts = np.zeros(5, int)
    for s in range(10000):
        counts[O.sample_token(lg, temperature=1.0, top_k=10, top_p=None, seed=s)] += 1
    assert counts[1] == 0 and counts[4] == 0
    assert np.abs(counts[[0, 2, 3]] / 10000.0 - p).max() <= 2e-4


# ---- nn-core OCP MXFP4 (crates/nn-core/src/layers/quantized/mxfp4.rs) ------------


def _ocp_block(O, values):
    v = np.zeros(32, np.float32)
    v[:len(values)] = values
    return O.ocp_quantize(v), v


def test_ocp_mxfp4_reference_cases(O):
    """The reference's own tests (crates/nn-core/src/layers/quantized/mxfp4_tests.rs)
    restated through the oracle's block and tensor functions."""
    b, _ = _ocp_block(O, [])
    assert b[0] == 0 and (O.ocp_dequantize(b, 32) == 0).all()  # zeros, shared_exp 0 (:10-18, :330-335)
    v = (np.arange(32, dtype=np.float32) / 31.0) * 2.0 - 1.0  # [-1, 1] round trip (:22-51)
    out = O.ocp_dequantize(O.ocp_quantize(v), 32)
    assert np.isfinite(out).all() and np.abs(out - v).max() < 1.0
    v = (np.arange(32, dtype=np.float32) - 16.0) * 100.0  # large values stay finite (:54-66)
    assert np.isfinite(O.ocp_dequantize(O.ocp_quantize(v), 32)).all()
    out = O.ocp_dequantize(O.ocp_quantize(np.full(32, 3.14, np.float32)), 32)  # constant block (:69-90)
    assert (out == out[0]).all() and abs(out[0] - 3.14) < 2.0
    v = -(np.arange(32, dtype=np.float32) + 1.0) * 0.1  # negatives stay non-positive (:93-107)
    assert (O.ocp_dequantize(O.ocp_quantize(v), 32) <= 0.0).all()
    b, _ = _ocp_block(O, [1e10, 1e-10])  # dynamic range: the tiny value becomes 0 (:112-131)
    out = O.ocp_dequantize(b, 32)
    assert np.isfinite(out[:2]).all() and out[1] == 0.0
    for bad in (np.nan, np.inf, -np.inf):  # non-finite rejected (:136-166, :232-236)
        v = np.zeros(64, np.float32)
        v[33] = bad
        with pytest.raises(O.OracleError):
            O.ocp_quantize(v)
    # tensor lengths: 64 -> 2 blocks, 50 -> 2 (padded), 1 -> 1, 0 -> 0 (:169-228)
    for n, nb in ((64, 2), (50, 2), (1, 1), (0, 0)):
        data = (np.arange(n, dtype=np.float32) - n / 2) * 0.1
        b = O.ocp_quantize(data)
        assert b.size == nb * 17
        assert O.ocp_dequantize(b, n).shape == (n,)
    assert O.ocp_quantize(np.ones(1024, np.float32)).size == 32 * 17  # 544 bytes (:241-252)
    # the eight magnitudes round-trip exactly at scale 1 (shared_exp 127), both signs (:258-283)
    for m in (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0):
        assert O.ocp_decode(O.ocp_encode(m, 1.0), 1.0) == m
        if m:
            assert O.ocp_decode(O.ocp_encode(-m, 1.0), 1.0) == -m
    assert O.ocp_encode(42.0, 0.0) == 0  # zero scale encodes 0 (:286-290)
    assert O.ocp_block_scale(127) == 1.0 and O.ocp_block_scale(128) == 2.0 and O.ocp_block_scale(126) == 0.5
    assert 0.0 < O.ocp_block_scale(0) < np.inf  # (:293-303)
    v = np.array([(1 if i % 2 == 0 else -1) * (i + 1) * 0.5 for i in range(32)], np.float32)  # signs (:306-333)
    out = O.ocp_dequantize(O.ocp_quantize(v), 32)
    assert ((v > 0) <= (out >= 0)).all() and ((v < 0) <= (out <= 0)).all()
    v = np.zeros(32, np.float32)
    v[:2] = (1.0, -1.0)  # unit range: the scale holds max |v| = 1 (:343-362)
    assert 6.0 * O.ocp_block_scale(O.ocp_shared_exp(v)) >= 1.0


def test_ocp_mxfp4_kani_invariants_exhaustive(O):
    """The Kani harnesses' properties (mxfp4.rs:350-770, kani_mxfp4_extra.rs), checked
    over every input they quantify: each scale byte 0..254 is a positive finite power of
    two with scale(127) = 1 and scale(e + 1) = 2 scale(e), and byte 0 is exactly 2^-127
    (the f64 computation keeps the f32 subnormal); codes 0..7 decode monotonically to
    the magnitudes <= 6, code 8 + i is the negation of code i, codes 0 and 8 are zeros;
    and every (scale byte, code) pair decodes to the exact value magnitude * 2^(e - 127)
    (closed form in f64, rounded once)."""
    mags = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    assert O.ocp_block_scale(0) == np.float32(2.0 ** -127)
    for e in range(255):
        s = O.ocp_block_scale(e)
        assert 0.0 < s < np.inf and np.frexp(s)[0] == 0.5
        if e < 254:
            assert O.ocp_block_scale(e + 1) == 2.0 * s
        prev = -1.0
        for code in range(16):
            got = O.ocp_decode(code, s)
            want = np.float32((-1.0 if code & 8 else 1.0) * mags[code & 7] * 2.0 ** (e - 127))
            assert np.float32(got).view(np.uint32) == want.view(np.uint32), (e, code)
            if code < 8:
                assert got >= prev and got <= np.float32(6.0) * np.float32(s)  # f32: 6 * 2^127 is +inf
                prev = got
    assert O.ocp_block_scale(127) == 1.0 and O.ocp_block_scale(255) == np.inf
    # nibble independence: the low nibble holds the even element, the high the odd one
    for code_lo in range(16):
        for code_hi in range(16):
            v = np.zeros(32, np.float32)
            v[0], v[1] = O.ocp_decode(code_lo, 1.0), O.ocp_decode(code_hi, 1.0)
            v[2] = 6.0  # fixes shared_exp at 127 (6 / 6 = 1 -> log2 0)
            b = O.ocp_quantize(v)
            # encode_e1m2 gives code 0 for either zero (:99-101), so code 8 re-encodes as 0
            lo, hi = (code_lo if code_lo & 7 else 0), (code_hi if code_hi & 7 else 0)
            assert b[0] == 127 and b[1] == (hi << 4) | lo, (code_lo, code_hi)


def test_ocp_mxfp4_shared_exp_brute_force(O):
    """compute_shared_exponent (mxfp4.rs:142-170) against an f64 brute force over 2000
    block maxima across the whole range: the smallest e with max |v| <= 6 * 2^(e - 127),
    clamped to [0, 254] (away from the few maxima where log2f rounding decides), and
    every value's code is its nearest magnitude at that scale (ties to the lower)."""
    rng = np.random.default_rng(7)
    mags = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    for _ in range(2000):
        mx = np.float32(6.0 * 2.0 ** rng.uniform(-140, 130))
        if not np.isfinite(mx) or mx == 0:
            continue
        v = (rng.uniform(-1, 1, 32) * mx).astype(np.float32)
        v[rng.integers(32)] = mx
        e = O.ocp_shared_exp(v)
        amax = float(np.abs(v).max())
        want = int(np.ceil(np.log2(amax / 6.0))) + 127
        r = np.log2(amax / 6.0)
        if abs(r - round(r)) > 1e-5:
            assert e == min(max(want, 0), 254), (amax, e, want)
        s = O.ocp_block_scale(e)
        b = O.ocp_quantize(v)
        assert b[0] == e
        for i in range(32):
            code = (b[1 + i // 2] >> (4 * (i % 2))) & 15
            q = abs(float(np.float32(abs(v[i]) / np.float32(s))))
            d = np.abs(q - mags)
            best = int(np.argmin(d)) if v[i] != 0 else 0
            assert code & 7 == best, (i, v[i], q, code)
            assert (code >> 3) == (1 if v[i] < 0 else 0)
