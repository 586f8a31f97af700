"""The CPU baseline bench.py times (oracle/cpu_baseline.*) computes the same path as
the oracle: its threaded decoders are bit-identical to the oracle's at any thread
count, and its MoE (numpy BLAS for the f32 products) is within f32 rounding of the
oracle's restatement, in both the faithful form (every expert decoded per expert call)
and the decode-once form.  A baseline that computed something else would time nothing."""
import numpy as np
import pytest

from oracle import cpu_baseline as CB


def test_host_info():
    h = CB.host_info()
    assert h["nproc"] >= 1 and h["affinity"] >= 1 and h["omp_num_threads"] >= 1
    assert 1 <= CB.all_threads() <= h["affinity"]


def test_decoders_match_oracle_any_threads(O):
    import nn_amd
    v = nn_amd.synth_normal(1, 1, (64, 1024), 0.02)
    b4 = O.quantize_q4_k(v)
    b6 = O.quantize_q6_k(v)
    p, s = O.mxfp4_quantize(v)
    for th in (1, 3):
        assert np.array_equal(CB.dequant_q4k(b4, v.size, th).view(np.uint32),
                              O.dequant_q4_k(b4, v.size).view(np.uint32))
        assert np.array_equal(CB.dequant_q6k(b6, v.size, th).view(np.uint32),
                              O.dequant_q6_k(b6, v.size).view(np.uint32))
        assert np.array_equal(CB.dequant_mxfp4(p, s, v.size, th).view(np.uint32),
                              O.mxfp4_dequantize(p, s, v.size).view(np.uint32))


@pytest.mark.parametrize("faithful", [False, True])
def test_moe_matches_oracle(O, faithful):
    import nn_amd
    E, H, I, T, K = 6, 64, 96, 21, 2
    gp, gs = O.mxfp4_quantize(nn_amd.synth_normal(5, 1, (E, H, 2 * I), 0.05))
    dp, ds = O.mxfp4_quantize(nn_amd.synth_normal(5, 2, (E, I, H), 0.05))
    gb = nn_amd.synth_normal(5, 3, (E, 2 * I), 0.05)
    db = nn_amd.synth_normal(5, 4, (E, H), 0.05)
    x = nn_amd.synth_normal(5, 5, (T, H), 1.0)
    lg = nn_amd.synth_normal(5, 6, (T, E), 1.0)
    ref = O.moe_forward(x, lg, K, gp, gs, gb, dp, ds, db, I)[0]
    with CB.blas_threads(2):
        got, ran = CB.moe_forward(x, lg, K, gp, gs, gb, dp, ds, db, I, faithful=faithful, threads=2)
        _, ran1 = CB.moe_forward(x, lg, K, gp, gs, gb, dp, ds, db, I, faithful=faithful, expert_limit=1)
    assert ran >= 1 and ran1 == 1
    assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()


@pytest.mark.parametrize("m,n,k", [(1, 37, 300), (5, 70, 1040), (8, 130, 2048)])
def test_matmul_and_qlinear_match_oracle(O, m, n, k):
    """The blocked f32 products (x . W^T and x . W; any m, n, k: register-block and vector
    tails) equal an f64 product to f32 rounding, at one and several threads; QLinear::forward's flow (decode,
    then the product) matches the oracle's decode followed by the same product."""
    rng = np.random.default_rng(m * 1000 + n)
    x = rng.standard_normal((m, k), dtype=np.float32)
    w = rng.standard_normal((n, k), dtype=np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    for th in (1, 3):
        y = CB.matmul_xwt(x, w, th)
        assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max() * np.sqrt(k)
        # the MoE experts' product x . W with W stored [k, n] (column strips of 64 and a
        # scalar tail, rows in fours and a ragged last group)
        y2 = CB.matmul_xw(x, np.ascontiguousarray(w.T), th)
        assert np.abs(y2 - ref).max() <= 1e-5 * np.abs(ref).max() * np.sqrt(k)
    if k % 256 == 0:
        import nn_amd
        wb = O.quantize_q4_k(nn_amd.synth_normal(7, 1, (n, k), 0.02))
        wbuf = np.empty(n * k, np.float32)
        y = np.empty((m, n), np.float32)
        CB.q4k_qlinear(wb, n, k, x, wbuf, y, 2)
        assert np.array_equal(wbuf.view(np.uint32), O.dequant_q4_k(wb, n * k).view(np.uint32))
        ref = x.astype(np.float64) @ wbuf.reshape(n, k).astype(np.float64).T
        assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max() * np.sqrt(k)
        assert CB.argmax(y[0]) == int(np.argmax(y[0]))
