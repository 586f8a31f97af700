"""GPU parity for token sampling (sample_token, crates/nn-gptoss/src/sampling.rs:136-185).

nnq_sample_token runs penalties, temperature, the top-k over the whole vocabulary (a
two-pass select up to 16384 candidates, every key sorted beyond), top-p, softmax and the
selector walk on the device.  The picked token must equal the
oracle's restatement of sample_token on the same logits, for every configuration and
seed tried (the only freedom the reference leaves, the order of exactly equal logits at
the k-th place, does not arise with these inputs).  nnq_linear_sample (Q6_K LM head +
sampling) is checked the same way on the logits it produced, and those logits against
the oracle's GEMV with the linear bars.
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


def pick(logits_np, dev, **cfg):
    import nn_amd
    t = torch.from_numpy(np.asarray(logits_np, np.float32)).to(dev)
    return int(nn_amd.sample_token(t, **cfg).item())


def test_sample_reference_cases(O, dev):
    greedy = dict(temperature=1e-7, top_k=1, top_p=None)
    assert pick([1.0, 5.0, 3.0, 0.5], dev, **greedy) == 1
    assert pick([3.9, 4.0, 3.8], dev, repetition_penalty=10.0, past_tokens=[1], **greedy) == 0
    assert pick([1.01, 1.0, 1.0, 1.0, 1.0], dev, temperature=1e-7, top_k=1, top_p=0.9) == 0
    assert pick([3.0, 1.0], dev, repetition_penalty=2.0, past_tokens=[0, 0], **greedy) == 1
    assert pick([5.0, 4.2], dev, frequency_penalty=0.5, past_tokens=[0, 0], **greedy) == 1
    assert pick([1.0, 2.0], dev, repetition_penalty=9.0, past_tokens=[5], **greedy) == 1
    assert pick([1.0, 3.0, 3.0, 2.0], dev, temperature=1.0, top_k=0, top_p=None) == 2  # argmax_slice: last max
    assert pick([0.0, 10.0, 0.0], dev, temperature=1.0, top_k=None, top_p=0.01, seed=7777) == 1


CONFIGS = [
    dict(temperature=0.7, top_k=50, top_p=0.9),
    dict(temperature=1.0, top_k=5, top_p=None),
    dict(temperature=1.3, top_k=200, top_p=0.5),
    dict(temperature=0.9, top_k=1, top_p=None),
    dict(temperature=1.0, top_k=40, top_p=0.95, repetition_penalty=1.3, frequency_penalty=0.4),
]


@pytest.mark.parametrize("n", [151936, 5000, 37])
@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_sample_vs_oracle(O, dev, n, ci):
    import nn_amd
    cfg = dict(CONFIGS[ci])
    lg = nn_amd.synth_normal(n + ci, 1, (n,), 2.0)
    lg[n // 3] = -np.inf
    if n > 100:
        lg[n // 2] = np.nan
    rng = np.random.default_rng(n + ci)
    past = rng.integers(0, n + 10, 40).tolist() + [int(np.argmax(lg))] * 3
    if "repetition_penalty" in cfg:
        cfg["past_tokens"] = past
    t = torch.from_numpy(lg).to(dev)
    for seed in (0, 1, 4999, 9999, 123456789, 31337):
        got = int(nn_amd.sample_token(t, seed=seed, **cfg).item())
        want = O.sample_token(lg, seed=seed, **cfg)
        assert got == want, (n, cfg, seed)


@pytest.mark.parametrize("top_p", [None, 0.8])
def test_sample_ties_around_register_tail(O, dev, top_p):
    """Top-k up to 64 is sorted and finished in registers, from 65 on in LDS: logits with
    few distinct values (many exact ties, broken by the lower index) for k on both sides
    of that boundary, against the oracle."""
    import nn_amd
    n = 5000
    lg = np.round(nn_amd.synth_normal(77, 1, (n,), 1.5) * 2.0).astype(np.float32) / 2.0
    t = torch.from_numpy(lg).to(dev)
    for k in (2, 17, 33, 63, 64, 65, 128):
        for seed in (0, 3333, 9999):
            got = int(nn_amd.sample_token(t, temperature=1.0, top_k=k, top_p=top_p, seed=seed).item())
            assert got == O.sample_token(lg, temperature=1.0, top_k=k, top_p=top_p, seed=seed), (k, top_p, seed)


def test_sample_top_k_none_small_vocab(O, dev):
    import nn_amd
    n = 3000
    lg = nn_amd.synth_normal(3, 1, (n,), 1.5)
    t = torch.from_numpy(lg).to(dev)
    for seed in (3, 5000, 9998):
        assert int(nn_amd.sample_token(t, temperature=1.0, top_k=None, top_p=None, seed=seed).item()) == \
            O.sample_token(lg, temperature=1.0, top_k=None, top_p=None, seed=seed)
        assert int(nn_amd.sample_token(t, temperature=0.8, top_k=None, top_p=0.7, seed=seed).item()) == \
            O.sample_token(lg, temperature=0.8, top_k=None, top_p=0.7, seed=seed)


def test_sample_errors(O, dev):
    import nn_amd
    t = torch.zeros(151936, device=dev)
    with pytest.raises(nn_amd.TensorError):
        nn_amd.sample_token(t, temperature=0.0)
    with pytest.raises(nn_amd.TensorError):
        nn_amd.sample_token(t, temperature=float("inf"))


def test_lm_head_sample_q6k(O, dev):
    """Config 3's LM head (Q6_K 151936 x 4096, nn-gguf layout) fused with sampling."""
    import nn_amd
    n, k = 151936, 4096
    wb = nn_amd.quantize_q6_k(nn_amd.synth_normal(3, 1, (n, k), 0.02))
    w = nn_amd.QuantizedWeight.from_quantized(wb, nn_amd.QuantType.Q6_K, (n, k), layout=nn_amd.Layout.NN_GGUF)
    x = torch.from_numpy(nn_amd.synth_normal(3, 2, (k,), 1.0)).to(dev)
    for seed, cfg in [(17, dict(temperature=0.7, top_k=50, top_p=0.9)), (4242, dict(temperature=1.0, top_k=1,
                                                                                   top_p=None))]:
        logits, tok = nn_amd.linear_sample(x, w, seed=seed, **cfg)
        lg = logits.cpu().numpy()
        assert int(tok.item()) == O.sample_token(lg, seed=seed, **cfg)
    ref = O.q6k_linear(x.cpu().numpy()[None, :], wb, n)
    check_close(ref, lg[None, :], "lm head logits")


@pytest.mark.parametrize("top_p", [None, 0.9])
def test_sample_infinite_logits(O, dev, top_p):
    """With top_k Some(k), +inf logits take top-k places but are not candidates
    (apply_top_k keeps finite values, sampling.rs:245-275); -inf and NaN sort last."""
    import nn_amd
    n = 9000
    lg = nn_amd.synth_normal(21, 1, (n,), 1.0)
    lg[[5, 77, 4000]] = np.inf
    lg[[6, 78]] = -np.inf
    lg[[7, 8000]] = np.nan
    t = torch.from_numpy(lg).to(dev)
    for seed in (0, 2500, 9999):
        for k in (3, 10, 64):
            got = int(nn_amd.sample_token(t, temperature=1.0, top_k=k, top_p=top_p, seed=seed).item())
            assert got == O.sample_token(lg, temperature=1.0, top_k=k, top_p=top_p, seed=seed), (k, seed)


@pytest.mark.parametrize("top_p", [None, 0.6, 0.999])
@pytest.mark.parametrize("n", [5, 9000, 16384])
def test_sample_top_k_none_pos_inf(O, dev, n, top_p):
    """top_k None: every logit v > -inf is a candidate, +inf included (sampling.rs:158-165),
    so a +inf logit makes the softmax uniform over all candidates (:371-391); the walk
    runs in index order, or in descending order after the top-p cut."""
    import nn_amd
    if n == 5:
        lg = np.array([0.0, np.inf, 1.0, 2.0, -np.inf], np.float32)
    else:
        lg = nn_amd.synth_normal(n + 7, 1, (n,), 1.5)
        lg[[3, n // 2, n - 1]] = np.inf
        lg[[4, 100]] = -np.inf
        lg[[5, n - 2]] = np.nan
    t = torch.from_numpy(lg).to(dev)
    for seed in (0, 1, 2600, 5100, 7499, 9999):
        got = int(nn_amd.sample_token(t, temperature=0.8, top_k=None, top_p=top_p, seed=seed).item())
        assert got == O.sample_token(lg, temperature=0.8, top_k=None, top_p=top_p, seed=seed), (n, top_p, seed)
    # without +inf, None keeps the finite logits: the ordinary softmax
    if n > 5:
        lg2 = lg.copy()
        lg2[~np.isfinite(lg2)] = -1.0
        t2 = torch.from_numpy(lg2).to(dev)
        for seed in (11, 4321):
            got = int(nn_amd.sample_token(t2, temperature=0.8, top_k=None, top_p=top_p, seed=seed).item())
            assert got == O.sample_token(lg2, temperature=0.8, top_k=None, top_p=top_p, seed=seed), (n, top_p, seed)


# Beyond the two-pass capacity (ceil(n / 2048) * min(k, 2048) > 16384 candidates) every
# key is sorted on the device: top_k None and large k over the Qwen3 vocabulary, with and
# without top-p, penalties, and infinite / NaN logits.
LARGE = [
    dict(temperature=0.7, top_k=None, top_p=None),
    dict(temperature=0.7, top_k=None, top_p=0.9),
    dict(temperature=1.0, top_k=None, top_p=0.5, repetition_penalty=1.3, frequency_penalty=0.2),
    dict(temperature=0.9, top_k=5000, top_p=None),
    dict(temperature=1.1, top_k=60000, top_p=0.95),
    dict(temperature=0.8, top_k=151936, top_p=None),
]


@pytest.mark.parametrize("ci", range(len(LARGE)))
@pytest.mark.parametrize("n", [151936, 20000])
def test_sample_large_candidate_sets(O, dev, n, ci):
    import nn_amd
    cfg = dict(LARGE[ci])
    lg = nn_amd.synth_normal(n + 31 * ci, 1, (n,), 3.0)
    past = [5, 5, 77, 1000, n - 1] if "repetition_penalty" in cfg else None
    t = torch.from_numpy(lg).to(dev)
    for seed in (0, 4321, 9999):
        got = int(nn_amd.sample_token(t, seed=seed, past_tokens=past, **cfg).item())
        want = O.sample_token(lg, seed=seed, past_tokens=past, **cfg)
        assert got == want, (n, cfg, seed)


@pytest.mark.parametrize("top_k,top_p", [(None, None), (None, 0.7), (30000, None), (30000, 0.99)])
def test_sample_large_infinite_logits(O, dev, top_k, top_p):
    """+inf, -inf and NaN logits in the sorted path: with top_k None a +inf logit is a
    candidate and the softmax uniform (sampling.rs:158-165, 371-391); with Some(k) only
    finite logits are candidates."""
    import nn_amd
    n = 40000
    lg = nn_amd.synth_normal(77, 1, (n,), 2.0)
    lg[[10, 20000]] = np.inf
    lg[[11, 39999]] = -np.inf
    lg[[12, 30000]] = np.nan
    t = torch.from_numpy(lg).to(dev)
    for seed in (1, 5000, 9998):
        got = int(nn_amd.sample_token(t, temperature=1.0, top_k=top_k, top_p=top_p, seed=seed).item())
        assert got == O.sample_token(lg, temperature=1.0, top_k=top_k, top_p=top_p, seed=seed), (top_k, top_p, seed)
