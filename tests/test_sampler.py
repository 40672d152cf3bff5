"""The oracle's restatement of Sampler (crates/nr-model/src/sample.rs), pinned by
what the mathematics fixes (the reference holds no sampler vectors):

* temperature <= 0 is argmax and leaves the state untouched (sample.rs:33-35);
* next_f32 gives multiples of 2^-24 in [0, 1), and Sampler::new keeps seed | 1;
* only the 64 largest logits are ever drawn (sample.rs:38-61);
* the empirical distribution of 60000 draws matches the closed form, computed
  in float64: softmax at temperature T over the top 64 in descending order,
  cut to the shortest prefix whose mass reaches top_p (chi-square);
* a tiny top_p always draws the maximum, and still advances the state once.
"""
import numpy as np
import pytest
from scipy import stats


def closed_form(logits, T, top_p):
    order = np.argsort(-logits.astype(np.float64), kind="stable")[:64]
    v = logits[order].astype(np.float64)
    p = np.exp((v - v[0]) / T)
    c = np.cumsum(p)
    cut = top_p * c[-1]
    n = int(np.searchsorted(c, cut) + 1)  # first prefix with mass >= cut
    margin = min(abs(c[n - 1] - cut), abs(c[n - 2] - cut) if n >= 2 else np.inf) / c[-1]
    return order[:n], p[:n] / c[n - 1], margin


def test_greedy_is_argmax(oracle):
    logits = np.random.default_rng(1).normal(0, 1, 5000).astype(np.float32)
    for T in (0.0, -1.0):
        s = oracle.Sampler(T, 0.9, 7)
        assert s.sample(logits) == int(np.argmax(logits))
        assert s.rng.value == 7


def test_next_f32_and_seed(oracle):
    assert oracle.Sampler(0.7, 0.9, 0).rng.value == 1
    assert oracle.Sampler(0.7, 0.9, 6).rng.value == 7
    s = oracle.Sampler(0.7, 0.9, 12345)
    xs = np.array([s.next_f32() for _ in range(100_000)], np.float64)
    assert xs.min() >= 0.0 and xs.max() < 1.0
    assert np.all(xs * (1 << 24) == np.floor(xs * (1 << 24)))
    assert abs(xs.mean() - 0.5) < 0.005


def test_only_the_top_64_are_drawn(oracle):
    logits = np.random.default_rng(2).normal(0, 1, 5000).astype(np.float32)
    top = set(np.argsort(-logits)[:64].tolist())
    s = oracle.Sampler(50.0, 1.0, 3)  # nearly flat over the candidates
    seen = {s.sample(logits) for _ in range(20_000)}
    assert seen <= top
    assert len(seen) == 64


@pytest.mark.parametrize("T,top_p,seed", [(0.8, 0.9, 99), (1.3, 0.6, 5), (0.5, 0.95, 17)])
def test_distribution_matches_closed_form(oracle, T, top_p, seed):
    logits = np.random.default_rng(seed).normal(0, 1.5, 300).astype(np.float32)
    ids, probs, margin = closed_form(logits, T, top_p)
    assert margin > 1e-4, "the f32 and f64 cuts could disagree for this case"
    s = oracle.Sampler(T, top_p, seed)
    n = 60_000
    draws = np.array([s.sample(logits) for _ in range(n)])
    assert set(np.unique(draws).tolist()) <= set(ids.tolist())
    obs = np.array([(draws == i).sum() for i in ids], np.float64)
    exp = probs * n
    keep = exp >= 5  # chi-square bins need expected counts >= 5; pool the rest
    o = np.append(obs[keep], obs[~keep].sum())
    e = np.append(exp[keep], exp[~keep].sum())
    if e[-1] < 5:
        o, e = o[:-1], e[:-1]
        o[-1] += obs[~keep].sum()
        e[-1] += exp[~keep].sum()
    chi2 = float(((o - e) ** 2 / e).sum())
    assert stats.chi2.sf(chi2, len(o) - 1) > 1e-4, chi2


def test_tiny_top_p_draws_the_max(oracle):
    logits = np.random.default_rng(4).normal(0, 1, 1000).astype(np.float32)
    s = oracle.Sampler(0.9, 1e-7, 11)
    ref = oracle.Sampler(0.9, 1e-7, 11)
    for _ in range(50):
        assert s.sample(logits) == int(np.argmax(logits))
        ref.next_f32()
    assert s.rng.value == ref.rng.value
