"""The oracle's sampler (sample_token, src/detail/generate.cpp:68-142, with
the uniform draw supplied) pinned by what the definition fixes, and the
product's host sampler checked against it.

Pins: over exhaustive draws on tiny vocabularies, each token's share of the
unit interval equals its renormalised probability inside the kept set, and
the kept set is the top-k prefix cut to the shortest nucleus reaching top_p
(computed here in float64 from the definition, not from the oracle's code);
draws map to tokens in descending-probability order; greedy forms are the
lowest-index argmax; equal logits give token floor(u * V)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from mt64 import first_uniform


def _kept_probs(lg, T, k, p):
    """Definition: softmax(l / T) in float64, descending order (index breaks
    ties), top-k cut, shortest prefix reaching top_p (>= 1 token)."""
    x = lg.astype(np.float64) / T
    e = np.exp(x - x.max())
    pr = e / e.sum()
    order = sorted(range(len(pr)), key=lambda i: (-pr[i], i))
    keep = len(pr) if k <= 0 or k >= len(pr) else k
    if p < 1.0:
        c = 0.0
        for n, i in enumerate(order[:keep]):
            c += pr[i]
            if c >= p:
                keep = n + 1
                break
    kept = order[:keep]
    w = np.array([pr[i] for i in kept])
    return kept, w / w.sum()


@pytest.mark.parametrize("V", [3, 5, 8])
@pytest.mark.parametrize("T,k,p", [(1.0, 0, 1.0), (0.5, 0, 1.0), (2.0, 0, 1.0), (1.0, 2, 1.0), (1.0, 3, 0.6),
                                   (1.0, 0, 0.5), (0.7, 0, 0.9), (1.5, 4, 0.95)])
def test_exhaustive_draws_give_kept_probabilities(V, T, k, p):
    rng = np.random.default_rng(V * 100 + k)
    lg = rng.standard_normal(V).astype(np.float32) * 2
    kept, w = _kept_probs(lg, T, k, p)
    n = 20000
    us = (np.arange(n) + 0.5) / n
    toks = [oracle.sample_token(lg, T, k, p, float(u))[0] for u in us]
    # every token drawn is kept; shares equal the renormalised probabilities
    assert set(toks) <= set(kept)
    share = np.array([toks.count(i) for i in kept]) / n
    np.testing.assert_allclose(share, w, atol=1.5 / n + 1e-6)
    # intervals follow descending probability: the draw sequence visits the
    # kept tokens in that order, each once
    runs = [t for j, t in enumerate(toks) if j == 0 or toks[j - 1] != t]
    assert runs == [i for i, wi in zip(kept, w) if wi * n >= 1.5]


def test_greedy_forms_and_uniform_closed_form():
    lg = np.array([0.5, 2.0, 2.0, -1.0, 1.9], np.float32)
    for T, k in ((0.0, 0), (-1.0, 40), (1.0, 1)):
        assert oracle.sample_token(lg, T, k, 0.9, 0.99)[0] == 1   # lowest index of the tied max
    V = 7
    flat = np.zeros(V, np.float32)
    for j in range(200):
        u = (j + 0.37) / 200
        assert oracle.sample_token(flat, 1.0, 0, 1.0, u)[0] == int(u * V)


def test_margin_locates_the_boundary():
    lg = np.log(np.array([0.5, 0.3, 0.2], np.float32))
    t, m = oracle.sample_token(lg, 1.0, 0, 1.0, 0.49)
    assert t == 0 and m == pytest.approx(0.01, abs=1e-6)
    t, m = oracle.sample_token(lg, 1.0, 0, 1.0, 0.81)
    assert t == 2 and m == pytest.approx(0.01, abs=1e-6)


def test_host_sampler_equals_oracle():
    """brolm_sample_token (generate.cpp's algorithm in the product, its draw
    from std::mt19937_64(seed)) picks the oracle's token for the same draw."""
    import brolm_amd as ba
    rng = np.random.default_rng(11)
    for V in (50, 1000, 151936):
        lg = (rng.standard_normal(V) * 3).astype(np.float32)
        for T, k, p in ((1.0, 0, 1.0), (0.8, 40, 0.95), (1.3, 0, 0.8), (0.6, 5, 1.0), (2.0, 100, 0.5)):
            for seed in range(4):
                want, _ = oracle.sample_token(lg, T, k, p, first_uniform(seed))
                got = ba.sample_token(lg, ba.SamplingParams(temperature=T, top_k=k, top_p=p), seed)
                assert got == want, (V, T, k, p, seed)
