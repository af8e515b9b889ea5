"""CPU checks of token sampling (include/ctd/sampling.h; reference
src/core/sampling.cpp) against oracle/sampling.py, and of oracle/sampling.py
against what fixes it independently:

- std::mt19937_64: the C++ standard's known answer (10000th output of a
  default-seeded engine is 9981545732273789042, [rand.predef]).
- The draw: the host sampler uses the real libstdc++ std::mt19937_64 and
  std::uniform_real_distribution<double>, so equal tokens over many seeds pin
  the oracle's restatement of both.
- The distribution: softmax(l / T) (scipy), top-k support = the k largest,
  top-p support = the shortest most-probable prefix reaching p, and empirical
  draw frequencies against the probabilities (chi-square).
- Greedy: the first index of the maximum; NaNs never win, NaN at index 0 does.
Nothing here touches the GPU.
"""
import math

import numpy as np
import pytest
from scipy.special import softmax as sp_softmax
from scipy.stats import chi2

from emberlm_amd import trainer as TR
from oracle import sampling as OS

F32 = np.float32


def oracle_draws(logits, seed, draws, **kw):
    rng = OS.MT19937_64(seed)
    return np.array([[OS.sample_row(row, rng, **kw) for row in logits] for _ in range(draws)])


# ------------------------------------------------------------- oracle pins
def test_mt19937_64_known_answer():
    r = OS.MT19937_64()
    for _ in range(9999):
        r()
    assert r() == 9981545732273789042


def test_uniform01_range_and_first_values():
    r = OS.MT19937_64(0)
    u = [OS.uniform01(r) for _ in range(20000)]
    assert min(u) >= 0.0 and max(u) < 1.0
    assert abs(np.mean(u) - 0.5) < 0.01 and abs(np.var(u) - 1 / 12) < 0.003


@pytest.mark.parametrize("T", [1.0, 0.7, 2.5])
def test_oracle_probabilities_are_tempered_softmax(T):
    rng = np.random.default_rng(1)
    z = rng.standard_normal(300).astype(F32) * 3
    p = OS.probabilities(z, T)
    ref = sp_softmax(z.astype(np.float64) / float(F32(T)))
    np.testing.assert_allclose(p, ref, rtol=2e-6, atol=1e-9)


def test_oracle_top_k_and_top_p_supports():
    rng = np.random.default_rng(2)
    z = rng.standard_normal(500).astype(F32) * 2
    k = 17
    p = OS.probabilities(z, 1.0, top_k=k)
    assert set(np.nonzero(p)[0]) == set(np.argsort(-z)[:k])
    assert math.isclose(float(p.sum(dtype=np.float64)), 1.0, rel_tol=1e-6)
    full = sp_softmax(z.astype(np.float64))
    for tp in (0.3, 0.9, 0.999):
        p = OS.probabilities(z, 1.0, top_p=tp)
        order = np.argsort(-full)
        n = int(np.searchsorted(np.cumsum(full[order]), tp) + 1)  # shortest prefix >= tp
        assert set(np.nonzero(p)[0]) == set(order[:n])
        np.testing.assert_allclose(p[order[:n]], full[order[:n]] / full[order[:n]].sum(),
                                   rtol=1e-5)


def test_oracle_draw_frequencies_follow_probabilities():
    z = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -3.0], F32)
    p = OS.probabilities(z, 0.8)
    rng = OS.MT19937_64(42)
    n = 20000
    counts = np.bincount([OS.sample_row(z, rng, 0.8) for _ in range(n)], minlength=z.size)
    stat = float(((counts - n * p) ** 2 / (n * p)).sum())
    assert stat < chi2.ppf(0.999, z.size - 1), (counts, n * p)


def test_oracle_argmax_scan_rules():
    nan, inf = float("nan"), float("inf")
    assert OS.argmax([1.0, 3.0, 3.0, 2.0]) == 1          # first of ties
    assert OS.argmax([nan, 5.0, 7.0]) == 0               # NaN first: nothing is greater
    assert OS.argmax([1.0, nan, 0.5]) == 0               # NaN later never wins
    assert OS.argmax([-inf, -inf, -inf]) == 0
    assert OS.argmax([-inf, 2.0, inf, inf]) == 2


# ------------------------------------------------ host sampler == oracle
@pytest.mark.parametrize("V,T,top_k,top_p", [
    (50, 1.0, 0, 0.0), (1000, 0.7, 0, 0.0), (1000, 1.3, 40, 0.0), (1000, 0.9, 0, 0.9),
    (257, 0.6, 25, 0.8), (1000, 1.0, 1, 0.0), (64, 2.0, 64, 0.5),
])
def test_host_sampler_matches_oracle(V, T, top_k, top_p):
    rng = np.random.default_rng(V + top_k)
    logits = (rng.standard_normal((3, V)) * 2.5).astype(F32)
    for seed in (0, 1, 12345, 2**63 + 7):
        got = TR.sample(logits, T, top_k, top_p, seed=seed, draws=4)
        ref = oracle_draws(logits, seed, 4, temperature=T, top_k=top_k, top_p=top_p)
        assert np.array_equal(got, ref), (seed, got, ref)


def test_top_k_one_is_greedy_and_tiny_top_p_is_greedy():
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((4, 300)).astype(F32)
    a = logits.argmax(1)
    for seed in range(5):
        assert np.array_equal(TR.sample(logits, 1.0, top_k=1, seed=seed)[0], a)
        assert np.array_equal(TR.sample(logits, 1.0, top_p=1e-6, seed=seed)[0], a)


def test_greedy_host_scan():
    nan, inf = float("nan"), float("inf")
    rows = np.array([[1.0, 3.0, 3.0, 2.0], [nan, 5.0, 7.0, 1.0], [1.0, nan, 0.5, 0.0],
                     [-inf, -inf, -inf, -inf], [-inf, 2.0, inf, inf]], F32)
    got = TR.sample(rows, 0.0)[0]
    assert list(got) == [OS.argmax(r) for r in rows] == [1, 0, 0, 0, 2]
    assert list(TR.sample(rows, -1.0)[0]) == [1, 0, 0, 0, 2]


def test_sampler_shape_errors():
    with pytest.raises(TR.CtdError, match="bad sizes"):
        TR.sample(np.zeros((2, 0), F32))
