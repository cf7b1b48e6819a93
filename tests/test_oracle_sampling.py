"""The sampling tail's oracle (oracle/model_oracle.py: splitmix64, uniform_draws, gumbel_scores, sample_token).

SplitMix64 against its published sequence for seed 0 (the generator of Steele, Lea and Flood as distributed with
xoshiro: 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F); the uniforms' grid, range and moments; the
Gumbel-max draw (reference server.py:1576-1583) against softmax(logits / temp) by a chi-square test over many
seeds, with a planted mistake (the temperature ignored) that fails it; temp -> 0 and temp <= 0 are the argmax.
"""
import numpy as np
from scipy.stats import chi2

from oracle.model_oracle import argmax_first, gumbel_scores, sample_token, splitmix64, uniform_draws

G = 0x9E3779B97F4A7C15
M = (1 << 64) - 1


def test_splitmix64_published_sequence():
    assert int(splitmix64(0)) == 0xE220A8397B1DCDAF
    assert int(splitmix64(G)) == 0x6E789E6AA1B965F4
    assert int(splitmix64((2 * G) & M)) == 0x06C45D188009454F


def test_uniform_draws_grid_range_and_moments():
    u = np.concatenate([uniform_draws(s, p, 4096) for s, p in ((0, 0), (1, 0), (0, 1), (12345, 4096))])
    assert u.dtype == np.float32 and u.min() >= 0 and u.max() < 1
    assert np.all(u * 2 ** 24 == np.floor(u * 2 ** 24))
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.005
    a, b, c = uniform_draws(7, 100, 64), uniform_draws(7, 101, 64), uniform_draws(8, 100, 64)
    assert not np.array_equal(a, b) and not np.array_equal(a, c)
    assert np.array_equal(a, uniform_draws(7, 100, 64))


def _chi2_stat(logits, temp, n, planted=False):
    p = np.exp((logits - logits.max()) / temp)
    p /= p.sum()
    counts = np.zeros(len(logits))
    for s in range(n):
        u = uniform_draws(s, 3, len(logits))
        counts[sample_token(logits, 1.0 if planted else temp, u)] += 1
    return float(((counts - n * p) ** 2 / (n * p)).sum())


def test_gumbel_max_draws_follow_the_softmax():
    logits = np.array([2.0, 1.0, 0.5, -1.0, 0.0, 1.5], np.float32)
    crit = chi2.ppf(1 - 1e-4, df=len(logits) - 1)
    assert _chi2_stat(logits, 0.7, 20000) < crit
    assert _chi2_stat(logits, 0.7, 20000, planted=True) > crit


def test_low_and_zero_temperature_are_argmax():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal(500).astype(np.float32)
    for s in range(20):
        assert sample_token(logits, 1e-4, uniform_draws(s, 0, 500)) == argmax_first(logits)
    assert sample_token(logits, 0.0, None) == argmax_first(logits)
    # clamp: u = 0 and u = 1 stay finite
    sc = gumbel_scores(np.zeros(2, np.float32), 1.0, np.array([0.0, 1.0], np.float32))
    assert np.all(np.isfinite(sc))
