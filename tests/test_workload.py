"""The synthetic workload helpers of the package (host side, no GPU): the counter RNG matches the
oracle's, and the Zipf router bias gives the intended expert load."""
from __future__ import annotations

import numpy as np

import oracle as O
import trmoe


def test_rng_matches_oracle():
    for seed, st, idx in [(1, 0, 0), (1, 5, 511), (7, (3 << 32) | 16, 123456789), (2**63 + 5, 2**40, 2**33)]:
        assert trmoe.rng_u64(seed, st, idx) == O.rng_u64(seed, st, idx)


def test_zipf_bias_is_scaled_log_zipf_over_a_permutation():
    E = 512
    b = trmoe.zipf_bias(1, E).astype(np.float64)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    want = np.sort((trmoe.ZIPF_BIAS_SCALE * np.log(p)).astype(np.float32).astype(np.float64))
    assert np.array_equal(np.sort(b), want)
    assert not np.array_equal(b, (trmoe.ZIPF_BIAS_SCALE * np.log(p)).astype(np.float32))  # permuted
    assert np.array_equal(trmoe.zipf_bias(1, E), trmoe.zipf_bias(1, E))


def test_zipf_bias_load_matches_distinct_zipf_draws():
    """Top-10 over N(0, 0.905^2) logits (router N(0, 0.02) rows against N(0, 1) x, H = 2048) plus
    the bias touches about as many experts, and leaves about as many empty, as drawing 10
    distinct experts per token from Zipf(1.1) (Gumbel-top-k: 464 touched, 48 empty at M = 512)."""
    E, M, K = 512, 512, 10
    b = trmoe.zipf_bias(1, E)
    rng = np.random.default_rng(3)
    touched, empty = [], []
    for _ in range(4):
        lg = rng.standard_normal((M, E)) * (0.02 * np.sqrt(2048)) + b[None, :]
        sel = np.argsort(-lg, axis=1)[:, :K]
        h = np.bincount(sel.ravel(), minlength=E)
        touched.append((h > 0).sum())
        empty.append((h == 0).sum())
    assert 430 <= np.mean(touched) <= 500, touched
    assert 25 <= np.mean(empty) <= 80, empty
