"""The synthetic workload helpers of the package (host side, no GPU): the counter RNG matches the
oracle's, and the Zipf router bias gives the intended expert load."""
from __future__ import annotations

import numpy as np

import oracle as O
import trmoe


def test_rng_matches_oracle():
    for seed, st, idx in [(1, 0, 0), (1, 5, 511), (7, (3 << 32) | 16, 123456789), (2**63 + 5, 2**40, 2**33)]:
        assert trmoe.rng_u64(seed, st, idx) == O.rng_u64(seed, st, idx)


def test_zipf_bias_is_the_fitted_rank_table_over_a_permutation():
    E = 512
    b = trmoe.zipf_bias(1, E).astype(np.float64)
    table = trmoe.zipf_rank_bias(E, 1.1)
    assert table is not None and table.size == E and np.all(np.diff(table) <= 0)
    assert np.array_equal(np.sort(b), np.sort(table.astype(np.float32).astype(np.float64)))
    assert not np.array_equal(b, table.astype(np.float32))  # permuted
    assert np.array_equal(trmoe.zipf_bias(1, E), trmoe.zipf_bias(1, E))
    # other shapes, or an explicit scale: the scaled log-Zipf form
    p = 1.0 / np.arange(1, 65) ** 1.1
    p /= p.sum()
    want = np.sort((0.4 * np.log(p)).astype(np.float32))
    assert np.array_equal(np.sort(trmoe.zipf_bias(1, 64)), want)


def test_zipf_table_inclusion_is_plackett_luce_of_zipf():
    """The table's target inclusion probabilities are those of drawing 10 distinct experts per
    token from Zipf(1.1) (Plackett-Luce): they sum to k, fall with rank, and a fresh Gumbel-top-k
    sample of the same law agrees with them."""
    import json
    t = json.load(open(trmoe.ZIPF_TABLE))
    pi = np.array(t["inclusion"])
    assert abs(pi.sum() - 10) < 1e-4 and np.all(np.diff(pi[:50]) < 0)  # stored to 6 decimals
    rng = np.random.default_rng(11)
    logp = -1.1 * np.log(np.arange(1, 513))
    g = logp[None, :] + rng.gumbel(size=(20_000, 512))
    ph = np.bincount(np.argpartition(-g, 10, axis=1)[:, :10].ravel(), minlength=512) / 20_000
    assert np.abs(ph - pi).max() < 0.012


def test_zipf_bias_load_matches_distinct_zipf_draws():
    """Top-10 over N(0, 0.905^2) logits (router N(0, 0.02) rows against N(0, 1) x, H = 2048) plus
    the bias loads the experts as drawing 10 distinct experts per token from Zipf(1.1) does: at
    M = 512 about 460 touched, about 50 empty, the largest group about 465 rows, median 3."""
    E, M, K = 512, 512, 10
    b = trmoe.zipf_bias(1, E)
    rng = np.random.default_rng(3)
    stats = []
    for _ in range(6):
        lg = rng.standard_normal((M, E)) * (0.02 * np.sqrt(2048)) + b[None, :]
        h = np.bincount(np.argsort(-lg, axis=1)[:, :K].ravel(), minlength=E)
        stats.append(((h > 0).sum(), (h == 0).sum(), h.max(), np.median(h[h > 0])))
    touched, empty, mx, med = np.mean(stats, axis=0)
    assert 440 <= touched <= 485 and 27 <= empty <= 72, stats
    assert 440 <= mx <= 490, stats
    assert 2 <= med <= 5, stats
