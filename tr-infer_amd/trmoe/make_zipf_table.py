"""Writes zipf_bias_table.json: the per-rank router bias under which top-10 routing over the
synthetic router's Gaussian logits has the expert load of config 3 (Zipf(1.1)
routing at M = 512).

The load the config describes is each token drawing k = 10 distinct experts from Zipf(1.1) over
E = 512, i.e. Plackett-Luce sampling, whose inclusion probability pi_r of the rank-r expert is
estimated here with Gumbel-top-k draws.  The bench's router logits are x . router_e with
router rows N(0, 0.02) and x N(0, 1) at H = 2048, so each expert's logit is N(0, sigma^2) with
sigma = 0.02 sqrt(2048).  The bias b_r is fitted, with common random numbers, so that top-10
over N(0, sigma^2) + b reproduces every pi_r:
    b_r <- b_r + 0.5 sigma (logit pi_r - logit pi_hat_r)
and finally made non-increasing in rank (the order the fit estimates with Monte-Carlo noise in
the tail).  Run: python tr-infer_amd/trmoe/make_zipf_table.py  (about two minutes, CPU)."""
from __future__ import annotations

import json
import os

import numpy as np


def fit(E=512, k=10, s=1.1, sigma=0.02 * np.sqrt(2048), n_target=400_000, n_fit=100_000, iters=80, seed=0):
    rng = np.random.default_rng(seed)
    logp = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    logp -= np.log(np.exp(logp).sum())
    incl = np.zeros(E)
    for _ in range(n_target // 20_000):
        g = logp[None, :] + rng.gumbel(size=(20_000, E))
        incl += np.bincount(np.argpartition(-g, k, axis=1)[:, :k].ravel(), minlength=E)
    pi = incl / n_target
    noise = (rng.standard_normal((n_fit, E)) * sigma).astype(np.float32)
    b = 0.4 * logp
    for _ in range(iters):
        sel = np.argpartition(-(noise + b[None, :].astype(np.float32)), k, axis=1)[:, :k]
        ph = np.clip(np.bincount(sel.ravel(), minlength=E) / n_fit, 0.5 / n_fit, 1 - 0.5 / n_fit)
        b = b + 0.5 * sigma * (np.log(pi / (1 - pi)) - np.log(ph / (1 - ph)))
        b -= b.max()
    b = -np.sort(-b)  # non-increasing in rank
    return pi, b


if __name__ == "__main__":
    E, k, s, sigma = 512, 10, 1.1, 0.02 * np.sqrt(2048)
    pi, b = fit(E, k, s, sigma)
    out = {"E": E, "k": k, "s": s, "sigma": sigma, "inclusion": [round(float(v), 6) for v in pi],
           "bias": [round(float(v), 6) for v in b]}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "zipf_bias_table.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print(path, "top pi", pi[:3], "bias", b[:3], b[-3:])
