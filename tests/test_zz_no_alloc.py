"""trk_moe_forward_noalloc (the layer with its workspace in the library's static device scratch, no
allocation) against trk_moe_forward on the same inputs: bit-identical outputs, on two calls in a row
whose second is smaller (the scratch keeps the first call's contents), for the decode and batch
paths and a dynamic-k policy."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle as O
import trmoe
from layerdata import Layer

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


_layers = {}


def layer(key, **kw):
    if key not in _layers:
        L = Layer(**kw)
        _layers[key] = (L, trmoe.LayerWeights.from_host(L))
    return _layers[key]


SHAPES = {"small": dict(seed=11, H=512, E=32, F=256), "full": dict(seed=1, H=2048, E=512, F=512, lazy=False)}


@pytest.mark.parametrize("shape,k,sizes,policy", [("full", 10, (40, 3), None), ("full", 10, (16, 1), None),
                                                  ("full", 10, (100, 7), None),  # 100: the largest M that fits
                                                  ("small", 4, (64, 5), None),
                                                  ("small", 4, (37, 1), (1, 8, 0.6, O.BASIS_TOP))])
def test_noalloc_matches_forward(shape, k, sizes, policy):
    import torch
    L, W = layer(shape, **SHAPES[shape])
    k_cap = 8 if policy else 0
    for i, M in enumerate(sizes):
        say(f"noalloc {shape} k={k} M={M} policy={policy} (call {i + 1} of {len(sizes)})")
        x = torch.from_numpy(L.x(M, tid=800 + M)).cuda()
        ref = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx = trmoe.Context(L.H, L.E, L.F, k, M, k_cap=k_cap)
        if policy:
            ctx.set_moe(policy)
        ctx.forward(W, x, ref)
        ctx.close()
        got = torch.full((M, L.H), float("nan"), dtype=torch.float32, device="cuda")
        trmoe.forward_noalloc(L.H, L.E, L.F, k, W, x, got, policy=policy, k_cap=k_cap)
        torch.cuda.synchronize()
        a, b = got.cpu().numpy(), ref.cpu().numpy()
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"M={M}: max {np.abs(a - b).max()}"
