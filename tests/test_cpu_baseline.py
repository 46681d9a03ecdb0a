"""The timed CPU baseline (oracle/cpu_moe.c: the reference's moe_block / moe_batch on AVX-512 VNNI,
threaded like one tile of the reference's pool) gives the scalar oracle's bits: the per-output
arithmetic order is one core's, whatever the thread count."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from layerdata import Layer

pytestmark = pytest.mark.skipif(not O.cpu_have_vnni(), reason="host without AVX-512 VNNI")


@pytest.fixture(scope="module")
def small():
    L = Layer(seed=41, H=512, E=24, F=256)
    orc = L.oracle()
    orc.ensure(range(L.E))
    return L, orc


@pytest.mark.parametrize("threads", [1, 3, 8])
@pytest.mark.parametrize("hiprec,policy", [(True, None), (False, None), (True, (1, 8, 0.7, O.BASIS_TOP))])
def test_block_matches_oracle(small, threads, hiprec, policy):
    L, orc = small
    cpu = O.CpuMoe(threads)
    for t in range(3):
        x = L.x(1, tid=900 + t)[0]
        want = orc.moe_block(x, k=4, policy=policy, hiprec=hiprec)
        got = cpu.block(orc, x, k=4, policy=policy, hiprec=hiprec)
        assert np.array_equal(got["ids"], want["ids"])
        assert np.array_equal(got["w"].view(np.uint32), want["w"].view(np.uint32))
        assert np.array_equal(got["out"].view(np.uint32), want["out"].view(np.uint32))
    cpu.close()


@pytest.mark.parametrize("threads", [1, 5])
@pytest.mark.parametrize("M,policy", [(5, None), (37, None), (37, (1, 8, 0.7, O.BASIS_TOP))])
def test_batch_matches_oracle(small, threads, M, policy):
    L, orc = small
    cpu = O.CpuMoe(threads)
    x = L.x(M, tid=950 + M)
    want = orc.moe_batch(x, k=4, policy=policy, router_dot_max_m=16)
    got = cpu.batch(orc, x, k=4, policy=policy, router_dot_max_m=16)
    assert got["n_ent"] == want["n_ent"]
    assert np.array_equal(got["out"].view(np.uint32), want["out"].view(np.uint32))
    cpu.close()


def test_q6k_down_layer(small):
    """The 8-bit TQ8_16 GEMV (config 4's Q6_K downs) on the VNNI path, bit-identical too."""
    L = Layer(seed=42, H=512, E=8, F=256, down_fmt=O.FMT_Q6_K)
    orc = L.oracle()
    orc.ensure(range(L.E))
    cpu = O.CpuMoe(4)
    x = L.x(9, tid=970)
    want = orc.moe_batch(x, k=3, router_dot_max_m=16)
    got = cpu.batch(orc, x, k=3, router_dot_max_m=16)
    assert np.array_equal(got["out"].view(np.uint32), want["out"].view(np.uint32))
    r = cpu.block(orc, x[0], k=3)
    assert np.array_equal(r["out"].view(np.uint32), orc.moe_block(x[0], k=3)["out"].view(np.uint32))
    cpu.close()
