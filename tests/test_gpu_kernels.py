"""Kernel-level parity on the GPU: each HIP kernel against the oracle on the same seeded inputs.

Bar: bit-exact for integer/byte work (quantisation, generators, routing ids) and for the f32
arithmetic the reference fixes (GEMV epilogue, dot orders, exp512/SwiGLU, RMSNorm).  Routing
weights use libm expf on the CPU and a double-rounded exp on the GPU: they may differ by one ulp
(tolerance written below)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle as O
import trmoe

pytestmark = pytest.mark.gpu


def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test on a host without a GPU"
    return torch


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(a):
    torch = torch_dev()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def ulp_diff(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


@pytest.mark.parametrize("fmt,rows,K", [(O.FMT_Q4_K, 33, 2048), (O.FMT_Q6_K, 17, 512), (O.FMT_Q8_0, 9, 768), (O.FMT_Q5_1, 9, 768)])
def test_generator_bytes_match_oracle(fmt, rows, K):
    say(f"gen_gguf fmt={fmt} rows={rows} K={K}")
    g = host(trmoe.gen_gguf(fmt, 7, (3 << 32) | 99, rows, K))
    o = O.gen_gguf(fmt, 7, (3 << 32) | 99, rows, K)
    assert np.array_equal(g, o)
    say("gen_normal")
    gn = host(trmoe.gen_normal(7, 5, 4096, 0.02))
    on = O.gen_normal(7, 5, 4096, 0.02)
    assert np.allclose(gn, on, rtol=1e-6, atol=1e-12)


@pytest.mark.parametrize("kb", [16, 32])
@pytest.mark.parametrize("m", [1, 5])
def test_quantize_rows_bit_exact(kb, m):
    say(f"quantize rows kb={kb} m={m}")
    rng = np.random.default_rng(kb + m)
    x = (rng.standard_normal((m, 2048)) * 3).astype(np.float32)
    x[0, :kb] = 0.0                                   # all-zero block
    x[0, kb:2 * kb] = np.arange(kb) - kb / 2 + 0.5    # exact .5 ties after scaling
    q, s, su = trmoe.quantize(to_dev(x), kb)
    oq, os_, osu = O.quant_rows(x, kb)
    assert np.array_equal(host(q), oq) and np.array_equal(host(s).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(host(su), osu)


@pytest.mark.parametrize("kb", [16, 32])
def test_quantize_pair_bit_exact(kb):
    say(f"quantize pair kb={kb}")
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(2048) * 2).astype(np.float32)
    q, s, su = trmoe.quantize(to_dev(x), kb, pair=True)
    oq, os_, osu = O.quant_pair(x, kb)
    assert np.array_equal(host(q), oq) and np.array_equal(host(s).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(host(su), osu)


@pytest.mark.parametrize("m", [1, 3, 16, 37])
def test_router_logits_bit_exact(m):
    say(f"router logits m={m}")
    E, H = 512, 2048
    router = O.gen_normal(1, 1, E * H, 0.02).reshape(E, H)
    shg = O.gen_normal(1, 2, H, 0.02)
    x = O.gen_normal(1, 3, m * H, 1.0).reshape(m, H)
    bias = (O.gen_normal(1, 4, E, 1.0)).astype(np.float32)
    dr, dx, ds, db = to_dev(router), to_dev(x), to_dev(shg), to_dev(bias)
    lg, sh = trmoe.router_logits(dr, dx, bias=db, shexp_gate=ds, gemm_order=False)
    want = np.array([[np.float32(O.dot(router[e], x[i]) + bias[e]) for e in range(E)] for i in range(m)], np.float32)
    assert np.array_equal(host(lg).view(np.uint32), want.view(np.uint32))
    wsh = np.array([O.dot(shg, x[i]) for i in range(m)], np.float32)
    assert np.array_equal(host(sh).view(np.uint32), wsh.view(np.uint32))
    lg2, _ = trmoe.router_logits(dr, dx, gemm_order=True)
    want2 = O.gemm_f32_nt(x, router)
    assert np.array_equal(host(lg2).view(np.uint32), want2.view(np.uint32))


@pytest.mark.parametrize("m", [70, 300])
def test_router_gemm_tiles_bit_exact(m):
    # the gemm tiles chosen for 64 <= m < 256 and m >= 256 (smallgemm.rs:8-59 order)
    say(f"router gemm m={m}")
    E, H = 512, 2048
    router = O.gen_normal(1, 1, E * H, 0.02).reshape(E, H)
    x = O.gen_normal(1, 5, m * H, 1.0).reshape(m, H)
    lg, _ = trmoe.router_logits(to_dev(router), to_dev(x), gemm_order=True)
    want = O.gemm_f32_nt(x, router)
    assert np.array_equal(host(lg).view(np.uint32), want.view(np.uint32))


def routing_cases(E=512):
    rng = np.random.default_rng(5)
    lg = [rng.standard_normal((8, E)).astype(np.float32),
          (rng.integers(0, 40, (8, E)) * 0.25).astype(np.float32),   # many exact ties (router.rs:277-312)
          np.tile(np.array([((i * 37) % 101) * 0.1 for i in range(E)], np.float32), (2, 1))]
    peaked = np.full((1, E), -12.0, np.float32)
    for i, p in enumerate([0.61, 0.19, 0.09, 0.05, 0.025, 0.015]):
        peaked[0, i * 7] = np.float32(np.log(np.float32(p)))
    lg.append(peaked)
    nanrow = rng.standard_normal((1, E)).astype(np.float32)
    nanrow[0, ::3] = np.nan
    nanrow[0, 1::7] = -np.inf
    lg.append(nanrow)
    # more than 64 keys at or above the selection threshold: every logit equal, and 100 copies
    # of the maximum (with -0.0 / +0.0 mixed, which compare equal)
    lg.append(np.zeros((1, E), np.float32))
    signed_zero = np.zeros((1, E), np.float32)
    signed_zero[0, 1::2] = -0.0
    lg.append(signed_zero)
    hundred = np.clip(rng.standard_normal((1, E)), -4, 2.9).astype(np.float32)
    hundred[0, rng.permutation(E)[:100]] = 3.0
    lg.append(hundred)
    return np.concatenate(lg)


@pytest.mark.parametrize("E", [512, 1000])
@pytest.mark.parametrize("policy", [None, (1, 10, 0.9, O.BASIS_TOP), (1, 10, 0.95, O.BASIS_ALL), (4, 4, 0.5, O.BASIS_TOP),
                                    (1, 32, 1.0, O.BASIS_ALL), (8, 10, 0.5, O.BASIS_ALL)])
def test_route_matches_oracle(policy, E):
    say(f"route policy={policy} E={E}")
    lg = routing_cases(E)
    ids, w, n = trmoe.route(to_dev(lg), 10, policy)
    ids, w, n = host(ids).view(np.uint32), host(w), host(n)
    worst = 0
    for r in range(lg.shape[0]):
        oi, ow = O.route_mass(lg[r], *policy) if policy else O.route_topk(lg[r], 10)
        assert n[r] == len(oi), r
        assert np.array_equal(ids[r, :n[r]], oi), r
        worst = max(worst, int(ulp_diff(w[r, :n[r]], ow).max()))
    assert worst <= 1  # libm expf vs correctly rounded exp


GEMV_CASES = [(O.FMT_Q4_K, 32, 64, 2048, False, 3), (O.FMT_Q4_K, 32, 48, 512, True, 2),
              (O.FMT_Q4_K, 16, 96, 512, True, 2), (O.FMT_Q4_K, 16, 32, 256, False, 5),
              (O.FMT_Q6_K, 16, 64, 512, False, 3), (O.FMT_Q6_K, 16, 32, 256, True, 2)]


@pytest.mark.parametrize("fmt,kb,rows,K,pair,m", GEMV_CASES)
def test_gemv_mirror_bit_exact(fmt, kb, rows, K, pair, m):
    say(f"gemv fmt={fmt} kb={kb} rows={rows} K={K} pair={pair} m={m}")
    raw = O.gen_gguf(fmt, 3, 40 + fmt + kb, rows, K)
    tq, bits = O.gguf_to_tq(fmt, raw, rows, K, kb)
    x = O.gen_normal(3, 41, m * K, 1.0).reshape(m, K)
    if pair:
        qs = [O.quant_pair(x[i], kb) for i in range(m)]
        q = np.concatenate([a[0] for a in qs])
        s = np.concatenate([a[1] for a in qs])
        su = np.concatenate([a[2] for a in qs])
    else:
        q, s, su = O.quant_rows(x, kb)
    want = O.gemv_tq(tq, K, bits, kb, rows, q, s, su, pair=pair)
    y = trmoe.gemv(to_dev(raw), rows, K, fmt, 0, 1, kb, to_dev(q), to_dev(s), to_dev(su), pair=pair)
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))
    # row map + accumulate (gemm_tq_rows with rows, accumulate = true)
    logical = m
    rmap = np.array([(3 * i + 1) % (logical + 2) for i in range(logical)], np.uint32)
    base = np.ones((logical + 2, rows), np.float32)
    want2 = O.gemv_tq(tq, K, bits, kb, rows, q, s, su, pair=pair, y=base.copy(), rows=rmap, accumulate=True)
    y2 = trmoe.gemv(to_dev(raw), rows, K, fmt, 0, 1, kb, to_dev(q), to_dev(s), to_dev(su), pair=pair,
                    y=to_dev(base.copy()), rowmap=to_dev(rmap.view(np.int32)), accumulate=True)
    assert np.array_equal(host(y2).view(np.uint32), want2.view(np.uint32))


def test_swiglu_and_rmsnorm_bit_exact():
    say("swiglu / rmsnorm")
    rng = np.random.default_rng(2)
    g = (rng.standard_normal(4096 + 7) * 4).astype(np.float32)
    u = rng.standard_normal(4096 + 7).astype(np.float32)
    y = host(trmoe.swiglu(to_dev(g), to_dev(u)))
    want = O.swiglu(g, u)
    body = g.size // 16 * 16  # exp512 body: bit-exact; scalar tail uses libm expf (<= 1 ulp apart)
    assert np.array_equal(y[:body].view(np.uint32), want[:body].view(np.uint32))
    assert np.allclose(y[body:], want[body:], rtol=1e-6, atol=0)
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    w = rng.uniform(0.9, 1.1, 2048).astype(np.float32)
    yn = host(trmoe.rmsnorm(to_dev(x), to_dev(w), 1e-6))
    want = np.stack([O.rmsnorm(x[i], w, 1e-6) for i in range(3)])
    assert np.array_equal(yn.view(np.uint32), want.view(np.uint32))
    # ragged width: one 1024-wide batch, a 64-wide step, a 16-wide tail and a scalar tail
    n = 1024 + 64 + 16 + 5
    x = rng.standard_normal((2, n)).astype(np.float32)
    w = rng.uniform(0.9, 1.1, n).astype(np.float32)
    yn = host(trmoe.rmsnorm(to_dev(x), to_dev(w), 1e-6))
    want = np.stack([O.rmsnorm(x[i], w, 1e-6) for i in range(2)])
    assert np.array_equal(yn.view(np.uint32), want.view(np.uint32))
