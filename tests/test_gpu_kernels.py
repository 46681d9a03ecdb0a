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


@pytest.mark.parametrize("m,E,H", [(512, 512, 2048), (700, 96, 768), (1024, 512, 2048), (1100, 80, 512),
                                   (1057, 96, 2560), (3072, 512, 2048)])
def test_router_mfma_bit_exact(m, E, H):
    """The matrix-core router gemm (m >= 512): the same bits as gemm_f32_nt's chains and halving
    tree, with ragged token and expert tiles, a bias, and the full shapes of configs 3 and 4."""
    say(f"router mfma m={m} E={E} H={H}")
    router = O.gen_normal(2, 1, E * H, 0.02).reshape(E, H)
    x = O.gen_normal(2, 5, m * H, 1.0).reshape(m, H)
    bias = O.gen_normal(2, 6, E, 1.0).astype(np.float32)
    lg, _ = trmoe.router_logits(to_dev(router), to_dev(x), bias=to_dev(bias), gemm_order=True)
    want = (O.gemm_f32_nt(x, router) + bias[None, :]).astype(np.float32)
    got = host(lg)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.abs(got - want).max()


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


def act_rows(x, kb, pair):
    """int8 activation rows as the reference quantises them: one row each, or (coarse, residual)
    pairs (quant.rs:36-53)."""
    if not pair:
        return O.quant_rows(x, kb)
    qs = [O.quant_pair(x[i], kb) for i in range(x.shape[0])]
    return tuple(np.concatenate([a[c] for a in qs]) for c in range(3))


def gemv_check(w_dev, w_tq, rows, K, fmt, bits, kb, x, pair, strips):
    """trk_gemv against the oracle's gemm_tq_rows on the same TQ bytes: identity rows, then a row
    map with repeats (accumulate and overwrite) into a wider y (ldy > rows)."""
    q, s, su = act_rows(x, kb, pair)
    m = x.shape[0]
    nstrips = (rows + 15) // 16
    s0, s1 = strips if strips else (0, nstrips)
    width = 16 * nstrips  # the oracle stores whole strips
    cut = width if fmt in trmoe.TQ_FMTS else rows  # GGUF rows past `rows` are never written
    want = O.gemv_tq(w_tq, K, bits, kb, width, q, s, su, pair=pair, s0=s0, s1=s1)
    y = trmoe.gemv(w_dev, rows, K, fmt, 0, 1, kb, to_dev(q), to_dev(s), to_dev(su), pair=pair, s0=s0, s1=s1,
                   y=to_dev(np.zeros((m, width), np.float32)), ldy=width)
    got = host(y)
    assert np.array_equal(got[:, :cut].view(np.uint32), want[:, :cut].view(np.uint32))
    assert not got[:, cut:].any()
    # a row map with repeats: logical rows in order onto 3 y rows of pitch width + 5
    rmap = np.array([(2 * i + 1) % 3 for i in range(m)], np.uint32)
    ldy = width + 5
    for acc in (True, False):
        base = np.arange(3 * ldy, dtype=np.float32).reshape(3, ldy) * 0.25
        want2 = O.gemv_tq(w_tq, K, bits, kb, width, q, s, su, pair=pair, y=base.copy(), rows=rmap,
                          accumulate=acc, s0=s0, s1=s1, ldy=ldy)
        y2 = trmoe.gemv(w_dev, rows, K, fmt, 0, 1, kb, to_dev(q), to_dev(s), to_dev(su), pair=pair,
                        y=to_dev(base.copy()), ldy=ldy, rowmap=to_dev(rmap.view(np.int32)), accumulate=acc,
                        s0=s0, s1=s1)
        got2 = host(y2)
        c0, c1 = 16 * s0, min(16 * s1, cut)
        assert np.array_equal(got2[:, c0:c1].view(np.uint32), want2[:, c0:c1].view(np.uint32)), acc
        keep = np.ones(ldy, bool)
        keep[c0:c1] = False
        assert np.array_equal(got2[:, keep], base[:, keep]), acc


# GGUF matrices read as their TQ conversion: every format and kb, sub-ranges of strips, rows not
# a multiple of 16, one to nine activation rows (passes of four), pairs
GEMV_GGUF_CASES = [(O.FMT_Q4_K, 32, 64, 2048, False, 3, None), (O.FMT_Q4_K, 32, 48, 512, True, 4, (1, 3)),
                   (O.FMT_Q4_K, 16, 96, 512, True, 6, (1, 5)), (O.FMT_Q4_K, 16, 40, 256, False, 5, None),
                   (O.FMT_Q6_K, 16, 64, 512, False, 3, (2, 4)), (O.FMT_Q6_K, 16, 40, 2048, True, 2, None),
                   (O.FMT_Q8_0, 32, 64, 512, False, 9, None), (O.FMT_Q8_0, 16, 48, 768, True, 4, (1, 3)),
                   (O.FMT_Q5_1, 32, 64, 1024, False, 1, None), (O.FMT_Q5_1, 16, 80, 512, False, 7, (2, 5))]


@pytest.mark.parametrize("fmt,kb,rows,K,pair,m,strips", GEMV_GGUF_CASES)
def test_gemv_gguf_bit_exact(fmt, kb, rows, K, pair, m, strips):
    say(f"gemv gguf fmt={fmt} kb={kb} rows={rows} K={K} pair={pair} m={m} strips={strips}")
    raw = O.gen_gguf(fmt, 3, 40 + fmt + kb, rows, K)
    tq, bits = O.gguf_to_tq(fmt, raw, rows, K, kb)
    x = O.gen_normal(3, 41 + m, m * K, 1.0).reshape(m, K)
    gemv_check(to_dev(raw), tq, rows, K, fmt, bits, kb, x, pair, strips)


def random_tq(seed, rows, K, bits, kb):
    """A packed TQ matrix (codec.rs:1-46) of uniform q and f16 scales / mins of real magnitudes."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 1 << bits, (rows, K), dtype=np.uint8)
    nb = K // kb
    d = (rng.uniform(1e-4, 3e-3, (rows, nb)) * rng.choice([-1, 1], (rows, nb))).astype(np.float16)
    m = (-d.astype(np.float32) * rng.uniform(0, 1 << (bits - 1), (rows, nb))).astype(np.float16)
    return O.pack_tq(q, d, m, bits, kb)


# The reference's own packed codecs: its real expert shapes (gate TQ4_32 [640][2560], down
# TQ5_16 [2560][640], python/tests/test_blocks_real.py:23-26), k not a multiple of 256, ragged
# slices (33 blocks), padded strips, sub-ranges, pairs and row maps
GEMV_TQ_CASES = [(4, 32, 640, 2560, False, 1, None), (5, 16, 2560, 640, False, 1, None),
                 (5, 16, 2560, 640, True, 2, (40, 100)), (4, 16, 40, 80, False, 5, None),
                 (8, 16, 64, 96, False, 9, (1, 3)), (8, 32, 48, 2048, True, 6, None),
                 (5, 32, 100, 320, False, 3, None), (4, 32, 64, 1056, False, 4, (0, 2)),
                 (8, 16, 2560, 640, False, 2, (3, 160))]


@pytest.mark.parametrize("bits,kb,rows,K,pair,m,strips", GEMV_TQ_CASES)
def test_gemv_tq_bit_exact(bits, kb, rows, K, pair, m, strips):
    say(f"gemv tq bits={bits} kb={kb} rows={rows} K={K} pair={pair} m={m} strips={strips}")
    fmt = (bits << 8) | kb
    tq = random_tq(7 + bits + kb + m, rows, K, bits, kb)
    assert tq.size == trmoe.matrix_bytes(fmt, rows, K)
    x = O.gen_normal(4, 50 + m, m * K, 1.0).reshape(m, K)
    gemv_check(to_dev(tq), tq, rows, K, fmt, bits, kb, x, pair, strips)


@pytest.mark.parametrize("m", [1, 70, 300, 512])
def test_designed_rounding_orders(m):
    """The designed cases that pin the oracle's f32 orders (test_oracle.py: test_gemv_epilogue_order,
    test_gemm_f32_nt_lane_map, test_rmsnorm_product_order) through the GPU kernels: the GEMV's
    two-FMA epilogue (gemv.rs:141-148), the router GEMM's lane / chain map on each of its tile paths
    (smallgemm.rs:8-59; m = 1 and 70 VALU tiles of two sizes, 300 the 16 x 16 tiles, 512 the matrix
    cores) and RMSNorm's (x r) w (elem.rs:255-262), each against the literal the case was built
    for."""
    from test_oracle import epilogue_order_case, rmsnorm_order_case
    say(f"designed rounding orders m={m}")
    w, k, bits, kb, xq, s, su = epilogue_order_case()
    y = host(trmoe.gemv(to_dev(w), 16, k, (bits << 8) | kb, 0, 1, kb, to_dev(xq), to_dev(s), to_dev(su)))
    assert y[0, 0] == np.float32(2.0 ** -10) and np.all(y[0, 1:] == 0)
    a = np.float32(1 + 2.0 ** -12)
    H, E = 256, 8
    router = np.zeros((E, H), np.float32)
    router[0, 0], router[0, 16] = a, a
    router[1, 0], router[1, 16], router[1, 1] = 1e8, -1e8, 1.0
    router[2, 0], router[2, 8], router[2, 1] = 1e8, 1.0, -1e8
    x = np.ones((m, H), np.float32)
    x[:, 0], x[:, 16] = a, -a
    # row 0: the fused chain of lane 0 leaves -2^-24; rows 1 and 2 see x = a at k = 0 and -a at
    # k = 16, so their designed sums are taken on rows of ones
    lg, _ = trmoe.router_logits(to_dev(router), to_dev(x), gemm_order=True)
    assert np.all(host(lg)[:, 0] == np.float32(-(2.0 ** -24)))
    lg, _ = trmoe.router_logits(to_dev(router), to_dev(np.ones((m, H), np.float32)), gemm_order=True)
    got = host(lg)
    assert np.all(got[:, 1] == 1.0) and np.all(got[:, 2] == 0.0)
    xr, wr, want = rmsnorm_order_case()
    yr = host(trmoe.rmsnorm(to_dev(np.tile(xr, (2, 1))), to_dev(wr), 0.0))
    assert np.array_equal(yr.view(np.uint32), np.tile(want, (2, 1)).view(np.uint32))


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
