"""Layer-level parity on the GPU: trk_moe_forward / trk_moe_residual against the oracle's
restatement of Model::moe_block (M = 1) and Model::moe_batch (M >= 2) on identical inputs.

Bar: top-k ids and the dispatch permutation bit-exact; Q8 activation
quantisation bit-exact; layer output within max-abs-rel 1e-3.  Where the routing weights agree
bit for bit (libm expf vs the GPU's correctly rounded exp, see test_gpu_kernels), the output is
required to be bit-identical too; otherwise within 1e-5 of the output scale."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle as O
import trmoe
from layerdata import Layer, zipf_bias

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    import torch
    assert torch.cuda.is_available()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def compare_out(got, want, w_equal, ctx=""):
    scale = float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    assert err <= 1e-3 * scale, f"{ctx}: max-abs {err} vs scale {scale}"
    if w_equal:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{ctx}: not bit-exact (max {err})"
    else:
        assert err <= 1e-5 * scale, f"{ctx}: {err} vs scale {scale}"


def ulp(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def slot_of(ids, toks, exps):
    """Slot index of expert exps[i] in token toks[i]'s selection (ids [M][k])."""
    return np.array([int(np.flatnonzero(ids[t] == e)[0]) for t, e in zip(toks, exps)], np.int64)


def _libm_expf():
    import ctypes as C
    f = C.CDLL("libm.so.6").expf
    f.restype, f.argtypes = C.c_float, [C.c_float]
    return f


_expf = None


def shared_gate_exact(L, x):
    """True when the host libm's expf, which the oracle's shared-gate sigmoid uses, gives the
    correctly rounded exp (what the GPU computes) for every row's gate logit."""
    global _expf
    if _expf is None:
        _expf = _libm_expf()
    for row in np.atleast_2d(x):
        s = np.float32(O.dot(row, L.shexp_gate))
        if np.float32(_expf(float(-s))) != np.float32(np.exp(np.float64(-s))):
            return False
    return True


_layers = {}


def layer(key, **kw):
    if key not in _layers:
        L = Layer(**kw)
        _layers[key] = (L, L.oracle(), trmoe.LayerWeights.from_host(L))
    return _layers[key]


SMALL = dict(seed=11, H=512, E=32, F=256)
FULL = dict(seed=1, H=2048, E=512, F=512, lazy=False)
WIDE = dict(seed=12, H=512, E=600, F=256)   # E > 512: 16 logits per routing lane
SHAPES = {"small": SMALL, "full": FULL, "wide": WIDE}


@pytest.mark.parametrize("shape,k,hiprec", [("small", 4, True), ("small", 4, False), ("full", 10, True),
                                            ("wide", 8, True)])
def test_decode_layer(shape, k, hiprec):
    say(f"decode layer {shape} k={k} hiprec={hiprec}")
    L, orc, W = layer(shape, **SHAPES[shape])
    ctx = trmoe.Context(L.H, L.E, L.F, k, 4, hiprec=hiprec)
    import torch
    for t in range(3):
        x = L.x(1, tid=100 + t)
        r = orc.moe_block(x[0], k=k, hiprec=hiprec)
        out = torch.empty((1, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        ids = ctx.read(trmoe.WS_IDS, 4 * 32, np.uint32)[:k]
        w = ctx.read(trmoe.WS_W, 4 * 32, np.float32)[:k]
        assert np.array_equal(ids, r["ids"])
        xq = ctx.read(trmoe.WS_XQ, 2 * L.H, np.int8)
        oq, _, _ = O.quant_pair(x[0], 32) if hiprec else O.quant_rows(x, 32)
        assert np.array_equal(xq[:oq.size], oq.reshape(-1))
        compare_out(host(out)[0], r["out"], np.array_equal(w, r["w"]) and shared_gate_exact(L, x), f"{shape} t={t}")
    assert ctx.stats() == (3, 3 * k)
    ctx.close()


@pytest.mark.parametrize("policy", [None, (1, 10, 0.9, O.BASIS_TOP), (2, 10, 0.8, O.BASIS_ALL)])
def test_decode_one_launch_matches_three(policy):
    """The one-launch decode layer (grid barriers) and the three-launch sequence give the same
    bits, both against the oracle; no barrier ever times out."""
    say(f"decode one launch vs three, policy {policy}")
    import torch
    L, orc, W = layer("full", **FULL)
    outs = {}
    for fused in (True, False):
        ctx = trmoe.Context(L.H, L.E, L.F, 10, 4)
        ctx.set_fusion(fused)
        if policy:
            ctx.set_moe(policy)
        res = []
        for t in range(3):
            x = L.x(1, tid=700 + t)
            out = torch.empty((1, L.H), dtype=torch.float32, device="cuda")
            ctx.forward(W, dev(x), out)
            res.append(host(out)[0].copy())
            if fused:
                r = orc.moe_block(x[0], k=10, hiprec=True, policy=policy)
                ids = ctx.read(trmoe.WS_IDS, 4 * 32, np.uint32)[:len(r["ids"])]
                assert np.array_equal(ids, r["ids"])
                w = ctx.read(trmoe.WS_W, 4 * 32, np.float32)[:len(r["ids"])]
                compare_out(res[-1], r["out"], np.array_equal(w, r["w"]) and shared_gate_exact(L, x), f"fused t={t}")
        assert ctx.read(trmoe.WS_BARRIER_ERR, 4, np.uint32)[0] == 0
        outs[fused] = res
        ctx.close()
    for a, b in zip(outs[True], outs[False]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("shape,M,k", [("small", 4, 4), ("small", 16, 4), ("small", 37, 6), ("full", 4, 10),
                                       ("full", 8, 10), ("full", 16, 10), ("small", 700, 3), ("small", 2200, 2),
                                       ("odd", 2100, 5)])
def test_batch_layer_and_dispatch(shape, M, k):
    # M = 700: the split (parallel) scatter; M = 2200: three rounds of 1024 tokens, 35 chunks;
    # from M = 2048 the gate/up runs item pairs of one expert as 32-row tiles (odd: 3 superblocks)
    say(f"batch layer {shape} M={M} k={k}")
    L, orc, W = layer(shape, **{"small": SMALL, "full": FULL, "odd": ODD}[shape])
    ctx = trmoe.Context(L.H, L.E, L.F, k, max(64, M))
    ctx.set_decode_rows(0)  # the grouped path, which writes the dispatch arrays
    import torch
    x = L.x(M, tid=200 + M)
    r = orc.moe_batch(x, k=k, router_dot_max_m=16)
    out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
    ctx.forward(W, dev(x), out)
    rlog = ctx.read(trmoe.WS_RLOG, M * L.E * 4, np.float32).reshape(M, L.E)
    assert np.array_equal(rlog.view(np.uint32), r["rlog"].view(np.uint32))
    ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)[:, :k]
    w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)[:, :k]
    assert np.array_equal(ids, r["ids"][:, :k])
    ng, n_ent = ctx.read(trmoe.WS_NGROUPS, 16, np.uint32)[:2]
    assert (ng, n_ent) == (r["n_groups"], r["n_ent"])
    assert ctx.stats() == (M, n_ent)  # MoeStats: rows and selected experts
    assert np.array_equal(ctx.read(trmoe.WS_ENT_TOK, 4 * n_ent, np.uint32), r["ent_tok"])
    assert np.array_equal(ctx.read(trmoe.WS_ENT_EXP, 4 * n_ent, np.uint32), r["ent_expert"])
    assert np.array_equal(ctx.read(trmoe.WS_GRP_START, 4 * (ng + 1), np.uint32), r["grp_start"])
    assert np.array_equal(ctx.read(trmoe.WS_GRP_EXP, 4 * ng, np.uint32), r["grp_expert"])
    # ent_w: the routing weights in entry order (exact where the GPU's weights equal the oracle's,
    # which differ by at most 1 ulp of libm expf otherwise)
    ent_w = ctx.read(trmoe.WS_ENT_W, 4 * n_ent, np.float32)
    if np.array_equal(w, r["w"][:, :k]):
        assert np.array_equal(ent_w.view(np.uint32), r["ent_w"].view(np.uint32))
    else:
        assert ulp(ent_w, r["ent_w"]).max() <= 3  # w = e / sum, e from libm expf (1 ulp)
    assert np.array_equal(ent_w.view(np.uint32), w[r["ent_tok"], slot_of(ids, r["ent_tok"], r["ent_expert"])].view(np.uint32))
    xq = ctx.read(trmoe.WS_XQ, M * L.H, np.int8).reshape(M, L.H)
    assert np.array_equal(xq, O.quant_rows(x, 32)[0])
    compare_out(host(out), r["out"], np.array_equal(w, r["w"][:, :k]) and shared_gate_exact(L, x), f"{shape} M={M}")
    ctx.close()


ODD = dict(seed=13, H=768, E=24, F=768)  # 3 superblocks per row: lanes of a row never straddle a wave


@pytest.mark.parametrize("shape,M,k", [("small", 4, 4), ("small", 16, 4), ("small", 37, 6), ("full", 4, 10),
                                       ("full", 16, 10), ("small", 700, 3), ("odd", 9, 5), ("odd", 40, 5),
                                       ("odd", 80, 5), ("small", 100, 3)])
def test_stream_items_match_mfma_tiles(shape, M, k):
    """Every split of the grouped items between the streaming GEMV and the int8 MFMA tiles gives
    the same bits, and matches the oracle's moe_batch."""
    say(f"stream vs mfma items {shape} M={M} k={k}")
    L, orc, W = layer(shape, **{"small": SMALL, "full": FULL, "odd": ODD}[shape])
    import torch
    x = L.x(M, tid=250 + M)
    r = orc.moe_batch(x, k=k, router_dot_max_m=16)
    outs = {}
    for rows in (0, 1, 4, 16, -1):
        ctx = trmoe.Context(L.H, L.E, L.F, k, max(64, M))
        ctx.set_stream_rows(rows)
        ctx.set_decode_rows(0)
        out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        outs[rows] = host(out).copy()
        w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)[:, :k]
        exact = np.array_equal(w, r["w"][:, :k]) and shared_gate_exact(L, x)
        compare_out(outs[rows], r["out"], exact, f"{shape} M={M} rows={rows}")
        ctx.close()
    for rows, o in outs.items():
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), f"rows={rows}"


@pytest.mark.parametrize("shape,M,k,policy", [("small", 2, 4, None), ("small", 3, 4, (1, 4, 0.9, O.BASIS_TOP)),
                                              ("full", 4, 10, None), ("full", 4, 10, (2, 10, 0.8, O.BASIS_ALL)),
                                              ("full", 16, 10, None), ("odd", 9, 5, None), ("wide", 5, 6, None)])
def test_decode_rows_match_grouped(shape, M, k, policy):
    """Batches run as per-token decode units (trk_set_decode_rows) give the grouped path's bits
    (the batch combine's order: shared expert first, then ascending expert), match the oracle's
    moe_batch, publish the same routing and count the same MoeStats."""
    say(f"decode rows {shape} M={M} k={k} policy={policy}")
    L, orc, W = layer(shape, **{"small": SMALL, "full": FULL, "odd": ODD, "wide": WIDE}[shape])
    import torch
    x = L.x(M, tid=270 + M)
    kcap = policy[1] if policy else k
    r = orc.moe_batch(x, k=k, router_dot_max_m=16, policy=policy)
    outs, routing = [], []
    for rows in (0, 16):
        ctx = trmoe.Context(L.H, L.E, L.F, k, max(64, M), k_cap=kcap)
        if policy:
            ctx.set_moe(policy)
        ctx.set_decode_rows(rows)
        out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        outs.append(host(out).copy())
        nsel = ctx.read(trmoe.WS_NSEL, 4 * M, np.uint32)
        ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
        w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)
        routing.append([(ids[t, :nsel[t]].copy(), w[t, :nsel[t]].copy()) for t in range(M)])
        assert ctx.stats() == (M, int(nsel.sum()))
        ctx.close()
    assert np.array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32)), f"{shape} M={M}: bits differ"
    for (i0, w0), (i1, w1) in zip(routing[0], routing[1]):
        assert np.array_equal(i0, i1) and np.array_equal(w0.view(np.uint32), w1.view(np.uint32))
    compare_out(outs[1], r["out"], False, f"decode rows {shape} M={M}")


def test_decode_odd_superblocks():
    """Decode with 3 superblocks per gate/up row and per down row (no power-of-two lane groups)."""
    say("decode odd superblocks")
    L, orc, W = layer("odd", **ODD)
    ctx = trmoe.Context(L.H, L.E, L.F, 5, 4)
    import torch
    for t in range(2):
        x = L.x(1, tid=120 + t)
        r = orc.moe_block(x[0], k=5)
        out = torch.empty((1, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        w = ctx.read(trmoe.WS_W, 4 * 32, np.float32)[:5]
        compare_out(host(out)[0], r["out"], np.array_equal(w, r["w"]) and shared_gate_exact(L, x), f"odd t={t}")
    ctx.close()


@pytest.mark.parametrize("M", [1, 5])
def test_dynamic_k_policy(M):
    say(f"dynamic-k M={M}")
    L, orc, W = layer("small", **SMALL)
    pol = (1, 8, 0.6, O.BASIS_TOP)
    ctx = trmoe.Context(L.H, L.E, L.F, 4, 8, k_cap=8)
    ctx.set_moe(pol)
    import torch
    x = L.x(M, tid=300)
    out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
    ctx.forward(W, dev(x), out)
    nsel = ctx.read(trmoe.WS_NSEL, 4 * M, np.uint32)
    if M == 1:
        r = orc.moe_block(x[0], k=4, policy=pol)
        assert nsel[0] == r["k"]
        w = ctx.read(trmoe.WS_W, 4 * 32, np.float32)[:r["k"]]
        compare_out(host(out)[0], r["out"], np.array_equal(w, r["w"]) and shared_gate_exact(L, x), "decode policy")
    else:
        r = orc.moe_batch(x, k=4, policy=pol)
        assert np.array_equal(nsel, r["n_sel"])
        assert 1 <= nsel.min() and nsel.max() <= 8
        ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
        w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)
        exact = shared_gate_exact(L, x)
        for t in range(M):
            assert np.array_equal(ids[t, :nsel[t]], r["ids"][t, :nsel[t]])
            exact = exact and np.array_equal(w[t, :nsel[t]], r["w"][t, :nsel[t]])
        compare_out(host(out), r["out"], exact, "batch policy")
    ctx.close()


def routing_exact(ctx, r, M, k, L, x):
    """True when the GPU's routing weights (and shared gate) equal the oracle's bit for bit: the
    outputs must then be identical too."""
    if M == 1:
        w = ctx.read(trmoe.WS_W, 4 * 32, np.float32)[:len(r["w"])]
        same = np.array_equal(w, r["w"])
    else:
        w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)[:, :k]
        same = np.array_equal(w, r["w"][:, :k])
    return same and shared_gate_exact(L, x)


@pytest.mark.parametrize("F", [256, 768])  # 768: three 256-value units per down row
@pytest.mark.parametrize("M", [1, 6, 40, 80])
def test_q6k_down(M, F):
    """Q6_K downs (unsigned 6-bit q, dd = f16(d sc), mm = f16(-32 dd)) on every down kernel: the
    decode path (M = 1), and for batches every split between the streaming GEMV and the MFMA tiles
    and the per-token path (M = 6) give the same bits, identical to the oracle's TQ8_16 path where
    the routing weights agree."""
    say(f"q6k down M={M} F={F}")
    L, orc, W = layer(f"q6F{F}", seed=4, H=512, E=16, F=F, down_fmt=O.FMT_Q6_K)
    import torch
    x = L.x(M, tid=400)
    r = orc.moe_block(x[0], k=3) if M == 1 else orc.moe_batch(x, k=3)
    want = r["out"][None] if M == 1 else r["out"]
    outs = []
    # batches: every stream / MFMA split of the grouped path, then (None) the default, which runs
    # each token as a decode up to 8 tokens
    for rows in ((-1,) if M == 1 else (0, 1, 4, 16, -1, None)):
        ctx = trmoe.Context(L.H, L.E, L.F, 3, max(64, M))
        if rows is not None:
            ctx.set_stream_rows(rows)
            ctx.set_decode_rows(0)
        out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        outs.append(host(out).copy())
        compare_out(outs[-1], want, routing_exact(ctx, r, M, 3, L, x), f"q6k M={M} F={F} rows={rows}")
        ctx.close()
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("F", [256, 768])  # 768: three 256-value units per down row
@pytest.mark.parametrize("fmt", [O.FMT_Q8_0, O.FMT_Q5_1])
@pytest.mark.parametrize("M", [1, 6, 40, 80])
def test_q80_q51_down(fmt, M, F):
    """Q8_0 and Q5_1 downs (the reference's q8_0_rows / q5_1_rows forms: q = int8 + 128 with
    m = f16(-128 d); 5-bit q with d, m as stored) on every down kernel: the decode path (M = 1),
    and for batches every split between the streaming GEMV and the MFMA tiles and the per-token
    path (M = 6) give the same bits, within tolerance of the oracle's TQ8_16 / TQ5_16 GEMV."""
    say(f"down fmt={fmt} M={M} F={F}")
    L, orc, W = layer(f"dfmt{fmt}F{F}", seed=6, H=512, E=16, F=F, down_fmt=fmt)
    import torch
    x = L.x(M, tid=410)
    r = orc.moe_block(x[0], k=3) if M == 1 else orc.moe_batch(x, k=3)
    want = r["out"][None] if M == 1 else r["out"]
    outs = []
    for rows in ((-1,) if M == 1 else (0, 16, -1, None)):
        ctx = trmoe.Context(L.H, L.E, L.F, 3, max(64, M))
        if rows is not None:
            ctx.set_stream_rows(rows)
            ctx.set_decode_rows(0)
        out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        outs.append(host(out).copy())
        compare_out(outs[-1], want, routing_exact(ctx, r, M, 3, L, x), f"fmt={fmt} M={M} rows={rows}")
        ctx.close()
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("M", [1, 3])
def test_residual_stack(M):
    """Config 5 in miniature: h <- h + MoE(rmsnorm(h)) through 3 layers."""
    say(f"residual stack M={M}")
    import torch
    layers = [Layer(seed=21 + i, H=512, E=16, F=256, layer=i) for i in range(3)]
    ws = [trmoe.LayerWeights.from_host(L) for L in layers]
    rms = [O.gen_uniform(21, (i << 32) | 4, 512, 0.9, 1.1) for i in range(3)]
    ctx = trmoe.Context(512, 16, 256, 3, 8)
    h0 = layers[0].x(M, tid=500)
    h = dev(h0.copy())
    hh = h0.copy()
    for i, L in enumerate(layers):
        ctx.residual(ws[i], dev(rms[i]), 1e-6, h)
        orc = L.oracle()
        xn = np.stack([O.rmsnorm(hh[t], rms[i], 1e-6) for t in range(M)])
        if M == 1:
            y = orc.moe_block(xn[0], k=3)["out"][None]
        else:
            y = orc.moe_batch(xn, k=3)["out"]
        hh = (hh + y).astype(np.float32)
    got = host(h)
    assert np.abs(got - hh).max() <= 1e-3 * np.abs(hh).max()
    ctx.close()


@pytest.mark.parametrize("M", [1, 3, 16])
def test_residual_norm_in_logits_launch(M):
    """Below the router GEMM threshold the config-5 layer normalises h inside the logits launch
    (no rmsnorm launch); the result has the same bits as rmsnorm into a copy and the layer on it
    (forced here through the one-launch decode setting, which keeps the separate rmsnorm).
    M = 16 takes the GEMM-order router and the separate rmsnorm on both sides."""
    say(f"residual norm fused M={M}")
    import torch
    L = Layer(seed=31, H=512, E=16, F=256)
    W = trmoe.LayerWeights.from_host(L)
    rms = dev(O.gen_uniform(31, 4, 512, 0.9, 1.1))
    h0 = L.x(M, tid=520)
    outs = []
    for fusion in (False, True):
        ctx = trmoe.Context(512, 16, 256, 3, 16)
        ctx.set_fusion(fusion)
        h = dev(h0.copy())
        for _ in range(2):
            ctx.residual(W, rms, 1e-6, h)
        outs.append(host(h).copy())
        ctx.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_prefill_zipf_full_size_sampled():
    """Config 3 (M = 512, Zipf(1.1) routing) at full size: dispatch bit-exact, properties of the
    grouping, and sampled tokens against the oracle (per-token batch arithmetic, gemm-order logits)."""
    say("prefill M=512 zipf full size")
    import torch
    E, H, F, M = 512, 2048, 512, 512
    bias = zipf_bias(1, E)
    L = Layer(seed=1, H=H, E=E, F=F, bias=bias, lazy=True)
    W = trmoe.LayerWeights.generate(1, 0, H, E, F, router_bias=dev(bias))
    # f32 normals may differ by an ulp between host and GPU libm: use the host's router / gate
    W.tensors["router"].copy_(dev(L.router.reshape(-1)))
    W.tensors["shexp_gate"].copy_(dev(L.shexp_gate))
    # the GPU generator and the host generator produce the same bytes
    for e in (0, 17, 511):
        assert np.array_equal(host(W.tensors["gate"][e]), L.gate(e))
    ctx = trmoe.Context(H, E, F, 10, M)
    x = L.x(M, tid=600)
    out = torch.empty((M, H), dtype=torch.float32, device="cuda")
    ctx.forward(W, dev(x), out)
    torch.cuda.synchronize()
    ng, n_ent = ctx.read(trmoe.WS_NGROUPS, 16, np.uint32)[:2]
    assert n_ent == M * 10
    ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)[:, :10]
    ent_tok = ctx.read(trmoe.WS_ENT_TOK, 4 * n_ent, np.uint32)
    ent_exp = ctx.read(trmoe.WS_ENT_EXP, 4 * n_ent, np.uint32)
    flat = [(int(ids[t, s]), t) for t in range(M) for s in range(10)]
    srt = sorted(flat)  # (expert, token) order == stable sort of token-major entries by expert
    assert list(zip(ent_exp.tolist(), ent_tok.tolist())) == srt
    sizes = np.bincount(ent_exp, minlength=E)
    assert ng == (sizes > 0).sum() and sizes.max() > 100  # skewed load
    got = host(out)
    assert np.isfinite(got).all()
    orc = L.oracle()
    rlog_gpu = ctx.read(trmoe.WS_RLOG, M * E * 4, np.float32).reshape(M, E)
    w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)[:, :10]
    # 32 tokens: 8 of the largest group's (the 16-row MFMA tiles and item pairs of the most popular
    # expert), the others spread over the batch
    big = int(np.argmax(sizes))
    big_toks = ent_tok[ent_exp == big]
    chosen = set(big_toks[np.linspace(0, len(big_toks) - 1, 8).astype(int)].tolist())
    for t in np.linspace(0, M - 1, 40).astype(int).tolist():
        if len(chosen) < 32:
            chosen.add(t)
    sample = sorted(chosen)
    assert len(sample) == 32 and sum(t in big_toks for t in sample) >= 8
    n_exact = 0
    for t in sample:
        xt = x[t:t + 1]
        want_lg = orc.logits(xt, dot_rows=False)
        assert np.array_equal(rlog_gpu[t].view(np.uint32), want_lg[0].view(np.uint32))
        r = orc.moe_batch(xt, k=10, router_dot_max_m=0)
        assert np.array_equal(r["ids"][0, :10], ids[t])
        exact = np.array_equal(w[t], r["w"][0, :10]) and shared_gate_exact(L, xt)
        n_exact += exact
        compare_out(got[t], r["out"][0], exact, f"token {t}")
    say(f"config 3: {len(sample)} tokens, {n_exact} with bit-identical routing weights and gate")
    assert n_exact >= len(sample) // 2
    ctx.close()


def full_layer_on_gpu(seed, layer_idx, down_fmt=O.FMT_Q4_K, bias=None):
    """A BASELINE-shape layer (H 2048, E 512, F 512) generated on the GPU, with the host's lazy twin
    for the oracle.  The router and shared-gate vector are uploaded from the host: f32 normals may
    differ by an ulp between the host's and the GPU's libm."""
    import torch
    H, E, F = 2048, 512, 512
    L = Layer(seed=seed, H=H, E=E, F=F, layer=layer_idx, down_fmt=down_fmt, bias=bias, lazy=True)
    W = trmoe.LayerWeights.generate(seed, layer_idx, H, E, F, down_fmt=down_fmt,
                                    router_bias=None if bias is None else dev(bias))
    W.tensors["router"].copy_(dev(L.router.reshape(-1)))
    W.tensors["shexp_gate"].copy_(dev(L.shexp_gate))
    torch.cuda.synchronize()
    for e in (0, 511):  # the GPU generator and the host generator produce the same bytes
        assert np.array_equal(host(W.tensors["down"][e]), L.down(e))
    return L, W


def test_config4_full_shape():
    """BASELINE config 4 at its own shape: M = 3072, Q4_K gate/up with Q6_K downs, dynamic-k
    routing MoePolicy{min 1, max 10, mass 0.9, basis Top}.  Every token's n_sel and ids against
    route_mass (router.rs:118-148) on the GPU's logits, the whole dispatch against the stable sort
    of exec_batch.rs:1428-1462, sampled logits rows against gemm_f32_nt, and sampled tokens'
    outputs against moe_batch (bit-identical where the routing weights agree)."""
    say("config 4 full shape M=3072")
    import torch
    M, k, pol = 3072, 10, (1, 10, 0.9, O.BASIS_TOP)
    L, W = full_layer_on_gpu(1, 0, down_fmt=O.FMT_Q6_K)
    ctx = trmoe.Context(L.H, L.E, L.F, k, M)
    ctx.set_moe(pol)
    x = L.x(M, tid=640)
    out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
    ctx.forward(W, dev(x), out)
    torch.cuda.synchronize()
    rlog = ctx.read(trmoe.WS_RLOG, M * L.E * 4, np.float32).reshape(M, L.E)
    ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
    w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)
    nsel = ctx.read(trmoe.WS_NSEL, M * 4, np.uint32)
    say("config 4: routing every token")
    w_exact = np.ones(M, bool)
    for t in range(M):
        oi, ow = O.route_mass(rlog[t], *pol)
        assert nsel[t] == len(oi), t
        assert np.array_equal(ids[t, :nsel[t]], oi), t
        # w = e / sum with e = exp(v - max): a 1-ulp difference of libm's expf in e (and in the
        # sum) moves the quotient by at most 3 ulps
        assert ulp(w[t, :nsel[t]], ow).max() <= 3, t
        w_exact[t] = np.array_equal(w[t, :nsel[t]], ow)
    assert 1 <= nsel.min() and nsel.max() <= 10 and 3 < nsel.mean() < 10
    say("config 4: dispatch")
    ng, n_ent = ctx.read(trmoe.WS_NGROUPS, 16, np.uint32)[:2]
    assert n_ent == nsel.sum()
    tok = np.repeat(np.arange(M), nsel)
    slot = np.concatenate([np.arange(n) for n in nsel])
    exp = ids[tok, slot]
    order = np.lexsort((tok, exp))  # stable sort of token-major entries by expert
    assert np.array_equal(ctx.read(trmoe.WS_ENT_TOK, 4 * n_ent, np.uint32), tok[order])
    assert np.array_equal(ctx.read(trmoe.WS_ENT_EXP, 4 * n_ent, np.uint32), exp[order])
    ent_w = ctx.read(trmoe.WS_ENT_W, 4 * n_ent, np.float32)
    assert np.array_equal(ent_w.view(np.uint32), w[tok, slot][order].view(np.uint32))
    sizes = np.bincount(exp, minlength=L.E)
    gs = np.concatenate([[0], np.cumsum(sizes[sizes > 0])]).astype(np.uint32)
    assert ng == (sizes > 0).sum()
    assert np.array_equal(ctx.read(trmoe.WS_GRP_START, 4 * (ng + 1), np.uint32), gs)
    assert np.array_equal(ctx.read(trmoe.WS_GRP_EXP, 4 * ng, np.uint32), np.flatnonzero(sizes).astype(np.uint32))
    assert ctx.stats() == (M, n_ent)
    got = host(out)
    assert np.isfinite(got).all()
    orc = L.oracle()
    for t in (0, 1, 1000, 2047, 3071):
        say(f"config 4: token {t}")
        xt = x[t:t + 1]
        assert np.array_equal(rlog[t].view(np.uint32), orc.logits(xt, dot_rows=False)[0].view(np.uint32))
        r = orc.moe_batch(xt, k=k, policy=pol, router_dot_max_m=0)
        assert np.array_equal(r["ids"][0, :nsel[t]], ids[t, :nsel[t]])
        compare_out(got[t], r["out"][0], bool(w_exact[t]) and shared_gate_exact(L, xt), f"C4 token {t}")
    ctx.close()


def test_config5_residual_full_m512():
    """BASELINE config 5 at M = 512 over two full-size layers: h <- h + MoE(rmsnorm(h)) through
    trk_moe_residual (rmsnorm_kernel, then the GEMM-order router).  After each layer, sampled rows
    against orc_rmsnorm + orc_moe_batch from the GPU's own input rows (elem.rs:255-262,
    exec_batch.rs:1404-1580); bit-identical where the routing weights agree."""
    say("config 5 M=512, two full layers")
    import torch
    M, k = 512, 10
    ctx = trmoe.Context(2048, 512, 512, k, M)
    h = dev(Layer(seed=1, H=2048, E=4, F=256, lazy=True).x(M, tid=660))
    for l in range(2):
        L, W = full_layer_on_gpu(1, l)
        rms = O.gen_uniform(1, (l << 32) | 4, 2048, 0.9, 1.1)
        h_in = host(h).copy()
        ctx.residual(W, dev(rms), 1e-6, h)
        torch.cuda.synchronize()
        h_out = host(h)
        assert np.isfinite(h_out).all()
        ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)[:, :k]
        w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)[:, :k]
        orc = L.oracle()
        for t in (0, 255, 511):
            say(f"config 5: layer {l} row {t}")
            xn = O.rmsnorm(h_in[t], rms, 1e-6)[None]
            r = orc.moe_batch(xn, k=k, router_dot_max_m=0)
            assert np.array_equal(r["ids"][0, :k], ids[t])
            want = (h_in[t] + r["out"][0]).astype(np.float32)
            exact = np.array_equal(r["w"][0, :k], w[t]) and shared_gate_exact(L, xn)
            compare_out(h_out[t], want, exact, f"C5 layer {l} row {t}")
    ctx.close()


def test_config5_residual_full_m1():
    """BASELINE config 5 at decode, M = 1, over two full-size layers (H 2048, E 512, F 512, top-10)
    through trk_moe_residual: the RMSNorm runs inside the dot-order logits launch, the decode down
    adds into h.  After each layer: the quantised normalised row (two levels) bit-exact against
    orc_rmsnorm + quant_pair, the routing against moe_block's, and h against h + moe_block(rmsnorm(h))
    (elem.rs:255-262, exec.rs:1540-1623), bit-identical where the routing weights agree."""
    say("config 5 M=1, two full layers")
    import torch
    k = 10
    ctx = trmoe.Context(2048, 512, 512, k, 16)
    h = dev(Layer(seed=1, H=2048, E=4, F=256, lazy=True).x(1, tid=661))
    for l in range(2):
        L, W = full_layer_on_gpu(1, l)
        rms = O.gen_uniform(1, (l << 32) | 4, 2048, 0.9, 1.1)
        h_in = host(h).copy()
        ctx.residual(W, dev(rms), 1e-6, h)
        torch.cuda.synchronize()
        h_out = host(h)
        xn = O.rmsnorm(h_in[0], rms, 1e-6)
        oq, _, _ = O.quant_pair(xn, 32)
        assert np.array_equal(ctx.read(trmoe.WS_XQ, 2 * 2048, np.int8)[:oq.size], oq.reshape(-1)), f"layer {l} xq"
        r = L.oracle().moe_block(xn, k=k, hiprec=True)
        ids = ctx.read(trmoe.WS_IDS, 4 * 32, np.uint32)[:k]
        w = ctx.read(trmoe.WS_W, 4 * 32, np.float32)[:k]
        assert np.array_equal(ids, r["ids"]), f"layer {l} ids"
        want = (h_in[0] + r["out"]).astype(np.float32)
        exact = np.array_equal(w, r["w"]) and shared_gate_exact(L, xn[None])
        say(f"config 5 M=1: layer {l} exact={exact}")
        compare_out(h_out[0], want, exact, f"C5 M=1 layer {l}")
    ctx.close()


@pytest.mark.parametrize("M", [1, 37])
def test_mass_profile(M):
    """MoeStats's router-mass profile (exec.rs:566-591, router.rs:152-166) on the GPU: the mean
    cumulative mass of the best 1..32 experts over every routed row, against the oracle's
    mass_profile in the same fixed point (1e-6 per row; the GPU's exp may differ from libm's expf
    by an ulp, so a row's fixed-point value may differ by a unit or two)."""
    say(f"mass profile M={M}")
    import torch
    L, orc, W = layer("small", **SMALL)
    ctx = trmoe.Context(L.H, L.E, L.F, 4, 64)
    ctx.profile_start()
    want = np.zeros(32)
    rows = 0
    for it in range(3):
        x = L.x(M, tid=680 + it)
        out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        lg = orc.logits(x, M < 16)
        for t in range(M):
            want += np.floor(O.mass_profile(lg[t]).astype(np.float64) * 1e6)
            rows += 1
    cum, n = ctx.profile_report()
    assert n == rows
    assert np.abs(cum - want * 1e-6 / rows).max() <= 3e-6
    assert np.all(np.diff(cum) >= -1e-12) and cum[-1] <= 1.0 + 1e-6
    ctx.profile_start(False)
    ctx.forward(W, dev(L.x(M, tid=690)), out)
    assert ctx.profile_report()[1] == rows  # off: nothing added
    ctx.close()


@pytest.mark.parametrize("M", [1, 4, 40])
def test_subset_pack_gguf(M):
    """A subset pack on the GGUF kernels (n_expert_packed = 8 of 32): the decode gate/up routes,
    folds (fold_ids, exec_batch.rs:214-225) and only then requests its slot's weights; the small and
    the general dispatch group the folded ids.  Against the oracle with the same fold."""
    say(f"subset pack gguf M={M}")
    import torch
    L, orc, W = layer("small", **SMALL)
    orc.packed = 8
    try:
        x = L.x(M, tid=820 + M)
        r = orc.moe_block(x[0], k=4) if M == 1 else orc.moe_batch(x, k=4)
        want = r["out"][None] if M == 1 else r["out"]
        ctx = trmoe.Context(L.H, L.E, L.F, 4, max(M, 16), n_expert_packed=8)
        out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)[:, :4]
        w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)[:, :4]
        rids = r["ids"][None] if M == 1 else r["ids"][:, :4]
        rw = r["w"][None] if M == 1 else r["w"][:, :4]
        assert np.array_equal(ids, rids) and ids.max() < 8
        compare_out(host(out), want, np.array_equal(w, rw) and shared_gate_exact(L, x), f"subset gguf M={M}")
        ctx.close()
    finally:
        orc.packed = 0
