"""The MoE layer on the reference's own packed TQ experts (k_tq.hip) against the oracle's
moe_block (M = 1) and moe_batch (M >= 2) on the same bytes.

Shapes: the real expert shape, gate/up TQ4_32 [640][2560] and down TQ5_16 [2560][640]
(python/tests/test_blocks_real.py:23-26), with 32 experts instead of 512; F = 640 and 80 are not
multiples of 256; every gate/down bit width.  Bar as for the GGUF layer: bit-identical where the
routing weights and the shared gate agree bit for bit, else within 1e-5 of the output scale."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

import oracle as O
import trmoe
from layerdata import TQLayer
from test_gpu_layer import compare_out, dev, host, routing_exact, say, shared_gate_exact

pytestmark = pytest.mark.gpu

_layers = {}


def tq_layer(key, **kw):
    if key not in _layers:
        L = TQLayer(**kw)
        W = trmoe.LayerWeights.from_tq(L.H, L.E, L.F, L.router, L.shexp_gate, L.gate, L.up, L.down, L.sh_gate,
                                       L.sh_up, L.sh_down, L.gate_fmt, L.down_fmt)
        _layers[key] = (L, L.oracle(), W)
    return _layers[key]


REAL = dict(seed=21, H=2560, E=32, F=640, gate_bits=4, down_bits=5)


def reference(orc, x, k, policy=None, hiprec=True):
    M = x.shape[0]
    if M == 1:
        r = orc.moe_block(x[0], k=k, policy=policy, hiprec=hiprec)
        return r, r["out"][None]
    if M > 16 and O.cpu_have_vnni():
        # the threaded VNNI restatement (bit-identical to the scalar oracle, tests/test_cpu_baseline.py);
        # the routing weights from the oracle's router and route functions
        cpu = O.CpuMoe(0)
        got = cpu.batch(orc, x, k=k, policy=policy)
        cpu.close()
        lg = orc.logits(x, False)
        w = np.zeros((M, 32), np.float32)
        ids = np.zeros((M, 32), np.uint32)
        n_sel = np.zeros(M, np.uint32)
        for t in range(M):
            it, wt = O.route_mass(lg[t], *policy) if policy else O.route_topk(lg[t], k)
            w[t, :len(wt)] = wt
            ids[t, :len(it)] = it
            n_sel[t] = len(wt)
        return {"w": w, "ids": ids, "n_sel": n_sel}, got["out"]
    r = orc.moe_batch(x, k=k, policy=policy)
    return r, r["out"]


def run_case(L, orc, W, M, k, hiprec=True, policy=None, tid=0, mfma=None):
    """The layer on L's TQ experts at M rows against the oracle.  mfma: require (True) or rule out
    (False) the int8 MFMA kernels, read from the launches the call made (the generic path runs a
    separate SwiGLU launch, tq_act)."""
    import torch
    x = L.x(M, tid=tid)
    r, want = reference(orc, x, k, policy, hiprec)
    ctx = trmoe.Context(L.H, L.E, L.F, k, max(M, 16), hiprec=hiprec, k_cap=policy[1] if policy else 0)
    if policy:
        ctx.set_moe(policy)
    out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
    if mfma is not None:
        ctx.set_timing(True)
    ctx.forward(W, dev(x), out)
    if mfma is not None:
        launched = ctx.timing()
        ctx.set_timing(False)
        assert "tq_gateup" in launched and ("tq_act" not in launched) == mfma, launched
    got = host(out).copy()
    exact = routing_exact(ctx, r, M, k, L, x) if not policy else policy_exact(ctx, r, M, L, x)
    # MoeStats: rows and selected experts, counted by whichever launch routed
    nsel = ctx.read(trmoe.WS_NSEL, M * 4, np.uint32)
    assert ctx.stats() == (M, int(nsel.sum()))
    ctx.close()
    return got, want, exact


def policy_exact(ctx, r, M, L, x):
    """Cumulative-mass routing: every token's count and ids equal the oracle's (asserted); True
    when the weights and the shared gate also agree bit for bit, so the outputs must too."""
    nsel = ctx.read(trmoe.WS_NSEL, M * 4, np.uint32)
    ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
    w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)
    if M == 1:
        want_n, want_ids, want_w = [r["k"]], [np.asarray(r["ids"])], [np.asarray(r["w"])]
    else:
        want_n, want_ids, want_w = r["n_sel"], r["ids"], r["w"]
    same = True
    for t in range(M):
        n = int(want_n[t])
        assert nsel[t] == n, (t, nsel[t], n)
        assert np.array_equal(ids[t, :n], np.asarray(want_ids[t])[:n]), t
        same = same and np.array_equal(w[t, :n], np.asarray(want_w[t])[:n])
    return same and shared_gate_exact(L, x)


@pytest.mark.parametrize("M,hiprec", [(1, True), (1, False), (3, True), (16, True), (64, True)])
def test_tq_layer_real_shape(M, hiprec):
    say(f"tq layer real shape M={M} hiprec={hiprec}")
    L, orc, W = tq_layer("real", **REAL)
    got, want, exact = run_case(L, orc, W, M, 8, hiprec=hiprec, tid=M)
    compare_out(got, want, exact, f"tq real M={M}")


@pytest.mark.parametrize("gate_bits,down_bits,F", [(5, 4, 96), (8, 8, 96), (4, 8, 96), (5, 5, 96), (8, 4, 160),
                                                   (5, 4, 80), (8, 8, 80)])
@pytest.mark.parametrize("M", [1, 9, 40])
def test_tq_layer_codecs(gate_bits, down_bits, F, M):
    """Every gate/up and down bit width.  F a multiple of 32 runs the int8 MFMA kernels (every
    instantiation of k_tqm.hip: the 8-bit codecs' byte-sum correction, TQ5_32 gate/up, TQ4_16 and
    TQ8_16 downs); F = 80 the generic grouped TQ GEMV."""
    say(f"tq layer codecs gate={gate_bits} down={down_bits} F={F} M={M}")
    L, orc, W = tq_layer(f"c{gate_bits}{down_bits}F{F}", seed=30 + gate_bits + down_bits + F, H=512, E=16, F=F,
                         gate_bits=gate_bits, down_bits=down_bits)
    got, want, exact = run_case(L, orc, W, M, 4, tid=100 + M, mfma=F % 32 == 0)
    compare_out(got, want, exact, f"tq codecs {gate_bits}/{down_bits} F={F} M={M}")


@pytest.mark.parametrize("M", [1, 24])
def test_tq_layer_dynamic_k(M):
    """Cumulative-mass routing (MoePolicy{1, 10, 0.9, Top}) on TQ experts: k varies per token."""
    say(f"tq layer dynamic k M={M}")
    L, orc, W = tq_layer("real", **REAL)
    pol = (1, 10, 0.9, O.BASIS_TOP)
    got, want, exact = run_case(L, orc, W, M, 8, policy=pol, tid=200 + M)
    say(f"tq dynamic-k M={M}: routing weights and shared gate bit-identical: {exact}")
    compare_out(got, want, exact, f"tq dynamic-k M={M}")


@pytest.mark.parametrize("M,policy", [(2, None), (3, (1, 8, 0.9, O.BASIS_TOP)), (8, None),
                                      (5, (2, 8, 0.8, O.BASIS_ALL))])
def test_tq_decode_rows_match_grouped(M, policy):
    """A batch of a few tokens run as per-token decodes (trk_set_decode_rows: each token's routing
    inside the gate/up launch, its rows added by the down + combine launch in the batch combine's
    order) gives the grouped path's bits, publishes the same routing and counts the same MoeStats;
    both against the oracle's moe_batch."""
    say(f"tq decode rows M={M} policy={policy}")
    L, orc, W = tq_layer("real", **REAL)
    import torch
    x = L.x(M, tid=260 + M)
    k = 8
    r, want = reference(orc, x, k, policy)
    outs, routing, launched = [], [], []
    for rows in (0, 8):
        ctx = trmoe.Context(L.H, L.E, L.F, k, M, k_cap=policy[1] if policy else 0)
        if policy:
            ctx.set_moe(policy)
        ctx.set_decode_rows(rows)
        ctx.set_timing(True)
        out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx.forward(W, dev(x), out)
        launched.append(set(ctx.timing()))
        ctx.set_timing(False)
        outs.append(host(out).copy())
        nsel = ctx.read(trmoe.WS_NSEL, 4 * M, np.uint32)
        ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
        w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)
        routing.append([(ids[t, :nsel[t]].copy(), w[t, :nsel[t]].copy()) for t in range(M)])
        assert ctx.stats() == (M, int(nsel.sum()))
        exact = policy_exact(ctx, r, M, L, x) if policy else routing_exact(ctx, r, M, k, L, x)
        ctx.close()
    assert "dispatch" in launched[0] and "dispatch" not in launched[1], launched  # the path asked for ran
    assert np.array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32)), f"M={M}: bits differ"
    for (i0, w0), (i1, w1) in zip(routing[0], routing[1]):
        assert np.array_equal(i0, i1) and np.array_equal(w0.view(np.uint32), w1.view(np.uint32))
    say(f"tq decode rows M={M}: routing weights and shared gate bit-identical: {exact}")
    compare_out(outs[1], want, exact, f"tq decode rows M={M}")


def test_tq_weights_rejected_when_mixed():
    """One gate/up codec and one down codec per layer, TQ and GGUF not mixed; gate/up must be
    kb 32 and down kb 16 (the activations' block sizes)."""
    import ctypes as C
    import torch
    L, orc, W = tq_layer("c54", seed=39, H=512, E=16, F=80, gate_bits=5, down_bits=4)
    ctx = trmoe.Context(L.H, L.E, L.F, 4, 4)
    x = torch.zeros((1, L.H), dtype=torch.float32, device="cuda")
    out = torch.empty_like(x)
    bad = trmoe.MoeW.from_buffer_copy(W.moew)
    bad.down.fmt = trmoe.FMT_TQ5_32
    rc = trmoe.lib().trk_moe_forward(ctx.h, C.byref(bad), C.c_void_p(x.data_ptr()), None, 1,
                                     C.c_void_p(out.data_ptr()), None)
    assert rc == -1 and b"kb" in trmoe.lib().trk_last_error()
    bad = trmoe.MoeW.from_buffer_copy(W.moew)
    bad.up.fmt = trmoe.FMT_TQ4_32
    rc = trmoe.lib().trk_moe_forward(ctx.h, C.byref(bad), C.c_void_p(x.data_ptr()), None, 1,
                                     C.c_void_p(out.data_ptr()), None)
    assert rc == -1 and b"formats" in trmoe.lib().trk_last_error()
    ctx.close()


@pytest.mark.parametrize("key,kw,M,k,hiprec", [("real", REAL, 1, 8, True), ("real", REAL, 1, 8, False),
                                               ("real", REAL, 16, 8, True), ("real", REAL, 64, 8, True),
                                               ("m88", dict(seed=46, H=512, E=16, F=96, gate_bits=8, down_bits=8), 40, 4, True),
                                               ("m88", dict(seed=46, H=512, E=16, F=96, gate_bits=8, down_bits=8), 1, 4, True),
                                               ("m54", dict(seed=39, H=512, E=16, F=96, gate_bits=5, down_bits=4), 1, 4, True),
                                               ("m54", dict(seed=39, H=512, E=16, F=96, gate_bits=5, down_bits=4), 300, 4, True),
                                               ("m48", dict(seed=42, H=512, E=16, F=160, gate_bits=4, down_bits=8), 9, 4, True),
                                               ("m48", dict(seed=42, H=512, E=16, F=160, gate_bits=4, down_bits=8), 300, 4, True)])
def test_tq_mfma_matches_generic(key, kw, M, k, hiprec):
    """The int8 MFMA kernels (a TQ block per MFMA, SwiGLU in the gate/up launch) and the generic
    grouped TQ GEMV give the same bits."""
    say(f"tq mfma vs generic {key} M={M}")
    import torch
    L, orc, W = tq_layer(key, **kw)
    x = dev(L.x(M, tid=300 + M))
    outs = []
    for mfma in (True, False):
        ctx = trmoe.Context(L.H, L.E, L.F, k, max(M, 16), hiprec=hiprec)
        ctx.set_tq_mfma(mfma)
        out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
        ctx.set_timing(True)
        ctx.forward(W, x, out)
        launched = ctx.timing()
        assert ("tq_act" not in launched) == mfma, launched  # the path asked for is the one that ran
        outs.append(host(out).copy())
        ctx.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), np.abs(outs[0] - outs[1]).max()


_full = {}


def tq_full_layer():
    """The real expert shape at the real expert count: H 2560, F 640, E 512, TQ4_32 gate/up and
    TQ5_16 down (1.78 GB of experts), generated on the GPU and copied back for the oracle."""
    if not _full:
        import torch
        gen = torch.Generator(device="cuda")
        gen.manual_seed(23)
        H, E, F = 2560, 512, 640
        bias = trmoe.zipf_bias(1, E)
        W = trmoe.LayerWeights.generate_tq(gen, H, E, F, router_bias=dev(bias))
        t = {k: host(v) for k, v in W.tensors.items() if k != "router_bias"}
        orc = O.TQOracleLayer(H, E, F, t["router"], t["shexp_gate"], t["gate"], t["up"], t["down"], t["sh_gate"],
                              t["sh_up"], t["sh_down"], 4, 5, bias)
        x = host(torch.randn((512, H), device="cuda", generator=gen))
        _full.update(W=W, orc=orc, x=x, H=H, E=E, F=F, shexp_gate=t["shexp_gate"])
    return _full


@pytest.mark.parametrize("policy", [None, (1, 10, 0.9, O.BASIS_TOP)])
def test_tq_full_shape_m512_sampled(policy):
    """The TQ layer at the bench's own configuration: E = 512, M = 512, Zipf(1.1)-biased router,
    top-10 or dynamic k.  The split dispatch, the MFMA batch gate/up over TQM_PAIRS strip pairs and
    the four-strip-group down all run.  Every token's ids against the oracle's route on the GPU's
    logits, and 16 sampled tokens (4 from the largest group) against moe_batch, bit-identical where
    the routing weights and the shared gate agree."""
    say(f"tq full shape M=512 policy={policy}")
    import torch
    from test_gpu_layer import shared_gate_exact, ulp
    d = tq_full_layer()
    W, orc, x, H, E, F = d["W"], d["orc"], d["x"], d["H"], d["E"], d["F"]
    M, k = 512, 10
    ctx = trmoe.Context(H, E, F, k, M, k_cap=policy[1] if policy else 0)
    if policy:
        ctx.set_moe(policy)
    out = torch.empty((M, H), dtype=torch.float32, device="cuda")
    ctx.set_timing(True)
    ctx.forward(W, dev(x), out)
    launched = ctx.timing()
    ctx.set_timing(False)
    assert "tq_act" not in launched and "tq_gateup" in launched, launched
    got = host(out)
    assert np.isfinite(got).all()
    rlog = ctx.read(trmoe.WS_RLOG, M * E * 4, np.float32).reshape(M, E)
    ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
    w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)
    nsel = ctx.read(trmoe.WS_NSEL, M * 4, np.uint32)
    w_exact = np.zeros(M, bool)
    for t in range(M):
        oi, ow = O.route_mass(rlog[t], *policy) if policy else O.route_topk(rlog[t], k)
        assert nsel[t] == len(oi) and np.array_equal(ids[t, :nsel[t]], oi), t
        assert ulp(w[t, :nsel[t]], ow).max() <= 3, t
        w_exact[t] = np.array_equal(w[t, :nsel[t]], ow)
    n_ent = int(nsel.sum())
    ent_tok = ctx.read(trmoe.WS_ENT_TOK, 4 * n_ent, np.uint32)
    ent_exp = ctx.read(trmoe.WS_ENT_EXP, 4 * n_ent, np.uint32)
    sizes = np.bincount(ent_exp, minlength=E)
    assert sizes.max() > 100  # the skewed load of the Zipf bias
    big_toks = ent_tok[ent_exp == int(np.argmax(sizes))]
    chosen = set(big_toks[np.linspace(0, len(big_toks) - 1, 4).astype(int)].tolist())
    for t in np.linspace(0, M - 1, 20).astype(int).tolist():
        if len(chosen) < 16:
            chosen.add(t)
    n_exact = 0
    for t in sorted(chosen):
        xt = x[t:t + 1]
        assert np.array_equal(rlog[t].view(np.uint32), orc.logits(xt, False)[0].view(np.uint32)), t
        r = orc.moe_batch(xt, k=k, policy=policy, router_dot_max_m=0)
        assert np.array_equal(r["ids"][0, :nsel[t]], ids[t, :nsel[t]])
        exact = bool(w_exact[t]) and shared_gate_exact(SimpleNamespace(shexp_gate=d["shexp_gate"]), xt)
        n_exact += exact
        compare_out(got[t], r["out"][0], exact, f"tq full M=512 token {t}")
    say(f"tq full shape: {len(chosen)} tokens, {n_exact} bit-identical")
    ctx.close()



# ---- packs written for T tiles, subset packs ---------------------------------------------------

_tiled = {}


def tiled_layer(key, **kw):
    from layerdata import TiledTQLayer
    if key not in _tiled:
        L = TiledTQLayer(**kw)
        W = trmoe.LayerWeights.from_tiled_tq(L.H, L.E, L.F, L.T, L.router, L.shexp_gate, L.gate, L.up, L.down,
                                             L.sh_gate, L.sh_up, L.sh_down, L.gate_fmt, L.down_fmt)
        _tiled[key] = (L, L.oracle(), W)
    return _tiled[key]


def run_tiled(L, orc, W, M, k, tid, policy=None):
    """The layer on L at M rows against the oracle: every token's ids (and count) exact; returns
    (out, oracle out, whether the routing weights and the shared gate agree bit for bit)."""
    import torch
    x = L.x(M, tid=tid)
    r = orc.moe_block(x[0], k=k, policy=policy) if M == 1 else orc.moe_batch(x, k=k, policy=policy)
    want = r["out"][None] if M == 1 else r["out"]
    if M == 1:
        rids, rws = [r["ids"]], [r["w"]]
    else:
        rids = [r["ids"][t, :r["n_sel"][t]] for t in range(M)]
        rws = [r["w"][t, :r["n_sel"][t]] for t in range(M)]
    ctx = trmoe.Context(L.H, L.E, L.F, k, max(M, 16), n_tiles=L.T, n_expert_packed=L.packed,
                        k_cap=policy[1] if policy else 0)
    if policy:
        ctx.set_moe(policy)
    out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
    ctx.forward(W, dev(x), out)
    got = host(out).copy()
    ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
    w = ctx.read(trmoe.WS_W, M * 32 * 4, np.float32).reshape(M, 32)
    nsel = ctx.read(trmoe.WS_NSEL, M * 4, np.uint32)
    same_w = True
    for t in range(M):
        n = len(rids[t])
        assert nsel[t] == n and np.array_equal(ids[t, :n], rids[t]), (t, ids[t, :nsel[t]], rids[t])
        same_w = same_w and np.array_equal(w[t, :n], rws[t])
    exact = same_w and shared_gate_exact_v(L.shexp_gate, x)
    ctx.close()
    return got, want, exact


def shared_gate_exact_v(shexp_gate, x):
    from test_gpu_layer import shared_gate_exact
    return shared_gate_exact(SimpleNamespace(shexp_gate=shexp_gate), x)


@pytest.mark.parametrize("T,M", [(2, 1), (2, 5), (2, 40), (8, 1), (8, 3), (8, 40)])
def test_tiled_pack(T, M):
    """A pack written for T tiles (python/trpack/plan.py:106-118,174-181), uploaded as it is: the
    K-split router's partials and each tile's down partials summed in tile order (exec.rs:1003-1038,
    exchange.rs:122-136, exec_batch.rs:821-849), against the oracle's T-tile restatement; bit-identical
    where the routing weights and the shared gate agree."""
    say(f"tiled pack T={T} M={M}")
    L, orc, W = tiled_layer(f"t{T}", seed=60 + T, H=512, E=16, F=256, T=T)
    got, want, exact = run_tiled(L, orc, W, M, 4, tid=10 + M)
    compare_out(got, want, exact, f"tiled T={T} M={M}")


@pytest.mark.parametrize("M", [1, 24])
def test_tiled_pack_real_shape(M):
    """The real expert shape packed for 8 tiles (H 2560, F 640: 80 rows / columns per tile, 320
    router columns per tile), TQ4_32 / TQ5_16, top-8 of 32 experts, and dynamic k at M = 24."""
    say(f"tiled pack real shape T=8 M={M}")
    L, orc, W = tiled_layer("real8", seed=71, H=2560, E=32, F=640, T=8, gate_bits=4, down_bits=5)
    got, want, exact = run_tiled(L, orc, W, M, 8, tid=20 + M)
    compare_out(got, want, exact, f"tiled real M={M}")
    if M > 1:
        got, want, _ = run_tiled(L, orc, W, M, 8, tid=30 + M, policy=(1, 10, 0.9, O.BASIS_TOP))
        compare_out(got, want, False, f"tiled real dynamic-k M={M}")


@pytest.mark.parametrize("M", [1, 4, 40, 300])
def test_subset_pack(M):
    """A subset pack (n_expert_packed = 16 of 64 experts, exec.rs:1545-1549): every token's routed ids
    folded onto the packed experts (fold_ids, exec_batch.rs:214-225) on the decode path, the small and
    the general dispatch, against the oracle."""
    say(f"subset pack M={M}")
    L, orc, W = tiled_layer("sub", seed=81, H=512, E=64, F=128, T=1, packed=16)
    got, want, exact = run_tiled(L, orc, W, M, 6, tid=40 + M)
    compare_out(got, want, exact, f"subset M={M}")
