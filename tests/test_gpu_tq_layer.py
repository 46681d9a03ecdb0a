"""The MoE layer on the reference's own packed TQ experts (k_tq.hip) against the oracle's
moe_block (M = 1) and moe_batch (M >= 2) on the same bytes.

Shapes: the real expert shape, gate/up TQ4_32 [640][2560] and down TQ5_16 [2560][640]
(python/tests/test_blocks_real.py:23-26), with 32 experts instead of 512; F = 640 and 80 are not
multiples of 256; every gate/down bit width.  Bar as for the GGUF layer: bit-identical where the
routing weights and the shared gate agree bit for bit, else within 1e-5 of the output scale."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import trmoe
from layerdata import TQLayer
from test_gpu_layer import compare_out, dev, host, routing_exact, say

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
        for t in range(M):
            _, wt = O.route_mass(lg[t], *policy) if policy else O.route_topk(lg[t], k)
            w[t, :len(wt)] = wt
        return {"w": w}, got["out"]
    r = orc.moe_batch(x, k=k, policy=policy)
    return r, r["out"]


def run_case(L, orc, W, M, k, hiprec=True, policy=None, tid=0):
    import torch
    x = L.x(M, tid=tid)
    r, want = reference(orc, x, k, policy, hiprec)
    ctx = trmoe.Context(L.H, L.E, L.F, k, max(M, 16), hiprec=hiprec, k_cap=policy[1] if policy else 0)
    if policy:
        ctx.set_moe(policy)
    out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
    ctx.forward(W, dev(x), out)
    got = host(out).copy()
    exact = routing_exact(ctx, r, M, policy[1] if policy else k, L, x) if not policy else False
    # MoeStats: rows and selected experts, counted by whichever launch routed
    nsel = ctx.read(trmoe.WS_NSEL, M * 4, np.uint32)
    assert ctx.stats() == (M, int(nsel.sum()))
    ctx.close()
    return got, want, exact


@pytest.mark.parametrize("M,hiprec", [(1, True), (1, False), (3, True), (16, True), (64, True)])
def test_tq_layer_real_shape(M, hiprec):
    say(f"tq layer real shape M={M} hiprec={hiprec}")
    L, orc, W = tq_layer("real", **REAL)
    got, want, exact = run_case(L, orc, W, M, 8, hiprec=hiprec, tid=M)
    compare_out(got, want, exact, f"tq real M={M}")


@pytest.mark.parametrize("gate_bits,down_bits", [(5, 4), (8, 8), (4, 8)])
@pytest.mark.parametrize("M", [1, 9, 40])
def test_tq_layer_codecs(gate_bits, down_bits, M):
    say(f"tq layer codecs gate={gate_bits} down={down_bits} M={M}")
    L, orc, W = tq_layer(f"c{gate_bits}{down_bits}", seed=30 + gate_bits + down_bits, H=512, E=16, F=80,
                         gate_bits=gate_bits, down_bits=down_bits)
    got, want, exact = run_case(L, orc, W, M, 4, tid=100 + M)
    compare_out(got, want, exact, f"tq codecs {gate_bits}/{down_bits} M={M}")


@pytest.mark.parametrize("M", [1, 24])
def test_tq_layer_dynamic_k(M):
    """Cumulative-mass routing (MoePolicy{1, 10, 0.9, Top}) on TQ experts: k varies per token."""
    say(f"tq layer dynamic k M={M}")
    L, orc, W = tq_layer("real", **REAL)
    pol = (1, 10, 0.9, O.BASIS_TOP)
    got, want, _ = run_case(L, orc, W, M, 8, policy=pol, tid=200 + M)
    compare_out(got, want, False, f"tq dynamic-k M={M}")


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
                                               ("c88", dict(seed=46, H=512, E=16, F=80, gate_bits=8, down_bits=8), 40, 4, True),
                                               ("c54", dict(seed=39, H=512, E=16, F=80, gate_bits=5, down_bits=4), 1, 4, True),
                                               ("c48", dict(seed=42, H=512, E=16, F=80, gate_bits=4, down_bits=8), 9, 4, True)])
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
        ctx.forward(W, x, out)
        outs.append(host(out).copy())
        ctx.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), np.abs(outs[0] - outs[1]).max()
