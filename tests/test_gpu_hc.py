"""The MoE layer with the hyper-connection mix as its input stage (trk_moe_forward_hc) against the
oracle: the mixed rows against orc_hc_mix (hc_mix_b at M = 1, hc_b_batch at M >= 2), then the
layer's output against moe_block / moe_batch on those rows.

The batch mix uses the reference's exp512 throughout: its rows are bit-identical.  The decode mix
uses the scalar sigmoid (f32::exp, the host libm's expf in the oracle, a correctly rounded exp on
the GPU): rows where the two exps agree are bit-identical, the others within 1e-6 of the scale."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import trmoe
from layerdata import Layer, TQLayer, random_tq
from test_gpu_layer import compare_out, dev, host, routing_exact, say

pytestmark = pytest.mark.gpu

HC, LR = 4, 128
_cache = {}


def layer(kind):
    if kind not in _cache:
        if kind == "tq":
            L = TQLayer(seed=41, H=512, E=16, F=80, gate_bits=4, down_bits=5)
            W = trmoe.LayerWeights.from_tq(L.H, L.E, L.F, L.router, L.shexp_gate, L.gate, L.up, L.down, L.sh_gate,
                                           L.sh_up, L.sh_down, L.gate_fmt, L.down_fmt)
            orc = L.oracle()
        else:
            L = Layer(seed=42, H=512, E=16, F=256)
            W = trmoe.LayerWeights.from_host(L)
            orc = L.oracle()
            orc.ensure(range(L.E))
        _cache[kind] = (L, orc, W)
    return _cache[kind]


@pytest.mark.parametrize("kind,M,hiprec,bits", [("tq", 1, True, 8), ("tq", 1, False, 4), ("gguf", 1, True, 5),
                                                ("tq", 5, True, 4), ("gguf", 3, True, 8), ("gguf", 40, True, 8),
                                                ("tq", 33, True, 5)])
def test_moe_forward_hc(kind, M, hiprec, bits):
    say(f"moe forward hc {kind} M={M} hiprec={hiprec} up bits={bits}")
    import torch
    L, orc, W = layer(kind)
    rng = np.random.default_rng(50 + M + bits)
    up = random_tq(rng, HC * L.H, LR, bits, 32)
    xn = rng.standard_normal((M, HC, L.H)).astype(np.float32)
    lo = (rng.standard_normal((M, LR)) * 3).astype(np.float32)
    decode = M == 1
    mixed_want = O.hc_mix(up, bits, HC, LR, xn, lo, decode, hiprec)
    ctx = trmoe.Context(L.H, L.E, L.F, 4, max(M, 8), hiprec=hiprec)
    out = torch.empty((M, L.H), dtype=torch.float32, device="cuda")
    ctx.forward_hc(W, (dev(up), (bits << 8) | 32), HC, LR, dev(xn), dev(lo), out)
    mixed = ctx.read(trmoe.WS_MIXED, M * L.H * 4, np.float32).reshape(M, L.H)
    same = np.array_equal(mixed.view(np.uint32), mixed_want.view(np.uint32))
    if not decode:
        assert same, np.abs(mixed - mixed_want).max()
    else:
        assert np.abs(mixed - mixed_want).max() <= 1e-6 * np.abs(mixed_want).max()
        assert (mixed == mixed_want).mean() >= 0.99
    # the layer on the GPU's own mixed rows against the oracle on the same rows
    if decode:
        r = orc.moe_block(mixed[0], k=4, hiprec=hiprec)
        want = r["out"][None]
    else:
        r = orc.moe_batch(mixed, k=4)
        want = r["out"]
    compare_out(host(out), want, routing_exact(ctx, r, M, 4, L, mixed), f"hc {kind} M={M}")
    ctx.close()


def test_moe_forward_hc_rejects_bad_shapes():
    import ctypes as C
    import torch
    L, orc, W = layer("tq")
    ctx = trmoe.Context(L.H, L.E, L.F, 4, 4)
    x = torch.zeros((1, HC, L.H), dtype=torch.float32, device="cuda")
    lo = torch.zeros((1, LR), dtype=torch.float32, device="cuda")
    out = torch.empty((1, L.H), dtype=torch.float32, device="cuda")
    up = torch.zeros(trmoe.matrix_bytes(trmoe.FMT_TQ4_16, HC * L.H, LR), dtype=torch.uint8, device="cuda")
    for hc, lr, fmt, msg in ((HC, LR, trmoe.FMT_TQ4_16, b"kb-32"), (9, LR, trmoe.FMT_TQ4_32, b"hc"),
                             (HC, 48, trmoe.FMT_TQ4_32, b"lr")):
        hw = trmoe.HcW(trmoe.Mat(up.data_ptr(), hc * L.H, lr, fmt, 1, 0), hc, lr)
        rc = trmoe.lib().trk_moe_forward_hc(ctx.h, C.byref(W.moew), C.byref(hw), C.c_void_p(x.data_ptr()),
                                            C.c_void_p(lo.data_ptr()), 1, C.c_void_p(out.data_ptr()), None)
        assert rc == -1 and msg in trmoe.lib().trk_last_error(), (hc, lr, fmt)
    ctx.close()
    # a batch's quantised lo rows (22 lr bytes per 16-row tile) beyond the per-entry output rows of
    # a context made for two rows and top-1 (4 (k + 1) m_max H bytes): a status, nothing launched
    ctx = trmoe.Context(L.H, L.E, L.F, 1, 2)
    lr = 512
    assert 22 * lr > 4 * 2 * 2 * L.H
    lo2 = torch.zeros((2, lr), dtype=torch.float32, device="cuda")
    x2 = torch.zeros((2, HC, L.H), dtype=torch.float32, device="cuda")
    out2 = torch.empty((2, L.H), dtype=torch.float32, device="cuda")
    hw = trmoe.HcW(trmoe.Mat(up.data_ptr(), HC * L.H, lr, trmoe.FMT_TQ4_32, 1, 0), HC, lr)
    rc = trmoe.lib().trk_moe_forward_hc(ctx.h, C.byref(W.moew), C.byref(hw), C.c_void_p(x2.data_ptr()),
                                        C.c_void_p(lo2.data_ptr()), 2, C.c_void_p(out2.data_ptr()), None)
    assert rc == -3 and b"per-entry" in trmoe.lib().trk_last_error()
    ctx.close()


def _mixed(ctx, W, up, bits, hc, lr, xn, lo, H):
    import torch
    M = lo.shape[0]
    out = torch.empty((M, H), dtype=torch.float32, device="cuda")
    ctx.forward_hc(W, (dev(up), (bits << 8) | 32), hc, lr, dev(xn), dev(lo), out)
    torch.cuda.synchronize()
    return ctx.read(trmoe.WS_MIXED, M * H * 4, np.float32).reshape(M, H)


@pytest.mark.parametrize("hc,M,bits", [(1, 40, 8), (3, 40, 5), (8, 40, 4), (1, 1, 4), (3, 1, 8), (8, 1, 5)])
def test_hc_streams(hc, M, bits):
    """Stream counts other than the real model's 4 (a wave per stream: 64, 192 and 512 threads)."""
    say(f"hc mix streams hc={hc} M={M} bits={bits}")
    L, orc, W = layer("tq")
    rng = np.random.default_rng(70 + hc + M)
    up = random_tq(rng, hc * L.H, LR, bits, 32)
    xn = rng.standard_normal((M, hc, L.H)).astype(np.float32)
    lo = (rng.standard_normal((M, LR)) * 3).astype(np.float32)
    ctx = trmoe.Context(L.H, L.E, L.F, 4, max(M, 8), hiprec=True)
    mixed = _mixed(ctx, W, up, bits, hc, LR, xn, lo, L.H)
    ctx.close()
    want = O.hc_mix(up, bits, hc, LR, xn, lo, M == 1, True)
    if M > 1:
        assert np.array_equal(mixed.view(np.uint32), want.view(np.uint32)), np.abs(mixed - want).max()
    else:
        assert np.abs(mixed - want).max() <= 1e-6 * np.abs(want).max()
        assert (mixed == want).mean() >= 0.99


_real = {}


@pytest.mark.parametrize("M", [1, 300, 512, 1000])
def test_hc_mix_real_shape(M):
    """The real model's mix shape (hc 4, lr 320, H 2560, up TQ8_32) at the token counts that take
    one, two and four 16-token tiles per workgroup, ragged ends included.  A batch row's mix depends
    on its own xn and lo rows only, so the oracle runs on a sample of rows (the first and last
    tiles among them)."""
    import torch
    H, hc, lr, bits = 2560, 4, 320, 8
    say(f"hc mix real shape M={M}")
    if "w" not in _real:
        gen = torch.Generator(device="cuda")
        gen.manual_seed(5)
        rng = np.random.default_rng(6)
        _real["w"] = trmoe.LayerWeights.generate_tq(gen, H, 16, 128)
        _real["up"] = random_tq(rng, hc * H, lr, bits, 32)
    W, up = _real["w"], _real["up"]
    rng = np.random.default_rng(80 + M)
    xn = rng.standard_normal((M, hc, H)).astype(np.float32)
    lo = (rng.standard_normal((M, lr)) * 3).astype(np.float32)
    ctx = trmoe.Context(H, 16, 128, 4, M, hiprec=True)
    mixed = _mixed(ctx, W, up, bits, hc, lr, xn, lo, H)
    ctx.close()
    if M == 1:
        want = O.hc_mix(up, bits, hc, lr, xn, lo, True, True)
        assert np.abs(mixed - want).max() <= 1e-6 * np.abs(want).max()
        assert (mixed == want).mean() >= 0.99
        return
    rows = np.unique(np.concatenate([np.arange(16), np.arange(M - 20, M), rng.choice(M, 16, replace=False)]))
    want = O.hc_mix(up, bits, hc, lr, xn[rows], lo[rows], False)
    got = mixed[rows]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.abs(got - want).max()
