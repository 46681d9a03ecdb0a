"""Pins the CPU oracle (a restatement of the reference's CPU MoE path) before it is trusted.

Each check is chosen so that a plausible restatement mistake fails it: golden vectors written by
the reference's own numpy packer (tests/golden/make_fixtures.py), hardware F16C conversions, the
reference's own Rust unit tests (ported; file:line cited), exact-arithmetic cases, and f64 brute
force on small shapes.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest

import oracle as O
from layerdata import Layer

GOLD = os.path.join(os.path.dirname(__file__), "golden", "blocks_codec.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


# ---- f16 ---------------------------------------------------------------------------------

def test_f16_matches_hardware_f16c():
    if not O.lib().orc_have_f16c():
        pytest.skip("no F16C on this host")
    assert O.lib().orc_selftest_f16(97) == 0


def test_f16_matches_numpy_golden(gold):
    fin, fout = gold["f16_in"], gold["f16_out"]
    got = np.array([O.f32_to_f16(v) for v in fin], np.uint16)
    assert np.array_equal(got, fout)
    allh = np.arange(65536, dtype=np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    mine = np.array([O.f16_to_f32(int(h)) for h in allh[::17]], np.float32)
    ok = np.isnan(ref[::17]) | (mine.view(np.uint32) == ref[::17].view(np.uint32))
    assert ok.all()


# ---- Q4_K / TQ layouts against the reference packer's own outputs ------------------------

def test_q4k_rows_golden(gold):
    raw = gold["q4k_raw"]
    rows, K = raw.shape[0], raw.shape[1] // 144 * 256
    q, dd, mm = O.q4k_rows(raw, rows, K)
    assert np.array_equal(q, gold["q4k_q"])
    assert np.array_equal(dd, gold["q4k_dd"])
    assert np.array_equal(mm, gold["q4k_mm"])


@pytest.mark.parametrize("fmt", ["q80", "q51"])
def test_q80_q51_rows_golden(gold, fmt):
    """orc_q80_rows / orc_q51_rows against the reference's q8_0_rows / q5_1_rows (blocks.py:57-78)
    on seeded blocks and edge cases: d where -128 d overflows f16, subnormal, zero and negative d,
    int8 extremes, qh all ones / zeros / alternating."""
    raw = gold[fmt + "_raw"]
    rows, K = raw.shape[0], raw.shape[1] // (34 if fmt == "q80" else 24) * 32
    q, d, m = (O.q80_rows if fmt == "q80" else O.q51_rows)(raw, rows, K)
    assert np.array_equal(q, gold[fmt + "_q"])
    assert np.array_equal(d, gold[fmt + "_d"])
    assert np.array_equal(m, gold[fmt + "_m"])


def test_q4k_to_tq_bytes_golden(gold):
    raw = gold["q4k_raw"]
    rows, K = raw.shape[0], raw.shape[1] // 144 * 256
    t32, b = O.gguf_to_tq(O.FMT_Q4_K, raw, rows, K, 32)
    assert b == 4 and np.array_equal(t32, gold["q4k_tq4_32"])
    t16, _ = O.gguf_to_tq(O.FMT_Q4_K, raw, rows, K, 16)
    assert np.array_equal(t16, gold["q4k_tq4_16"])


@pytest.mark.parametrize("bits,kb,r,k", [(4, 32, 32, 64), (5, 32, 16, 96), (8, 32, 40, 64), (5, 16, 48, 80),
                                         (8, 16, 16, 32), (4, 16, 16, 48), (4, 32, 5, 64)])
def test_pack_tq_golden(gold, bits, kb, r, k):
    tag = f"tq{bits}_{kb}_{r}x{k}"
    buf = O.pack_tq(gold[tag + "_q"], gold[tag + "_d"], gold[tag + "_m"], bits, kb)
    assert np.array_equal(buf, gold[tag + "_bytes"])
    deq = O.dequant_tq(buf, r, k, bits, kb)
    assert np.array_equal(deq, gold[tag + "_deq"])


def test_tq_block_bytes_match_reference():
    # codec.rs:106-113 sizes_match_python
    L = O.lib()
    assert L.orc_tq_block_bytes(4, 32) == 64 + 256
    assert L.orc_tq_block_bytes(5, 32) == 64 + 256 + 64
    assert L.orc_tq_block_bytes(8, 32) == 64 + 512
    assert L.orc_tq_block_bytes(5, 16) == 64 + 128 + 32
    assert O.tq_matrix_bytes(80, 2560, 4, 32) == 5 * 80 * 320
    assert O.tq_matrix_bytes(2560, 80, 5, 16) == 160 * 5 * 224


def test_q6k_mapping_bruteforce():
    """Q6_K has no reference converter (extension): pin the mapping to ggml's published
    dequantisation d*sc*(q-32), evaluated independently in f64 from the raw bytes."""
    rows, K = 3, 512
    raw = O.gen_gguf(O.FMT_Q6_K, 5, 77, rows, K).reshape(rows, -1)
    want = np.zeros((rows, K))
    for r in range(rows):
        for sb in range(K // 256):
            b = raw[r, sb * 210:(sb + 1) * 210]
            ql, qh, sc = b[:128].astype(int), b[128:192].astype(int), b[192:208].view(np.int8).astype(int)
            d = float(b[208:210].view(np.float16)[0])
            for i in range(256):
                n, rem = divmod(i, 128)
                g, l = divmod(rem, 32)
                lo = ql[64 * n + l + (32 if g in (1, 3) else 0)]
                lo = (lo & 15) if g < 2 else (lo >> 4)
                hi = (qh[32 * n + l] >> (2 * g)) & 3
                q = lo | (hi << 4)
                dd = float(np.float16(d * sc[i // 16]))  # the only rounding: f16(d*sc)
                want[r, sb * 256 + i] = dd * (q - 32)
    got = O.gguf_dequant(O.FMT_Q6_K, raw, rows, K)
    assert np.allclose(got, want, rtol=0, atol=1e-7 * np.abs(want).max())


def test_q80_dequant_closed_form():
    """Q8_0 through the offset-folded unsigned form (q + 128, m = f16(-128 d)) dequantises to
    exactly d * int8, ggml's definition of the block; the generator keeps d in its range and puts
    it at the start of every 34-byte block."""
    rows, K = 3, 512
    raw = O.gen_gguf(O.FMT_Q8_0, 9, 5, rows, K).reshape(rows, -1)
    assert raw.shape[1] == K // 32 * 34 == O.gguf_row_bytes(O.FMT_Q8_0, K)
    blk = raw.reshape(rows, K // 32, 34)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float32)[:, :, 0]
    assert (d >= np.float16(1e-4)).all() and (d <= np.float16(2e-3)).all()
    want = (d[:, :, None] * blk[:, :, 2:].view(np.int8).astype(np.float32)).reshape(rows, K)
    got = O.gguf_dequant(O.FMT_Q8_0, raw, rows, K)
    assert np.array_equal(got, want)
    # the TQ form at both block widths holds the same weights
    for kb in (16, 32):
        tq, bits = O.gguf_to_tq(O.FMT_Q8_0, raw, rows, K, kb)
        assert bits == 8 and np.array_equal(O.dequant_tq(tq, rows, K, 8, kb), want)


def test_q51_dequant_bruteforce():
    """Q5_1 through q5_1_rows' form against an evaluation of ggml's layout: element i of a block
    is nibble i % 16 of qs (low for i < 16, high after) with bit i of qh on top, w = d q + m."""
    rows, K = 2, 512
    raw = O.gen_gguf(O.FMT_Q5_1, 9, 6, rows, K).reshape(rows, -1)
    assert raw.shape[1] == K // 32 * 24 == O.gguf_row_bytes(O.FMT_Q5_1, K)
    want = np.zeros((rows, K), np.float32)
    for r in range(rows):
        for b in range(K // 32):
            blk = raw[r, 24 * b:24 * b + 24]
            d, m = (np.float32(v) for v in blk[:4].view(np.float16))
            qh = int(blk[4:8].view(np.uint32)[0])
            for i in range(32):
                nib = (int(blk[8 + i % 16]) >> (4 * (i // 16))) & 15
                q = nib | (((qh >> i) & 1) << 4)
                want[r, 32 * b + i] = np.float32(d * np.float32(q)) + m
    got = O.gguf_dequant(O.FMT_Q5_1, raw, rows, K)
    assert np.array_equal(got, want)
    for kb in (16, 32):
        tq, bits = O.gguf_to_tq(O.FMT_Q5_1, raw, rows, K, kb)
        assert bits == 5 and np.array_equal(O.dequant_tq(tq, rows, K, 5, kb), want)


def test_q4k_dequant_bruteforce():
    """Q4_K dequant via (q, f16(d*sc), f16(-dmin*mn)) against an f64 evaluation of ggml's layout."""
    rows, K = 2, 512
    raw = O.gen_gguf(O.FMT_Q4_K, 9, 3, rows, K).reshape(rows, -1)
    want = np.zeros((rows, K))
    for r in range(rows):
        for sb in range(K // 256):
            b = raw[r, sb * 144:(sb + 1) * 144]
            d, dmin = (float(v) for v in b[:4].view(np.float16))
            s = b[4:16].astype(int)
            for j in range(8):
                if j < 4:
                    sc, mn = s[j] & 63, s[4 + j] & 63
                else:
                    sc = (s[8 + j - 4] & 15) | ((s[j - 4] >> 6) << 4)
                    mn = (s[8 + j - 4] >> 4) | ((s[4 + j - 4] >> 6) << 4)
                c, h = divmod(j, 2)
                for i in range(32):
                    byte = int(b[16 + 32 * c + i])
                    q = (byte & 15) if h == 0 else (byte >> 4)
                    want[r, sb * 256 + 32 * j + i] = float(np.float16(d * sc)) * q + float(np.float16(-(dmin * mn)))
    got = O.gguf_dequant(O.FMT_Q4_K, raw, rows, K)
    assert np.allclose(got, want, rtol=0, atol=2e-7 * np.abs(want).max())


# ---- activation quantisation (quant.rs) ---------------------------------------------------

def test_quant_block_known_answers():
    # amax = 127 -> scale 1, inv 1: q = rint_even(x)
    x = np.zeros(32, np.float32)
    x[:9] = [0.5, 1.5, 2.5, -0.5, -1.5, 127.0, -126.5, 3.49999, -2.5]
    q, s, su = O.quant_block(x)
    assert s == 1.0
    assert list(q[:9]) == [0, 2, 2, 0, -2, 127, -126, 3, -2]
    assert su == int(q.astype(np.int32).sum())
    # all zeros: scale 0, inv 0, q 0
    q, s, su = O.quant_block(np.zeros(16, np.float32))
    assert s == 0.0 and su == 0 and not q.any()


def test_quant_multiplies_by_the_rounded_inverse():
    """quant.rs:158-160 rounds x * f32(127 / amax), not x / f32(amax / 127): blocks where the two
    forms give different int8 values are found by search, and the oracle must give the first."""
    rng = np.random.default_rng(17)
    hits = 0
    for kb in (16, 32):
        # values aimed at the rounding boundaries: x = f32((j + 1/2) * amax / 127), a few ulps apart
        n = 20000
        amax0 = rng.uniform(0.01, 50, n).astype(np.float32)
        j = rng.integers(-126, 126, (n, kb - 1))
        aim = ((j + 0.5) * amax0[:, None].astype(np.float64) / 127).astype(np.float32)
        aim = (aim.view(np.int32) + rng.integers(-2, 3, aim.shape).astype(np.int32)).view(np.float32)
        x = np.concatenate([amax0[:, None], aim], 1).astype(np.float32)
        amax = np.abs(x).max(1, keepdims=True)
        inv = np.float32(127) / amax
        by_inv = np.rint(x * inv).astype(np.int32)
        by_div = np.rint(x / (amax / np.float32(127))).astype(np.int32)
        differ = np.flatnonzero((by_inv != by_div).any(1))
        assert differ.size > 0
        q, s, su = O.quant_rows(x[differ], kb)
        assert np.array_equal(q.reshape(-1, kb).astype(np.int32), by_inv[differ])
        assert not np.array_equal(q.reshape(-1, kb).astype(np.int32), by_div[differ])
        assert np.array_equal(su.reshape(-1), by_inv[differ].sum(1))
        hits += differ.size
    assert hits >= 10


def test_quant_invariants_and_pair_residual():
    rng = np.random.default_rng(3)
    for kb in (16, 32):
        x = (rng.standard_normal(4 * 512) * 3).astype(np.float32).reshape(4, 512)
        q, s, su = O.quant_rows(x, kb)
        nb = 512 // kb
        assert np.abs(q.astype(int)).max() <= 127
        assert np.array_equal(su, q.reshape(4, nb, kb).astype(np.int32).sum(-1))
        deq = q.reshape(4, nb, kb) * s[:, :, None]
        assert (np.abs(deq - x.reshape(4, nb, kb)) <= s[:, :, None] / 2 * (1 + 1e-5) + 1e-30).all()
        amax = np.abs(x.reshape(4, nb, kb)).max(-1)
        assert np.array_equal(s, (amax / np.float32(127)).astype(np.float32))
        # pair: residual row quantises x - q*scale (one rounding: fnmadd)
        qp, sp, sup = O.quant_pair(x[0], kb)
        r = (x[0].astype(np.float64) - qp[0].astype(np.float64) * np.repeat(sp[0], kb)).astype(np.float32)
        q2, s2, su2 = O.quant_rows(r[None], kb)
        assert np.array_equal(qp[1], q2[0]) and np.array_equal(sp[1], s2[0]) and np.array_equal(sup[1], su2[0])


# ---- GEMV (gemv.rs) ----------------------------------------------------------------------

class Lcg:
    """gemv.rs:181-190"""

    def __init__(self, s):
        self.s = s

    def next(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & (2 ** 64 - 1)
        return self.s >> 33

    def unif(self):
        return np.float32((self.next() % 100000) / 100000.0)


def synth_tq(rows, k, bits, kb, rng):
    """gemv.rs:192-198"""
    nb = k // kb
    q = np.array([rng.next() % (1 << bits) for _ in range(rows * k)], np.uint8).reshape(rows, k)
    d = np.array([O.f32_to_f16(np.float32(rng.unif() * np.float32(0.02) + np.float32(0.001)))
                  for _ in range(rows * nb)], np.uint16).reshape(rows, nb)
    m = np.array([O.f32_to_f16(np.float32(-rng.unif() * np.float32(0.2))) for _ in range(rows * nb)],
                 np.uint16).reshape(rows, nb)
    return O.pack_tq(q, d, m, bits, kb)


@pytest.mark.parametrize("bits,kb,rows,k,m", [(4, 32, 80, 2560, 1), (5, 32, 48, 256, 3), (8, 32, 32, 320, 8),
                                              (5, 16, 160, 80, 1), (8, 16, 32, 80, 4), (4, 16, 16, 32, 2)])
def test_gemv_matches_reference_all_codecs(bits, kb, rows, k, m):
    """gemv.rs:200-227: 1e-4*scale against the f64 product of the quantised activations,
    2e-2*scale against f32 activations, and the accumulate path."""
    rng = Lcg(7 + bits * 31 + kb)
    w = synth_tq(rows, k, bits, kb, rng)
    wf = O.dequant_tq(w, rows, k, bits, kb).astype(np.float64)
    x = np.array([rng.unif() * 2 - 1 for _ in range(m * k)], np.float32).reshape(m, k)
    q, s, su = O.quant_rows(x, kb)
    y = O.gemv_tq(w, k, bits, kb, rows, q, s, su)
    xd = q.astype(np.float64) * np.repeat(s, kb, axis=1)
    want_q = xd @ wf.T
    want_f = x.astype(np.float64) @ wf.T
    scale = max(np.abs(want_f).max(), 1e-6)
    assert (np.abs(y - want_q) <= 1e-4 * scale + 1e-5).all()
    assert (np.abs(y - want_f) <= 2e-2 * scale).all()
    y2 = O.gemv_tq(w, k, bits, kb, rows, q, s, su, y=y.copy(), accumulate=True)
    assert (np.abs(y2 - 2 * want_q) <= 2e-4 * scale + 1e-5).all()


def test_gemv_exact_arithmetic():
    """With power-of-two scales and small integers every f32 operation is exact, so the result
    must equal the integer formula sum_b d*sx*dot_b + m*sx*sum_b exactly (a dropped min term,
    a swapped nibble or a wrong block index fails)."""
    rows, k, kb, bits = 16, 128, 32, 4
    rng = np.random.default_rng(1)
    nb = k // kb
    q = rng.integers(0, 16, (rows, k), dtype=np.uint8)
    d = np.array([O.f32_to_f16(2.0 ** -int(e)) for e in rng.integers(2, 6, rows * nb)], np.uint16).reshape(rows, nb)
    mv = np.array([O.f32_to_f16(-(2.0 ** -int(e))) for e in rng.integers(1, 5, rows * nb)], np.uint16).reshape(rows, nb)
    w = O.pack_tq(q, d, mv, bits, kb)
    xq = rng.integers(-127, 128, (2, k)).astype(np.int8)
    s = (2.0 ** -rng.integers(0, 4, (2, nb))).astype(np.float32)
    su = xq.reshape(2, nb, kb).astype(np.int32).sum(-1)
    y = O.gemv_tq(w, k, bits, kb, rows, xq, s, su)
    df = np.array([[O.f16_to_f32(v) for v in r] for r in d])
    mf = np.array([[O.f16_to_f32(v) for v in r] for r in mv])
    want = np.zeros((2, rows))
    for mi in range(2):
        for r in range(rows):
            for b in range(nb):
                dot = int((q[r, b * kb:(b + 1) * kb].astype(int) * xq[mi, b * kb:(b + 1) * kb]).sum())
                want[mi, r] += mf[r, b] * s[mi, b] * su[mi, b] + df[r, b] * s[mi, b] * dot
    assert np.array_equal(y.astype(np.float64), want)


def test_gemm_many_rows_and_row_map():
    """gemv.rs:256-273 plus the row-map accumulate used by the batch down projection."""
    rng = Lcg(21)
    rows, k, m = 48, 256, 21
    w = synth_tq(rows, k, 4, 32, rng)
    x = np.array([rng.unif() - 0.5 for _ in range(m * k)], np.float32).reshape(m, k)
    q, s, su = O.quant_rows(x, 32)
    y = O.gemv_tq(w, k, 4, 32, rows, q, s, su)
    for mi in range(m):
        y1 = O.gemv_tq(w, k, 4, 32, rows, q[mi:mi + 1], s[mi:mi + 1], su[mi:mi + 1])
        assert np.array_equal(y1[0], y[mi])  # chunking into MAX_M passes does not change a row
    rmap = np.array([(5 * i) % m for i in range(m)], np.uint32)
    base = np.ones((m, rows), np.float32)
    got = O.gemv_tq(w, k, 4, 32, rows, q, s, su, y=base.copy(), rows=rmap, accumulate=True)
    want = base.copy()
    want[rmap] = want[rmap] + y
    assert np.array_equal(got, want)


def test_pair_mode_is_much_more_accurate():
    """gemv.rs:229-254"""
    rng = Lcg(11)
    rows, k = 256, 768
    w = synth_tq(rows, k, 8, 32, rng)
    wf = O.dequant_tq(w, rows, k, 8, 32).astype(np.float64)
    x = np.array([0.5 if i % 32 == 5 else (rng.unif() - 0.5) * 0.01 for i in range(k)], np.float32)
    want = wf @ x.astype(np.float64)
    q1, s1, su1 = O.quant_rows(x[None], 32)
    q2, s2, su2 = O.quant_pair(x, 32)
    y1 = O.gemv_tq(w, k, 8, 32, rows, q1, s1, su1)[0]
    y2 = O.gemv_tq(w, k, 8, 32, rows, q2, s2, su2, pair=True)[0]
    e1, e2 = np.abs(y1 - want).sum(), np.abs(y2 - want).sum()
    assert e2 < e1 / 20


# ---- router (router.rs) ------------------------------------------------------------------

def probs(lg):
    p = np.exp(lg.astype(np.float64) - lg.max())
    return p / p.sum()


def test_picks_top_and_renormalises():
    """router.rs:168-193"""
    lg = np.array([((i * 37) % 101) * 0.1 for i in range(512)], np.float32)
    ids, w = O.route_topk(lg, 10)
    srt = np.sort(lg)[::-1]
    assert np.array_equal(lg[ids], srt[:10])
    assert abs(w.sum() - 1) < 1e-5 and w[0] >= w[9]
    p = probs(lg)
    assert np.allclose(w, p[ids] / p[ids].sum(), atol=1e-6)


def test_ties_match_sequential_selection():
    """router.rs:277-312 (200 LCG trials with many exact ties)"""
    seed = 3
    for _ in range(200):
        lg = np.zeros(512, np.float32)
        for i in range(512):
            seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
            lg[i] = ((seed >> 20) % 40) * 0.25
        ids, _ = O.route_topk(lg, 10)
        taken = np.zeros(512, bool)
        ref = []
        for _ in range(10):
            best, bv = None, -np.inf
            for i in range(512):
                if not taken[i] and lg[i] > bv:
                    bv, best = lg[i], i
            taken[best] = True
            ref.append(best)
        assert list(ids) == ref


def test_mass_policy():
    """router.rs:198-247 (stops_at_the_target_mass_within_bounds)"""
    lg = np.full(512, -12.0, np.float32)
    for i, p in enumerate([0.61, 0.19, 0.09, 0.05, 0.025, 0.015]):
        lg[i * 7] = np.float32(math.log(np.float32(p)))
    pr = probs(lg)
    ids, w = O.route_mass(lg, 1, 10, 0.95, O.BASIS_ALL)
    n = len(ids)
    cum = np.cumsum([pr[i * 7] for i in range(6)])
    assert n == int(np.argmax(cum >= 0.95)) + 1
    assert list(ids) == [i * 7 for i in range(n)]
    assert abs(w.sum() - 1) < 1e-5
    tid, tw = O.route_topk(lg, n)
    assert np.array_equal(ids, tid) and np.allclose(w, tw, atol=1e-6)
    assert len(O.route_mass(lg, 8, 10, 0.5, O.BASIS_ALL)[0]) == 8
    assert len(O.route_mass(lg, 1, 3, 0.999, O.BASIS_ALL)[0]) == 3
    assert len(O.route_mass(lg, 1, 32, 1.0, O.BASIS_ALL)[0]) == 32
    flat = np.full(512, 0.5, np.float32)
    ids, _ = O.route_mass(flat, 1, 10, 0.95, O.BASIS_ALL)
    assert list(ids) == list(range(10))
    assert len(O.route_mass(flat, 1, 10, 0.95, O.BASIS_TOP)[0]) == 10
    assert len(O.route_mass(flat, 1, 10, 0.05, O.BASIS_TOP)[0]) == 1
    tid, tw = O.route_topk(lg, 10)
    acc, expect = np.float32(0), None
    for j, v in enumerate(tw):
        acc = np.float32(acc + v)
        if acc >= np.float32(0.9):
            expect = j + 1
            break
    ids, _ = O.route_mass(lg, 1, 10, 0.9, O.BASIS_TOP)
    assert len(ids) == expect and np.array_equal(ids, tid[:expect])
    lg2 = np.array([((i * 37) % 101) * 0.1 for i in range(512)], np.float32)
    tid, tw = O.route_topk(lg2, 10)
    for basis in (O.BASIS_ALL, O.BASIS_TOP):
        ids, w = O.route_mass(lg2, 10, 10, 0.5, basis)
        assert np.array_equal(ids, tid) and np.array_equal(w, tw)  # bit-identical
    assert O.policy_validate(0, 10, 0.9, 512)[0] != 0
    assert O.policy_validate(1, 33, 0.9, 512)[0] != 0
    assert O.policy_validate(1, 20, 0.9, 16)[0] != 0
    assert O.policy_validate(1, 10, 0.0, 512)[0] != 0
    assert O.policy_validate(1, 10, 0.9, 512)[0] == 0
    cum = O.mass_profile(lg2)
    srt = np.sort(probs(lg2))[::-1]
    assert np.allclose(cum, np.cumsum(srt[:32]), atol=1e-5)


def test_nan_and_neg_inf_never_selected():
    lg = np.full(64, np.nan, np.float32)
    lg[[3, 9]] = [1.0, 2.0]
    lg[10] = -np.inf
    ids, w = O.route_topk(lg, 3)
    assert list(ids[:2]) == [9, 3] and ids[2] == 0xFFFFFFFF


# ---- elementwise (elem.rs, smallgemm.rs, attn.rs) ----------------------------------------

def test_exp_sigmoid_silu_accuracy():
    """elem.rs:286-303"""
    L = O.lib()
    for i in range(-2000, 2000, 7):
        x = np.float32(i * 0.04)
        y = L.orc_exp512(float(x))
        want = math.exp(float(x))
        assert abs(y - want) <= 2e-6 * want + 1e-30
        s = L.orc_silu512(float(x))
        assert abs(s - float(x) * L.orc_sigmoid(float(x))) <= 1e-5 * (1 + abs(float(x)))
    assert L.orc_exp512(0.0) == 1.0


def test_rmsnorm():
    """elem.rs:305-321"""
    x = np.sin(np.arange(128) * 0.37).astype(np.float32)
    w = (1 + np.arange(128) * 0.01).astype(np.float32)
    y = O.rmsnorm(x, w, 1e-6)
    ms = (x.astype(np.float64) ** 2).mean()
    assert np.allclose(y, x / np.sqrt(ms + 1e-6) * w, atol=1e-5)


def test_gemm_f32_nt_and_dot_against_f64():
    """smallgemm.rs:61-85 and the dot used for router logits"""
    rng = np.random.default_rng(7)
    x = (rng.random((9, 320)) - 0.5).astype(np.float32)
    w = (rng.random((12, 320)) - 0.5).astype(np.float32)
    y = O.gemm_f32_nt(x, w)
    assert np.abs(y - x.astype(np.float64) @ w.astype(np.float64).T).max() < 1e-4
    for n in (2048, 2048 + 16, 2048 + 48 + 5):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        assert abs(O.dot(a, b) - a.astype(np.float64) @ b) < 1e-3


def test_dot_chain_order():
    """The 4-chain order is observable: put a large value and its negation in the same lane of
    chains 0/1 (they cancel before the tree) versus lanes that only meet in the tree."""
    a = np.zeros(64, np.float32)
    b = np.ones(64, np.float32)
    a[0], a[16], a[1] = 1e8, -1e8, 1.0  # chain0 lane0, chain1 lane0 cancel exactly; lane1 keeps 1
    assert O.dot(a, b) == 1.0
    a = np.zeros(64, np.float32)
    a[0], a[8], a[1] = 1e8, 1.0, -1e8  # lane0 + lane8 first: 1e8+1 rounds to 1e8, then -1e8 -> 0
    assert O.dot(a, b) == 0.0


def epilogue_order_case():
    """One TQ8_32 strip whose row 0 makes the order of gemv.rs:141-148 observable (the other rows
    are zero).  Activation scale sx = 1, so u = sx * sum = sum and t = d * sx = d exactly.
    d = 1 + 2^-10 (f16 0x3C01), dot = 127 * 7 + 104 * 149 = 16385, so dot * d = 16401 + 2^-10:
    between the floats 16401 and 16401 + 2^-9, a tie that rounds to even, 16401.  m = -71 and
    sum = 127 + 104 = 231 give m * u = -16401 exactly.  The reference's order, fma(m, u, 0) =
    -16401 then fma(dot, t, acc) = 2^-10 exactly (the fused product keeps the half-ulp).  Plain
    mul + add gives round(dot * d) - 16401 = 0; the terms swapped give round(dot * d) then
    fma(m, u, 16401) = 0."""
    k, kb, bits = 32, 32, 8
    q = np.zeros((16, k), np.uint8)
    q[0, 0], q[0, 1] = 7, 149
    d = np.full((16, 1), 0x3C00, np.uint16)
    d[0, 0] = 0x3C01
    m = np.zeros((16, 1), np.uint16)
    m[0, 0] = O.f32_to_f16(-71.0)
    assert O.f16_to_f32(m[0, 0]) == -71.0 and O.f16_to_f32(d[0, 0]) == 1 + 2.0 ** -10
    w = O.pack_tq(q, d, m, bits, kb)
    xq = np.zeros((1, k), np.int8)
    xq[0, 0], xq[0, 1] = 127, 104
    return w, k, bits, kb, xq, np.ones((1, 1), np.float32), np.array([[231]], np.int32)


def test_gemv_epilogue_order():
    """The two-FMA epilogue of gemv.rs:141-148, pinned by a designed case (epilogue_order_case):
    acc = fma(m, sx * sum, acc) first, then fma(cvt(dot), d * sx, acc), both fused."""
    w, k, bits, kb, xq, s, su = epilogue_order_case()
    y = O.gemv_tq(w, k, bits, kb, 16, xq, s, su)
    assert y[0, 0] == np.float32(2.0 ** -10)
    assert np.all(y[0, 1:] == 0)


def test_gemm_f32_nt_lane_map():
    """smallgemm.rs:8-59: output (i, j) accumulates k = 16 s + l in lane l with one fused
    multiply-add per step, then _mm512_reduce_add_ps's halving tree (lanes l and l + 8, then
    + 4, + 2, + 1).  Designed cases:
    - (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 rounds (a tie, to even) to 1 + 2^-11; the same product
      negated at k = 16, in the same lane, leaves -2^-24 with a fused chain and 0 with mul + add;
    - 1e8 at k = 0 and -1e8 at k = 16 cancel inside lane 0, so the 1 at k = 1 survives: 1;
    - 1e8 (lane 0) and 1 (lane 8) meet first in the tree (1e8 + 1 rounds to 1e8), and -1e8
      (lane 1) only at the last step: 0."""
    a = np.float32(1 + 2.0 ** -12)
    x = np.ones((1, 32), np.float32)
    x[0, 0], x[0, 16] = a, -a
    w = np.zeros((4, 32), np.float32)
    w[0, 0], w[0, 16] = a, a
    y = O.gemm_f32_nt(x, w)
    assert y[0, 0] == np.float32(-(2.0 ** -24)) and y[0, 1] == 0.0
    w = np.zeros((4, 32), np.float32)
    w[0, 0], w[0, 16], w[0, 1] = 1e8, -1e8, 1.0
    w[1, 0], w[1, 8], w[1, 1] = 1e8, 1.0, -1e8
    y = O.gemm_f32_nt(np.ones((1, 32), np.float32), w)
    assert y[0, 0] == 1.0 and y[0, 1] == 0.0


def rmsnorm_order_case():
    """n = 64; sixteen entries 2^-30 make sumsq = 2^-56 exactly, the mean 2^-62, r = 1 / sqrt(2^-62)
    = 2^31 (eps = 0).  Two probes p = 2^-90 (1 + 2^-23), whose squares vanish below the sum's ulp:
    with w = 2^-60 the reference's (x r) w gives 2^-119 (1 + 2^-23), while (x w) r underflows
    through the subnormals (2^-150 (1 + 2^-23) -> 2^-149) to 2^-118; with w = 2^100, (x r) w gives
    2^41 (1 + 2^-23), while x (r w) overflows (2^131 -> inf)."""
    x = np.zeros(64, np.float32)
    w = np.ones(64, np.float32)
    x[::4] = np.float32(2.0 ** -30)
    p = np.float32(2.0 ** -90 * (1 + 2.0 ** -23))
    x[1], w[1] = p, np.float32(2.0 ** -60)
    x[2], w[2] = p, np.float32(2.0 ** 100)
    want = np.zeros(64, np.float32)
    want[::4] = 2.0
    want[1] = np.float32(2.0 ** -119 * (1 + 2.0 ** -23))
    want[2] = np.float32(2.0 ** 41 * (1 + 2.0 ** -23))
    return x, w, want


def test_rmsnorm_product_order():
    """elem.rs:255-262: y = (x * r) * w with r = 1 / sqrt(sumsq / n + eps), pinned by a designed
    case (rmsnorm_order_case) that (x w) r and x (r w) both miss."""
    x, w, want = rmsnorm_order_case()
    y = O.rmsnorm(x, w, 0.0)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


# ---- the MoE block -----------------------------------------------------------------------

def f64_moe(layer, x, ids, w, sh_scale):
    """Textbook MoE in f64 (tools/oracle/check_layer.py:52-64): sum_j w_j down_j(silu(g x) u x) +
    sigmoid(shexp_gate . x) shared(x), with the f16-rounded dequantised weights."""
    H, F = layer.H, layer.F

    def ffn(g, u, d):
        G = O.gguf_dequant(layer.gate_fmt, g, F, H).astype(np.float64)
        U = O.gguf_dequant(layer.gate_fmt, u, F, H).astype(np.float64)
        D = O.gguf_dequant(layer.down_fmt, d, H, F).astype(np.float64)
        a = G @ x
        return D @ (a / (1 + np.exp(-a)) * (U @ x))

    out = sh_scale * ffn(layer.sh_gate, layer.sh_up, layer.sh_down)
    for e, wj in zip(ids, w):
        out += float(wj) * ffn(*layer.expert(int(e)))
    return out


@pytest.fixture(scope="module")
def small_layer():
    return Layer(seed=11, H=512, E=32, F=256)


def test_moe_block_against_f64(small_layer):
    L = small_layer
    orc = L.oracle()
    x = L.x(1)[0]
    r = orc.moe_block(x, k=4, hiprec=True)
    sh = 1 / (1 + math.exp(-float(np.dot(L.shexp_gate.astype(np.float64), x))))
    want = f64_moe(L, x.astype(np.float64), r["ids"], r["w"].astype(np.float64), sh)
    scale = np.abs(want).max()
    # pair (two-level) activations: error ~1e-4 of the output scale
    assert np.abs(r["out"] - want).max() <= 3e-3 * scale
    r1 = orc.moe_block(x, k=4, hiprec=False)
    assert np.abs(r1["out"] - want).max() <= 0.06 * scale  # single-level int8 (moe_mass.rs:67 bound)
    assert np.abs(r["out"] - want).max() < np.abs(r1["out"] - want).max()
    assert r["stats"] == (1, 4)


def test_moe_batch_dispatch_and_against_decode(small_layer):
    """moe_mass.rs:61-68: batch vs decode within 0.06*scale + 0.05; dispatch is the stable sort."""
    L = small_layer
    orc = L.oracle()
    X = L.x(6)
    rb = orc.moe_batch(X, k=4, router_dot_max_m=16)
    ids = rb["ids"][:, :4]
    flat = [(t, s, int(ids[t, s])) for t in range(6) for s in range(4)]
    order = sorted(range(len(flat)), key=lambda i: flat[i][2])  # python sort is stable
    assert list(rb["ent_tok"]) == [flat[i][0] for i in order]
    assert list(rb["ent_expert"]) == [flat[i][2] for i in order]
    uniq = sorted(set(f[2] for f in flat))
    assert list(rb["grp_expert"]) == uniq
    sizes = np.diff(rb["grp_start"])
    assert list(sizes[rb["grp_order"]]) == sorted(sizes, reverse=True)
    for t in range(6):
        rd = orc.moe_block(X[t], k=4, hiprec=True)
        assert np.array_equal(rd["ids"], ids[t])
        scale = np.abs(rd["out"]).max()
        assert np.abs(rb["out"][t] - rd["out"]).max() <= 0.06 * scale + 0.05


def test_policy_min_eq_max_is_topk(small_layer):
    """moe_mass.rs:36-44: min = max = k is bit-identical to top-k on both paths."""
    orc = small_layer.oracle()
    X = small_layer.x(3)
    a = orc.moe_block(X[0], k=4)
    b = orc.moe_block(X[0], k=4, policy=(4, 4, 0.5, O.BASIS_TOP))
    assert np.array_equal(a["out"], b["out"])
    a = orc.moe_batch(X, k=4)
    b = orc.moe_batch(X, k=4, policy=(4, 4, 0.5, O.BASIS_ALL))
    assert np.array_equal(a["out"], b["out"])


def test_q6k_down_layer_runs(small_layer):
    L = Layer(seed=4, H=512, E=16, F=256, down_fmt=O.FMT_Q6_K)
    orc = L.oracle()
    x = L.x(1)[0]
    r = orc.moe_block(x, k=3)
    sh = 1 / (1 + math.exp(-float(np.dot(L.shexp_gate.astype(np.float64), x))))
    want = f64_moe(L, x.astype(np.float64), r["ids"], r["w"].astype(np.float64), sh)
    assert np.abs(r["out"] - want).max() <= 3e-3 * np.abs(want).max()


def _tq_from(q, d, m, bits):
    return O.pack_tq(q.astype(np.uint8), d.astype(np.float16), m.astype(np.float16), bits, 32)


def test_hc_mix_half_gate_when_up_is_zero():
    """With every up block's d = m = 0 the gate is sigmoid(0) = 1/2 exactly, so mixed is the
    stream sum times 1/hc in the reference's order: decode accumulates from 0 with a separate
    multiply and add (exec.rs:1221-1227), batch multiplies stream 0 and fuses the rest
    (exec_batch.rs:953-959); with a gate of 1/2 both are the same float32 sequence.  This fixes the
    [hc][hh] stream layout, the 1/hc factor and sigmoid(0)."""
    hc, hh, lr, M = 3, 64, 64, 4
    rows = hc * hh
    up = _tq_from(np.zeros((rows, lr)), np.zeros((rows, lr // 32)), np.zeros((rows, lr // 32)), 8)
    rng = np.random.default_rng(5)
    xn = rng.standard_normal((M, hc, hh)).astype(np.float32)
    lo = rng.standard_normal((M, lr)).astype(np.float32)
    inv = np.float32(1.0) / np.float32(hc)
    want = np.zeros((M, hh), np.float32)
    for mi in range(M):
        acc = np.zeros(hh, np.float32)
        for s in range(hc):
            acc = (acc + xn[mi, s] * np.float32(0.5)).astype(np.float32)
        want[mi] = acc * inv
    got_dec = O.hc_mix(up, 8, hc, lr, xn[:1], lo[:1], True)
    got_bat = O.hc_mix(up, 8, hc, lr, xn, lo, False)
    assert np.array_equal(got_dec.view(np.uint32), want[:1].view(np.uint32))
    assert np.array_equal(got_bat.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [4, 5, 8])
def test_hc_mix_against_f64(bits):
    """mixed = sum_s xn_s * sigmoid(W_up . silu(lo / hc)) / hc in f64 on the dequantised up
    matrix: the only differences are the int8 quantisation of silu(lo / hc) (per 32, two-level at
    decode with hiprec) and f32 rounding."""
    hc, hh, lr, M = 4, 96, 128, 3
    rows = hc * hh
    rng = np.random.default_rng(6 + bits)
    q = rng.integers(0, 1 << bits, (rows, lr))
    d = rng.uniform(5e-3, 2e-2, (rows, lr // 32)).astype(np.float16)
    mm = (-d.astype(np.float32) * rng.uniform(0, 1 << (bits - 1), (rows, lr // 32))).astype(np.float16)
    up = _tq_from(q, d, mm, bits)
    W = q * np.repeat(d.astype(np.float64), 32, axis=1) + np.repeat(mm.astype(np.float64), 32, axis=1)
    xn = rng.standard_normal((M, hc, hh)).astype(np.float32)
    lo = (rng.standard_normal((M, lr)) * 3).astype(np.float32)
    lsil = (lo / hc) / (1 + np.exp(-(lo.astype(np.float64) / hc)))
    g = 1 / (1 + np.exp(-(lsil @ W.T)))                      # [M][hc*hh]
    want = (xn.astype(np.float64) * g.reshape(M, hc, hh)).sum(axis=1) / hc
    scale = np.abs(want).max()
    for decode, hiprec, tol in ((True, True, 5e-5), (True, False, 3e-3), (False, False, 3e-3)):
        got = O.hc_mix(up, bits, hc, lr, xn[:1] if decode else xn, lo[:1] if decode else lo, decode, hiprec)
        err = np.abs(got - want[:got.shape[0]]).max()
        assert err <= tol * scale, (decode, hiprec, err, scale)


# ---- subset packs and packs written for T tiles --------------------------------------------

def test_fold_ids():
    """exec_batch.rs:214-225, designed cases: each id taken mod packed, then stepped (mod packed)
    past the ids already folded; more ids than packed experts is refused (the reference asserts)."""
    assert O.fold_ids([3, 19, 35], 16).tolist() == [3, 4, 5]
    assert O.fold_ids([15, 31, 0], 16).tolist() == [15, 0, 1]
    assert O.fold_ids([7, 2, 9, 40], 8).tolist() == [7, 2, 1, 0]
    assert O.fold_ids([5], 16).tolist() == [5]
    with pytest.raises(ValueError):
        O.fold_ids(list(range(9)), 8)
    rng = np.random.default_rng(3)
    for _ in range(50):  # distinct, inside the pack, and unchanged where nothing collides
        ids = rng.choice(512, 10, replace=False).astype(np.uint32)
        f = O.fold_ids(ids, 16)
        assert len(set(f.tolist())) == 10 and f.max() < 16 and f[0] == ids[0] % 16


def test_tiled_router_tile_order():
    """exec.rs:1003-1011 + exchange.rs:122-136: with T tiles each logit is the tiles' partial dots
    over their H/T columns, summed in tile order.  Designed partials 1e8, 1, -1e8 (one nonzero per
    tile slice against x = 1) give (1e8 + 1) - 1e8 = 0; 1e8, -1e8, 1 give 1."""
    from layerdata import TiledTQLayer
    L = TiledTQLayer(seed=5, H=192, E=16, F=96, T=3)
    L.router[:] = 0
    L.router[0, 0, 0], L.router[1, 0, 5], L.router[2, 0, 63] = 1e8, 1.0, -1e8
    L.router[0, 1, 1], L.router[1, 1, 2], L.router[2, 1, 3] = 1e8, -1e8, 1.0
    orc = L.oracle()
    x = np.ones((2, 192), np.float32)
    for dot_rows in (True, False):
        lg = orc.logits(x, dot_rows)
        assert lg[0, 0] == 0.0 and lg[0, 1] == 1.0 and np.all(lg[:, 2:] == 0), dot_rows


@pytest.mark.parametrize("T", [2, 4])
def test_tiled_layer_against_untiled(T):
    """A pack written for T tiles computes the same layer as the untiled pack of the same bytes,
    up to the order of the f32 sums (the router's and the down's partials per tile): ids equal,
    outputs within 2e-6 of the output scale, decode and batch.  A tile reading another tile's rows
    or columns would be off by the whole term."""
    from layerdata import TiledTQLayer, untile
    L = TiledTQLayer(seed=7, H=512, E=16, F=256, T=T)
    tiled, flat = L.oracle(), untile(L)
    x = L.x(6, tid=3)
    a, b = tiled.moe_block(x[0], k=4), flat.moe_block(x[0], k=4)
    assert np.array_equal(a["ids"], b["ids"])
    assert np.abs(a["out"] - b["out"]).max() <= 2e-6 * np.abs(b["out"]).max()
    a, b = tiled.moe_batch(x, k=4), flat.moe_batch(x, k=4)
    assert np.array_equal(a["ids"], b["ids"])
    assert np.abs(a["out"] - b["out"]).max() <= 2e-6 * np.abs(b["out"]).max()
    # and the tiles are not interchangeable: swapping two down tiles changes the output
    before = tiled.moe_block(x[0], k=4)["out"]
    L.down[[0, 1]] = L.down[[1, 0]]
    after = L.oracle().moe_block(x[0], k=4)["out"]
    assert np.abs(after - before).max() > 1e-2 * np.abs(before).max()


def test_subset_pack_folds_ids():
    """A subset pack (n_expert_packed < E): the layer routes on all E logits, then folds the ids
    onto the packed experts (exec.rs:1545-1549, exec_batch.rs:1418-1420); the result equals the
    full pack's layer with the folded ids' experts."""
    from layerdata import TiledTQLayer
    L = TiledTQLayer(seed=9, H=512, E=64, F=128, T=1, packed=16)
    orc = L.oracle()
    x = L.x(3, tid=4)
    r = orc.moe_block(x[0], k=6)
    lg = orc.logits(x[:1], True)[0]
    ids, w = O.route_topk(lg, 6)
    assert np.array_equal(r["ids"], O.fold_ids(ids, 16)) and np.array_equal(r["w"], w)
    rb = orc.moe_batch(x, k=6)
    lgb = orc.logits(x, False)
    for t in range(3):
        assert np.array_equal(rb["ids"][t, :6], O.fold_ids(O.route_topk(lgb[t], 6)[0], 16))
    assert rb["ent_expert"].max() < 16
