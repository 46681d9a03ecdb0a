"""ctypes wrapper of the CPU oracle (liboracle.so) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.
It restates the reference's CPU MoE path (tokenring-ai/tr-infer) and is the checker for the HIP
library, never a fallback for it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

FMT_Q4_K = 12
FMT_Q6_K = 14
FMT_Q8_0 = 8
FMT_Q5_1 = 7
MOE_K_MAX = 32
BASIS_ALL = 0
BASIS_TOP = 1


def build(force: bool = False) -> str:
    """Compile liboracle.so with its Makefile (gcc)."""
    if force and os.path.exists(LIB_PATH):
        os.remove(LIB_PATH)
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


class QAct(C.Structure):
    _fields_ = [("m", C.c_int), ("k", C.c_int), ("kb", C.c_int), ("q", C.c_void_p),
                ("scale", C.c_void_p), ("sum", C.c_void_p), ("pair", C.c_int)]


class Policy(C.Structure):
    _fields_ = [("min", C.c_uint32), ("max", C.c_uint32), ("mass", C.c_float), ("basis", C.c_uint32)]


class MoeW(C.Structure):
    _fields_ = [("H", C.c_int), ("E", C.c_int), ("F", C.c_int), ("router", C.c_void_p),
                ("router_bias", C.c_void_p), ("shexp_gate", C.c_void_p), ("gate_bits", C.c_int),
                ("down_bits", C.c_int), ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
                ("sh_gate_bits", C.c_int), ("sh_down_bits", C.c_int), ("sh_gate", C.c_void_p),
                ("sh_up", C.c_void_p), ("sh_down", C.c_void_p), ("tiles", C.c_int), ("packed", C.c_int)]


class Stats(C.Structure):
    _fields_ = [("rows", C.c_uint64), ("experts", C.c_uint64)]


def _declare(L):
    vp, i, f, u64, u32, sz = C.c_void_p, C.c_int, C.c_float, C.c_uint64, C.c_uint32, C.c_size_t
    L.orc_f16_to_f32.argtypes = [C.c_uint16]
    L.orc_f16_to_f32.restype = f
    L.orc_f32_to_f16.argtypes = [f]
    L.orc_f32_to_f16.restype = C.c_uint16
    L.orc_selftest_f16.argtypes = [u32]
    L.orc_selftest_f16.restype = u64
    L.orc_have_f16c.restype = i
    L.orc_tq_block_bytes.argtypes = [i, i]
    L.orc_tq_block_bytes.restype = sz
    L.orc_tq_matrix_bytes.argtypes = [i, i, i, i]
    L.orc_tq_matrix_bytes.restype = sz
    L.orc_pack_tq.argtypes = [i, i, i, i, vp, vp, vp, vp]
    L.orc_dequant_tq.argtypes = [vp, i, i, i, i, vp]
    L.orc_q4k_rows.argtypes = [vp, i, i, vp, vp, vp]
    L.orc_q6k_rows.argtypes = [vp, i, i, vp, vp, vp]
    L.orc_gguf_to_tq.argtypes = [i, vp, i, i, i, vp]
    L.orc_gguf_to_tq.restype = i
    L.orc_gguf_row_bytes.argtypes = [i, i]
    L.orc_gguf_row_bytes.restype = sz
    L.orc_gguf_dequant.argtypes = [i, vp, i, i, vp]
    L.orc_quant_block.argtypes = [vp, i, vp, vp, vp]
    L.orc_quant_rows.argtypes = [vp, i, i, i, vp, vp, vp]
    L.orc_quant_pair.argtypes = [vp, i, i, vp, vp, vp]
    L.orc_gemv_tq_rows.argtypes = [vp, i, i, i, i, i, C.POINTER(QAct), vp, sz, vp, i]
    L.orc_gemm_tq_rows.argtypes = [vp, i, i, i, i, i, C.POINTER(QAct), vp, sz, vp, i]
    L.orc_hc_mix.argtypes = [vp, i, i, i, i, vp, vp, i, i, i, vp]
    L.orc_dot.argtypes = [vp, vp, i]
    L.orc_dot.restype = f
    L.orc_gemm_f32_nt.argtypes = [vp, i, i, vp, i, i, i, vp, i]
    L.orc_sumsq.argtypes = [vp, i]
    L.orc_sumsq.restype = f
    L.orc_rmsnorm.argtypes = [vp, vp, f, vp, i]
    for n in ("orc_exp512", "orc_sigmoid512", "orc_silu512", "orc_sigmoid"):
        getattr(L, n).argtypes = [f]
        getattr(L, n).restype = f
    L.orc_swiglu.argtypes = [vp, vp, vp, i]
    L.orc_add_inplace.argtypes = [vp, vp, i]
    L.orc_policy_validate.argtypes = [C.POINTER(Policy), i, C.c_char_p, i]
    L.orc_policy_validate.restype = i
    L.orc_route_topk.argtypes = [vp, i, i, vp, vp]
    L.orc_route_mass.argtypes = [vp, i, C.POINTER(Policy), vp, vp]
    L.orc_route_mass.restype = i
    L.orc_mass_profile.argtypes = [vp, i, vp]
    L.orc_moe_block.argtypes = [C.POINTER(MoeW), vp, vp, i, C.POINTER(Policy), i, vp, vp, vp, vp, C.POINTER(Stats)]
    L.orc_moe_logits.argtypes = [C.POINTER(MoeW), vp, i, i, vp]
    L.orc_fold_ids.argtypes = [vp, i, C.c_uint32]
    L.orc_moe_block.restype = i
    L.orc_moe_batch.argtypes = [C.POINTER(MoeW), vp, vp, i, i, C.POINTER(Policy), i, vp, vp, vp, vp, vp,
                                vp, vp, vp, vp, vp, vp, vp, C.POINTER(Stats)]
    L.orc_moe_batch.restype = i
    L.orc_rng_u64.argtypes = [u64, u64, u64]
    L.orc_rng_u64.restype = u64
    L.orc_gen_gguf.argtypes = [i, u64, u64, i, i, f, f, vp]
    L.orc_gen_normal.argtypes = [u64, u64, sz, C.c_double, vp]
    L.orc_gen_uniform.argtypes = [u64, u64, sz, f, f, vp]


# ---- numpy conveniences ------------------------------------------------------------------

def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(float(x))


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(int(h))


def tq_matrix_bytes(rows, k, bits, kb):
    return lib().orc_tq_matrix_bytes(rows, k, bits, kb)


def pack_tq(q, d, m, bits, kb):
    rows, k = q.shape
    q = np.ascontiguousarray(q, np.uint8)
    d = np.ascontiguousarray(d).view(np.uint16)
    m = np.ascontiguousarray(m).view(np.uint16)
    out = np.zeros(tq_matrix_bytes(rows, k, bits, kb), np.uint8)
    lib().orc_pack_tq(rows, k, bits, kb, _p(q), _p(d), _p(m), _p(out))
    return out


def dequant_tq(buf, rows, k, bits, kb):
    out = np.zeros((rows, k), np.float32)
    lib().orc_dequant_tq(_p(np.ascontiguousarray(buf, np.uint8)), rows, k, bits, kb, _p(out))
    return out


def q4k_rows(raw, rows, K):
    raw = np.ascontiguousarray(raw, np.uint8)
    q = np.zeros((rows, K), np.uint8)
    dd = np.zeros((rows, K // 32), np.uint16)
    mm = np.zeros((rows, K // 32), np.uint16)
    lib().orc_q4k_rows(_p(raw), rows, K, _p(q), _p(dd), _p(mm))
    return q, dd, mm


def q6k_rows(raw, rows, K):
    raw = np.ascontiguousarray(raw, np.uint8)
    q = np.zeros((rows, K), np.uint8)
    dd = np.zeros((rows, K // 16), np.uint16)
    mm = np.zeros((rows, K // 16), np.uint16)
    lib().orc_q6k_rows(_p(raw), rows, K, _p(q), _p(dd), _p(mm))
    return q, dd, mm


def q80_rows(raw, rows, K):
    """blocks.py:71-78 q8_0_rows: (q = int8 + 128, d, m = f16(-128 d)) per 32."""
    raw = np.ascontiguousarray(raw, np.uint8)
    q = np.zeros((rows, K), np.uint8)
    d = np.zeros((rows, K // 32), np.uint16)
    m = np.zeros((rows, K // 32), np.uint16)
    lib().orc_q80_rows(_p(raw), rows, K, _p(q), _p(d), _p(m))
    return q, d, m


def q51_rows(raw, rows, K):
    """blocks.py:57-68 q5_1_rows: (5-bit q, d, m as stored) per 32."""
    raw = np.ascontiguousarray(raw, np.uint8)
    q = np.zeros((rows, K), np.uint8)
    d = np.zeros((rows, K // 32), np.uint16)
    m = np.zeros((rows, K // 32), np.uint16)
    lib().orc_q51_rows(_p(raw), rows, K, _p(q), _p(d), _p(m))
    return q, d, m


def gguf_row_bytes(fmt, K):
    return lib().orc_gguf_row_bytes(fmt, K)


def gguf_to_tq(fmt, raw, rows, K, kb):
    bits = {FMT_Q6_K: 8, FMT_Q8_0: 8, FMT_Q5_1: 5}.get(fmt, 4)
    out = np.zeros(tq_matrix_bytes(rows, K, bits, kb), np.uint8)
    got = lib().orc_gguf_to_tq(fmt, _p(np.ascontiguousarray(raw, np.uint8)), rows, K, kb, _p(out))
    if got != bits:
        raise ValueError(f"unsupported conversion fmt={fmt} kb={kb}")
    return out, bits


def gguf_dequant(fmt, raw, rows, K):
    out = np.zeros((rows, K), np.float32)
    lib().orc_gguf_dequant(fmt, _p(np.ascontiguousarray(raw, np.uint8)), rows, K, _p(out))
    return out


def quant_block(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.size, np.int8)
    s = C.c_float()
    su = C.c_int32()
    lib().orc_quant_block(_p(x), x.size, _p(q), C.byref(s), C.byref(su))
    return q, s.value, su.value


def quant_rows(x, kb):
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    q = np.zeros((m, k), np.int8)
    s = np.zeros((m, k // kb), np.float32)
    su = np.zeros((m, k // kb), np.int32)
    lib().orc_quant_rows(_p(x), m, k, kb, _p(q), _p(s), _p(su))
    return q, s, su


def quant_pair(x, kb):
    x = np.ascontiguousarray(x, np.float32)
    k = x.size
    q = np.zeros((2, k), np.int8)
    s = np.zeros((2, k // kb), np.float32)
    su = np.zeros((2, k // kb), np.int32)
    lib().orc_quant_pair(_p(x), k, kb, _p(q), _p(s), _p(su))
    return q, s, su


def gemv_tq(w, k, bits, kb, rows_out, q, s, su, pair=False, y=None, rows=None, accumulate=False, gemm=True,
            s0=0, s1=None, ldy=None):
    """y[mi][r] (+)= W x_mi over strips [s0, s1) (default: all rows_out // 16) of a packed TQ
    matrix w (the whole matrix: the strip-s0 pointer is taken here, as the reference's callers
    do); q/s/su as returned by quant_rows/quant_pair."""
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(s, np.float32)
    su = np.ascontiguousarray(su, np.int32)
    m = q.shape[0]
    logical = m // 2 if pair else m
    s1 = rows_out // 16 if s1 is None else s1
    ldy = rows_out if ldy is None else ldy
    if y is None:
        y = np.zeros((logical if rows is None else int(np.max(rows)) + 1, ldy), np.float32)
    qa = QAct(m, k, kb, _p(q), _p(s), _p(su), int(pair))
    rp = _p(np.ascontiguousarray(rows, np.uint32)) if rows is not None else None
    w = np.ascontiguousarray(w, np.uint8)
    off = s0 * (k // kb) * lib().orc_tq_block_bytes(bits, kb)
    fn = lib().orc_gemm_tq_rows if gemm else lib().orc_gemv_tq_rows
    fn(C.c_void_p(w.ctypes.data + off), k, bits, kb, s0, s1, C.byref(qa), _p(y), ldy, rp, int(accumulate))
    return y


def hc_mix(up, bits, hc, lr, xn, lo, decode, hiprec=True):
    """Hyper-connection mix part B (exec.rs:1196-1234 when decode, exec_batch.rs:929-968
    otherwise): mixed [m][hh] from xn [m][hc][hh], lo [m][lr] and the TQ up matrix [hc*hh][lr]."""
    xn = np.ascontiguousarray(xn, np.float32)
    lo = np.ascontiguousarray(lo, np.float32)
    m, hh = lo.shape[0], xn.shape[-1]
    out = np.zeros((m, hh), np.float32)
    lib().orc_hc_mix(_p(np.ascontiguousarray(up, np.uint8)), bits, hc, hh, lr, _p(xn), _p(lo), m, int(decode),
                     int(hiprec), _p(out))
    return out


def dot(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().orc_dot(_p(a), _p(b), a.size)


def gemm_f32_nt(x, w):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    mr, k = x.shape
    n = w.shape[0]
    y = np.zeros((mr, n), np.float32)
    lib().orc_gemm_f32_nt(_p(x), k, mr, _p(w), k, n, k, _p(y), n)
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros_like(x)
    lib().orc_rmsnorm(_p(x), _p(np.ascontiguousarray(w, np.float32)) if w is not None else None, eps, _p(y),
                      x.size)
    return y


def swiglu(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    y = np.zeros_like(g)
    lib().orc_swiglu(_p(g), _p(u), _p(y), g.size)
    return y


def route_topk(logits, k):
    lg = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(MOE_K_MAX, np.uint32)
    w = np.zeros(MOE_K_MAX, np.float32)
    lib().orc_route_topk(_p(lg), lg.size, k, _p(ids), _p(w))
    return ids[:k].copy(), w[:k].copy()


def fold_ids(ids, packed):
    """fold_ids (exec_batch.rs:214-225) on a copy of ids."""
    out = np.ascontiguousarray(ids, np.uint32).copy()
    if lib().orc_fold_ids(_p(out), out.size, packed) != 0:
        raise ValueError("more routed experts than packed experts")
    return out


def route_mass(logits, mn, mx, mass, basis=BASIS_TOP):
    lg = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(MOE_K_MAX, np.uint32)
    w = np.zeros(MOE_K_MAX, np.float32)
    pol = Policy(mn, mx, mass, basis)
    n = lib().orc_route_mass(_p(lg), lg.size, C.byref(pol), _p(ids), _p(w))
    return ids[:n].copy(), w[:n].copy()


def policy_validate(mn, mx, mass, n_expert, basis=BASIS_TOP):
    buf = C.create_string_buffer(256)
    pol = Policy(mn, mx, mass, basis)
    rc = lib().orc_policy_validate(C.byref(pol), n_expert, buf, 256)
    return rc, buf.value.decode()


def mass_profile(logits):
    lg = np.ascontiguousarray(logits, np.float32)
    cum = np.zeros(MOE_K_MAX, np.float32)
    lib().orc_mass_profile(_p(lg), lg.size, _p(cum))
    return cum


def rng_u64(seed, stream, idx):
    return lib().orc_rng_u64(seed, stream, idx)


def gen_gguf(fmt, seed, stream, rows, K, dlo=1e-4, dhi=2e-3):
    out = np.zeros(rows * gguf_row_bytes(fmt, K), np.uint8)
    lib().orc_gen_gguf(fmt, seed, stream, rows, K, dlo, dhi, _p(out))
    return out


def gen_normal(seed, stream, n, sigma=1.0):
    out = np.zeros(n, np.float32)
    lib().orc_gen_normal(seed, stream, n, sigma, _p(out))
    return out


def gen_uniform(seed, stream, n, lo, hi):
    out = np.zeros(n, np.float32)
    lib().orc_gen_uniform(seed, stream, n, lo, hi, _p(out))
    return out


# ---- the MoE layer ------------------------------------------------------------------------

class OracleLayer:
    """One MoE layer's weights in the reference's TQ format, converted lazily per expert from
    the raw GGUF bytes (the reference packs offline: python/trpack/blocks.py + codec.py)."""

    def __init__(self, H, E, F, router, shexp_gate, gate_raw, up_raw, down_raw, sh_gate_raw, sh_up_raw,
                 sh_down_raw, gate_fmt=FMT_Q4_K, down_fmt=FMT_Q4_K, router_bias=None):
        self.H, self.E, self.F = H, E, F
        self.router = np.ascontiguousarray(router, np.float32)
        self.router_bias = None if router_bias is None else np.ascontiguousarray(router_bias, np.float32)
        self.shexp_gate = np.ascontiguousarray(shexp_gate, np.float32)
        self.gate_fmt, self.down_fmt = gate_fmt, down_fmt
        self.gate_raw, self.up_raw, self.down_raw = gate_raw, up_raw, down_raw  # callables e -> bytes or arrays [E]
        self._tq = {}
        self.sh_gate, self.gate_bits = gguf_to_tq(gate_fmt, sh_gate_raw, F, H, 32)
        self.sh_up, _ = gguf_to_tq(gate_fmt, sh_up_raw, F, H, 32)
        self.sh_down, self.sh_down_bits = gguf_to_tq(down_fmt, sh_down_raw, H, F, 16)
        self.down_bits = {FMT_Q6_K: 8, FMT_Q8_0: 8, FMT_Q5_1: 5}.get(down_fmt, 4)
        self._gate_ptrs = (C.c_void_p * E)()
        self._up_ptrs = (C.c_void_p * E)()
        self._down_ptrs = (C.c_void_p * E)()

    def _raw(self, src, e):
        return src(e) if callable(src) else src[e]

    def ensure(self, experts):
        for e in sorted(set(int(v) for v in experts)):
            if e in self._tq:
                continue
            g, _ = gguf_to_tq(self.gate_fmt, self._raw(self.gate_raw, e), self.F, self.H, 32)
            u, _ = gguf_to_tq(self.gate_fmt, self._raw(self.up_raw, e), self.F, self.H, 32)
            d, _ = gguf_to_tq(self.down_fmt, self._raw(self.down_raw, e), self.H, self.F, 16)
            self._tq[e] = (g, u, d)
            self._gate_ptrs[e] = g.ctypes.data
            self._up_ptrs[e] = u.ctypes.data
            self._down_ptrs[e] = d.ctypes.data

    tiles = 1   # the reference's T tiles (plan.py:106-118): see TQOracleLayer
    packed = 0  # n_expert_packed of a subset pack (fold_ids); 0: all E experts packed

    def _w(self):
        return MoeW(self.H, self.E, self.F, self.router.ctypes.data,
                    None if self.router_bias is None else self.router_bias.ctypes.data,
                    self.shexp_gate.ctypes.data, self.gate_bits, self.down_bits,
                    C.cast(self._gate_ptrs, C.c_void_p), C.cast(self._up_ptrs, C.c_void_p),
                    C.cast(self._down_ptrs, C.c_void_p), self.gate_bits, self.sh_down_bits,
                    self.sh_gate.ctypes.data, self.sh_up.ctypes.data, self.sh_down.ctypes.data, self.tiles,
                    self.packed)

    def logits(self, x, dot_rows=True):
        """Router logits as the decode path (dot) or batch gemm path computes them (tiles: the
        tiles' partials in tile order)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.H)
        lg = np.zeros((x.shape[0], self.E), np.float32)
        W = self._w()
        lib().orc_moe_logits(C.byref(W), _p(x), x.shape[0], int(bool(dot_rows)), _p(lg))
        return lg

    def _routed(self, lg, k, policy):
        """The experts a row's routing uses (folded onto the packed experts of a subset pack)."""
        ids, _ = (route_mass(lg, *policy) if policy else route_topk(lg, k))
        if self.packed and self.packed < self.E:
            ids = fold_ids(ids, self.packed)
        return ids

    def moe_block(self, x, k=10, policy=None, hiprec=True, rlog=None):
        x = np.ascontiguousarray(x, np.float32)
        if rlog is None:
            rlog = self.logits(x, True)[0]
        rlog = np.ascontiguousarray(rlog, np.float32)
        self.ensure(self._routed(rlog, k, policy))
        out = np.zeros(self.H, np.float32)
        ids_o = np.zeros(MOE_K_MAX, np.uint32)
        w_o = np.zeros(MOE_K_MAX, np.float32)
        st = Stats()
        pol = Policy(*policy) if policy else None
        W = self._w()
        n = lib().orc_moe_block(C.byref(W), _p(x), _p(rlog), k, C.byref(pol) if pol else None, int(hiprec),
                                _p(out), None, _p(ids_o), _p(w_o), C.byref(st))
        if n < 0:
            raise RuntimeError("oracle moe_block failed")
        return dict(out=out, ids=ids_o[:n].copy(), w=w_o[:n].copy(), k=n, rlog=rlog, stats=(st.rows, st.experts))

    def moe_batch(self, x, k=10, policy=None, router_dot_max_m=16, rlog=None):
        x = np.ascontiguousarray(x, np.float32)
        M = x.shape[0]
        if rlog is None:
            rlog = self.logits(x, M < router_dot_max_m)
        rlog = np.ascontiguousarray(rlog, np.float32)
        ids = np.zeros((M, MOE_K_MAX), np.uint32)
        w = np.zeros((M, MOE_K_MAX), np.float32)
        for mi in range(M):
            self.ensure(self._routed(rlog[mi], k, policy))
        E = self.E
        out = np.zeros((M, self.H), np.float32)
        n_sel = np.zeros(M, np.uint32)
        cap = M * MOE_K_MAX
        ent_tok = np.zeros(cap, np.uint32)
        ent_w = np.zeros(cap, np.float32)
        ent_expert = np.zeros(cap, np.uint32)
        grp_start = np.zeros(E + 1, np.uint32)
        grp_expert = np.zeros(E + 1, np.uint32)
        grp_order = np.zeros(E + 1, np.uint32)
        n_groups = np.zeros(2, np.uint32)
        st = Stats()
        pol = Policy(*policy) if policy else None
        W = self._w()
        n_ent = lib().orc_moe_batch(C.byref(W), _p(x), _p(rlog), M, k, C.byref(pol) if pol else None,
                                    router_dot_max_m, _p(out), None, _p(ids), _p(w), _p(n_sel), _p(ent_tok),
                                    _p(ent_w), _p(ent_expert), _p(grp_start), _p(grp_expert), _p(grp_order),
                                    _p(n_groups), C.byref(st))
        if n_ent < 0:
            raise RuntimeError("oracle moe_batch failed")
        ng = int(n_groups[0])
        return dict(out=out, ids=ids, w=w, n_sel=n_sel, ent_tok=ent_tok[:n_ent].copy(), ent_w=ent_w[:n_ent].copy(),
                    ent_expert=ent_expert[:n_ent].copy(), grp_start=grp_start[:ng + 1].copy(),
                    grp_expert=grp_expert[:ng].copy(), grp_order=grp_order[:ng].copy(), n_ent=n_ent, n_groups=ng,
                    rlog=rlog, stats=(st.rows, st.experts))


# ---- the timed CPU baseline (libcpumoe.so: AVX-512 VNNI, threaded) ----------------------------

CPU_LIB_PATH = os.path.join(HERE, "libcpumoe.so")
_cpu = None


def cpu_lib() -> C.CDLL:
    """libcpumoe.so (cpu_moe.c): the reference's CPU MoE path on AVX-512 VNNI over a pinned pool."""
    global _cpu
    if _cpu is None:
        if not os.path.exists(CPU_LIB_PATH):
            build()
        L = C.CDLL(CPU_LIB_PATH)
        vp = C.c_void_p
        L.cpu_have_vnni.restype = C.c_int
        L.cpu_amx_available.restype = C.c_int
        L.cpu_pool_create.restype = vp
        L.cpu_pool_create.argtypes = [C.c_int]
        L.cpu_pool_destroy.argtypes = [vp]
        L.cpu_pool_size.argtypes = [vp]
        L.cpu_pool_cpu.argtypes = [vp, C.c_int]
        L.cpu_moe_block.argtypes = [vp, C.POINTER(MoeW), vp, C.c_int, C.POINTER(Policy), C.c_int, vp, vp, vp]
        L.cpu_moe_batch.argtypes = [vp, C.POINTER(MoeW), vp, C.c_int, C.c_int, C.POINTER(Policy), C.c_int, vp]
        _cpu = L
    return _cpu


def cpu_have_vnni() -> bool:
    return bool(cpu_lib().cpu_have_vnni())


class TQOracleLayer(OracleLayer):
    """A layer whose experts are already the reference's packed TQ strips (what trpack writes):
    gate / up [E] arrays of a kb-32 codec, down [E] of a kb-16 codec, used as they are."""

    def __init__(self, H, E, F, router, shexp_gate, gate_tq, up_tq, down_tq, sh_gate, sh_up, sh_down, gate_bits,
                 down_bits, router_bias=None, tiles=1, packed=0):
        """tiles = T > 1: a pack written for T tiles (plan.py:106-118,174-181).  router is then
        [T][E][H/T] (tile t: columns [H/T t, H/T (t+1))); each expert's gate / up array holds its T
        tiles' [F/T][H] matrices back to back and its down array the T tiles' [H][F/T] matrices;
        the shared expert's likewise.  packed: n_expert_packed of a subset pack (fold_ids)."""
        self.H, self.E, self.F = H, E, F
        self.tiles, self.packed = tiles, packed
        self.router = np.ascontiguousarray(router, np.float32)
        self.router_bias = None if router_bias is None else np.ascontiguousarray(router_bias, np.float32)
        self.shexp_gate = np.ascontiguousarray(shexp_gate, np.float32)
        self.gate_fmt = self.down_fmt = None
        self.gate_bits, self.down_bits, self.sh_down_bits = gate_bits, down_bits, down_bits
        self.sh_gate, self.sh_up, self.sh_down = (np.ascontiguousarray(a, np.uint8) for a in (sh_gate, sh_up, sh_down))
        self._gate_ptrs = (C.c_void_p * E)()
        self._up_ptrs = (C.c_void_p * E)()
        self._down_ptrs = (C.c_void_p * E)()
        self._tq = {}
        for e in range(min(E, len(gate_tq))):  # a subset pack holds only its first experts
            g, u, d = (np.ascontiguousarray(a[e], np.uint8) for a in (gate_tq, up_tq, down_tq))
            self._tq[e] = (g, u, d)
            self._gate_ptrs[e] = g.ctypes.data
            self._up_ptrs[e] = u.ctypes.data
            self._down_ptrs[e] = d.ctypes.data

    def ensure(self, experts):
        pass


class CpuMoe:
    """A pool of `threads` pinned threads (0: one per allowed CPU, at most 16 = one tile) running
    the VNNI restatement of moe_block / moe_batch on an OracleLayer's TQ weights."""

    def __init__(self, threads=0):
        self.L = cpu_lib()
        if not self.L.cpu_have_vnni():
            raise RuntimeError("this host has no AVX-512 VNNI")
        self.p = self.L.cpu_pool_create(threads)
        self.threads = self.L.cpu_pool_size(self.p)
        self.cpus = [self.L.cpu_pool_cpu(self.p, i) for i in range(self.threads)]

    def close(self):
        if self.p:
            self.L.cpu_pool_destroy(self.p)
            self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def block(self, layer, x, k=10, policy=None, hiprec=True):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(layer.H, np.float32)
        ids = np.zeros(MOE_K_MAX, np.uint32)
        w = np.zeros(MOE_K_MAX, np.float32)
        pol = Policy(*policy) if policy else None
        W = layer._w()
        n = self.L.cpu_moe_block(self.p, C.byref(W), _p(x), k, C.byref(pol) if pol else None, int(hiprec), _p(out),
                                 _p(ids), _p(w))
        if n < 0:
            raise RuntimeError("cpu_moe_block failed")
        return dict(out=out, ids=ids[:n].copy(), w=w[:n].copy(), k=n)

    def batch(self, layer, x, k=10, policy=None, router_dot_max_m=16):
        x = np.ascontiguousarray(x, np.float32)
        M = x.shape[0]
        out = np.zeros((M, layer.H), np.float32)
        pol = Policy(*policy) if policy else None
        W = layer._w()
        n = self.L.cpu_moe_batch(self.p, C.byref(W), _p(x), M, k, C.byref(pol) if pol else None, router_dot_max_m,
                                 _p(out))
        if n < 0:
            raise RuntimeError("cpu_moe_batch failed")
        return dict(out=out, n_ent=n)
