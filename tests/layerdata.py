"""Seeded synthetic MoE layers for the parity tests (test helper).

Every tensor is drawn from the oracle's counter-based generator, keyed by (seed, stream, index),
so the host (for the oracle) and the GPU generator (for the bench) produce the same bytes.
Stream ids: (layer << 32) | tensor id, with the tensor ids below.
"""
from __future__ import annotations

import numpy as np

import oracle as O

T_ROUTER, T_SHEXP_GATE, T_X, T_RMS_W, T_BIAS = 1, 2, 3, 4, 5
T_SH_GATE, T_SH_UP, T_SH_DOWN = 8, 9, 10


def t_gate(e):
    return 16 + 3 * e


def t_up(e):
    return 17 + 3 * e


def t_down(e):
    return 18 + 3 * e


def stream(layer, tid):
    return (layer << 32) | tid


def zipf_bias(seed, E, s=1.1, layer=0):
    """The package's Zipf router bias on this layer's bias stream."""
    import trmoe
    return trmoe.zipf_bias(seed, E, s, stream_id=stream(layer, T_BIAS))


class Layer:
    """Raw GGUF bytes for one MoE layer: experts [E][rows*row_bytes] for gate/up/down."""

    def __init__(self, seed=1, H=2048, E=512, F=512, layer=0, down_fmt=O.FMT_Q4_K, gate_fmt=O.FMT_Q4_K,
                 bias=None, lazy=False):
        self.seed, self.H, self.E, self.F, self.layer = seed, H, E, F, layer
        self.gate_fmt, self.down_fmt = gate_fmt, down_fmt
        self.router = O.gen_normal(seed, stream(layer, T_ROUTER), E * H, 0.02).reshape(E, H)
        self.shexp_gate = O.gen_normal(seed, stream(layer, T_SHEXP_GATE), H, 0.02)
        self.bias = bias
        self.sh_gate = O.gen_gguf(gate_fmt, seed, stream(layer, T_SH_GATE), F, H)
        self.sh_up = O.gen_gguf(gate_fmt, seed, stream(layer, T_SH_UP), F, H)
        self.sh_down = O.gen_gguf(down_fmt, seed, stream(layer, T_SH_DOWN), H, F)
        self._cache = {}
        if not lazy:
            for e in range(E):
                self.expert(e)

    def expert(self, e):
        if e not in self._cache:
            s = self.seed
            self._cache[e] = (O.gen_gguf(self.gate_fmt, s, stream(self.layer, t_gate(e)), self.F, self.H),
                              O.gen_gguf(self.gate_fmt, s, stream(self.layer, t_up(e)), self.F, self.H),
                              O.gen_gguf(self.down_fmt, s, stream(self.layer, t_down(e)), self.H, self.F))
        return self._cache[e]

    def gate(self, e):
        return self.expert(e)[0]

    def up(self, e):
        return self.expert(e)[1]

    def down(self, e):
        return self.expert(e)[2]

    def oracle(self):
        return O.OracleLayer(self.H, self.E, self.F, self.router, self.shexp_gate, self.gate, self.up, self.down,
                             self.sh_gate, self.sh_up, self.sh_down, gate_fmt=self.gate_fmt,
                             down_fmt=self.down_fmt, router_bias=self.bias)

    def x(self, M, tid=T_X, sigma=1.0):
        return O.gen_normal(self.seed, stream(self.layer, tid), M * self.H, sigma).reshape(M, self.H)

    def stacked(self, which):
        """[E][bytes] contiguous expert stack (what the GPU library takes)."""
        idx = {"gate": 0, "up": 1, "down": 2}[which]
        return np.stack([self.expert(e)[idx] for e in range(self.E)])


def random_tq(rng, rows, K, bits, kb):
    """One packed TQ matrix (codec.rs:1-46): uniform q, f16 d > 0 and m = -d * U(0, 2^(bits-1)),
    the sign pattern of weights converted from GGUF (d * sc >= 0, -(dmin * mn) <= 0)."""
    q = rng.integers(0, 1 << bits, (rows, K), dtype=np.uint8)
    nb = K // kb
    d = rng.uniform(5e-4, 3e-3, (rows, nb)).astype(np.float16)
    m = (-d.astype(np.float32) * rng.uniform(0, 1 << (bits - 1), (rows, nb))).astype(np.float16)
    return O.pack_tq(q, d, m, bits, kb)


class TQLayer:
    """A layer whose experts are the reference's packed TQ strips: gate / up [E][F][H] in a kb-32
    codec, down [E][H][F] in a kb-16 codec (the real packs: TQ4_32 / TQ5_16), shared expert alike."""

    def __init__(self, seed=1, H=2560, E=32, F=640, gate_bits=4, down_bits=5, bias=None):
        rng = np.random.default_rng(seed)
        self.H, self.E, self.F, self.seed = H, E, F, seed
        self.gate_bits, self.down_bits = gate_bits, down_bits
        self.gate_fmt, self.down_fmt = (gate_bits << 8) | 32, (down_bits << 8) | 16
        self.router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        self.shexp_gate = (rng.standard_normal(H) * 0.02).astype(np.float32)
        self.bias = bias
        self.gate = np.stack([random_tq(rng, F, H, gate_bits, 32) for _ in range(E)])
        self.up = np.stack([random_tq(rng, F, H, gate_bits, 32) for _ in range(E)])
        self.down = np.stack([random_tq(rng, H, F, down_bits, 16) for _ in range(E)])
        self.sh_gate = random_tq(rng, F, H, gate_bits, 32)
        self.sh_up = random_tq(rng, F, H, gate_bits, 32)
        self.sh_down = random_tq(rng, H, F, down_bits, 16)

    def oracle(self):
        return O.TQOracleLayer(self.H, self.E, self.F, self.router, self.shexp_gate, self.gate, self.up, self.down,
                               self.sh_gate, self.sh_up, self.sh_down, self.gate_bits, self.down_bits, self.bias)

    def x(self, M, tid=0, sigma=1.0):
        return O.gen_normal(self.seed, stream(0, 900 + tid), M * self.H, sigma).reshape(M, self.H)


class TiledTQLayer:
    """A layer as a pack written for T tiles stores it (python/trpack/plan.py:106-118,174-181):
    the router K-split into [T][E][H/T], every expert's gate / up split by rows into T [F/T][H]
    TQ matrices and its down split by columns into T [H][F/T] matrices, the shared expert alike.
    Tile arrays are tile-major, [T][E][bytes] (how the GPU takes them: tile t at t * tile_stride);
    the oracle takes each expert's tiles back to back.  packed: a subset pack of the first
    `packed` experts (the router still scores all E)."""

    def __init__(self, seed=1, H=2560, E=32, F=640, T=2, gate_bits=4, down_bits=5, packed=0):
        rng = np.random.default_rng(seed)
        assert F % (16 * T) == 0 and H % T == 0
        self.H, self.E, self.F, self.T, self.seed, self.packed = H, E, F, T, seed, packed
        self.gate_bits, self.down_bits = gate_bits, down_bits
        self.gate_fmt, self.down_fmt = (gate_bits << 8) | 32, (down_bits << 8) | 16
        per, hl = F // T, H // T
        Ep = packed or E
        self.router_full = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        self.router = np.ascontiguousarray(self.router_full.reshape(E, T, hl).transpose(1, 0, 2))  # [T][E][hl]
        self.shexp_gate = (rng.standard_normal(H) * 0.02).astype(np.float32)
        self.gate = np.stack([np.stack([random_tq(rng, per, H, gate_bits, 32) for _ in range(Ep)]) for _ in range(T)])
        self.up = np.stack([np.stack([random_tq(rng, per, H, gate_bits, 32) for _ in range(Ep)]) for _ in range(T)])
        self.down = np.stack([np.stack([random_tq(rng, H, per, down_bits, 16) for _ in range(Ep)]) for _ in range(T)])
        self.sh_gate = np.stack([random_tq(rng, per, H, gate_bits, 32) for _ in range(T)])
        self.sh_up = np.stack([random_tq(rng, per, H, gate_bits, 32) for _ in range(T)])
        self.sh_down = np.stack([random_tq(rng, H, per, down_bits, 16) for _ in range(T)])

    def oracle(self):
        def per_expert(a):  # [T][E][bytes] -> [E][T * bytes]
            return np.ascontiguousarray(a.transpose(1, 0, 2)).reshape(a.shape[1], -1)
        return O.TQOracleLayer(self.H, self.E, self.F, self.router, self.shexp_gate, per_expert(self.gate),
                               per_expert(self.up), per_expert(self.down), self.sh_gate.reshape(-1),
                               self.sh_up.reshape(-1), self.sh_down.reshape(-1), self.gate_bits, self.down_bits,
                               tiles=self.T, packed=self.packed)

    def x(self, M, tid=0, sigma=1.0):
        return O.gen_normal(self.seed, stream(0, 950 + tid), M * self.H, sigma).reshape(M, self.H)


def untile(L):
    """The untiled layer holding the same weights as TiledTQLayer L: gate / up tiles concatenated
    by rows (a TQ strip is a self-contained 16-row unit), each down strip's blocks concatenated
    over the tiles in column order (a TQ block is self-contained), the router rows rejoined."""
    T, E, H, F = L.T, L.packed or L.E, L.H, L.F
    per = F // T
    bb = O.tq_matrix_bytes(16, 16, L.down_bits, 16)  # one block
    sb = per // 16 * bb  # one strip of a down tile

    def down_full(tiles):  # [T][bytes of [H][per]] -> bytes of [H][F]
        strips = [t.reshape(H // 16, sb) for t in tiles]
        return np.concatenate(strips, axis=1).reshape(-1)

    gate = np.stack([np.concatenate([L.gate[t][e] for t in range(T)]) for e in range(E)])
    up = np.stack([np.concatenate([L.up[t][e] for t in range(T)]) for e in range(E)])
    down = np.stack([down_full([L.down[t][e] for t in range(T)]) for e in range(E)])
    return O.TQOracleLayer(H, L.E, F, L.router_full, L.shexp_gate, gate, up, down, L.sh_gate.reshape(-1),
                           L.sh_up.reshape(-1), down_full(list(L.sh_down)), L.gate_bits, L.down_bits,
                           packed=L.packed)
