"""Python host side of the trmoe C ABI (include/trmoe.h) — ctypes bindings plus a small layer
object that keeps one MoE layer's weights in HBM.

This mirrors the reference's Rust call sites (tr_model::exec::Model::moe_block /
exec_batch::moe_batch) for tests and the benchmark; device memory and streams come from torch.
There is no CPU fallback: without the built HIP library every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG_ROOT, "libtrmoe.so")
HEADER = os.path.join(os.path.dirname(PKG_ROOT), "include", "trmoe.h")

FMT_Q4_K, FMT_Q6_K, FMT_Q8_0, FMT_Q5_1 = 12, 14, 8, 7
# the reference's TQ codecs (codec.rs:1-46): bits << 8 | kb
FMT_TQ4_16, FMT_TQ4_32, FMT_TQ5_16, FMT_TQ5_32, FMT_TQ8_16, FMT_TQ8_32 = 0x410, 0x420, 0x510, 0x520, 0x810, 0x820
TQ_FMTS = (FMT_TQ4_16, FMT_TQ4_32, FMT_TQ5_16, FMT_TQ5_32, FMT_TQ8_16, FMT_TQ8_32)
BASIS_ALL, BASIS_TOP = 0, 1
K_MAX = 32
(WS_RLOG, WS_IDS, WS_W, WS_NSEL, WS_ENT_TOK, WS_ENT_W, WS_ENT_EXP, WS_GRP_START, WS_GRP_EXP, WS_NGROUPS, WS_XQ,
 WS_XS, WS_ACTQ, WS_ACTS, WS_SHLOGIT, WS_BARRIER_ERR, WS_MIXED) = range(1, 18)


class TrkError(RuntimeError):
    pass


class Mat(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("rows", C.c_uint32), ("k", C.c_uint32), ("fmt", C.c_uint32),
                ("count", C.c_uint32), ("stride", C.c_uint64), ("tile_stride", C.c_uint64)]


class HcW(C.Structure):
    """trk_hc_w: the hyper-connection up projection [hc * hidden][lr] (a kb-32 TQ codec)."""
    _fields_ = [("up", Mat), ("hc", C.c_uint32), ("lr", C.c_uint32)]


class MoeW(C.Structure):
    _fields_ = [("router", C.c_void_p), ("router_bias", C.c_void_p), ("shexp_gate", C.c_void_p),
                ("gate", Mat), ("up", Mat), ("down", Mat), ("sh_gate", Mat), ("sh_up", Mat), ("sh_down", Mat)]


class Policy(C.Structure):
    _fields_ = [("min", C.c_uint32), ("max", C.c_uint32), ("mass", C.c_float), ("basis", C.c_uint32)]


class Cfg(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("n_expert", C.c_uint32), ("n_ff", C.c_uint32),
                ("n_expert_used", C.c_uint32), ("m_max", C.c_uint32), ("k_cap", C.c_uint32),
                ("router_dot_max_m", C.c_uint32), ("hiprec", C.c_int32), ("n_tiles", C.c_uint32),
                ("n_expert_packed", C.c_uint32)]


class Stats(C.Structure):
    _fields_ = [("rows", C.c_uint64), ("experts", C.c_uint64)]


_lib = None


def lib() -> C.CDLL:
    """Load libtrmoe.so (built by `make -C tr-infer_amd` / __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TrkError(f"{LIB_PATH} is not built: run __graft_entry__.build() (make -C tr-infer_amd)")
        L = C.CDLL(LIB_PATH)
        vp, u32, u64, i, f, sz = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_float, C.c_size_t
        L.trk_last_error.restype = C.c_char_p
        L.trk_create.argtypes = [C.POINTER(Cfg), C.POINTER(vp)]
        L.trk_workspace_bytes.argtypes = [C.POINTER(Cfg), u32, C.POINTER(sz)]
        L.trk_destroy.argtypes = [vp]
        L.trk_set_moe.argtypes = [vp, C.POINTER(Policy)]
        L.trk_moe_forward.argtypes = [vp, C.POINTER(MoeW), vp, vp, u32, vp, vp]
        L.trk_moe_residual.argtypes = [vp, C.POINTER(MoeW), vp, f, vp, u32, vp]
        L.trk_moe_forward_hc.argtypes = [vp, C.POINTER(MoeW), C.POINTER(HcW), vp, vp, u32, vp, vp]
        L.trk_moe_forward_noalloc.argtypes = [C.POINTER(Cfg), C.POINTER(Policy), C.POINTER(MoeW), vp, vp, u32, vp,
                                              vp]
        L.trk_get_stats.argtypes = [vp, C.POINTER(Stats), i, vp]
        L.trk_profile_start.argtypes = [vp, i, vp]
        L.trk_profile_report.argtypes = [vp, C.POINTER(C.c_double), C.POINTER(C.c_uint64), vp]
        L.trk_router_logits.argtypes = [vp, vp, vp, vp, u32, u32, u32, i, vp, vp, vp]
        L.trk_route.argtypes = [vp, u32, u32, u32, C.POINTER(Policy), vp, vp, vp, vp]
        L.trk_quantize.argtypes = [vp, u32, u32, u32, i, vp, vp, vp, vp]
        L.trk_gemv.argtypes = [C.POINTER(Mat), u32, u32, u32, u32, vp, vp, vp, u32, i, vp, u32, vp, i, vp]
        L.trk_swiglu.argtypes = [vp, vp, vp, sz, vp]
        L.trk_rmsnorm.argtypes = [vp, vp, f, u32, u32, vp, vp]
        L.trk_add_inplace.argtypes = [vp, vp, sz, vp]
        L.trk_gen_gguf.argtypes = [u32, u64, u64, u32, u32, f, f, vp, vp]
        L.trk_gen_gguf_stack.argtypes = [u32, u64, u64, u64, u32, u32, u32, f, f, vp, u64, vp]
        L.trk_gen_normal.argtypes = [u64, u64, sz, C.c_double, vp, vp]
        L.trk_debug_read.argtypes = [vp, i, vp, sz, vp]
        L.trk_launch_kernel.argtypes = [vp, C.POINTER(MoeW), vp, vp, u32, vp, C.c_char_p, vp]
        L.trk_set_timing.argtypes = [vp, i]
        L.trk_set_fusion.argtypes = [vp, i]
        L.trk_set_stream_rows.argtypes = [vp, i]
        L.trk_set_decode_rows.argtypes = [vp, i]
        L.trk_set_tq_mfma.argtypes = [vp, i]
        L.trk_get_timing.argtypes = [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_double), C.POINTER(C.c_uint64), i]
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise TrkError(f"trmoe error {rc}: {lib().trk_last_error().decode()}")


def header_functions() -> list[str]:
    """Names of the functions include/trmoe.h declares."""
    import re
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(trk_\w+)\s*\(", txt, re.M)))


def row_bytes(fmt: int, k: int) -> int:
    return k // 256 * {FMT_Q4_K: 144, FMT_Q6_K: 210, FMT_Q8_0: 272, FMT_Q5_1: 192}[fmt]


def tq_block_bytes(fmt: int) -> int:
    """Codec::block_bytes (codec.rs:22-29)."""
    bits, kb = fmt >> 8, fmt & 0xFF
    return 64 + (16 * kb if bits == 8 else 8 * kb) + (2 * kb if bits == 5 else 0)


def matrix_bytes(fmt: int, rows: int, k: int) -> int:
    """Bytes of one [rows][k] matrix: TQ strips (rows padded to 16) or GGUF rows."""
    if fmt in TQ_FMTS:
        return (rows + 15) // 16 * (k // (fmt & 0xFF)) * tq_block_bytes(fmt)
    return rows * row_bytes(fmt, k)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class Context:
    """trk_create/trk_destroy around one layer shape (Model::load_with's workspace sizing)."""

    def __init__(self, hidden, n_expert, n_ff, k, m_max, k_cap=0, router_dot_max_m=16, hiprec=True, n_tiles=1,
                 n_expert_packed=0):
        self.cfg = Cfg(hidden, n_expert, n_ff, k, m_max, k_cap, router_dot_max_m, int(hiprec), n_tiles,
                       n_expert_packed)
        h = C.c_void_p()
        check(lib().trk_create(C.byref(self.cfg), C.byref(h)))
        self.h = h
        self.k = k

    def close(self):
        if self.h:
            lib().trk_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_moe(self, policy):
        """policy: None or (min, max, mass, basis) (Model::set_moe)."""
        if policy is None:
            check(lib().trk_set_moe(self.h, None))
        else:
            p = Policy(*policy)
            check(lib().trk_set_moe(self.h, C.byref(p)))

    def forward(self, w: "LayerWeights", x, out, rlog=None, stream=None):
        check(lib().trk_moe_forward(self.h, C.byref(w.moew), _ptr(x), _ptr(rlog), x.shape[0], _ptr(out),
                                    _stream(stream)))

    def forward_hc(self, w: "LayerWeights", up, hc, lr, xn, lo, out, stream=None):
        """trk_moe_forward_hc: out = MoE(the hyper-connection mix of xn [M][hc][H] and lo [M][lr]);
        up: a uint8 tensor holding the TQ matrix [hc * H][lr] in `up_fmt` = (bits << 8) | 32."""
        upt, fmt = up
        hw = HcW(Mat(upt.data_ptr(), hc * w.H, lr, fmt, 1, matrix_bytes(fmt, hc * w.H, lr)), hc, lr)
        check(lib().trk_moe_forward_hc(self.h, C.byref(w.moew), C.byref(hw), _ptr(xn), _ptr(lo), lo.shape[0],
                                       _ptr(out), _stream(stream)))

    def launch_kernel(self, name: str, w: "LayerWeights", x, out, rlog=None, stream=None):
        """Launch one kernel of the forward sequence (timing in isolation; see trk_launch_kernel)."""
        check(lib().trk_launch_kernel(self.h, C.byref(w.moew), _ptr(x), _ptr(rlog), x.shape[0], _ptr(out),
                                      name.encode(), _stream(stream)))

    def residual(self, w: "LayerWeights", rms_w, eps, h, stream=None):
        check(lib().trk_moe_residual(self.h, C.byref(w.moew), _ptr(rms_w), eps, _ptr(h), h.shape[0], _stream(stream)))

    def stats(self, reset=False, stream=None):
        """(rows, experts) routed since the last reset (MoeStats::snapshot); raises on TRK_E_TIMEOUT."""
        s = Stats()
        check(lib().trk_get_stats(self.h, C.byref(s), int(reset), _stream(stream)))
        return s.rows, s.experts

    def profile_start(self, on=True, stream=None):
        """MoeStats::profile_start: zero the router-mass profile and collect it on later forwards."""
        check(lib().trk_profile_start(self.h, int(on), _stream(stream)))

    def profile_report(self, stream=None):
        """MoeStats::profile_report: (mean cumulative mass of the best 1..32 experts, rows profiled)."""
        import numpy as np
        cum = np.zeros(K_MAX, np.float64)
        rows = C.c_uint64()
        check(lib().trk_profile_report(self.h, cum.ctypes.data_as(C.POINTER(C.c_double)), C.byref(rows),
                                       _stream(stream)))
        return cum, rows.value

    def set_fusion(self, on: bool):
        check(lib().trk_set_fusion(self.h, int(on)))

    def set_tq_mfma(self, on: bool):
        """TQ layers on the int8 MFMA kernels (True) or the generic grouped TQ GEMV (False)."""
        check(lib().trk_set_tq_mfma(self.h, int(bool(on))))

    def set_stream_rows(self, rows: int):
        """Batch items of at most `rows` rows on the streaming GEMV (-1 automatic, 0 none)."""
        check(lib().trk_set_stream_rows(self.h, int(rows)))

    def set_decode_rows(self, rows: int):
        """GGUF batches of 2..rows tokens as per-token decode units (0 never, default 8)."""
        check(lib().trk_set_decode_rows(self.h, int(rows)))

    def set_timing(self, on: bool):
        check(lib().trk_set_timing(self.h, int(on)))

    def timing(self):
        """{kernel: (total ms, launches)} since the last call (synchronises)."""
        cap = 16
        names = (C.c_char_p * cap)()
        ms = (C.c_double * cap)()
        cnt = (C.c_uint64 * cap)()
        n = lib().trk_get_timing(self.h, names, ms, cnt, cap)
        if n < 0:
            check(n)
        return {names[i].decode(): (ms[i], int(cnt[i])) for i in range(min(n, cap))}

    def read(self, which, nbytes, dtype, stream=None):
        import numpy as np
        buf = np.zeros(nbytes, np.uint8)
        check(lib().trk_debug_read(self.h, which, buf.ctypes.data_as(C.c_void_p), nbytes, _stream(stream)))
        return buf.view(dtype)


class LayerWeights:
    """One layer's weights resident on the GPU: expert stacks [E][rows*row_bytes] as uint8 tensors."""

    def __init__(self, H, E, F, router, shexp_gate, gate, up, down, sh_gate, sh_up, sh_down, gate_fmt=FMT_Q4_K,
                 down_fmt=FMT_Q4_K, router_bias=None):
        self.H, self.E, self.F = H, E, F
        self.tensors = dict(router=router, shexp_gate=shexp_gate, gate=gate, up=up, down=down, sh_gate=sh_gate,
                            sh_up=sh_up, sh_down=sh_down, router_bias=router_bias)
        gm, dmb = matrix_bytes(gate_fmt, F, H), matrix_bytes(down_fmt, H, F)

        def mat(t, rows, k, fmt, count, mb):
            return Mat(t.data_ptr(), rows, k, fmt, count, mb, 0)

        self.moew = MoeW(router.data_ptr() if router is not None else None,
                         router_bias.data_ptr() if router_bias is not None else None, shexp_gate.data_ptr(),
                         mat(gate, F, H, gate_fmt, E, gm), mat(up, F, H, gate_fmt, E, gm), mat(down, H, F, down_fmt, E, dmb),
                         mat(sh_gate, F, H, gate_fmt, 1, gm), mat(sh_up, F, H, gate_fmt, 1, gm),
                         mat(sh_down, H, F, down_fmt, 1, dmb))
        self.bytes_per_expert = 2 * gm + dmb

    @classmethod
    def from_host(cls, layer, device="cuda"):
        """Upload a host-side layer (raw GGUF bytes; see tests/layerdata.py)."""
        import numpy as np
        import torch

        def dev(a, dtype=None):
            return torch.from_numpy(np.ascontiguousarray(a)).to(device)

        return cls(layer.H, layer.E, layer.F, dev(layer.router), dev(layer.shexp_gate), dev(layer.stacked("gate")),
                   dev(layer.stacked("up")), dev(layer.stacked("down")), dev(layer.sh_gate), dev(layer.sh_up),
                   dev(layer.sh_down), layer.gate_fmt, layer.down_fmt,
                   None if layer.bias is None else dev(layer.bias))

    @classmethod
    def from_tq(cls, H, E, F, router, shexp_gate, gate, up, down, sh_gate, sh_up, sh_down, gate_fmt, down_fmt,
                router_bias=None, device="cuda"):
        """Upload a layer whose experts are the reference's packed TQ strips (host arrays: gate /
        up / down as [E][matrix bytes], the shared expert's as one matrix each), unchanged."""
        import numpy as np
        import torch

        def dev(a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(device)

        return cls(H, E, F, dev(router), dev(shexp_gate), dev(gate), dev(up), dev(down), dev(sh_gate), dev(sh_up),
                   dev(sh_down), gate_fmt, down_fmt, None if router_bias is None else dev(router_bias))

    @classmethod
    def generate(cls, seed, layer, H, E, F, down_fmt=FMT_Q4_K, router_bias=None, device="cuda", stream=None):
        """Synthesise a layer on the GPU with the same generator the test oracle uses."""
        import torch
        gb, db = row_bytes(FMT_Q4_K, H), row_bytes(down_fmt, F)
        L = lib()
        st = _stream(stream)

        def sid(t):
            return (layer << 32) | t

        router = torch.empty(E * H, dtype=torch.float32, device=device)
        check(L.trk_gen_normal(seed, sid(1), E * H, 0.02, _ptr(router), st))
        shg = torch.empty(H, dtype=torch.float32, device=device)
        check(L.trk_gen_normal(seed, sid(2), H, 0.02, _ptr(shg), st))
        gate = torch.empty((E, F * gb), dtype=torch.uint8, device=device)
        up = torch.empty((E, F * gb), dtype=torch.uint8, device=device)
        down = torch.empty((E, H * db), dtype=torch.uint8, device=device)
        # expert e: gate / up / down from streams 16 + 3e, 17 + 3e, 18 + 3e of this layer
        for t, fmt, rows, k, buf in ((gate, FMT_Q4_K, F, H, 16), (up, FMT_Q4_K, F, H, 17), (down, down_fmt, H, F, 18)):
            check(L.trk_gen_gguf_stack(fmt, seed, sid(buf), 3, E, rows, k, 1e-4, 2e-3, _ptr(t), t.stride(0), st))
        sh_gate = torch.empty(F * gb, dtype=torch.uint8, device=device)
        sh_up = torch.empty(F * gb, dtype=torch.uint8, device=device)
        sh_down = torch.empty(H * db, dtype=torch.uint8, device=device)
        check(L.trk_gen_gguf(FMT_Q4_K, seed, sid(8), F, H, 1e-4, 2e-3, _ptr(sh_gate), st))
        check(L.trk_gen_gguf(FMT_Q4_K, seed, sid(9), F, H, 1e-4, 2e-3, _ptr(sh_up), st))
        check(L.trk_gen_gguf(down_fmt, seed, sid(10), H, F, 1e-4, 2e-3, _ptr(sh_down), st))
        return cls(H, E, F, router, shg, gate, up, down, sh_gate, sh_up, sh_down, FMT_Q4_K, down_fmt, router_bias)


    @classmethod
    def from_tiled_tq(cls, H, E, F, T, router, shexp_gate, gate, up, down, sh_gate, sh_up, sh_down, gate_fmt,
                      down_fmt, router_bias=None, device="cuda"):
        """A layer as a pack written for T tiles holds it (python/trpack/plan.py:106-118,174-181),
        uploaded unchanged: router [T][E][H/T]; gate / up [T][count][tile bytes] (tile t: rows
        [F/T t, F/T (t+1)) as a [F/T][H] TQ matrix), down [T][count][tile bytes] (columns
        [F/T t, F/T (t+1)), [H][F/T]); the shared expert's as [T][tile bytes].  count < E: a
        subset pack of the first `count` experts."""
        import numpy as np
        import torch

        def dev(a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(device)

        self = cls.__new__(cls)
        self.H, self.E, self.F = H, E, F
        t = dict(router=dev(router), shexp_gate=dev(shexp_gate), gate=dev(gate), up=dev(up), down=dev(down),
                 sh_gate=dev(sh_gate), sh_up=dev(sh_up), sh_down=dev(sh_down),
                 router_bias=None if router_bias is None else dev(router_bias))
        self.tensors = t
        per = F // T

        def mat(name, rows, k, fmt):
            a = t[name]
            if a.dim() == 2:  # [T][bytes]: one matrix per tile
                return Mat(a.data_ptr(), rows, k, fmt, 1, a.shape[1], a.stride(0))
            return Mat(a.data_ptr(), rows, k, fmt, a.shape[1], a.stride(1), a.stride(0))

        self.moew = MoeW(t["router"].data_ptr(), None if router_bias is None else t["router_bias"].data_ptr(),
                         t["shexp_gate"].data_ptr(), mat("gate", per, H, gate_fmt), mat("up", per, H, gate_fmt),
                         mat("down", H, per, down_fmt), mat("sh_gate", per, H, gate_fmt),
                         mat("sh_up", per, H, gate_fmt), mat("sh_down", H, per, down_fmt))
        self.bytes_per_expert = T * (2 * matrix_bytes(gate_fmt, per, H) + matrix_bytes(down_fmt, H, per))
        return self

    @classmethod
    def generate_tq(cls, gen, H, E, F, gate_fmt=None, down_fmt=None, router_bias=None, device="cuda"):
        """A synthetic layer of packed TQ experts generated on the GPU from a torch Generator:
        router and shared-gate vector ~ N(0, 0.02), every TQ matrix as `gen_tq_stack`."""
        import torch
        gf = FMT_TQ4_32 if gate_fmt is None else gate_fmt
        df = FMT_TQ5_16 if down_fmt is None else down_fmt
        router = torch.randn((E, H), device=device, generator=gen) * 0.02
        shg = torch.randn(H, device=device, generator=gen) * 0.02
        gate, up = (gen_tq_stack(gen, E, F, H, gf, device) for _ in range(2))
        down = gen_tq_stack(gen, E, H, F, df, device)
        sg, su = (gen_tq_stack(gen, 1, F, H, gf, device)[0] for _ in range(2))
        sd = gen_tq_stack(gen, 1, H, F, df, device)[0]
        return cls(H, E, F, router, shg, gate, up, down, sg, su, sd, gf, df, router_bias)

    def with_down(self, down_fmt, seed, layer, device="cuda", stream=None):
        """The same layer with its routed and shared down projections regenerated in `down_fmt`
        (config 4: Q4_K gate/up, Q6_K down); every other tensor is shared with this one."""
        import torch
        H, E, F = self.H, self.E, self.F
        db = row_bytes(down_fmt, F)
        L = lib()
        st = _stream(stream)
        down = torch.empty((E, H * db), dtype=torch.uint8, device=device)
        check(L.trk_gen_gguf_stack(down_fmt, seed, (layer << 32) | 18, 3, E, H, F, 1e-4, 2e-3, _ptr(down),
                                   down.stride(0), st))
        sh_down = torch.empty(H * db, dtype=torch.uint8, device=device)
        check(L.trk_gen_gguf(down_fmt, seed, (layer << 32) | 10, H, F, 1e-4, 2e-3, _ptr(sh_down), st))
        t = self.tensors
        return LayerWeights(H, E, F, t["router"], t["shexp_gate"], t["gate"], t["up"], down, t["sh_gate"],
                            t["sh_up"], sh_down, FMT_Q4_K, down_fmt, t["router_bias"])


def gen_tq_stack(gen, count, rows, k, fmt, device="cuda"):
    """A stack of `count` packed TQ matrices [rows][k] on the GPU (codec.rs:1-46): uniform q bytes
    (and 5-bit planes), each block's f16 d in [5e-4, 3e-3] and m = -d * U(0, 2^(bits-1)), the sign
    pattern of converted GGUF weights.  `gen` is a torch Generator on `device`."""
    import torch
    mb = matrix_bytes(fmt, rows, k)
    bb, bits = tq_block_bytes(fmt), fmt >> 8
    t = torch.randint(0, 256, (count, mb), dtype=torch.uint8, device=device, generator=gen)
    blocks = t.view(count, mb // bb, bb)
    d = torch.empty((count, mb // bb, 16), device=device).uniform_(5e-4, 3e-3, generator=gen)
    m = -d * torch.empty_like(d).uniform_(0, float(1 << (bits - 1)), generator=gen)
    blocks[:, :, 0:32] = d.half().view(torch.uint8)
    blocks[:, :, 32:64] = m.half().view(torch.uint8)
    return t


NOALLOC_SCRATCH_BYTES = 16 << 20


def workspace_bytes(hidden, n_expert, n_ff, k, m, k_cap=0):
    """trk_workspace_bytes: the device workspace of the layer for m rows (host-side sizing)."""
    out = C.c_size_t()
    cfg = Cfg(hidden, n_expert, n_ff, k, m, k_cap, 16, 1)
    check(lib().trk_workspace_bytes(C.byref(cfg), m, C.byref(out)))
    return out.value


def noalloc_max_m(hidden, n_expert, n_ff, k, k_cap=0):
    """The largest M whose workspace fits trk_moe_forward_noalloc's static scratch (the need grows
    with M)."""
    lo, hi = 0, 1
    while workspace_bytes(hidden, n_expert, n_ff, k, hi, k_cap) <= NOALLOC_SCRATCH_BYTES:
        lo, hi = hi, 2 * hi
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if workspace_bytes(hidden, n_expert, n_ff, k, mid, k_cap) <= NOALLOC_SCRATCH_BYTES:
            lo = mid
        else:
            hi = mid
    return lo


def forward_noalloc(hidden, n_expert, n_ff, k, w: "LayerWeights", x, out, policy=None, k_cap=0, router_dot_max_m=16,
                    hiprec=True, rlog=None, stream=None):
    """trk_moe_forward_noalloc: the layer without a context, its workspace in the library's static
    device scratch (no allocation)."""
    cfg = Cfg(hidden, n_expert, n_ff, k, 0, k_cap, router_dot_max_m, int(hiprec))
    p = C.byref(Policy(*policy)) if policy is not None else None
    check(lib().trk_moe_forward_noalloc(C.byref(cfg), p, C.byref(w.moew), _ptr(x), _ptr(rlog), x.shape[0], _ptr(out),
                                        _stream(stream)))


# ---- kernel-level wrappers (torch tensors on the GPU) ----------------------------------------

def quantize(x, kb, pair=False, stream=None):
    import torch
    m, k = (1, x.numel()) if pair else x.shape
    rows = 2 if pair else m
    q = torch.empty((rows, k), dtype=torch.int8, device=x.device)
    s = torch.empty((rows, k // kb), dtype=torch.float32, device=x.device)
    su = torch.empty((rows, k // kb), dtype=torch.int32, device=x.device)
    check(lib().trk_quantize(_ptr(x), m, k, kb, int(pair), _ptr(q), _ptr(s), _ptr(su), _stream(stream)))
    return q, s, su


def router_logits(router, x, bias=None, shexp_gate=None, gemm_order=False, stream=None):
    import torch
    m, H = x.shape
    E = router.shape[0] if router is not None else 0
    rlog = torch.empty((m, max(E, 1)), dtype=torch.float32, device=x.device)
    sh = torch.empty(m, dtype=torch.float32, device=x.device)
    check(lib().trk_router_logits(_ptr(router), _ptr(bias), _ptr(shexp_gate), _ptr(x), m, E, H, int(gemm_order),
                                  _ptr(rlog), _ptr(sh), _stream(stream)))
    return rlog[:, :E], sh


def route(logits, k, policy=None, stream=None):
    import torch
    m, E = logits.shape
    ids = torch.zeros((m, K_MAX), dtype=torch.int32, device=logits.device)
    w = torch.zeros((m, K_MAX), dtype=torch.float32, device=logits.device)
    n = torch.zeros(m, dtype=torch.int32, device=logits.device)
    p = C.byref(Policy(*policy)) if policy is not None else None
    check(lib().trk_route(_ptr(logits), m, E, k, p, _ptr(ids), _ptr(w), _ptr(n), _stream(stream)))
    return ids, w, n


def gemv(wt, rows, k, fmt, item, count, kb, q, s, su, pair=False, y=None, ldy=None, rowmap=None, accumulate=False,
         s0=0, s1=None, stream=None):
    """trk_gemv over strips [s0, s1) (all strips by default) of matrix `item` of a stack of
    `count` [rows][k] matrices in `fmt` (GGUF or TQ) held in `wt`."""
    import torch
    m = q.shape[0]
    logical = m // 2 if pair else m
    strips = (rows + 15) // 16
    s1 = strips if s1 is None else s1
    width = 16 * strips if fmt in TQ_FMTS else rows
    if y is None:
        y = torch.zeros((logical, width), dtype=torch.float32, device=q.device)
    mat = Mat(wt.data_ptr(), rows, k, fmt, count, matrix_bytes(fmt, rows, k))
    check(lib().trk_gemv(C.byref(mat), item, s0, s1, kb, _ptr(q), _ptr(s), _ptr(su), m, int(pair), _ptr(y),
                         ldy if ldy is not None else width, _ptr(rowmap), int(accumulate), _stream(stream)))
    return y


def swiglu(g, u, stream=None):
    import torch
    y = torch.empty_like(g)
    check(lib().trk_swiglu(_ptr(g), _ptr(u), _ptr(y), g.numel(), _stream(stream)))
    return y


def rmsnorm(x, w, eps, stream=None):
    import torch
    y = torch.empty_like(x)
    m, n = x.shape
    check(lib().trk_rmsnorm(_ptr(x), _ptr(w), eps, m, n, _ptr(y), _stream(stream)))
    return y


def gen_gguf(fmt, seed, stream_id, rows, k, dlo=1e-4, dhi=2e-3, device="cuda", stream=None):
    import torch
    out = torch.empty(rows * row_bytes(fmt, k), dtype=torch.uint8, device=device)
    check(lib().trk_gen_gguf(fmt, seed, stream_id, rows, k, dlo, dhi, _ptr(out), _stream(stream)))
    return out


def gen_normal(seed, stream_id, n, sigma=1.0, device="cuda", stream=None):
    import torch
    out = torch.empty(n, dtype=torch.float32, device=device)
    check(lib().trk_gen_normal(seed, stream_id, n, sigma, _ptr(out), _stream(stream)))
    return out


# ---- synthetic workloads ------------------------------------------------------------------------

_M64 = (1 << 64) - 1


def _mix64(z: int) -> int:
    z = (z + 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def rng_u64(seed: int, stream_id: int, idx: int) -> int:
    """The counter-based draw that trk_gen_gguf / trk_gen_normal use: one u64 per (seed, stream, idx)."""
    key = _mix64((seed ^ _mix64(stream_id)) & _M64)
    return _mix64((key + idx * 0xD1B54A32D192ED03) & _M64)


# Config 3's Zipf(1.1) load as a router bias.  Top-k over logits + log p (with the router's
# N(0, 0.905^2) logits) concentrates the load far beyond Zipf: only ~99 experts are touched at
# M = 512.  The load the config describes is drawing k distinct experts per token from p
# (Plackett-Luce; at M = 512, k = 10: ~460 experts touched, ~50 empty, largest group ~465, median
# 3).  zipf_bias_table.json holds the per-rank bias fitted to reproduce every rank's inclusion
# probability (make_zipf_table.py); ZIPF_BIAS_SCALE * log p is the fallback for other (E, s),
# which matches the touched and empty counts but not the largest group (~290).
ZIPF_BIAS_SCALE = 0.40
ZIPF_TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "zipf_bias_table.json")


def zipf_rank_bias(E: int, s: float = 1.1):
    """The fitted per-rank bias of zipf_bias_table.json (make_zipf_table.py) when it was fitted for
    this E and s, else None."""
    import json
    import numpy as np
    try:
        with open(ZIPF_TABLE) as f:
            t = json.load(f)
    except OSError:
        return None
    if t["E"] != E or abs(t["s"] - s) > 1e-12:
        return None
    return np.array(t["bias"], np.float64)


def zipf_bias(seed: int, E: int, s: float = 1.1, scale: float = None, stream_id: int = 5):
    """Router bias for config 3's Zipf(s) load, over the permutation pi that sorts
    rng_u64(seed, stream_id, e): the expert of rank j gets b_j (float32 numpy array of E).

    b_j is the fitted per-rank bias of zipf_bias_table.json when one exists for (E, s): top-10
    over the synthetic router's N(0, 0.905^2) logits plus b then includes each expert as often as
    drawing 10 distinct experts per token from Zipf(s) does (make_zipf_table.py).  Otherwise, or
    with an explicit scale, b_j = scale * log p_j with p_j ~ j^-s (scale 0.40 by default)."""
    import numpy as np
    keys = np.array([rng_u64(seed, stream_id, e) for e in range(E)], np.uint64)
    perm = np.argsort(keys, kind="stable")  # perm[j] = the expert of rank j
    rank_b = zipf_rank_bias(E, s) if scale is None else None
    if rank_b is None:
        p = 1.0 / np.arange(1, E + 1, dtype=np.float64) ** s
        p /= p.sum()
        rank_b = (ZIPF_BIAS_SCALE if scale is None else scale) * np.log(p)
    b = np.zeros(E, np.float32)
    b[perm] = rank_b.astype(np.float32)
    return b
