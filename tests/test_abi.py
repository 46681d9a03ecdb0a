"""CPU-side checks of the C ABI: the library builds for gfx950, loads, and exports every entry
point include/trmoe.h declares; argument validation returns the documented status codes without
touching a GPU."""
from __future__ import annotations

import ctypes as C
import os

import pytest

import trmoe


def test_library_exports_every_declared_symbol():
    L = trmoe.lib()
    names = trmoe.header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_header_declares_the_boundary():
    names = set(trmoe.header_functions())
    for n in ("trk_create", "trk_destroy", "trk_set_moe", "trk_moe_forward", "trk_moe_residual", "trk_route",
              "trk_quantize", "trk_gemv", "trk_router_logits", "trk_last_error"):
        assert n in names


def test_invalid_arguments_are_rejected_on_the_host():
    L = trmoe.lib()
    # QAct::zeros asserts kb in {16, 32} (quant.rs:68-71): status, not a crash
    rc = L.trk_quantize(C.c_void_p(16), 1, 48, 24, 0, C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), None)
    assert rc == -1 and b"kb" in L.trk_last_error()
    # MoePolicy::validate (router.rs:32-44)
    for pol in [(0, 10, 0.9, 1), (1, 33, 0.9, 1), (1, 10, 0.0, 1), (3, 2, 0.5, 0)]:
        p = trmoe.Policy(*pol)
        rc = L.trk_route(C.c_void_p(16), 1, 512, 10, C.byref(p), C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), None)
        assert rc == -2, pol
    p = trmoe.Policy(1, 20, 0.9, 1)
    assert L.trk_route(C.c_void_p(16), 1, 16, 10, C.byref(p), C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), None) == -2
    # bad shapes for trk_create
    h = C.c_void_p()
    bad = trmoe.Cfg(2000, 512, 512, 10, 1, 0, 16, 1)
    assert L.trk_create(C.byref(bad), C.byref(h)) == -1
    bad = trmoe.Cfg(2048, 512, 512, 33, 1, 0, 16, 1)
    assert L.trk_create(C.byref(bad), C.byref(h)) == -1


def test_build_flags_keep_numerics_contract():
    mk = open(os.path.join(trmoe.PKG_ROOT, "Makefile")).read()
    for flag in ("-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt", "-packed-fp32-ops",
                 "--offload-arch=$(ARCH)"):
        assert flag in mk


def test_generator_rejects_undersized_stride():
    """trk_gen_gguf_stack sizes each matrix by its own format (Q8_0: 272 B and Q5_1: 192 B per 256
    values), so a stride one piece short is refused before anything is written."""
    L = trmoe.lib()
    rows, k = 4, 512
    for fmt in (trmoe.FMT_Q4_K, trmoe.FMT_Q6_K, trmoe.FMT_Q8_0, trmoe.FMT_Q5_1):
        need = rows * trmoe.row_bytes(fmt, k)
        rc = L.trk_gen_gguf_stack(fmt, 1, 0, 1, 2, rows, k, 1e-4, 2e-3, C.c_void_p(256), need - 16, None)
        assert rc == -1 and b"stride" in L.trk_last_error(), fmt


def test_stats_and_profile_reject_null_arguments():
    L = trmoe.lib()
    assert L.trk_get_stats(None, None, 0, None) == -1
    assert L.trk_profile_report(None, None, None, None) == -1
    assert L.trk_profile_start(None, 1, None) == -1


def test_noalloc_rejects_a_workspace_above_the_scratch():
    """trk_moe_forward_noalloc lays its workspace out on the host and refuses a call whose workspace
    does not fit the static scratch before touching a GPU."""
    L = trmoe.lib()
    cfg = trmoe.Cfg(2048, 512, 512, 10, 0, 0, 16, 1)
    rc = L.trk_moe_forward_noalloc(C.byref(cfg), None, None, C.c_void_p(256), None, 4096, C.c_void_p(256), None)
    assert rc == -3 and b"scratch" in L.trk_last_error()
    bad = trmoe.Cfg(2000, 512, 512, 10, 0, 0, 16, 1)
    assert L.trk_moe_forward_noalloc(C.byref(bad), None, None, C.c_void_p(256), None, 1, C.c_void_p(256), None) == -1
    # the boundary at BASELINE's shape: trk_workspace_bytes is the layout noalloc checks
    m_max = trmoe.noalloc_max_m(2048, 512, 512, 10)
    assert m_max == 100
    assert trmoe.workspace_bytes(2048, 512, 512, 10, m_max) <= trmoe.NOALLOC_SCRATCH_BYTES
    assert trmoe.workspace_bytes(2048, 512, 512, 10, m_max + 1) > trmoe.NOALLOC_SCRATCH_BYTES
    rc = L.trk_moe_forward_noalloc(C.byref(cfg), None, None, C.c_void_p(256), None, m_max + 1, C.c_void_p(256), None)
    assert rc == -3 and b"scratch" in L.trk_last_error()
    assert L.trk_workspace_bytes(None, 1, None) == -1


def test_gemv_rejects_bad_codecs_and_ranges():
    """gemv_tq_rows' contract (gemv.rs:16-40): kb equal to the codec's, k a multiple of kb, strips
    inside the matrix; GGUF formats with the kb their TQ conversion has."""
    L = trmoe.lib()

    def call(fmt, rows, k, kb, s0=0, s1=1, m=1, pair=0, q=64, ldy=4096, ptr=256):
        mat = trmoe.Mat(C.c_void_p(ptr), rows, k, fmt, 1, 0)
        return L.trk_gemv(C.byref(mat), 0, s0, s1, kb, C.c_void_p(q), C.c_void_p(64), C.c_void_p(64), m, pair,
                          C.c_void_p(64), ldy, None, 0, None)

    assert call(trmoe.FMT_TQ4_32, 64, 2560, 16) == -1 and b"codec" in L.trk_last_error()
    assert call(trmoe.FMT_TQ5_16, 64, 648, 16) == -1 and b"multiple of kb" in L.trk_last_error()
    assert call(trmoe.FMT_TQ8_16, 40, 640, 16, s0=0, s1=4) == -1 and b"strips" in L.trk_last_error()
    assert call(trmoe.FMT_TQ8_16, 40, 640, 16, s0=2, s1=1) == -1
    assert call(trmoe.FMT_Q6_K, 64, 512, 32) == -1 and b"unsupported" in L.trk_last_error()
    assert call(trmoe.FMT_Q8_0, 64, 640, 32) == -1 and b"256" in L.trk_last_error()
    assert call(trmoe.FMT_Q5_1, 64, 512, 16, q=72) == -1 and b"aligned" in L.trk_last_error()
    # TQ strips are read in 16-byte pieces: a pointer 4-byte but not 16-byte aligned is refused
    assert call(trmoe.FMT_TQ4_32, 64, 2560, 32, ptr=260) == -1 and b"16-byte" in L.trk_last_error()
    assert call(trmoe.FMT_TQ4_16, 64, 640, 16, m=3, pair=1) == -1 and b"twos" in L.trk_last_error()
    assert call(trmoe.FMT_TQ4_16, 64, 640, 16, s1=4, m=2, ldy=63) == -1 and b"ldy" in L.trk_last_error()
    # within the contract and with nothing to do: no device work, status OK
    assert call(trmoe.FMT_TQ5_16, 2560, 640, 16, s0=7, s1=7) == 0
    assert call(trmoe.FMT_Q4_K, 64, 2048, 32, m=0) == 0
