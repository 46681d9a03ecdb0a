// C ABI of the MoE library: argument checks, workspace ownership and the launch sequence of the
// decode (M = 1) and batch (M >= 2) paths.  Kernels live in k_*.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "trmoe_internal.h"

using namespace trk;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

#define HIP_TRY(expr)                                                                             \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess) return fail(TRK_E_HIP, "%s: %s", #expr, hipGetErrorString(e_));    \
    } while (0)

uint32_t row_bytes(uint32_t fmt, uint32_t k) {
    if (fmt == TRK_FMT_Q4_K) return k / 256 * 144;
    if (fmt == TRK_FMT_Q6_K) return k / 256 * 210;
    if (fmt == TRK_FMT_Q8_0) return k / 256 * 272;
    if (fmt == TRK_FMT_Q5_1) return k / 256 * 192;
    return 0;
}

}  // namespace

// Kernel ids for trk_get_timing.
enum KernelId { K_LOGITS, K_ROUTE, K_QUANT, K_DEC_GATEUP, K_DEC_DOWN, K_DEC_LAYER, K_DISPATCH, K_B_GATEUP, K_B_DOWN,
                K_S_GATEUP, K_S_DOWN, K_B_COMBINE, K_RMSNORM, K_PROFILE, K_TQ_GATEUP, K_TQ_ACT, K_TQ_DOWN,
                K_TQ_COMBINE, K_HC_MIX, K_COUNT };
static const char* const kKernelNames[K_COUNT] = {"router_logits", "route", "quantize", "decode_gateup",
                                                  "decode_down", "decode_layer", "dispatch", "batch_gateup",
                                                  "batch_down", "stream_gateup", "stream_down", "batch_combine",
                                                  "rmsnorm", "mass_profile", "tq_gateup", "tq_act", "tq_down",
                                                  "tq_combine", "hc_mix"};

// Which grouped items run on the streaming GEMV (the rest on the MFMA tiles), when the caller has
// not chosen: all of them up to 16 tokens; the items of at most 4 rows while the selections
// average at most two per expert (most routed items hold one or two rows, the shared expert's
// 16); none beyond, where tail items share their expert's weights with its full tiles and a
// split costs more than it saves (measured at M = 512 and 3072).
// Items of at most this many rows take the streaming kernels: every item up to BR tokens, items of
// up to 4 rows while few rows share an expert, none beyond.
static uint32_t auto_stream_rows(uint32_t m, uint32_t kcap, uint32_t E) {
    if (m <= BR) return BR;
    return (uint64_t)m * kcap <= 2ull * E ? 4u : 0u;
}

struct TimedLaunch {
    int kid;
    hipEvent_t start, stop;
};

struct trk_ctx {
    trk_cfg cfg;
    Workspace ws;
    Policy pol;
    int device;
    void* block;  // one device allocation holding every workspace buffer
    int timing;
    std::vector<TimedLaunch> timed;
    std::vector<hipEvent_t> spare;
    int fusion = 0;   // decode: one launch per layer (when the shape and the GPU allow it) if set
    int stream_rows = -1;  // batch: items of at most this many rows on the streaming GEMV (-1: automatic)
    int tq_mfma = 1;       // TQ layers: the MFMA kernels where the shape fits (0: the generic TQ GEMV)
    int profile = 0;       // MoeStats::profile: add every routed row's mass profile to ws.prof
    int decode_rows = 8;   // batch: up to this many tokens run as per-token decode units (0: never)
};

extern "C" const char* trk_last_error(void) { return g_err; }

static int check_policy(const trk_ctx* c, const trk_moe_policy* p) {
    // MoePolicy::validate (router.rs:32-44), plus the workspace capacity
    if (p->min < 1 || p->min > p->max)
        return fail(TRK_E_POLICY, "moe policy: need 1 <= min (%u) <= max (%u)", p->min, p->max);
    uint32_t lim = std::min<uint32_t>(TRK_MOE_K_MAX, c->cfg.n_expert);
    if (p->max > TRK_MOE_K_MAX || p->max > c->cfg.n_expert)
        return fail(TRK_E_POLICY, "moe policy: max (%u) above the limit (%u)", p->max, lim);
    if (!(p->mass > 0.0f) || p->mass != p->mass)
        return fail(TRK_E_POLICY, "moe policy: target mass (%g) must be positive", (double)p->mass);
    if (p->max > c->ws.k_cap)
        return fail(TRK_E_POLICY, "moe policy: max (%u) above the context's k_cap (%u)", p->max, c->ws.k_cap);
    return TRK_OK;
}

// Shape checks of a layer configuration (trk_create and the no-allocation entry point); k_cap
// comes back resolved (0 = n_expert_used).
static int check_cfg(const trk_cfg* cfg, uint32_t m_max, uint32_t& k_cap) {
    const uint32_t H = cfg->hidden, E = cfg->n_expert, F = cfg->n_ff, k = cfg->n_expert_used;
    // n_ff: a multiple of 256 for GGUF experts (checked per call), of 16 for TQ experts
    if (H == 0 || H % 256 || F == 0 || F % 16)
        return fail(TRK_E_INVALID, "hidden (%u) must be a positive multiple of 256 and n_ff (%u) of 16", H, F);
    if (E == 0 || E > 1024) return fail(TRK_E_INVALID, "n_expert (%u) must be in 1..1024", E);
    if (k < 1 || k > TRK_MOE_K_MAX || k > E) return fail(TRK_E_INVALID, "n_expert_used (%u) must be in 1..min(32, E)", k);
    if (m_max == 0) return fail(TRK_E_INVALID, "m_max must be positive");
    k_cap = cfg->k_cap ? cfg->k_cap : k;
    if (k_cap < k || k_cap > TRK_MOE_K_MAX) return fail(TRK_E_INVALID, "k_cap (%u) must be in n_expert_used..32", k_cap);
    const geo::Caps caps{H, E, F, m_max, k_cap};
    if (geo::ent_cap(caps) > 0xffffffffull || geo::item_cap(caps) > 0xffffffffull)
        return fail(TRK_E_INVALID, "m_max * k_cap (%u * %u) too large", m_max, k_cap);
    // a pack written for T tiles (plan.py:86-90): n_ff splits into 16-row strips per tile, the
    // router's K into T slices (of a multiple of 16 columns: the dot and gemm orders step by 16)
    const uint32_t T = cfg->n_tiles > 1 ? cfg->n_tiles : 1;
    if (T > 64 || F % (16 * T) || H % (16 * T))
        return fail(TRK_E_INVALID, "n_tiles (%u): n_ff (%u) must split into 16-row strips per tile and hidden (%u) "
                    "into multiples of 16 per tile (at most 64 tiles)", T, F, H);
    // fold_ids asserts at most `packed` routed ids per token (exec_batch.rs:217)
    if (cfg->n_expert_packed && (cfg->n_expert_packed > E || cfg->n_expert_packed < k_cap))
        return fail(TRK_E_INVALID, "n_expert_packed (%u) must be in k_cap (%u) .. n_expert (%u)", cfg->n_expert_packed,
                    k_cap, E);
    return TRK_OK;
}

// The subset pack's expert count as the routing takes it (0: every expert is packed).
static uint32_t packed_of(const trk_cfg& cfg) {
    return cfg.n_expert_packed && cfg.n_expert_packed < cfg.n_expert ? cfg.n_expert_packed : 0u;
}
static uint32_t tiles_of(const trk_cfg& cfg) { return cfg.n_tiles > 1 ? cfg.n_tiles : 1u; }

// The workspace of a layer configuration for m_max rows: sizes, then 256-byte aligned pieces cut
// from base (nullptr: sizes only).  Returns the bytes the pieces take.
static size_t layout_workspace(Workspace& ws, const trk_cfg& cfg, uint32_t m_max, uint32_t k_cap, char* base) {
    const uint32_t H = cfg.hidden, E = cfg.n_expert, F = cfg.n_ff;
    const size_t M = m_max, rows_x = std::max<size_t>(2, M);
    ws.H = H;
    ws.E = E;
    ws.F = F;
    ws.m_max = m_max;
    ws.k_cap = k_cap;
    const geo::Caps caps{H, E, F, m_max, k_cap};
    ws.ent_cap = (uint32_t)geo::ent_cap(caps);
    ws.item_cap = (uint32_t)geo::item_cap(caps);  // items of <= 16 rows
    ws.act_rows = geo::act_rows(caps);
    const uint32_t T = tiles_of(cfg);
    ws.tiles = T;
    struct Piece {
        void** p;
        size_t bytes;
    };
    const size_t yrows = geo::yent_rows(caps);
    ws.yent_tile = yrows * H;
    Piece pieces[] = {
        {(void**)&ws.xq, rows_x * H},
        {(void**)&ws.xs, rows_x * (H / 32) * 4},
        {(void**)&ws.xsum, rows_x * (H / 32) * 4},
        {(void**)&ws.xu, rows_x * (H / 32) * 4},
        {(void**)&ws.xn, M * H * 4},
        {(void**)&ws.rlog, M * E * 4},
        {(void**)&ws.shl, M * 4},
        {(void**)&ws.ids, M * TRK_MOE_K_MAX * 4},
        {(void**)&ws.w, M * TRK_MOE_K_MAX * 4},
        {(void**)&ws.n_sel, M * 4},
        {(void**)&ws.ent_tok, (size_t)ws.ent_cap * 4},
        {(void**)&ws.ent_w, (size_t)ws.ent_cap * 4},
        {(void**)&ws.ent_exp, (size_t)ws.ent_cap * 4},
        {(void**)&ws.ent_of, M * TRK_MOE_K_MAX * 4},
        {(void**)&ws.grp_start, (E + 2) * 4},
        {(void**)&ws.grp_exp, (E + 1) * 4},
        {(void**)&ws.n_groups, 32},
        {(void**)&ws.doff, geo::doff_elems(m_max, E) * 4},  // [ceil(m / 64)][E] per-chunk offsets
        {(void**)&ws.items, (size_t)ws.item_cap * sizeof(Item)},
        {(void**)&ws.pairs, ((size_t)ws.item_cap / 2 + 1) * 4},
        {(void**)&ws.single, (size_t)ws.item_cap * 4},
        {(void**)&ws.actq, ws.act_rows * F},
        {(void**)&ws.acts, ws.act_rows * (F / 16) * 4},
        {(void**)&ws.actsum, ws.act_rows * (F / 16) * 4},
        {(void**)&ws.actu, ws.act_rows * (F / 16) * 4},
        {(void**)&ws.yent, T * yrows * H * 4},
        {(void**)&ws.plog, T > 1 ? (size_t)T * M * E * 4 : 0},
        {(void**)&ws.xt, T > 1 ? M * H * 4 : 0},
        {(void**)&ws.hgu, yrows * 2 * F * 4},
        {(void**)&ws.out_tmp, M * H * 4},
        {(void**)&ws.stats, 16},
        {(void**)&ws.prof, (K_MAX + 1) * 8},
        {(void**)&ws.counters, (size_t)BAR_LINE * 4 * (BAR_GROUPS + 2)},
    };
    size_t off = 0;
    for (auto& pc : pieces) {
        *pc.p = base ? base + off : nullptr;
        off += (pc.bytes + 255) / 256 * 256;
    }
    return off;
}

extern "C" int trk_workspace_bytes(const trk_cfg* cfg, uint32_t m, size_t* bytes) {
    if (!cfg || !bytes) return fail(TRK_E_INVALID, "trk_workspace_bytes: null argument");
    uint32_t k_cap = 0;
    const int rc = check_cfg(cfg, m, k_cap);
    if (rc) return rc;
    Workspace ws{};
    *bytes = layout_workspace(ws, *cfg, m, k_cap, nullptr);
    return TRK_OK;
}

extern "C" int trk_create(const trk_cfg* cfg, trk_ctx** out) {
    if (!cfg || !out) return fail(TRK_E_INVALID, "trk_create: null argument");
    uint32_t k_cap = 0;
    int rc = check_cfg(cfg, cfg->m_max, k_cap);
    if (rc) return rc;
    int device = 0;
    HIP_TRY(hipGetDevice(&device));
    trk_ctx* c = new (std::nothrow) trk_ctx();
    if (!c) return fail(TRK_E_NOMEM, "host allocation failed");
    c->cfg = *cfg;
    if (!c->cfg.router_dot_max_m) c->cfg.router_dot_max_m = 16;
    c->pol = Policy{0, 0, 0, 0, 0.0f, packed_of(c->cfg)};
    c->device = device;
    const size_t total = layout_workspace(c->ws, c->cfg, cfg->m_max, k_cap, nullptr);
    hipError_t e = hipMalloc(&c->block, total);
    if (e != hipSuccess) {
        delete c;
        return fail(TRK_E_NOMEM, "hipMalloc(%zu): %s", total, hipGetErrorString(e));
    }
    e = hipMemset(c->block, 0, total);
    if (e != hipSuccess) {
        (void)hipFree(c->block);
        delete c;
        return fail(TRK_E_HIP, "workspace clear: %s", hipGetErrorString(e));
    }
    layout_workspace(c->ws, c->cfg, cfg->m_max, k_cap, (char*)c->block);
    e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(c->block);
        delete c;
        return fail(TRK_E_HIP, "workspace init: %s", hipGetErrorString(e));
    }
    *out = c;
    return TRK_OK;
}

extern "C" int trk_destroy(trk_ctx* c) {
    if (!c) return TRK_OK;
    for (auto& t : c->timed) {
        (void)hipEventDestroy(t.start);
        (void)hipEventDestroy(t.stop);
    }
    for (auto ev : c->spare) (void)hipEventDestroy(ev);
    (void)hipFree(c->block);
    delete c;
    return TRK_OK;
}

extern "C" int trk_set_moe(trk_ctx* c, const trk_moe_policy* p) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    if (!p) {
        c->pol = Policy{0, 0, 0, 0, 0.0f, packed_of(c->cfg)};
        return TRK_OK;
    }
    int rc = check_policy(c, p);
    if (rc) return rc;
    c->pol = Policy{1, p->min, p->max, p->basis, p->mass, packed_of(c->cfg)};
    return TRK_OK;
}

// tiles > 1: m describes one tile's stack (rows / k of one tile), the T stacks tile_stride apart
static int make_mat(const trk_mat& m, uint32_t rows, uint32_t k, bool down_ok_q6, uint32_t min_count, const char* name,
                    Mat& out, uint32_t tiles = 1) {
    if (!m.ptr) return fail(TRK_E_INVALID, "%s: null weight pointer", name);
    if (m.rows != rows || m.k != k)
        return fail(TRK_E_INVALID, "%s: shape [%u][%u], expected [%u][%u]", name, m.rows, m.k, rows, k);
    if (m.count < min_count) return fail(TRK_E_INVALID, "%s: %u matrices, need %u", name, m.count, min_count);
    uint64_t pitch, mb, align;
    if (fmt_is_tq(m.fmt)) {
        // the reference's packed strips: gate/up blocks of 32 values (x is quantised per 32), down
        // blocks of 16 (the SwiGLU output is quantised per 16), exec.rs:1563-1606
        const uint32_t kb = tq_kb(m.fmt);
        if (kb != (down_ok_q6 ? 16u : 32u))
            return fail(TRK_E_INVALID, "%s: TQ codec with kb %u, this projection needs kb %u", name, kb, down_ok_q6 ? 16u : 32u);
        if (k % kb) return fail(TRK_E_INVALID, "%s: k %u is not a multiple of kb %u", name, k, kb);
        pitch = (uint64_t)(k / kb) * tq_block_bytes(m.fmt);  // one 16-row strip
        mb = pitch * ((rows + 15) / 16);
        align = 16;  // blocks are read with 16-byte loads
    } else {
        if (!(m.fmt == TRK_FMT_Q4_K || (down_ok_q6 && (m.fmt == TRK_FMT_Q6_K || m.fmt == TRK_FMT_Q8_0 || m.fmt == TRK_FMT_Q5_1))))
            return fail(TRK_E_INVALID, "%s: unsupported format %u", name, m.fmt);
        if (k % 256 || rows % 256)
            return fail(TRK_E_INVALID, "%s: GGUF experts need rows and k multiples of 256 ([%u][%u])", name, rows, k);
        pitch = row_bytes(m.fmt, k);
        mb = pitch * rows;
        // Q4_K superblocks and Q8_0 / Q5_1 units of 8 blocks (272 / 192 bytes) are read with 16- and
        // 8-byte loads
        align = m.fmt == TRK_FMT_Q6_K ? 2 : 16;
    }
    if (m.count > 1 && m.stride < mb) return fail(TRK_E_INVALID, "%s: stride %llu below matrix bytes %llu", name,
                                                  (unsigned long long)m.stride, (unsigned long long)mb);
    if ((uintptr_t)m.ptr % align || (m.count > 1 && m.stride % align))
        return fail(TRK_E_INVALID, "%s: pointer/stride must be %llu-byte aligned", name, (unsigned long long)align);
    const uint64_t stride = m.count > 1 ? m.stride : mb;
    out = Mat{(const uint8_t*)m.ptr, stride, rows, k, m.fmt, (uint32_t)pitch, 0, (rows + 15) / 16};
    if (tiles > 1) {
        if (!fmt_is_tq(m.fmt)) return fail(TRK_E_INVALID, "%s: a pack written for tiles holds TQ experts", name);
        // the tiles' stacks follow one another without overlapping
        const uint64_t stack = (uint64_t)(m.count - 1) * stride + mb;
        if (m.tile_stride < stack || m.tile_stride % 16)
            return fail(TRK_E_INVALID, "%s: tile_stride %llu below a tile's %llu bytes or not 16-byte aligned", name,
                        (unsigned long long)m.tile_stride, (unsigned long long)stack);
        out.tile_stride = m.tile_stride;
    }
    return TRK_OK;
}

struct Mats {
    Mat gate, up, down, shg, shu, shd;
};

static int check_weights(trk_ctx* c, const trk_moe_w* w, Mats& M) {
    const uint32_t H = c->cfg.hidden, F = c->cfg.n_ff, E = c->cfg.n_expert;
    // a subset pack holds only its first n_expert_packed experts; with T tiles every stack is one
    // tile's: gate/up [F / T][H] (rows split), down [H][F / T] (columns split)
    const uint32_t T = tiles_of(c->cfg), Ep = packed_of(c->cfg) ? packed_of(c->cfg) : E, Ft = F / T;
    if (!w || !w->shexp_gate) return fail(TRK_E_INVALID, "weights: null pointer");
    int rc;
    if ((rc = make_mat(w->gate, Ft, H, false, Ep, "gate", M.gate, T))) return rc;
    if ((rc = make_mat(w->up, Ft, H, false, Ep, "up", M.up, T))) return rc;
    if ((rc = make_mat(w->down, H, Ft, true, Ep, "down", M.down, T))) return rc;
    if ((rc = make_mat(w->sh_gate, Ft, H, false, 1, "sh_gate", M.shg, T))) return rc;
    if ((rc = make_mat(w->sh_up, Ft, H, false, 1, "sh_up", M.shu, T))) return rc;
    if ((rc = make_mat(w->sh_down, H, Ft, true, 1, "sh_down", M.shd, T))) return rc;
    if (M.shd.fmt != M.down.fmt) return fail(TRK_E_INVALID, "sh_down: format %u, down: %u (one down format per layer)",
                                             M.shd.fmt, M.down.fmt);
    // one gate/up format per layer; TQ and GGUF experts are not mixed within a layer
    if (M.up.fmt != M.gate.fmt || M.shg.fmt != M.gate.fmt || M.shu.fmt != M.gate.fmt)
        return fail(TRK_E_INVALID, "gate/up: formats %u/%u (shared %u/%u) differ (one gate/up format per layer)",
                    M.gate.fmt, M.up.fmt, M.shg.fmt, M.shu.fmt);
    if (fmt_is_tq(M.gate.fmt) != fmt_is_tq(M.down.fmt))
        return fail(TRK_E_INVALID, "gate/up and down: TQ and GGUF experts in one layer");
    return TRK_OK;
}

static hipError_t take_event(trk_ctx* c, hipEvent_t* ev) {
    if (!c->spare.empty()) {
        *ev = c->spare.back();
        c->spare.pop_back();
        return hipSuccess;
    }
    return hipEventCreate(ev);
}

// Run one launch; with timing on, bracket it with events on the launch's stream.
template <typename F>
static hipError_t timed(trk_ctx* c, int kid, hipStream_t st, F&& launch) {
    if (!c->timing) return launch();
    TimedLaunch t{kid, nullptr, nullptr};
    hipError_t e;
    if ((e = take_event(c, &t.start)) != hipSuccess || (e = take_event(c, &t.stop)) != hipSuccess) return e;
    if ((e = hipEventRecord(t.start, st)) != hipSuccess) return e;
    e = launch();
    if (e != hipSuccess) return e;
    if ((e = hipEventRecord(t.stop, st)) != hipSuccess) return e;
    c->timed.push_back(t);
    return hipSuccess;
}
// One launch of the forward sequence; with `only` >= 0, only the kernel of that id is launched.
#define TIMED(kid, expr)                                                              \
    do {                                                                              \
        if (only < 0 || only == (kid)) HIP_TRY(timed(c, kid, st, [&]() { return (expr); })); \
    } while (0)

// The MoE block on x (already normed, or normed inside the logits launch when norm is set; only
// the logits launch reads x).  residual: out += moe instead of out = moe.
static int forward(trk_ctx* c, const trk_moe_w* w, const float* x, const float* rlog, uint32_t m, float* out,
                   int residual, hipStream_t st, int only = -1, const XNorm* norm = nullptr) {
    Mats M;
    int rc = check_weights(c, w, M);
    if (rc) return rc;
    if (!x || !out) return fail(TRK_E_INVALID, "null x/out");
    if (m == 0) return TRK_OK;
    if (m > c->cfg.m_max) return fail(TRK_E_CAPACITY, "M (%u) above m_max (%u)", m, c->cfg.m_max);
    if (!rlog && !w->router) return fail(TRK_E_INVALID, "need router weights or precomputed logits");
    Workspace& ws = c->ws;
    const uint32_t H = ws.H, E = ws.E, k = c->cfg.n_expert_used;
    const uint32_t kcap = c->pol.enabled ? c->pol.max : k;
    const float* lg = rlog ? rlog : ws.rlog;
    const int gemm_order = m >= c->cfg.router_dot_max_m ? 1 : 0;
    const bool tq = fmt_is_tq(M.gate.fmt);
    // every grid below and every workspace extent its kernels index, checked on the host
    if (const char* why = geo::check_call(geo::Caps{H, E, ws.F, ws.m_max, ws.k_cap}, m, kcap, tq))
        return fail(TRK_E_INVALID, "launch geometry: %s", why);
    if (tq) {
        // the layer on the reference's packed TQ experts (k_tq.hip): the logits launch quantises x
        // (two levels at M = 1 with hiprec), routing and dispatch as below, then the grouped TQ
        // GEMVs, SwiGLU + quantisation + fold between them, and the combine
        const int pair = m == 1 && c->cfg.hiprec ? 1 : 0;
        const XQuant xq{ws.xq, ws.xs, ws.xsum, ws.xu, pair};
        const uint32_t T = ws.tiles;
        if (rlog || T > 1)
            TIMED(K_LOGITS, launch_router_logits(nullptr, nullptr, w->shexp_gate, x, m, 0, H, 0, nullptr, ws.shl, st,
                                                 &xq, norm));
        else
            TIMED(K_LOGITS, launch_router_logits(w->router, w->router_bias, w->shexp_gate, x, m, E, H,
                                                 m == 1 ? 0 : gemm_order, ws.rlog, ws.shl, st, &xq, norm));
        if (!rlog && T > 1) {
            // the K-split router of a pack written for T tiles (exec.rs:1003-1011, exec_batch.rs:
            // 1008-1016): each tile's partial over its H / T columns of x, in the dot or gemm order,
            // then the partials summed in tile order (exchange.rs:122-136) and the bias added
            const uint32_t hl = H / T;
            TIMED(K_LOGITS, launch_tile_split(x, m, H, T, ws.xt, st));
            for (uint32_t t = 0; t < T; t++)
                TIMED(K_LOGITS, launch_router_logits(w->router + (size_t)t * E * hl, nullptr, nullptr,
                                                     ws.xt + (size_t)t * m * hl, m, E, hl, m == 1 ? 0 : gemm_order,
                                                     ws.plog + (size_t)t * m * E, nullptr, st, nullptr, nullptr));
            TIMED(K_LOGITS, launch_tile_reduce(ws.plog, m, E, T, w->router_bias, ws.rlog, st));
        }
        // tiles: the generic grouped TQ GEMV, which takes each tile's rows and columns
        const bool mfma = c->tq_mfma && tqm_fits(H, ws.F) && T == 1;
        // a few tokens: each one a decode (routing inside the gate/up launch, its rows added by the
        // down in the batch combine's order), no routing, dispatch or combine launch
        if (m >= 2 && m <= (uint32_t)c->decode_rows && mfma && tqd_tokens_fit(ws, m, kcap) &&
            tqd_gateup_ok(M.gate, M.up, M.shg, M.shu, ws, c->pol) && tqd_dc_ok(M.down, M.shd, ws, kcap)) {
            TIMED(K_TQ_GATEUP, launch_tqm_gateup(M.gate, M.up, M.shg, M.shu, ws, m, kcap, 0, lg, k, c->pol, st));
            TIMED(K_TQ_DOWN, launch_tqd_down_combine(M.down, M.shd, ws, kcap, 0, out, residual, st, m));
            if (c->profile) TIMED(K_PROFILE, launch_mass_profile(lg, m, E, ws.prof, st));
            return TRK_OK;
        }
        if (m == 1) {
            // the MFMA gate/up launch routes for itself
            if (!mfma) TIMED(K_ROUTE, launch_route(lg, 1, E, k, c->pol, ws.ids, ws.w, ws.n_sel, ws.stats, st));
        } else if (m <= 4 && m * kcap <= 1024) {
            TIMED(K_DISPATCH, launch_dispatch_small(ws, m, kcap, lg, k, c->pol, st));
        } else if (m <= 16 && m * kcap <= 1024) {
            TIMED(K_ROUTE, launch_route(lg, m, E, k, c->pol, ws.ids, ws.w, ws.n_sel, nullptr, st));
            TIMED(K_DISPATCH, launch_dispatch_small(ws, m, kcap, nullptr, k, c->pol, st));
        } else {
            TIMED(K_ROUTE, launch_route(lg, m, E, k, c->pol, ws.ids, ws.w, ws.n_sel, nullptr, st));
            TIMED(K_DISPATCH, launch_dispatch(ws, m, kcap, st));
        }
        if (mfma) {
            // int8 MFMA per TQ block, SwiGLU + quantisation + fold in the gate/up launch
            TIMED(K_TQ_GATEUP, launch_tqm_gateup(M.gate, M.up, M.shg, M.shu, ws, m, kcap, pair, m == 1 ? lg : nullptr, k,
                                                 c->pol, st));
            if (m == 1 && tqd_dc_ok(M.down, M.shd, ws, kcap)) {
                // decode: the down adds the slots' rows in order itself (no combine launch)
                TIMED(K_TQ_DOWN, launch_tqd_down_combine(M.down, M.shd, ws, kcap, pair, out, residual, st));
                if (c->profile) TIMED(K_PROFILE, launch_mass_profile(lg, m, E, ws.prof, st));
                return TRK_OK;
            }
            TIMED(K_TQ_DOWN, launch_tqm_down(M.down, M.shd, ws, m, kcap, pair, st));
        } else {
            TIMED(K_TQ_GATEUP, launch_tq_gateup(M.gate, M.up, M.shg, M.shu, ws, ws.hgu, m, kcap, pair, st));
            TIMED(K_TQ_ACT, launch_tq_act(ws, ws.hgu, m, kcap, pair, st));
            TIMED(K_TQ_DOWN, launch_tq_down(M.down, M.shd, ws, m, kcap, pair, st));
        }
        if (m == 1)
            TIMED(K_TQ_COMBINE, launch_tq_combine(ws, out, residual, st));
        else
            TIMED(K_B_COMBINE, launch_batch_combine(ws, m, out, residual, st));
        if (c->profile) TIMED(K_PROFILE, launch_mass_profile(lg, m, E, ws.prof, st));
        return TRK_OK;
    }
    if (m == 1) {
        // logits (and the shared gate's logit), then routing + gate/up in one launch, then down
        const int pair = c->cfg.hiprec ? 1 : 0;
        // the one-launch layer where this layer's shape has one (checked per call: the formats may
        // change from layer to layer)
        const bool fuse = c->fusion && ws.counters &&
                          launch_decode_layer(w->router, w->router_bias, w->shexp_gate, M.gate, M.up, M.down, M.shg,
                                              M.shu, M.shd, x, rlog, ws, k, c->pol, pair, kcap, out, residual, true,
                                              st) == hipSuccess;
        if (fuse) {
            TIMED(K_DEC_LAYER, launch_decode_layer(w->router, w->router_bias, w->shexp_gate, M.gate, M.up, M.down, M.shg,
                                                   M.shu, M.shd, x, rlog, ws, k, c->pol, pair, kcap, out, residual,
                                                   false, st));
            if (c->profile) TIMED(K_PROFILE, launch_mass_profile(lg, m, E, ws.prof, st));
            return TRK_OK;
        }
        // the logits launch also quantises x for gate/up
        const XQuant xq{ws.xq, ws.xs, ws.xsum, ws.xu, pair};
        if (rlog)
            TIMED(K_LOGITS,
                  launch_router_logits(nullptr, nullptr, w->shexp_gate, x, 1, 0, H, 0, nullptr, ws.shl, st, &xq, norm));
        else
            TIMED(K_LOGITS, launch_router_logits(w->router, w->router_bias, w->shexp_gate, x, 1, E, H, 0, ws.rlog,
                                                 ws.shl, st, &xq, norm));
        TIMED(K_DEC_GATEUP, launch_decode_gateup(M.gate, M.up, M.shg, M.shu, x, lg, ws, k, c->pol, pair, kcap, st));
        TIMED(K_DEC_DOWN, launch_decode_down(M.down, M.shd, ws, pair, kcap, out, residual, st));
    } else if (m <= (uint32_t)c->decode_rows && ws.tiles == 1) {
        // a few tokens: each one a decode (routing inside its gate/up units, its rows added by the
        // down in the batch combine's order), so no routing, dispatch or combine launch and no
        // grouped items; the logits and quantised x exactly as for a batch
        const XQuant xq{ws.xq, ws.xs, ws.xsum, ws.xu, 0};
        if (rlog)
            TIMED(K_LOGITS, launch_router_logits(nullptr, nullptr, w->shexp_gate, x, m, 0, H, 0, nullptr, ws.shl, st,
                                                 &xq, norm));
        else
            TIMED(K_LOGITS, launch_router_logits(w->router, w->router_bias, w->shexp_gate, x, m, E, H, gemm_order,
                                                 ws.rlog, ws.shl, st, &xq, norm));
        TIMED(K_DEC_GATEUP, launch_decode_gateup(M.gate, M.up, M.shg, M.shu, x, lg, ws, k, c->pol, 0, kcap, st, m));
        TIMED(K_DEC_DOWN, launch_decode_down(M.down, M.shd, ws, 0, kcap, out, residual, st, m));
    } else {
        // the logits launch also quantises x (single level, per 32) for the grouped kernels
        const XQuant xq{ws.xq, ws.xs, ws.xsum, ws.xu, 0};
        if (rlog)
            TIMED(K_LOGITS, launch_router_logits(nullptr, nullptr, w->shexp_gate, x, m, 0, H, 0, nullptr, ws.shl, st,
                                                 &xq, norm));
        else
            TIMED(K_LOGITS, launch_router_logits(w->router, w->router_bias, w->shexp_gate, x, m, E, H, gemm_order,
                                                 ws.rlog, ws.shl, st, &xq, norm));
        // the dispatch kernel counts the routed rows (one atomic per call, not per token).  Up to 4
        // tokens one launch routes (a wave per token, one per SIMD) and dispatches; up to 16 the
        // routing has a launch of its own (spread over CUs) and the dispatch is the small one
        if (m <= 4 && m * kcap <= 1024) {
            TIMED(K_DISPATCH, launch_dispatch_small(ws, m, kcap, lg, k, c->pol, st));
        } else if (m <= 16 && m * kcap <= 1024) {
            TIMED(K_ROUTE, launch_route(lg, m, E, k, c->pol, ws.ids, ws.w, ws.n_sel, nullptr, st));
            TIMED(K_DISPATCH, launch_dispatch_small(ws, m, kcap, nullptr, k, c->pol, st));
        } else {
            TIMED(K_ROUTE, launch_route(lg, m, E, k, c->pol, ws.ids, ws.w, ws.n_sel, nullptr, st));
            TIMED(K_DISPATCH, launch_dispatch(ws, m, kcap, st));
        }
        // items of few rows on the streaming GEMV, the others on the MFMA tiles (same bits)
        const uint32_t sr = c->stream_rows >= 0 ? (uint32_t)c->stream_rows : auto_stream_rows(m, kcap, E);
        if (sr > 0) TIMED(K_S_GATEUP, launch_stream_gateup(M.gate, M.up, M.shg, M.shu, ws, m, sr, st));
        if (sr < BR) TIMED(K_B_GATEUP, launch_batch_gateup(M.gate, M.up, M.shg, M.shu, ws, m, sr, st));
        if (sr > 0) TIMED(K_S_DOWN, launch_stream_down(M.down, M.shd, ws, m, sr, st));
        if (sr < BR) TIMED(K_B_DOWN, launch_batch_down(M.down, M.shd, ws, m, sr, st));
        TIMED(K_B_COMBINE, launch_batch_combine(ws, m, out, residual, st));
    }
    // MoeStats::profile_row on every routed row (exec.rs:1552, exec_batch.rs:1456), off the layer's
    // critical path
    if (c->profile) TIMED(K_PROFILE, launch_mass_profile(lg, m, E, ws.prof, st));
    return TRK_OK;
}

extern "C" int trk_moe_forward(trk_ctx* c, const trk_moe_w* w, const float* x, const float* rlog, uint32_t m,
                               float* out, void* stream) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    return forward(c, w, x, rlog, m, out, 0, (hipStream_t)stream);
}

extern "C" int trk_moe_forward_hc(trk_ctx* c, const trk_moe_w* w, const trk_hc_w* hc, const float* xn, const float* lo,
                                  uint32_t m, float* out, void* stream) {
    if (!c || !hc || !xn || !lo || !out) return fail(TRK_E_INVALID, "null argument");
    if (hc->hc == 0 || hc->hc > 8) return fail(TRK_E_INVALID, "hc (%u) must be in 1..8", hc->hc);
    if (hc->lr == 0 || hc->lr % 32 || hc->lr > 1024) return fail(TRK_E_INVALID, "lr (%u): a multiple of 32 up to 1024", hc->lr);
    if (!fmt_is_tq(hc->up.fmt) || tq_kb(hc->up.fmt) != 32)
        return fail(TRK_E_INVALID, "up: a kb-32 TQ codec (the low-rank row is quantised per 32)");
    if (m == 0) return TRK_OK;
    if (m > c->cfg.m_max) return fail(TRK_E_CAPACITY, "M (%u) above m_max (%u)", m, c->cfg.m_max);
    const size_t img = hc_image_bytes(m, hc->lr), yent = (size_t)c->ws.tiles * c->ws.yent_tile * 4;
    if (m > 1 && img > yent)
        return fail(TRK_E_CAPACITY, "the mix's quantised rows (%zu bytes) exceed the per-entry output rows (%zu bytes)",
                    img, yent);
    const uint32_t H = c->cfg.hidden;
    Mat up;
    int rc = make_mat(hc->up, hc->hc * H, hc->lr, false, 1, "hc up", up);
    if (rc) return rc;
    Mats M;
    if ((rc = check_weights(c, w, M))) return rc;
    hipStream_t st = (hipStream_t)stream;
    const int only = -1;
    TIMED(K_HC_MIX, launch_hc_mix(up, hc->hc, H, hc->lr, xn, lo, m, c->cfg.hiprec, c->ws, c->ws.xn, st));
    return forward(c, w, c->ws.xn, nullptr, m, out, 0, st);
}

// ---- the layer without a context and without allocating ------------------------------------
//
// The workspace lives in one file-scope device array, `scratch`, of TRK_NOALLOC_SCRATCH_BYTES; every
// GPU the library runs on holds its own copy until the process ends.  Host code never uses the
// array's name as an address: on a device's first call hipGetSymbolAddress gives that device's
// address, kept per device, and only that address reaches the kernels.  Nothing in the sequence
// reads the workspace before writing it in the same call (routing, dispatch, activations and
// per-entry outputs are all produced before they are consumed), so no clear is needed; the
// MoeStats counters, the mass profile and the one-launch layer's barrier words belong to a
// context and are not used here.  Calls that overlap on one GPU share the array and race.
static __device__ __align__(256) uint8_t scratch[TRK_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
constexpr int SCRATCH_DEVICES = 64;
static void* g_scratch_ptr[SCRATCH_DEVICES];  // device address of `scratch`, per device

static int scratch_of_current_device(void** out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= SCRATCH_DEVICES) return fail(TRK_E_INVALID, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(TRK_E_HIP, "hipGetSymbolAddress gave no address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return TRK_OK;
}

extern "C" int trk_moe_forward_noalloc(const trk_cfg* cfg, const trk_moe_policy* policy, const trk_moe_w* w,
                                       const float* x, const float* rlog, uint32_t m, float* out, void* stream) {
    if (!cfg) return fail(TRK_E_INVALID, "null configuration");
    if (m == 0) return TRK_OK;
    uint32_t k_cap = 0;
    int rc = check_cfg(cfg, m, k_cap);
    if (rc) return rc;
    trk_ctx c;  // host-side bookkeeping on the stack; its event lists stay empty (timing off)
    c.cfg = *cfg;
    c.cfg.m_max = m;
    if (!c.cfg.router_dot_max_m) c.cfg.router_dot_max_m = 16;
    c.pol = Policy{0, 0, 0, 0, 0.0f, packed_of(c.cfg)};
    c.block = nullptr;
    c.timing = 0;
    const size_t need = layout_workspace(c.ws, c.cfg, m, k_cap, nullptr);
    if (need > TRK_NOALLOC_SCRATCH_BYTES)
        return fail(TRK_E_CAPACITY, "workspace for M=%u needs %zu bytes, above the static scratch of %zu bytes", m,
                    need, (size_t)TRK_NOALLOC_SCRATCH_BYTES);
    if (policy) {
        if ((rc = check_policy(&c, policy))) return rc;
        c.pol = Policy{1, policy->min, policy->max, policy->basis, policy->mass, packed_of(c.cfg)};
    }
    void* base = nullptr;
    if ((rc = scratch_of_current_device(&base))) return rc;
    layout_workspace(c.ws, c.cfg, m, k_cap, (char*)base);
    c.ws.stats = nullptr;  // MoeStats, the mass profile and the barrier words belong to a context
    c.ws.prof = nullptr;
    c.ws.counters = nullptr;
    HIP_TRY(hipGetDevice(&c.device));
    return forward(&c, w, x, rlog, m, out, 0, (hipStream_t)stream);
}

extern "C" int trk_launch_kernel(trk_ctx* c, const trk_moe_w* w, const float* x, const float* rlog, uint32_t m,
                                 float* out, const char* name, void* stream) {
    if (!c || !name) return fail(TRK_E_INVALID, "null argument");
    for (int kid = 0; kid < K_COUNT; kid++)
        if (std::strcmp(name, kKernelNames[kid]) == 0) return forward(c, w, x, rlog, m, out, 0, (hipStream_t)stream, kid);
    return fail(TRK_E_INVALID, "no kernel named '%s'", name);
}

extern "C" int trk_moe_residual(trk_ctx* c, const trk_moe_w* w, const float* rms_w, float eps, float* h, uint32_t m,
                                void* stream) {
    if (!c || !h) return fail(TRK_E_INVALID, "null argument");
    if (m > c->cfg.m_max) return fail(TRK_E_CAPACITY, "M (%u) above m_max (%u)", m, c->cfg.m_max);
    hipStream_t st = (hipStream_t)stream;
    const int only = -1;
    // Below the router GEMM threshold (and off the one-launch decode layer, which reads x itself)
    // the logits launch normalises h where it reads it: no rmsnorm launch, no normed copy
    if (!c->fusion && m < c->cfg.router_dot_max_m && w->router && c->ws.tiles == 1) {
        const XNorm nrm{rms_w, eps};
        return forward(c, w, h, nullptr, m, h, 1, st, only, &nrm);
    }
    TIMED(K_RMSNORM, launch_rmsnorm(h, rms_w, eps, m, c->cfg.hidden, c->ws.xn, st));
    return forward(c, w, c->ws.xn, nullptr, m, h, 1, st);
}

extern "C" int trk_get_stats(trk_ctx* c, trk_moe_stats* out, int reset, void* stream) {
    if (!c || !out) return fail(TRK_E_INVALID, "null argument");
    hipStream_t st = (hipStream_t)stream;
    unsigned long long v[2];
    uint32_t timed_out = 0;
    HIP_TRY(hipMemcpyAsync(v, c->ws.stats, sizeof v, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipMemcpyAsync(&timed_out, c->ws.counters + 2, 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    out->rows = v[0];
    out->experts = v[1];
    if (reset) HIP_TRY(hipMemsetAsync(c->ws.stats, 0, sizeof v, st));
    if (timed_out) {
        HIP_TRY(hipMemsetAsync(c->ws.counters + 2, 0, 4, st));
        HIP_TRY(hipStreamSynchronize(st));
        return fail(TRK_E_TIMEOUT, "a device-side wait of the one-launch decode layer timed out: the outputs of "
                                   "the calls since the last trk_get_stats are invalid");
    }
    if (reset) HIP_TRY(hipStreamSynchronize(st));
    return TRK_OK;
}

extern "C" int trk_profile_start(trk_ctx* c, int on, void* stream) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    // MoeStats::profile_start (exec.rs:567-573): zero the sums, then count
    if (on) HIP_TRY(hipMemsetAsync(c->ws.prof, 0, (K_MAX + 1) * sizeof(unsigned long long), (hipStream_t)stream));
    c->profile = on ? 1 : 0;
    return TRK_OK;
}

extern "C" int trk_profile_report(trk_ctx* c, double* cum, uint64_t* rows, void* stream) {
    if (!c || !cum || !rows) return fail(TRK_E_INVALID, "null argument");
    hipStream_t st = (hipStream_t)stream;
    unsigned long long v[K_MAX + 1];
    HIP_TRY(hipMemcpyAsync(v, c->ws.prof, sizeof v, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    // MoeStats::profile_report (exec.rs:575-581): fixed point 1e-6, mean over the profiled rows
    const unsigned long long n = v[K_MAX];
    *rows = n;
    for (int j = 0; j < K_MAX; j++) cum[j] = n ? (double)v[j] * 1e-6 / (double)n : 0.0;
    return TRK_OK;
}

extern "C" int trk_set_fusion(trk_ctx* c, int on) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    c->fusion = on ? 1 : 0;
    return TRK_OK;
}

extern "C" int trk_set_tq_mfma(trk_ctx* c, int on) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    c->tq_mfma = on ? 1 : 0;
    return TRK_OK;
}

extern "C" int trk_set_stream_rows(trk_ctx* c, int rows) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    if (rows < -1 || rows > (int)BR) return fail(TRK_E_INVALID, "stream rows (%d) must be in -1..%u", rows, BR);
    c->stream_rows = rows;
    return TRK_OK;
}

extern "C" int trk_set_decode_rows(trk_ctx* c, int rows) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    if (rows < 0 || rows > 16) return fail(TRK_E_INVALID, "decode rows (%d) must be in 0..16", rows);
    c->decode_rows = rows;
    return TRK_OK;
}

extern "C" int trk_set_timing(trk_ctx* c, int on) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    c->timing = on ? 1 : 0;
    return TRK_OK;
}

extern "C" int trk_get_timing(trk_ctx* c, const char** names, double* ms, uint64_t* launches, int cap) {
    if (!c) return fail(TRK_E_INVALID, "null context");
    double tot[K_COUNT] = {0};
    uint64_t cnt[K_COUNT] = {0};
    for (auto& t : c->timed) {
        HIP_TRY(hipEventSynchronize(t.stop));
        float v = 0.0f;
        HIP_TRY(hipEventElapsedTime(&v, t.start, t.stop));
        tot[t.kid] += v;
        cnt[t.kid]++;
        c->spare.push_back(t.start);
        c->spare.push_back(t.stop);
    }
    c->timed.clear();
    int n = 0;
    for (int k = 0; k < K_COUNT; k++) {
        if (!cnt[k]) continue;
        if (n < cap) {
            if (names) names[n] = kKernelNames[k];
            if (ms) ms[n] = tot[k];
            if (launches) launches[n] = cnt[k];
        }
        n++;
    }
    return n;
}

extern "C" int trk_debug_read(trk_ctx* c, int which, void* host, size_t bytes, void* stream) {
    if (!c || !host) return fail(TRK_E_INVALID, "null argument");
    const Workspace& ws = c->ws;
    const void* src = nullptr;
    size_t cap = 0;
    const size_t M = ws.m_max, rows_x = std::max<size_t>(2, M);
    switch (which) {
    case TRK_WS_RLOG: src = ws.rlog; cap = M * ws.E * 4; break;
    case TRK_WS_IDS: src = ws.ids; cap = M * TRK_MOE_K_MAX * 4; break;
    case TRK_WS_W: src = ws.w; cap = M * TRK_MOE_K_MAX * 4; break;
    case TRK_WS_NSEL: src = ws.n_sel; cap = M * 4; break;
    case TRK_WS_ENT_TOK: src = ws.ent_tok; cap = (size_t)ws.ent_cap * 4; break;
    case TRK_WS_ENT_W: src = ws.ent_w; cap = (size_t)ws.ent_cap * 4; break;
    case TRK_WS_ENT_EXP: src = ws.ent_exp; cap = (size_t)ws.ent_cap * 4; break;
    case TRK_WS_GRP_START: src = ws.grp_start; cap = (ws.E + 2) * 4; break;
    case TRK_WS_GRP_EXP: src = ws.grp_exp; cap = (ws.E + 1) * 4; break;
    case TRK_WS_NGROUPS: src = ws.n_groups; cap = 16; break;
    case TRK_WS_XQ: src = ws.xq; cap = rows_x * ws.H; break;
    case TRK_WS_XS: src = ws.xs; cap = rows_x * (ws.H / 32) * 4; break;
    case TRK_WS_ACTQ: src = ws.actq; cap = ws.act_rows * ws.F; break;
    case TRK_WS_ACTS: src = ws.acts; cap = ws.act_rows * (ws.F / 16) * 4; break;
    case TRK_WS_BARRIER_ERR: src = ws.counters + 2; cap = 4; break;
    case TRK_WS_SHLOGIT: src = ws.shl; cap = M * 4; break;
    case TRK_WS_MIXED: src = ws.xn; cap = M * ws.H * 4; break;
    default: return fail(TRK_E_INVALID, "unknown workspace buffer %d", which);
    }
    if (bytes > cap) return fail(TRK_E_INVALID, "read of %zu bytes above the buffer's %zu", bytes, cap);
    HIP_TRY(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return TRK_OK;
}

// ---- kernel-level entry points --------------------------------------------------------------

extern "C" int trk_router_logits(const float* router, const float* bias, const float* shexp_gate, const float* x,
                                 uint32_t m, uint32_t n_expert, uint32_t hidden, int gemm_order, float* rlog, float* sh,
                                 void* stream) {
    if (!x || (n_expert && (!router || !rlog)) || (shexp_gate && !sh)) return fail(TRK_E_INVALID, "null argument");
    if (hidden == 0 || hidden % 16) return fail(TRK_E_INVALID, "hidden (%u) must be a positive multiple of 16", hidden);
    if (m == 0) return TRK_OK;
    HIP_TRY(launch_router_logits(router, bias, shexp_gate, x, m, n_expert, hidden, gemm_order, rlog, sh,
                                 (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_route(const float* logits, uint32_t m, uint32_t n_expert, uint32_t k, const trk_moe_policy* p,
                         uint32_t* ids, float* w, uint32_t* n_sel, void* stream) {
    if (!logits || !ids || !w || !n_sel) return fail(TRK_E_INVALID, "null argument");
    if (n_expert == 0 || n_expert > 1024) return fail(TRK_E_INVALID, "n_expert (%u) must be in 1..1024", n_expert);
    Policy pol{0, 0, 0, 0, 0.0f};
    if (p) {
        if (p->min < 1 || p->min > p->max)
            return fail(TRK_E_POLICY, "moe policy: need 1 <= min (%u) <= max (%u)", p->min, p->max);
        if (p->max > TRK_MOE_K_MAX || p->max > n_expert)
            return fail(TRK_E_POLICY, "moe policy: max (%u) above the limit (%u)", p->max,
                        std::min<uint32_t>(TRK_MOE_K_MAX, n_expert));
        if (!(p->mass > 0.0f) || p->mass != p->mass)
            return fail(TRK_E_POLICY, "moe policy: target mass (%g) must be positive", (double)p->mass);
        pol = Policy{1, p->min, p->max, p->basis, p->mass, 0};
    } else if (k < 1 || k > TRK_MOE_K_MAX || k > n_expert) {
        return fail(TRK_E_INVALID, "k (%u) must be in 1..min(32, n_expert)", k);
    }
    if (m == 0) return TRK_OK;
    HIP_TRY(launch_route(logits, m, n_expert, k, pol, ids, w, n_sel, nullptr, (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_quantize(const float* x, uint32_t m, uint32_t k, uint32_t kb, int pair, int8_t* q, float* scale,
                            int32_t* sum, void* stream) {
    // QAct::zeros asserts kb in {16, 32} and k % kb == 0 (quant.rs:68-71)
    if (!x || !q || !scale || !sum) return fail(TRK_E_INVALID, "null argument");
    if (!(kb == 16 || kb == 32) || k == 0 || k % kb) return fail(TRK_E_INVALID, "need kb in {16,32} and k %% kb == 0");
    if ((uintptr_t)x % 16 || k % 4) return fail(TRK_E_INVALID, "x must be 16-byte aligned");
    if (pair && m != 1) return fail(TRK_E_INVALID, "pair quantisation takes one row");
    if (m == 0) return TRK_OK;
    HIP_TRY(launch_quantize(x, m, k, kb, pair, q, scale, sum, nullptr, (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_gemv(const trk_mat* w, uint32_t item, uint32_t s0, uint32_t s1, uint32_t kb, const int8_t* q,
                        const float* scale, const int32_t* sum, uint32_t m, int pair, float* y, uint32_t ldy,
                        const uint32_t* rows, int accumulate, void* stream) {
    if (!w || !q || !scale || !sum || !y) return fail(TRK_E_INVALID, "null argument");
    if (!w->ptr || w->k == 0 || w->rows == 0) return fail(TRK_E_INVALID, "bad matrix");
    const bool tq = fmt_is_tq(w->fmt);
    uint64_t pitch, mbytes;  // row (GGUF) or strip (TQ) bytes, matrix bytes
    if (tq) {
        // gemv_tq_rows asserts xq.kb == c.kb (gemv.rs:27); blocks never straddle k
        if (kb != tq_kb(w->fmt)) return fail(TRK_E_INVALID, "kb %u differs from the codec's %u", kb, tq_kb(w->fmt));
        if (w->k % kb) return fail(TRK_E_INVALID, "k %u is not a multiple of kb %u", w->k, kb);
        // the block readers take 16-byte pieces; every codec's block is a multiple of 16 bytes
        if ((uintptr_t)w->ptr % 16 || (w->count > 1 && w->stride % 16))
            return fail(TRK_E_INVALID, "TQ matrix pointer/stride must be 16-byte aligned");
        pitch = (uint64_t)(w->k / kb) * tq_block_bytes(w->fmt);
        mbytes = pitch * ((w->rows + 15) / 16);
    } else {
        const bool ok = ((w->fmt == TRK_FMT_Q4_K || w->fmt == TRK_FMT_Q8_0 || w->fmt == TRK_FMT_Q5_1) && (kb == 32 || kb == 16)) ||
                        (w->fmt == TRK_FMT_Q6_K && kb == 16);
        if (!ok) return fail(TRK_E_INVALID, "unsupported (fmt %u, kb %u)", w->fmt, kb);
        if (w->k % 256) return fail(TRK_E_INVALID, "k %u is not a multiple of 256", w->k);
        const uint32_t al = w->fmt == TRK_FMT_Q6_K ? 2 : 16;
        if ((uintptr_t)w->ptr % al || (w->count > 1 && w->stride % al)) return fail(TRK_E_INVALID, "matrix misaligned");
        pitch = row_bytes(w->fmt, w->k);
        mbytes = pitch * w->rows;
    }
    if (item >= (w->count ? w->count : 1)) return fail(TRK_E_INVALID, "item %u out of range", item);
    if (w->count > 1 && w->stride < mbytes) return fail(TRK_E_INVALID, "stride below the matrix size");
    const uint32_t strips = (w->rows + 15) / 16;
    if (s0 > s1 || s1 > strips) return fail(TRK_E_INVALID, "strips [%u, %u) outside [0, %u)", s0, s1, strips);
    if (pair && m % 2) return fail(TRK_E_INVALID, "pair rows come in twos");
    if ((uintptr_t)q % 16) return fail(TRK_E_INVALID, "q must be 16-byte aligned");
    const uint32_t r_hi = tq ? 16 * s1 : (16 * s1 < w->rows ? 16 * s1 : w->rows);
    if (ldy < r_hi && !(m == (pair ? 2u : 1u) && !rows)) return fail(TRK_E_INVALID, "ldy %u below row %u", ldy, r_hi);
    if (m == 0 || s0 == s1) return TRK_OK;
    Mat M{(const uint8_t*)w->ptr, w->count > 1 ? w->stride : mbytes, w->rows, w->k, w->fmt, (uint32_t)pitch};
    HIP_TRY(launch_gemv(M, item, s0, s1, kb, q, scale, sum, m, pair, y, ldy, rows, accumulate, (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_swiglu(const float* g, const float* u, float* y, size_t n, void* stream) {
    if (!g || !u || !y) return fail(TRK_E_INVALID, "null argument");
    if (n == 0) return TRK_OK;
    HIP_TRY(launch_swiglu(g, u, y, n, (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_rmsnorm(const float* x, const float* w, float eps, uint32_t m, uint32_t n, float* y, void* stream) {
    if (!x || !y) return fail(TRK_E_INVALID, "null argument");
    if (m == 0 || n == 0) return TRK_OK;
    HIP_TRY(launch_rmsnorm(x, w, eps, m, n, y, (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_add_inplace(float* y, const float* a, size_t n, void* stream) {
    if (!y || !a) return fail(TRK_E_INVALID, "null argument");
    if (n == 0) return TRK_OK;
    HIP_TRY(launch_add(y, a, n, (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_gen_gguf(uint32_t fmt, uint64_t seed, uint64_t stream_id, uint32_t rows, uint32_t k, float dlo,
                            float dhi, void* out, void* stream) {
    if (!out) return fail(TRK_E_INVALID, "null argument");
    if (!(fmt == TRK_FMT_Q4_K || fmt == TRK_FMT_Q6_K || fmt == TRK_FMT_Q8_0 || fmt == TRK_FMT_Q5_1) || k % 256)
        return fail(TRK_E_INVALID, "bad format/k");
    if (rows == 0) return TRK_OK;
    HIP_TRY(launch_gen_gguf(fmt, seed, stream_id, 0, 1, rows, k, dlo, dhi, out, 0, (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_gen_gguf_stack(uint32_t fmt, uint64_t seed, uint64_t stream0, uint64_t stream_step,
                                  uint32_t count, uint32_t rows, uint32_t k, float dlo, float dhi, void* out,
                                  uint64_t stride, void* stream) {
    if (!out) return fail(TRK_E_INVALID, "null argument");
    if (!(fmt == TRK_FMT_Q4_K || fmt == TRK_FMT_Q6_K || fmt == TRK_FMT_Q8_0 || fmt == TRK_FMT_Q5_1) || k % 256)
        return fail(TRK_E_INVALID, "bad format/k");
    const uint64_t mb = (uint64_t)rows * row_bytes(fmt, k);
    if (count > 1 && stride < mb) return fail(TRK_E_INVALID, "stride %llu below matrix bytes %llu",
                                              (unsigned long long)stride, (unsigned long long)mb);
    if (count > 65535) return fail(TRK_E_INVALID, "count (%u) above 65535", count);
    if (rows == 0 || count == 0) return TRK_OK;
    HIP_TRY(launch_gen_gguf(fmt, seed, stream0, stream_step, count, rows, k, dlo, dhi, out, stride,
                            (hipStream_t)stream));
    return TRK_OK;
}

extern "C" int trk_gen_normal(uint64_t seed, uint64_t stream_id, size_t n, double sigma, float* out, void* stream) {
    if (!out) return fail(TRK_E_INVALID, "null argument");
    if (n == 0) return TRK_OK;
    HIP_TRY(launch_gen_normal(seed, stream_id, n, sigma, out, (hipStream_t)stream));
    return TRK_OK;
}
