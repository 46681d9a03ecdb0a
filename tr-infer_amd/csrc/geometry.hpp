// Launch geometry and workspace extents of the MoE kernels, as plain host arithmetic (no HIP
// types), shared by the launchers, the workspace sizing of trk_create and a CPU-only check that
// sweeps shapes (tests/geometry_check.cpp).  Every grid a launcher builds and every workspace
// extent a kernel indexes is computed here, so a grid that addresses strips past F or a buffer
// sized below what a dispatch writes shows up on the host, without a GPU.
#pragma once

#include <stdint.h>

namespace trk {
namespace geo {

constexpr uint32_t KMAX = 32;      // router.rs:6 MOE_K_MAX: stride of the per-token id / weight rows
constexpr uint32_t ITEM_ROWS = 16; // rows of a grouped work item (one 16-row MFMA tile)
constexpr uint32_t CHUNK = 64;     // tokens per dispatch chunk (one wave's lane mask)
constexpr uint32_t DN_R = 4;       // output rows per decode down workgroup

struct Caps {  // what trk_create sizes for (m_max rows, k_cap selections per token)
    uint32_t H, E, F, m_max, k_cap;
};

inline uint64_t ent_cap(const Caps& c) { return (uint64_t)c.m_max * c.k_cap; }
// work items: every non-empty expert's entries in items of <= 16 rows (at most E + entries / 16 of
// them), then the shared expert's tokens in items of <= 16
inline uint64_t item_cap(const Caps& c) {
    return c.E + (ent_cap(c) + ITEM_ROWS - 1) / ITEM_ROWS + (c.m_max + ITEM_ROWS - 1) / ITEM_ROWS + 1;
}
inline uint64_t items_max(uint32_t E, uint32_t m, uint32_t kcap) {
    const uint64_t ent = (uint64_t)m * kcap;
    const uint64_t nonempty = ent < E ? ent : E;
    return nonempty + ent / ITEM_ROWS + (m + ITEM_ROWS - 1) / ITEM_ROWS;
}
// activation rows of the down input: one per entry and one per token (shared), the decode slots
// (K_MAX routed + the shared one, two levels each), and a TQ batch of up to 16 tokens run as
// per-token decodes (k_cap + 1 slots of two rows per token)
inline uint64_t act_rows(const Caps& c) {
    const uint64_t a = ent_cap(c) + c.m_max, d = (uint64_t)(KMAX + 1) * 2;
    const uint64_t t = 2ull * (c.m_max < 16 ? c.m_max : 16) * (c.k_cap + 1);
    const uint64_t ad = a > d ? a : d;
    return ad > t ? ad : t;
}
inline uint64_t yent_rows(const Caps& c) { return ent_cap(c) + c.m_max; }
// dispatch chunks of 64 tokens, and the per-(chunk, expert) offsets the split dispatch writes
inline uint32_t chunks(uint32_t m) { return (m + CHUNK - 1) / CHUNK; }
inline uint64_t doff_elems(uint32_t m, uint32_t E) { return (uint64_t)chunks(m) * E; }
inline bool dispatch_split(uint32_t m) { return m >= 256; }

// MFMA gate/up: grid.x column blocks of F / 16 / grid.x strips, four waves taking every fourth.
// A wave's strips run one after another, so with few items (one or two rounds of workgroups on
// the GPU) the kernel time is a wave's chain of strips: 128-wide blocks below 2048 rows (M = 512:
// gate/up 210 -> 197 us), 256-wide from 2048 (config 4: 507 against 512 us with 128), 64-wide for
// small batches.
inline uint32_t mfma_gateup_cols(uint32_t m, uint32_t F) {
    return m >= 2048 && F % 256 == 0 ? F / 256 : m >= 64 && F % 128 == 0 ? F / 128 : F / 64;
}
inline uint32_t mfma_gateup_strips(uint32_t m, uint32_t F) { return F / 16 / mfma_gateup_cols(m, F); }
// MFMA gate/up over item pairs from 2048 rows: two items of one expert run as one 32-row tile
// (v_mfma_i32_32x32x32_i8) in a workgroup of eight waves, each taking every eighth strip of the
// column block.  The pair's activations and scales take 40 H bytes of LDS, which leaves room for
// two workgroups per CU up to H = 2048.
inline bool gateup_pairs(uint32_t m, uint32_t H) { return m >= 2048 && H <= 2048; }
inline uint64_t gateup_pair_lds(uint32_t H) { return (uint64_t)H * 40; }
// a pair's workgroup takes 32 strips (four per wave) where F allows: the 80 KB of staged
// activations then serve twice the weights (config 4 gate/up 500 -> 483 us against 16 strips)
inline uint32_t gateup_pair_cols(uint32_t m, uint32_t F) { return F % 512 == 0 ? F / 512 : mfma_gateup_cols(m, F); }
inline uint32_t gateup_pair_strips(uint32_t m, uint32_t F) { return F / 16 / gateup_pair_cols(m, F); }
// MFMA down: grid.x blocks of 256 or 64 output rows, four waves of 16-row strips
inline uint32_t mfma_down_cols(uint32_t m, uint32_t H) { return m >= 64 ? H / 256 : H / 64; }
inline uint32_t mfma_down_rows(uint32_t m, uint32_t H) { return H / mfma_down_cols(m, H); }
// MFMA down over item pairs (two items of one expert share each weight load, unpack and scale
// decode) from 256 rows: config 4's Q6_K down 457 -> 416 us, M = 512's Q4_K down 123 -> 120 us
inline bool down_pairs(uint32_t m) { return m >= 256; }
// streaming down: 4 waves of 64 / (2 NSB) units of 2 NSB lanes (half a superblock each)
inline uint32_t stream_down_rows_per_wg(uint32_t F) { return 4 * (64 / (2 * (F / 256))); }
inline uint32_t stream_down_cols(uint32_t H, uint32_t F) {
    const uint32_t r = stream_down_rows_per_wg(F);
    return (H + r - 1) / r;
}
// decode: gate/up (F / 16 strips, kcap + 1 slots), down H / 4 workgroups
inline uint32_t decode_gateup_strips(uint32_t F) { return F / 16; }
inline uint32_t decode_down_wgs(uint32_t H) { return H / DN_R; }

// TQ layer (k_tq.hip): gate/up strips of 16 over F twice (gate, up), down strips of 16 over H;
// grid.y: the decode slots (kcap + 1) or the work items
inline uint32_t tq_gateup_tiles(uint32_t F) { return 2 * F / 16; }
inline uint32_t tq_down_tiles(uint32_t H) { return H / 16; }

// Every invariant a call of m rows with kcap selections per token relies on; returns nullptr when
// they hold, else what failed.  tq: the experts are TQ strips (k_tq.hip), not GGUF superblocks.
inline const char* check_call(const Caps& c, uint32_t m, uint32_t kcap, bool tq = false) {
    if (c.H == 0 || c.H % 256) return "H must be a multiple of 256";
    if (c.F == 0 || c.F % (tq ? 16 : 256)) return tq ? "F must be a multiple of 16" : "F must be a multiple of 256";
    if (m == 0 || m > c.m_max) return "m outside 1..m_max";
    if (kcap == 0 || kcap > c.k_cap || kcap > KMAX) return "kcap outside 1..k_cap";
    if ((uint64_t)m * kcap > ent_cap(c)) return "entries above the entry capacity";
    if (items_max(c.E, m, kcap) > item_cap(c)) return "work items above the item capacity";
    if ((uint64_t)m * kcap + m > act_rows(c) || (uint64_t)m * kcap + m > yent_rows(c))
        return "activation rows above capacity";
    if (doff_elems(m, c.E) > doff_elems(c.m_max, c.E)) return "dispatch offsets above capacity";
    if (tq) {
        if (tq_gateup_tiles(c.F) * 16 != 2 * c.F || tq_down_tiles(c.H) * 16 != c.H) return "TQ strips do not tile F / H";
        // decode: slots 0..kcap (the shared one last) in h / yent rows and in the [33][2] act rows
        if (m == 1 && ((uint64_t)kcap + 1 > yent_rows(c) || (uint64_t)(KMAX + 1) * 2 > act_rows(c)))
            return "decode slots above capacity";
        return nullptr;
    }
    {  // MFMA gate/up: the column blocks tile F's strips exactly, four waves each
        const uint32_t cols = mfma_gateup_cols(m, c.F), s = mfma_gateup_strips(m, c.F);
        if (cols == 0 || cols * s * 16 != c.F || s % 4) return "MFMA gate/up grid does not tile F";
        // the pairs' workgroups: eight waves over the block's strips (the launcher runs every item
        // on the 16-row path otherwise), and two workgroups' LDS per CU
        if (gateup_pairs(m, c.H) && gateup_pair_strips(m, c.F) % 8 == 0 && 2 * gateup_pair_lds(c.H) > 160 * 1024)
            return "MFMA gate/up pair LDS above 80 KiB";
    }
    {  // MFMA down: the row blocks tile H exactly, 16-row strips over four waves
        const uint32_t cols = mfma_down_cols(m, c.H), r = mfma_down_rows(m, c.H);
        if (cols == 0 || cols * r != c.H || r % 64) return "MFMA down grid does not tile H";
    }
    {  // streaming down: the row blocks cover H (the kernel guards rows past H)
        const uint32_t r = stream_down_rows_per_wg(c.F);
        if (r == 0 || (uint64_t)stream_down_cols(c.H, c.F) * r < c.H) return "stream down grid does not cover H";
    }
    if (m == 1) {  // decode: slots 0..kcap-1 and the shared slot, strips of F, rows of H
        if (decode_gateup_strips(c.F) * 16 != c.F) return "decode gate/up strips do not tile F";
        if (decode_down_wgs(c.H) * DN_R != c.H) return "decode down workgroups do not tile H";
        if ((uint64_t)(KMAX + 1) * 2 > act_rows(c)) return "decode activation slots above capacity";
    }
    return nullptr;
}

}  // namespace geo
}  // namespace trk
