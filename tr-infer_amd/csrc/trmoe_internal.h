// Internal interfaces between the C ABI (abi.cpp) and the kernel translation units (*.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/trmoe.h"
#include "geometry.hpp"

namespace trk {

constexpr int K_MAX = TRK_MOE_K_MAX;

// Routing policy as the kernels take it (enabled == 0: fixed top-k).  packed: n_expert_packed of a
// subset pack, the routed ids are folded onto experts 0 .. packed - 1 (fold_ids); 0: no folding.
struct Policy {
    uint32_t enabled, min, max, basis;
    float mass;
    uint32_t packed;
};

// TQ codecs (codec.rs:1-46): fmt = bits << 8 | kb
__host__ __device__ inline bool fmt_is_tq(uint32_t fmt) {
    return fmt == TRK_FMT_TQ4_16 || fmt == TRK_FMT_TQ4_32 || fmt == TRK_FMT_TQ5_16 || fmt == TRK_FMT_TQ5_32 ||
           fmt == TRK_FMT_TQ8_16 || fmt == TRK_FMT_TQ8_32;
}
__host__ __device__ inline uint32_t tq_bits(uint32_t fmt) { return fmt >> 8; }
__host__ __device__ inline uint32_t tq_kb(uint32_t fmt) { return fmt & 0xff; }
// Codec::block_bytes: a 64-byte header (d[16], m[16] f16), 16 x kb q values, 5-bit: 2 kb plane bytes
__host__ __device__ inline uint32_t tq_block_bytes(uint32_t fmt) {
    const uint32_t b = tq_bits(fmt), kb = tq_kb(fmt);
    return 64 + (b == 8 ? 16 * kb : 8 * kb) + (b == 5 ? 2 * kb : 0);
}

// A weight stack as the kernels take it.  With tiles (a pack written for T tiles), rows / k are one
// tile's shape and tile t's stack starts at ptr + t * tile_stride; gate/up strip s of the full
// F rows is strip s % tile_strips of tile s / tile_strips.
struct Mat {
    const uint8_t* ptr;
    uint64_t stride;  // bytes between experts
    uint32_t rows, k, fmt;
    uint32_t row_bytes;     // a GGUF row or a TQ strip (of one tile's matrix)
    uint64_t tile_stride;   // 0: one tile
    uint32_t tile_strips;   // strips of one tile's rows
};

// Strip `strip` (16 rows, counted over all tiles' rows) of expert e.
__host__ __device__ inline const uint8_t* mat_strip(const Mat& M, uint32_t e, uint32_t strip) {
    if (M.tile_stride) {
        const uint32_t t = strip / M.tile_strips, s = strip % M.tile_strips;
        return M.ptr + (size_t)t * M.tile_stride + (size_t)e * M.stride + (size_t)s * M.row_bytes;
    }
    return M.ptr + (size_t)e * M.stride + (size_t)strip * M.row_bytes;
}
// Expert e of tile t (a down stack split by columns: each tile a [rows][k] matrix of its own).
__host__ __device__ inline const uint8_t* mat_tile(const Mat& M, uint32_t e, uint32_t t) {
    return M.ptr + (size_t)t * M.tile_stride + (size_t)e * M.stride;
}

// Grouped-GEMM work item: `nrows` entry rows starting at `row0` of the sorted entries, all of
// expert `expert` (expert == 0xffffffff: the shared expert, rows are tokens); `part` is the item's
// index among its expert's items (row0 = the expert's first entry + 16 part).
struct Item {
    uint32_t expert, row0, nrows, part;
};
constexpr uint32_t BR = 16;                  // most entry rows of an item: one 16-row MFMA tile
constexpr uint32_t NO_EXPERT = 0xffffffffu;  // Item::expert of the shared expert's items

// Device workspace (sized at trk_create).
// grid barrier of the one-launch decode layer: workgroups arrive on BAR_GROUPS counters, BAR_LINE
// u32 words apart
constexpr uint32_t BAR_GROUPS = 32;
constexpr uint32_t BAR_LINE = 64;

struct Workspace {
    uint32_t H, E, F, m_max, k_cap, ent_cap, item_cap;
    uint32_t tiles;       // T of a pack written for T tiles (1: one)
    int8_t* xq;           // [max(2, m_max)][H]
    float* xs;            // [max(2, m_max)][H/32]
    int32_t* xsum;
    float* xu;            // [max(2, m_max)][H/32]: scale * (float)sum, the epilogue's u term
    float* xn;            // [m_max][H]: normed input (config-5 layers)
    float* rlog;          // [m_max][E]
    float* shl;           // [m_max]: shared-gate logits
    uint32_t* ids;        // [m_max][32]
    float* w;             // [m_max][32]
    uint32_t* n_sel;      // [m_max]
    uint32_t* ent_tok;    // [ent_cap]
    float* ent_w;
    uint32_t* ent_exp;
    uint32_t* ent_of;     // [m_max][32]: entry index of (token, slot)
    uint32_t* grp_start;  // [E + 2]
    uint32_t* grp_exp;    // [E + 1]
    uint32_t* n_groups;   // [8]: n_groups, n_ent, n_items, pad, n_pairs, n_single, pad, pad
    uint32_t* doff;       // dispatch: [ceil(m_max / 64)][E] first entry of each (64-token chunk, expert)
    Item* items;          // [item_cap]
    uint32_t* pairs;      // [item_cap / 2 + 1]: first item of each pair (parts 2j, 2j + 1 of one expert)
    uint32_t* single;     // [item_cap]: the items in no pair (an expert's last when its count is odd)
    int8_t* actq;         // [act_rows][F] (decode: [kcap + 1][P][F], the shared expert's slot last)
    float* acts;          // [act_rows][F/16]
    int32_t* actsum;
    float* actu;          // [act_rows][F/16]: folded scale * (float)sum
    float* yent;          // [tiles][ent_cap + m_max][H] per-entry down outputs (batch), per tile
    size_t yent_tile;     // floats between two tiles' yent blocks
    float* plog;          // [tiles][m_max][E] router partials of a tiled layer
    float* xt;            // [tiles][m_max][H / tiles] x by tile (the router's K-split)
    float* hgu;           // [ent_cap + m_max][2F] gate / up outputs of the TQ layer
    float* out_tmp;       // [m_max][H]
    unsigned long long* stats;  // [2] rows, experts
    unsigned long long* prof;   // [33] router-mass profile: fixed-point sums per k, then the row count
    uint32_t* counters;   // [BAR_LINE * (BAR_GROUPS + 2)]: grid-barrier words (k_decode.hip): [0..1] top
                          // counter, [2] time-out flag, group g's counter and release word at BAR_LINE * (1 + g)
    size_t act_rows;
};

// ---- launchers (return hipError_t of the launch) ----
hipError_t launch_quantize(const float* x, uint32_t m, uint32_t k, uint32_t kb, int pair, int8_t* q, float* s,
                           int32_t* su, float* u, hipStream_t st);
// x of one row quantised per 32 (pair: coarse + residual) into q [P][H], s / sum / u [P][H/32]
struct XQuant {
    int8_t* q;
    float* s;
    int32_t* sum;
    float* u;  // s * (float)sum
    int pair;
};
// rmsnorm applied to x inside the logits launch (elem.rs:255-262): weights w (null: none), eps
struct XNorm {
    const float* w;
    float eps;
};
hipError_t launch_router_logits(const float* router, const float* bias, const float* shexp_gate, const float* x,
                                uint32_t m, uint32_t E, uint32_t H, int gemm_order, float* rlog, float* sh,
                                hipStream_t st, const XQuant* xquant = nullptr, const XNorm* norm = nullptr);
hipError_t launch_mass_profile(const float* logits, uint32_t m, uint32_t E, unsigned long long* prof,
                               hipStream_t st);
hipError_t launch_route(const float* logits, uint32_t m, uint32_t E, uint32_t k, Policy pol, uint32_t* ids,
                        float* w, uint32_t* n_sel, unsigned long long* stats, hipStream_t st);
hipError_t launch_decode_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const float* x,
                                const float* lg, const Workspace& ws, uint32_t k, Policy pol, int pair, uint32_t kcap,
                                hipStream_t st, uint32_t m = 1);
hipError_t launch_decode_layer(const float* router, const float* bias, const float* shexp_gate, const Mat& gate,
                               const Mat& up, const Mat& down, const Mat& sh_gate, const Mat& sh_up,
                               const Mat& sh_down, const float* x, const float* rlog, const Workspace& ws, uint32_t k,
                               Policy pol, int pair, uint32_t kcap, float* out, int residual, bool check_only,
                               hipStream_t st);
bool decode_layer_supported(const Mat& gate, const Mat& down, const Mat& sh_down, uint32_t E, int pair,
                            uint32_t kcap);
// m >= 2 (pair = 0): m tokens as per-token decode units, each token's rows added in the batch
// combine's order; the routing, x rows and activation slots of token t at t times the decode's
hipError_t launch_decode_down(const Mat& down, const Mat& sh_down, const Workspace& ws, int pair,
                              uint32_t kcap, float* out, int residual, hipStream_t st, uint32_t m = 1);
hipError_t launch_dispatch(const Workspace& ws, uint32_t m, uint32_t kcap, hipStream_t st);
// m <= 16 (m * kcap <= 1024): the same dispatch in one launch with the routing (lg != null) or
// from ws.ids / w / n_sel (lg == null)
hipError_t launch_dispatch_small(const Workspace& ws, uint32_t m, uint32_t kcap, const float* lg, uint32_t k,
                                 Policy pol, hipStream_t st);
// grouped expert products: the MFMA tiles take the items of more than skip_rows rows, the
// streaming GEMV the items of at most max_rows rows
uint32_t grouped_item_rows(const Workspace& ws, uint32_t m);  // grid rows covering every item
hipError_t launch_batch_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up,
                               const Workspace& ws, uint32_t m, uint32_t skip_rows, hipStream_t st);
hipError_t launch_batch_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m,
                             uint32_t skip_rows, hipStream_t st);
hipError_t launch_stream_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up,
                                const Workspace& ws, uint32_t m, uint32_t max_rows, hipStream_t st);
hipError_t launch_stream_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m,
                              uint32_t max_rows, hipStream_t st);
hipError_t launch_batch_combine(const Workspace& ws, uint32_t m, float* out, int residual, hipStream_t st);
// Mat for a TQ matrix: row_bytes holds the bytes of one 16-row strip
hipError_t launch_gemv(const Mat& w, uint32_t item, uint32_t s0, uint32_t s1, uint32_t kb, const int8_t* q,
                       const float* s, const int32_t* su, uint32_t m, int pair, float* y, uint32_t ldy,
                       const uint32_t* rows, int accumulate, hipStream_t st);
// the layer on TQ experts (k_tq.hip): gate/up into h [rows][2F], SwiGLU + quantisation + fold,
// down into yent, and (decode) the slot-order combine
hipError_t launch_tq_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const Workspace& ws,
                            float* h, uint32_t m, uint32_t kcap, int pair, hipStream_t st);
hipError_t launch_tq_act(const Workspace& ws, const float* h, uint32_t m, uint32_t kcap, int pair, hipStream_t st);
hipError_t launch_tq_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m, uint32_t kcap, int pair,
                          hipStream_t st);
hipError_t launch_tq_combine(const Workspace& ws, float* out, int residual, hipStream_t st);
// the K-split router of a tiled layer: x [m][H] -> xt [T][m][H / T]; then the tiles' partial logits
// plog [T][m][E] -> rlog [m][E] summed in tile order, plus the bias (k_basic.hip)
hipError_t launch_tile_split(const float* x, uint32_t m, uint32_t H, uint32_t T, float* xt, hipStream_t st);
hipError_t launch_tile_reduce(const float* plog, uint32_t m, uint32_t E, uint32_t T, const float* bias, float* rlog,
                              hipStream_t st);
// the TQ layer's expert products on int8 MFMA (k_tqm.hip): gate/up + SwiGLU + quantisation + fold,
// and down into yent; tqm_fits: the shapes whose staged activations fit a workgroup's LDS
// lg != null at m = 1: the decode routing (top-k or mass policy) runs inside the launch; at m >= 2
// (pair = 0, tqd_gateup_ok, tqd_tokens_fit): every token runs as such a decode (lg [m][E])
hipError_t launch_tqm_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const Workspace& ws,
                             uint32_t m, uint32_t kcap, int pair, const float* lg, uint32_t k, Policy pol,
                             hipStream_t st);
// decode down and combine in one launch (k_tqm.hip) where the shape allows (tqd_dc_ok): out (+)= the
// slots' down rows in slot order, no per-slot rows in yent.  m >= 2 (pair = 0, tqd_tokens_fit): m
// tokens as per-token decodes, each token's rows in the batch combine's order
bool tqd_dc_ok(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t kcap);
hipError_t launch_tqd_down_combine(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t kcap, int pair,
                                   float* out, int residual, hipStream_t st, uint32_t m = 1);
// the decode gate/up from LDS copies of the strips takes this layer's shape; m tokens' decode
// slots (two activation rows each) fit the workspace
bool tqd_gateup_ok(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const Workspace& ws,
                   const Policy& pol);
bool tqd_tokens_fit(const Workspace& ws, uint32_t m, uint32_t kcap);
hipError_t launch_tqm_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m, uint32_t kcap, int pair,
                           hipStream_t st);
inline bool tqm_fits(uint32_t H, uint32_t F) {
    const size_t gu = (size_t)(H / 32) * 64 * 8 + (size_t)(H / 32) * 16 * 16;
    const size_t dn = (size_t)(F / 32) * 64 * 8 + (size_t)(F / 16) * 16 * 16;
    return H % 64 == 0 && F % 32 == 0 && gu + 1024 * 4 <= 64 * 1024 && dn <= 64 * 1024;
}
// the hyper-connection mix part B (k_tqm.hip): mixed [m][hh] from xn [m][hc][hh] and lo [m][lr]; a
// batch quantises lo first into an operand image of hc_image_bytes in ws.yent (free until the down
// stage): 704 bytes per 16-token tile and 32-wide block
inline size_t hc_image_bytes(uint32_t m, uint32_t lr) { return (size_t)(m + 15) / 16 * 22 * lr; }
hipError_t launch_hc_mix(const Mat& up, uint32_t hc, uint32_t hh, uint32_t lr, const float* xn, const float* lo,
                         uint32_t m, int pair, const Workspace& ws, float* mixed, hipStream_t st);
hipError_t launch_swiglu(const float* g, const float* u, float* y, size_t n, hipStream_t st);
hipError_t launch_rmsnorm(const float* x, const float* w, float eps, uint32_t m, uint32_t n, float* y,
                          hipStream_t st);
hipError_t launch_add(float* y, const float* a, size_t n, hipStream_t st);
hipError_t launch_gen_gguf(uint32_t fmt, uint64_t seed, uint64_t stream0, uint64_t step, uint32_t count,
                           uint32_t rows, uint32_t k, float dlo, float dhi, void* out, uint64_t stride,
                           hipStream_t st);
hipError_t launch_gen_normal(uint64_t seed, uint64_t stream_id, size_t n, double sigma, float* out,
                             hipStream_t st);

}  // namespace trk
