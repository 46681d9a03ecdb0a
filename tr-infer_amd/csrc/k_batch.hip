// Batch path (M >= 2): Model::moe_batch (crates/tr-model/src/exec_batch.rs:1404-1580).
//
//   dispatch: the stable sort of (token, slot) entries by expert (exec_batch.rs:1428-1462) as a
//             histogram + exclusive scan + rank-within-expert scatter (ranks from per-wave token
//             bitmaps, so the order is the reference's token-major order), plus the compressed
//             group table and the grouped-GEMM work list.
//   gate/up:  per work item (an expert and up to BR of its entry rows, or up to BR tokens of the
//             shared expert) and 16-row strip of F: int8 MFMA per 32-block, the reference's
//             per-block f32 epilogue per output in registers; SwiGLU, the per-16 requantisation
//             and the weight fold follow in the same workgroup.
//   down:     per work item and 64-row strip of H, int8 MFMA per 16-block: per-entry outputs
//             into yent.
//   combine:  per token, shared row first, then its entries in ascending expert order (the
//             reference's overwrite-then-accumulate order, exec_batch.rs:1539-1561).
#include "common.hpp"
#include "gemv.hpp"
#include "route.hpp"

#include <type_traits>

namespace trk {

constexpr uint32_t DISPATCH_WAVES = 8;

__device__ __forceinline__ uint32_t popc64(unsigned long long v) { return (uint32_t)__popcll(v); }

// A token's selected experts: the first ceil(kcap / 4) 16-byte pieces of its id row, all requested
// at once; returns n_sel.
__device__ __forceinline__ uint32_t load_ids(const Workspace& ws, uint32_t t, uint32_t kc4, uint32_t (&id)[K_MAX]) {
    const uint32_t ns = ws.n_sel[t];
#pragma unroll
    for (uint32_t q = 0; q < K_MAX / 4; q++)
        if (q < kc4) {
            const uint4 v = reinterpret_cast<const uint4*>(ws.ids + (size_t)t * K_MAX)[q];
            id[4 * q] = v.x; id[4 * q + 1] = v.y; id[4 * q + 2] = v.z; id[4 * q + 3] = v.w;
        }
    return ns;
}

// Single workgroup of DISPATCH_WAVES waves, one token per thread per round of DT tokens (ids and
// weights stay in registers).  Per round each wave ORs its 64 tokens into a per-(wave, expert) lane
// mask, so a token's rank within its expert is the popcount of the lower lanes' bits plus the
// counts of the earlier waves and rounds: the reference's token-major order.  Expert starts,
// group indices and work-item offsets come from one block-wide scan (a DPP scan per wave, then
// the wave totals).  kc4 = ceil(largest selection / 4).
constexpr uint32_t DT = DISPATCH_WAVES * 64;  // tokens per round
// split: leave the scatter to scatter_kernel (many workgroups) and store the per-(64-token chunk,
// expert) first positions in ws.doff instead: pass 1 stores each chunk's counts there, and one
// prefix per expert over the chunks turns them into positions (no second pass over the tokens).
__global__ __launch_bounds__(DISPATCH_WAVES * 64) void dispatch_kernel(Workspace ws, uint32_t m, uint32_t kc4,
                                                                       int split) {
    const uint32_t E = ws.E, tid = threadIdx.x;
    const uint32_t wv = tid / 64, lane = tid % 64;
    extern __shared__ __align__(16) uint8_t smem[];
    unsigned long long* masks = reinterpret_cast<unsigned long long*>(smem);  // [W][E]
    uint32_t* cnt = reinterpret_cast<uint32_t*>(masks + DISPATCH_WAVES * E);  // [E]
    uint32_t* run = cnt + E;                                                  // [E]
    uint32_t* off = run + E;                                                  // [W][E]
    uint32_t* wtot = off + DISPATCH_WAVES * E;                                // [W][5]
    const uint32_t rounds = (m + DT - 1) / DT, nchunks = (m + 63) / 64;
    const uint32_t ept = (E + DT - 1) / DT;  // experts per thread in the scans (contiguous)

    uint32_t id[K_MAX], ns = 0;
    float wt[K_MAX];
    auto load_tok = [&](uint32_t r) {
        const uint32_t t = r * DT + tid;
        ns = t < m ? load_ids(ws, t, kc4, id) : 0u;
        if (t < m) {
#pragma unroll
            for (uint32_t q = 0; q < K_MAX / 4; q++)
                if (q < kc4) {
                    const float4 v = reinterpret_cast<const float4*>(ws.w + (size_t)t * K_MAX)[q];
                    wt[4 * q] = v.x; wt[4 * q + 1] = v.y; wt[4 * q + 2] = v.z; wt[4 * q + 3] = v.w;
                }
        }
    };
    auto build_masks = [&]() {  // ends with the masks complete
        for (uint32_t i = tid; i < DISPATCH_WAVES * E; i += DT) masks[i] = 0ull;
        __syncthreads();
        uint32_t* mw = reinterpret_cast<uint32_t*>(masks + wv * E);
#pragma unroll
        for (uint32_t s = 0; s < K_MAX; s++)
            if (s < ns) atomicOr(&mw[id[s] * 2 + (lane >> 5)], 1u << (lane & 31));
        __syncthreads();
    };

    // pass 1: per-expert counts
    for (uint32_t e = tid; e < E; e += DT) cnt[e] = 0;
    for (uint32_t r = 0; r < rounds; r++) {
        load_tok(r);
        build_masks();
        for (uint32_t e = tid; e < E; e += DT) {
            uint32_t c = cnt[e];
            for (uint32_t w = 0; w < DISPATCH_WAVES; w++) {
                const uint32_t pc = popc64(masks[w * E + e]);
                const uint32_t ch = r * DISPATCH_WAVES + w;  // 64-token chunk
                if (split && rounds > 1 && ch < nchunks) ws.doff[(size_t)ch * E + e] = pc;  // its count, for now
                c += pc;
            }
            cnt[e] = c;
        }
        if (rounds > 1) __syncthreads();
    }
    __syncthreads();

    // block-wide exclusive scans of (entries, non-empty, items, item pairs, unpaired items) over the
    // experts
    uint32_t loc[5] = {0, 0, 0, 0, 0};
    for (uint32_t i = 0; i < ept; i++) {
        const uint32_t e = tid * ept + i;
        const uint32_t c = e < E ? cnt[e] : 0u, nc = (c + BR - 1) / BR;
        loc[0] += c;
        loc[1] += c ? 1u : 0u;
        loc[2] += nc;
        loc[3] += nc / 2;
        loc[4] += nc % 2;
    }
    uint32_t inc[5];
#pragma unroll
    for (int v = 0; v < 5; v++) {
        inc[v] = wave_incl_scan_u32(loc[v]);
        if (lane == 63) wtot[wv * 5 + v] = inc[v];
    }
    __syncthreads();
    uint32_t base[5] = {0, 0, 0, 0, 0}, tot[5] = {0, 0, 0, 0, 0};
    for (uint32_t w = 0; w < DISPATCH_WAVES; w++)
#pragma unroll
        for (int v = 0; v < 5; v++) {
            const uint32_t x = wtot[w * 5 + v];
            if (w < wv) base[v] += x;
            tot[v] += x;
        }
    const uint32_t n_ent = tot[0], ng = tot[1], n_routed_items = tot[2];
    {
        uint32_t st = base[0] + inc[0] - loc[0], gi = base[1] + inc[1] - loc[1], it = base[2] + inc[2] - loc[2];
        uint32_t pi = base[3] + inc[3] - loc[3], si = base[4] + inc[4] - loc[4];
        for (uint32_t i = 0; i < ept; i++) {
            const uint32_t e = tid * ept + i;
            if (e >= E) break;
            const uint32_t c = cnt[e], nc = (c + BR - 1) / BR;
            run[e] = st;
            if (c) {  // group table: non-empty experts ascending; work items of BR rows
                ws.grp_start[gi] = st;
                ws.grp_exp[gi] = e;
                for (uint32_t q = 0; q < nc; q++) {
                    const uint32_t nr = c - q * BR < BR ? c - q * BR : BR;
                    ws.items[it + q] = Item{e, st + q * BR, nr, q};
                }
                for (uint32_t q = 0; q < nc / 2; q++) ws.pairs[pi + q] = it + 2 * q;
                if (nc % 2) ws.single[si] = it + nc - 1;
            }
            st += c;
            gi += c ? 1u : 0u;
            it += nc;
            pi += nc / 2;
            si += nc % 2;
        }
    }
    const uint32_t n_sh = (m + BR - 1) / BR;  // the shared expert over the tokens, last
    for (uint32_t q = tid; q < n_sh; q += DT) {
        const uint32_t r0 = q * BR;
        ws.items[n_routed_items + q] = Item{NO_EXPERT, r0, m - r0 < BR ? m - r0 : BR, q};
        if (q % 2 == 0 && q + 1 < n_sh) ws.pairs[tot[3] + q / 2] = n_routed_items + q;
        if (q % 2 == 0 && q + 1 == n_sh) ws.single[tot[4]] = n_routed_items + q;
    }
    if (tid == 0) {
        if (ws.stats) {  // MoeStats: rows and selected experts of this call
            atomicAdd(&ws.stats[0], (unsigned long long)m);
            atomicAdd(&ws.stats[1], (unsigned long long)n_ent);
        }
        ws.grp_start[ng] = n_ent;
        ws.n_groups[0] = ng;
        ws.n_groups[1] = n_ent;
        ws.n_groups[2] = n_routed_items + n_sh;
        ws.n_groups[4] = tot[3] + n_sh / 2;
        ws.n_groups[5] = tot[4] + n_sh % 2;
    }
    __syncthreads();

    if (split && rounds == 1) {  // one round: the chunk counts are the masks still in LDS
        for (uint32_t e = tid; e < E; e += DT) {
            uint32_t o = run[e];
            for (uint32_t w = 0; w < DISPATCH_WAVES && w < nchunks; w++) {
                ws.doff[(size_t)w * E + e] = o;
                o += popc64(masks[w * E + e]);
            }
        }
        return;
    }
    if (split) {  // the chunk counts become each chunk's first position per expert
        for (uint32_t e = tid; e < E; e += DT) {
            uint32_t o = run[e];
            for (uint32_t ch0 = 0; ch0 < nchunks; ch0 += 16) {  // 16 counts requested at once
                uint32_t c[16];
#pragma unroll
                for (int j = 0; j < 16; j++) c[j] = ch0 + j < nchunks ? ws.doff[(size_t)(ch0 + j) * E + e] : 0u;
#pragma unroll
                for (int j = 0; j < 16; j++)
                    if (ch0 + j < nchunks) {
                        ws.doff[(size_t)(ch0 + j) * E + e] = o;
                        o += c[j];
                    }
            }
        }
        return;
    }
    // pass 2: scatter (the single-round case reuses the masks and the registers of pass 1)
    const unsigned long long below = lane ? ((1ull << lane) - 1ull) : 0ull;
    for (uint32_t r = 0; r < rounds; r++) {
        if (rounds > 1) {
            load_tok(r);
            build_masks();
        }
        for (uint32_t e = tid; e < E; e += DT) {
            uint32_t o = run[e];
            for (uint32_t w = 0; w < DISPATCH_WAVES; w++) {
                off[w * E + e] = o;
                o += popc64(masks[w * E + e]);
            }
            run[e] = o;
        }
        __syncthreads();
        const uint32_t t = r * DT + tid;
#pragma unroll
        for (uint32_t s = 0; s < K_MAX; s++)
            if (s < ns) {
                const uint32_t e = id[s];
                const uint32_t pos = off[wv * E + e] + popc64(masks[wv * E + e] & below);
                ws.ent_tok[pos] = t;
                ws.ent_w[pos] = wt[s];
                ws.ent_exp[pos] = e;
                ws.ent_of[(size_t)t * K_MAX + s] = pos;
            }
        if (rounds > 1) __syncthreads();
    }
}

// The scatter of a split dispatch: one wave per 64-token chunk, the same lane-mask ranks.
__global__ __launch_bounds__(64) void scatter_kernel(Workspace ws, uint32_t m, uint32_t kc4) {
    const uint32_t E = ws.E, c = blockIdx.x, lane = threadIdx.x, t = c * 64 + lane;
    extern __shared__ __align__(16) uint8_t smem[];
    unsigned long long* masks = reinterpret_cast<unsigned long long*>(smem);  // [E]
    uint32_t* first = reinterpret_cast<uint32_t*>(masks + E);                // [E] the chunk's first positions
    uint32_t id[K_MAX];
    float wt[K_MAX];
    const uint32_t ns = t < m ? load_ids(ws, t, kc4, id) : 0u;
    if (t < m) {
#pragma unroll
        for (uint32_t q = 0; q < K_MAX / 4; q++)
            if (q < kc4) {
                const float4 v = reinterpret_cast<const float4*>(ws.w + (size_t)t * K_MAX)[q];
                wt[4 * q] = v.x; wt[4 * q + 1] = v.y; wt[4 * q + 2] = v.z; wt[4 * q + 3] = v.w;
            }
    }
    // the chunk's row of first positions, requested together with the ids (one round trip)
    for (uint32_t e0 = 0; e0 < E; e0 += 512) {
        uint32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t e = e0 + lane + 64 * j;
            v[j] = e < E ? ws.doff[(size_t)c * E + e] : 0u;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t e = e0 + lane + 64 * j;
            if (e < E) {
                first[e] = v[j];
                masks[e] = 0ull;
            }
        }
    }
    wave_sync();
    uint32_t* mw = reinterpret_cast<uint32_t*>(masks);
#pragma unroll
    for (uint32_t s = 0; s < K_MAX; s++)
        if (s < ns) atomicOr(&mw[id[s] * 2 + (lane >> 5)], 1u << (lane & 31));
    wave_sync();
    const unsigned long long below = lane ? ((1ull << lane) - 1ull) : 0ull;
#pragma unroll
    for (uint32_t s = 0; s < K_MAX; s++)
        if (s < ns) {
            const uint32_t e = id[s];
            const uint32_t pos = first[e] + popc64(masks[e] & below);
            ws.ent_tok[pos] = t;
            ws.ent_w[pos] = wt[s];
            ws.ent_exp[pos] = e;
            ws.ent_of[(size_t)t * K_MAX + s] = pos;
        }
}

// Routing and dispatch of a batch of at most 16 tokens in one launch (every expert's group then
// fits one work item).  One workgroup of 16 waves: wave t routes token t (route_topk /
// route_mass, router.rs:70-148, as route_kernel does) into ws.ids / w / n_sel; then thread
// (token, slot) ranks its selection's key (expert, token) against every other key, broadcast
// from LDS: the rank is the entry's position in moe_batch's order (experts ascending, tokens
// ascending within one), and the keys of the same expert give its group size.  Group indices
// come from one block scan of the group-start flags over the sorted keys.
constexpr uint32_t SMALL_WAVES = 16;
constexpr uint32_t SMALL_T = SMALL_WAVES * 64;
template <int NJ>
__global__ __launch_bounds__(SMALL_T) void dispatch_small_kernel(Workspace ws, uint32_t m, uint32_t kcap,
                                                               const float* __restrict__ lg, uint32_t k, Policy pol) {
    const uint32_t E = ws.E, tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
    extern __shared__ __align__(16) uint8_t smem[];
    if (lg) {  // route (the scratch below is reused once every wave is past the barrier)
        uint2* cand = reinterpret_cast<uint2*>(smem) + wv * ROUTE_CAND;                           // [16][96]
        float* ex = reinterpret_cast<float*>(smem + SMALL_WAVES * ROUTE_CAND * 8) + (size_t)wv * E;  // [16][E]
        if (wv < m) {
            const uint32_t n = route_row<NJ>(lg + (size_t)wv * E, E, k, pol, lane, cand, ex,
                                             ws.ids + (size_t)wv * K_MAX, ws.w + (size_t)wv * K_MAX);
            if (lane == 0) ws.n_sel[wv] = n;
        }
        __syncthreads();  // orders the routing's global stores before the loads below
    }
    uint32_t* keys = reinterpret_cast<uint32_t*>(smem);  // [SMALL_T] (expert << 16 | token), ~0 = none
    uint32_t* skey = keys + SMALL_T;                     // [SMALL_T] keys in entry order
    float* sw = reinterpret_cast<float*>(skey + SMALL_T);  // [SMALL_T] their routing weights
    uint32_t* scnt = reinterpret_cast<uint32_t*>(sw + SMALL_T);  // [SMALL_T] their group sizes
    uint32_t* wtot = scnt + SMALL_T;                     // [16]
    const uint32_t N = m * kcap, t = tid / kcap, s = tid % kcap;
    // n_sel: lane i of every wave loads token i's (a per-lane vector load, which sees the routing's
    // stores), then the wave sums them and each thread takes its token's by a lane shuffle
    const uint32_t ns_l = lane < m ? ws.n_sel[lane] : 0u;
    const uint32_t n_ent = (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan_u32(ns_l), 63);
    const uint32_t ns_t = (uint32_t)__shfl((int)ns_l, (int)(t < m ? t : 0));
    const bool valid = tid < N && s < ns_t;
    const uint32_t key = valid ? (ws.ids[(size_t)t * K_MAX + s] << 16) | t : 0xffffffffu;
    const float w = valid ? ws.w[(size_t)t * K_MAX + s] : 0.0f;
    keys[tid] = key;
    __syncthreads();
    uint32_t rank = 0, same = 0;
    // only the waves holding selections rank (broadcast LDS reads still cost full bandwidth)
    const uint32_t N16 = wv * 64 < N ? (N + 15) / 16 : 0u;
    for (uint32_t j = 0; j < N16; j++) {  // keys past N are ~0 from the store above (tid >= N)
        uint4 kv[4];
#pragma unroll
        for (int c = 0; c < 4; c++) kv[c] = reinterpret_cast<const uint4*>(keys)[4 * j + c];  // all four in flight
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t ka[4] = {kv[c].x, kv[c].y, kv[c].z, kv[c].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                rank += ka[i] < key ? 1u : 0u;
                same += (ka[i] >> 16) == (key >> 16) ? 1u : 0u;
            }
        }
    }
    if (valid) {
        skey[rank] = key;
        sw[rank] = w;
        scnt[rank] = same;
        ws.ent_of[(size_t)t * K_MAX + s] = rank;
    }
    __syncthreads();
    // entry p = tid: its group starts here when the expert changes
    const uint32_t p = tid;
    const uint32_t kp = p < n_ent ? skey[p] : 0u;
    const bool head = p < n_ent && (p == 0 || (skey[p - 1] >> 16) != (kp >> 16));
    const uint32_t inc = wave_incl_scan_u32(head ? 1u : 0u);
    if (lane == 63) wtot[wv] = inc;
    if (p < n_ent) {
        ws.ent_tok[p] = kp & 0xffffu;
        ws.ent_exp[p] = kp >> 16;
        ws.ent_w[p] = sw[p];
    }
    __syncthreads();
    uint32_t base = 0, ng = 0;
    for (uint32_t v = 0; v < SMALL_WAVES; v++) {
        const uint32_t x = wtot[v];
        base += v < wv ? x : 0u;
        ng += x;
    }
    if (head) {
        const uint32_t g = base + inc - 1, e = kp >> 16;
        ws.grp_start[g] = p;
        ws.grp_exp[g] = e;
        ws.items[g] = Item{e, p, scnt[p], 0};
    }
    if (tid == 0) {
        ws.items[ng] = Item{NO_EXPERT, 0, m, 0};  // the shared expert over the tokens, last
        if (ws.stats) {  // MoeStats: rows and selected experts of this call
            atomicAdd(&ws.stats[0], (unsigned long long)m);
            atomicAdd(&ws.stats[1], (unsigned long long)n_ent);
        }
        ws.grp_start[ng] = n_ent;
        ws.n_groups[0] = ng;
        ws.n_groups[1] = n_ent;
        ws.n_groups[2] = ng + 1;
    }
}

hipError_t launch_dispatch_small(const Workspace& ws, uint32_t m, uint32_t kcap, const float* lg, uint32_t k,
                                 Policy pol, hipStream_t st) {
    const size_t E = ws.E;
    if (m > SMALL_WAVES || m * kcap > SMALL_T || E > 1024) return hipErrorInvalidValue;
    size_t lds = (size_t)SMALL_T * 16 + SMALL_WAVES * 4;
    if (lg) {
        const size_t rl = SMALL_WAVES * ROUTE_CAND * 8 +
                          ((pol.enabled && pol.basis == TRK_BASIS_ALL) ? SMALL_WAVES * E * 4 : 0);
        lds = lds > rl ? lds : rl;
    }
    if (route_nj(ws.E) == 8)
        dispatch_small_kernel<8><<<1, SMALL_T, lds, st>>>(ws, m, kcap, lg, k, pol);
    else
        dispatch_small_kernel<16><<<1, SMALL_T, lds, st>>>(ws, m, kcap, lg, k, pol);
    return hipGetLastError();
}

hipError_t launch_dispatch(const Workspace& ws, uint32_t m, uint32_t kcap, hipStream_t st) {
    const size_t E = ws.E;
    if (E > 2 * DT) return hipErrorInvalidValue;
    const size_t lds = DISPATCH_WAVES * E * 8 + (2 * E + DISPATCH_WAVES * E + DISPATCH_WAVES * 5) * 4;
    // from a few hundred tokens on, one workgroup's scattered stores dominate: spread them
    const int split = geo::dispatch_split(m) ? 1 : 0;
    if (split && geo::doff_elems(m, ws.E) > geo::doff_elems(ws.m_max, ws.E)) return hipErrorInvalidValue;
    dispatch_kernel<<<1, DT, lds, st>>>(ws, m, (kcap + 3) / 4, split);
    if (split) scatter_kernel<<<geo::chunks(m), 64, E * 12, st>>>(ws, m, (kcap + 3) / 4);
    return hipGetLastError();
}

// ---- grouped expert products on int8 MFMA ----------------------------------------------------
//
// v_mfma_i32_16x16x32_i8 with A = 16 entry rows x 32 activation bytes, B = 32 weight values x 16
// weight rows gives, per 32-block, the exact int32 dot of every (entry, weight row) pair in one
// instruction; lane l then holds D[entry 4(l/16) + v][weight row l%16], v = 0..3, and runs the
// reference's per-block f32 epilogue (gemv.rs:141-148) on its four outputs in block order, so
// the result is the same float as the CPU chain.  Operand layouts (lane l, k-group g = l/16):
// A[row l%16][k 8g..8g+7], B[k 8g..8g+7][col l%16], 8 bytes each.

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// 8 bytes of packed Q4_K nibbles -> 8 int8 values of nibble h
__device__ __forceinline__ long unpack8(uint2 p, int h) {
    const uint32_t lo = (p.x >> (4 * h)) & 0x0f0f0f0fu, hi = (p.y >> (4 * h)) & 0x0f0f0f0fu;
    return (long)(((unsigned long long)hi << 32) | lo);
}

// Shared by the two grouped kernels.  A workgroup takes one item (<= 16 entry rows of one expert,
// or <= 16 tokens of the shared expert) and a range of 16-row weight strips, one strip per wave at
// a time.  The item's int8 activations are staged once in LDS in MFMA operand order (block b,
// lane l -> the 8 bytes A[row l%16][k 8(l/16)..]), with their per-block scales; every wave then
// streams its strips' weights straight from HBM into registers, one superblock ahead.  The
// (dd, mm) pairs of a superblock are decoded cooperatively by the wave (each lane a quarter) into
// a per-wave LDS table.

// (dd, mm) of Q4_K sub-block j (runtime) from the header words: blocks.py:16-22 with the byte
// selected by shifts
__device__ __forceinline__ float2 q4k_dm_rt(uint4 hdr, uint32_t j) {
    const uint32_t sh = 8 * (j & 3);
    const uint32_t b1 = (hdr.y >> sh) & 0xffu, b2 = (hdr.z >> sh) & 0xffu, b3 = (hdr.w >> sh) & 0xffu;
    const int sc = j < 4 ? (int)(b1 & 63u) : (int)((b3 & 15u) | ((b1 >> 6) << 4));
    const int mn = j < 4 ? (int)(b2 & 63u) : (int)((b3 >> 4) | ((b2 >> 6) << 4));
    float dd, mm;
    q4k_dm(h2f((uint16_t)(hdr.x & 0xffff)), h2f((uint16_t)(hdr.x >> 16)), sc, mn, dd, mm);
    return make_float2(dd, mm);
}

// Q4_K operands of one superblock for lane (g, r): the header and, per sub-block pair c, the
// 8 qs bytes 32c + 8g .. 32c + 8g + 7 (k-group g of both sub-blocks 2c and 2c+1).
struct Q4Sb {
    uint4 hdr;
    uint2 qs[4];
};
__device__ __forceinline__ void load_q4sb(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t g, Q4Sb& w) {
    const uint8_t* p = rowp + sb * 144;
    w.hdr = *reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int c = 0; c < 4; c++) w.qs[c] = *reinterpret_cast<const uint2*>(p + 16 + 32 * c + 8 * g);
}

__device__ __forceinline__ const Q4Sb& settle(const Q4Sb& w) { return w; }

// ---- gate/up on v_mfma_i32_16x16x64_i8 ------------------------------------------------------
//
// A Q4_K superblock's 128 qs bytes are chunk pairs p = 0, 1 of 64 bytes (sub-blocks 4p .. 4p+3:
// chunk 2p holds 4p / 4p+1 in its low / high nibbles, chunk 2p+1 holds 4p+2 / 4p+3).  Lane (g, r)
// loads the 16 bytes 64p + 16g .. +15 of row r: the four lanes of a row read 64 contiguous bytes
// (one 16-byte load each) instead of four scattered 8-byte pieces.  Its low nibbles are 16 values
// of sub-block 4p + 2 (g / 2), at positions 16 (g % 2) ..; the high nibbles those of the next
// sub-block.  One 64-wide MFMA per sub-block, with the activation operand zero in the lanes of the
// other chunk, gives each 32-block's exact dot on its own: the pairing of A and B elements within
// a lane is all the dot depends on.
typedef int v4i_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4i mfma_i8_64(v4i_t a, v4i_t b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, z, 0, 0, 0);
}
struct Q4Sb16 {
    uint4 hdr;
    v4i_t q[2];  // chunk pair p: bytes 64p + 16g .. +15
};
__device__ __forceinline__ void load_q4sb16(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t g, Q4Sb16& w) {
    const uint8_t* p = rowp + sb * 144;
    w.hdr = *reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int c = 0; c < 2; c++) w.q[c] = *reinterpret_cast<const v4i_t*>(p + 16 + 64 * c + 16 * g);
}
// Activation rows staged as [block][half][row] 16-byte pieces: lane (g, r) reads half g % 2 of a
// block of entry row r.  The row of piece p sits at slot r ^ a16_swz(p) of the piece's 16: each
// four consecutive staging lanes read 64 contiguous bytes of one row (pieces 4j .. 4j + 3), and the
// swizzle puts the 16 lanes of a quarter-wave (four rows, four pieces) in 16 different 16-byte
// bank groups, also its two halves in 8; the plain [piece][row] order put them all in one.
__device__ __forceinline__ uint32_t a16_swz(uint32_t p) {
    const uint32_t b = p % 4;
    return 4 * b + 2 * (b / 2);
}
__device__ __forceinline__ void stage_a16(const int8_t* __restrict__ src_rows, const uint32_t* rowoff, uint32_t K,
                                          v4i_t* As, uint32_t tid) {
    const uint32_t pieces = K / 16;  // 16-byte pieces per row = (block, half); a multiple of 4
    for (uint32_t i0 = 0; i0 < 16 * pieces; i0 += 2048) {
        v4i_t v[8];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const uint32_t i = i0 + tid + 256 * c, ic = i < 16 * pieces ? i : 16 * pieces - 1;
            const uint32_t row = (ic / 4) % 16, pc = 4 * (ic / 64) + ic % 4;
            v[c] = *reinterpret_cast<const v4i_t*>(src_rows + (size_t)rowoff[row] + pc * 16);
        }
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const uint32_t i = i0 + tid + 256 * c;
            const uint32_t row = (i / 4) % 16, pc = 4 * (i / 64) + i % 4;
            if (i < 16 * pieces) As[pc * 16 + (row ^ a16_swz(pc))] = v[c];
        }
    }
}

constexpr uint32_t DM_STRIDE = 17;  // float2 per row of a wave's (dd, mm) table (16 + 1 against bank conflicts)
constexpr uint32_t DM_GU = 9;       // the same for gate/up's 8 sub-blocks per row
constexpr uint32_t DN_ZERO = 512;   // longs of zeros in the down's LDS: 8 chunks of 64 lanes apart

__device__ __forceinline__ v4i mfma_i8_64_acc(v4i_t a, v4i_t b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// The f32 epilogue of one 32-block of gate and up (gemv.rs:141-148 per output, blocks in order):
// acc = fma(mm, u, acc), then acc = fma(dot, dd * sx, acc).  The fma with mm and the products
// dd * sx run as rank-1 MFMAs (the same bits as the VALU forms); sx, su are this lane's row's.
__device__ __forceinline__ void gateup_block(v4f& accg, v4f& accu, const v4i& dg, const v4i& du, float2 mg, float2 mu,
                                             float sx, float su) {
    const v4f dsg = rank1(sx, mg.x, neg_zero4()), dsu = rank1(sx, mu.x, neg_zero4());
    accg = rank1(su, mg.y, accg);
    accu = rank1(su, mu.y, accu);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        accg[i] = __builtin_fmaf((float)dg[i], dsg[i], accg[i]);
        accu[i] = __builtin_fmaf((float)du[i], dsu[i], accu[i]);
    }
}

// gate/up for items of at most 16 / S rows, S strips per MFMA output: the activation rows split
// into S slots of R = 16 / S rows as in the down kernel's down_strips_q4.  Lane (g, r) ends with
// strip g * S / 4 (of the S) of weight row r at activation rows (4g) % R .. +3; the 16 lanes of
// one lane group still hold one strip's 16 weight rows, so the per-16 requantisation reduces
// across the same lanes as with one strip.
template <int NSB, int S>
__device__ __forceinline__ void gateup_strips(const Mat& G, const Mat& U, uint32_t e, const Item& item, bool shared,
                                              uint32_t n_ent, uint32_t F, const v4i_t* As, const float* Sx,
                                              const float* Su, const Workspace& ws, uint32_t wv, uint32_t lane,
                                              uint32_t strips, uint32_t bx) {
    constexpr uint32_t R = 16 / S;
    const uint32_t g = lane / 16, r = lane % 16, nbf = F / 16;
    const uint32_t own = g * S / 4, orow = (4 * g) % R;
    const uint32_t arl = r % R, sel = r / R;
    const uint32_t nstep = (strips / 4 / S) * NSB;
    float wgt[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = orow + i < item.nrows ? orow + i : 0u;
        wgt[i] = shared ? sigmoid_libm(ws.shl[item.row0 + row]) : ws.ent_w[item.row0 + row];
    }
    // the qs pieces load in row order (lane l: row l / 4, piece l % 4; each four lanes 64 contiguous
    // bytes) and move to MFMA lane (g, r) by ds_bpermute from lane 4r + g; the headers load per row
    // piece lpc ^ 2 (lane / 32) (the four lanes of a row still read its 64 bytes): MFMA lane (g, r)
    // then takes its piece from lane 4r + (g ^ 2 (r / 8)), and any 32 consecutive lanes read 32
    // sources distinct modulo 32
    const uint32_t lrow = lane / 4, lpc = (lane % 4) ^ (2 * (lane / 32));
    const int paddr = (int)(4 * r + (g ^ (2 * (r / 8)))) * 4;
    auto rowp = [&](const Mat& M, uint32_t step, uint32_t s, uint32_t row) -> const uint8_t* {
        const uint32_t strip = bx * strips + wv + 4 * ((step / NSB) * S + s);
        return M.ptr + (size_t)e * M.stride + (size_t)(strip * 16 + row) * M.row_bytes + (step % NSB) * 144;
    };
    auto to_mfma = [&](const v4i_t& v) -> v4i_t {
        v4i_t o;
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = __builtin_amdgcn_ds_bpermute(paddr, v[i]);
        return o;
    };
    struct W {
        uint4 hg, hu;
        v4i_t qg[S][2], qu[S][2];
    };
    auto load = [&](uint32_t step, W& w) {
#pragma unroll
        for (int s = 0; s < S; s++) {
            const uint8_t* pg = rowp(G, step, s, lrow);
            const uint8_t* pu = rowp(U, step, s, lrow);
#pragma unroll
            for (int c = 0; c < 2; c++) {
                w.qg[s][c] = *reinterpret_cast<const v4i_t*>(pg + 16 + 64 * c + 16 * lpc);
                w.qu[s][c] = *reinterpret_cast<const v4i_t*>(pu + 16 + 64 * c + 16 * lpc);
            }
        }
        w.hg = *reinterpret_cast<const uint4*>(rowp(G, step, own, r));
        w.hu = *reinterpret_cast<const uint4*>(rowp(U, step, own, r));
    };
    W cw;
    load(0, cw);
    v4f accg = {0.0f, 0.0f, 0.0f, 0.0f}, accu = {0.0f, 0.0f, 0.0f, 0.0f};
    const v4i_t zero4 = {0, 0, 0, 0};
    const v4i z = {0, 0, 0, 0};
    const bool first = g < 2;
    const uint32_t tl = orow + (r & 3);  // the row whose scales this lane feeds the rank-1 MFMAs
    // staged slots of row arl in the pieces read below (block bl even: piece % 4 = g % 2, 2 + g % 2)
    const uint32_t arl_l = arl ^ a16_swz(g % 2), arl_h = arl ^ a16_swz(2 + g % 2);
    for (uint32_t step = 0; step < nstep; step++) {
        const uint32_t sb = step % NSB;
        W nw = cw;
        if (step + 1 < nstep) load(step + 1, nw);
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            const uint32_t bl = sb * 8 + 4 * pp + (first ? 0u : 2u);
            const v4i_t al = As[(bl * 2 + g % 2) * 16 + arl_l], ah = As[((bl + 1) * 2 + g % 2) * 16 + arl_h];
            const v4i_t a0 = first ? al : zero4, a2 = first ? zero4 : al;
            const v4i_t a1 = first ? ah : zero4, a3 = first ? zero4 : ah;
            v4i dgv[4] = {z, z, z, z}, duv[4] = {z, z, z, z};
#pragma unroll
            for (int s = 0; s < S; s++) {
                const bool m = sel == (uint32_t)s;
                const v4i_t b0 = m ? a0 : zero4, b1 = m ? a1 : zero4, b2 = m ? a2 : zero4, b3 = m ? a3 : zero4;
                const v4i_t qgs = to_mfma(cw.qg[s][pp]), qus = to_mfma(cw.qu[s][pp]);
                const v4i_t wgl = qgs & 0x0f0f0f0f, wgh = (qgs >> 4) & 0x0f0f0f0f;
                const v4i_t wul = qus & 0x0f0f0f0f, wuh = (qus >> 4) & 0x0f0f0f0f;
                dgv[0] = mfma_i8_64_acc(b0, wgl, dgv[0]);
                duv[0] = mfma_i8_64_acc(b0, wul, duv[0]);
                dgv[1] = mfma_i8_64_acc(b1, wgh, dgv[1]);
                duv[1] = mfma_i8_64_acc(b1, wuh, duv[1]);
                dgv[2] = mfma_i8_64_acc(b2, wgl, dgv[2]);
                duv[2] = mfma_i8_64_acc(b2, wul, duv[2]);
                dgv[3] = mfma_i8_64_acc(b3, wgh, dgv[3]);
                duv[3] = mfma_i8_64_acc(b3, wuh, duv[3]);
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int j = 4 * pp + jj;
                const uint32_t B = sb * 8 + j;
                const v4i dg = dgv[jj], du = duv[jj];
                const float2 mg = q4k_dm_rt(cw.hg, j), mu = q4k_dm_rt(cw.hu, j);
                gateup_block(accg, accu, dg, du, mg, mu, Sx[B * 16 + tl], Su[B * 16 + tl]);
            }
        }
        cw = nw;
        if (sb == NSB - 1) {
            const uint32_t strip = bx * strips + wv + 4 * ((step / NSB) * S + own);
            // the item's first output row, opaque to the compiler so that it does not hoist the row
            // addresses below out of the strip loop into scratch memory
            uint32_t arow0 = shared ? n_ent + item.row0 : item.row0;
            asm volatile("" : "+v"(arow0));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t row = orow + i;
                const float v = silu512(accg[i]) * accu[i];
                const float amax =
                        row16_allreduce(__builtin_fabsf(v), [](float x, float y) { return mx_ps(x, y); });
                const float sc = amax / 127.0f;
                const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
                const int32_t qi = cvt_rne(v * inv);
                const int32_t sum = row16_allreduce(qi, [](int32_t x, int32_t y) { return x + y; });
                if (row < item.nrows) {
                    const uint32_t arow = arow0 + row;
                    ws.actq[(size_t)arow * F + strip * 16 + r] = sat_i8(qi);
                    if (r == 0) {
                        const float sf = sc * wgt[i];  // exec_batch.rs:1533-1535
                        ws.acts[(size_t)arow * nbf + strip] = sf;
                        ws.actsum[(size_t)arow * nbf + strip] = sum;
                        ws.actu[(size_t)arow * nbf + strip] = sf * (float)sum;
                    }
                }
                accg[i] = 0.0f;
                accu[i] = 0.0f;
            }
        }
    }
}

// gate/up + SwiGLU + per-16 requantisation + weight fold (tasks A and B of moe_batch) of one
// item over column block bx: the block's strips of 16 rows, each wave every fourth of them.
template <int NSB>
__device__ __forceinline__ void gateup_item(const Mat& gate, const Mat& up, const Mat& shg, const Mat& shu,
                                            const Workspace& ws, uint32_t skip_rows, uint32_t bx, uint32_t itn,
                                            uint8_t* smem) {
    constexpr uint32_t H = NSB * 256, nb = NSB * 8;
    const uint32_t F = gate.rows, nbf = F / 16;
    const uint32_t tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
    const Item item = ws.items[itn];
    if (item.nrows <= skip_rows) return;  // a streaming-GEMV item (k_stream.hip)
    const bool shared = item.expert == NO_EXPERT;
    const uint32_t n_ent = ws.n_groups[1];
    const Mat& G = shared ? shg : gate;
    const Mat& U = shared ? shu : up;
    const uint32_t e = shared ? 0u : item.expert;

    v4i_t* As = reinterpret_cast<v4i_t*>(smem);                      // [nb][2 halves][16 rows]
    float* Sx = reinterpret_cast<float*>(smem + nb * 64 * 8);        // [nb][16] activation scales
    float* Su = Sx + nb * 16;                                        // [nb][16] scale * sum
    float2* Dm = reinterpret_cast<float2*>(Su + nb * 16);            // [4 waves][2][16][DM_GU]
    uint32_t* rowoff = reinterpret_cast<uint32_t*>(Dm + 4 * 2 * 16 * DM_GU);  // [16]
    uint32_t* tokv = rowoff + 16;                                    // [16]

    if (tid < 16) {
        const uint32_t tok = item_token(ws, item, shared, tid);
        tokv[tid] = tok;
        rowoff[tid] = tok * H;
    }
    __syncthreads();
    stage_a16(ws.xq, rowoff, H, As, tid);
    for (uint32_t i0 = 0; i0 < 16 * nb; i0 += 1024) {
        float a[4], c2[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = i0 + tid + 256 * c, ic = i < 16 * nb ? i : 16 * nb - 1;  // row ic % 16, block ic / 16
            a[c] = ws.xs[(size_t)tokv[ic % 16] * nb + ic / 16];
            c2[c] = ws.xu[(size_t)tokv[ic % 16] * nb + ic / 16];
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = i0 + tid + 256 * c;
            if (i < 16 * nb) {
                Sx[i] = a[c];
                Su[i] = c2[c];
            }
        }
    }
    const uint32_t strips = F / 16 / gridDim.x;  // per workgroup
    if (item.nrows <= 8 && strips % 8 == 0) {
        __syncthreads();
        gateup_strips<NSB, 2>(G, U, e, item, shared, n_ent, F, As, Sx, Su, ws, wv, lane, strips, bx);
        return;
    }
    const uint32_t g = lane / 16, r = lane % 16;
    // routing weight of this lane's four entry rows (exec_batch.rs:1533-1535; shared: the gate)
    float wgt[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = 4 * g + i < item.nrows ? 4 * g + i : 0u;
        wgt[i] = shared ? sigmoid_libm(ws.shl[item.row0 + row]) : ws.ent_w[item.row0 + row];
    }
    __syncthreads();

    float2* dmw = Dm + wv * 2 * 16 * DM_GU;
    const uint32_t nstep = (strips / 4) * NSB;   // (strip, superblock) steps of this wave
    // Loads go out in row order: lane l reads row l / 4, 16-byte piece l % 4, so each four
    // consecutive lanes read 64 contiguous bytes (the vector L1 serves that about 3x faster from L2
    // than the MFMA order, where consecutive lanes read different rows).  ds_bpermute then moves
    // each piece to MFMA lane (g, r) = (piece, row), from lane 4r + g.
    const uint32_t lrow = lane / 4, lpc = (lane % 4) ^ (2 * (lane / 32));  // as in gateup_strips
    const int paddr = (int)(4 * r + (g ^ (2 * (r / 8)))) * 4;
    auto rows_of = [&](uint32_t step, const uint8_t*& rg, const uint8_t*& ru) {
        const uint32_t strip = bx * strips + wv + 4 * (step / NSB);
        rg = G.ptr + (size_t)e * G.stride + (size_t)(strip * 16 + lrow) * G.row_bytes;
        ru = U.ptr + (size_t)e * U.stride + (size_t)(strip * 16 + lrow) * U.row_bytes;
    };
    auto to_mfma = [&](const v4i_t& v) -> v4i_t {
        v4i_t o;
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = __builtin_amdgcn_ds_bpermute(paddr, v[i]);
        return o;
    };
    Q4Sb16 cg, cu;
    {
        const uint8_t *rg, *ru;
        rows_of(0, rg, ru);
        load_q4sb16(rg, 0, lpc, cg);
        load_q4sb16(ru, 0, lpc, cu);
    }
    v4f accg = {0.0f, 0.0f, 0.0f, 0.0f}, accu = {0.0f, 0.0f, 0.0f, 0.0f};
    const v4i_t zero4 = {0, 0, 0, 0};
    const bool first = g < 2;  // this lane's bytes are of the pair's first chunk
    const uint32_t tl = 4 * g + (r & 3);  // the token whose scales this lane feeds the rank-1 MFMAs
    // staged slots of row r in the pieces read below (block bl even: piece % 4 = g % 2, 2 + g % 2)
    const uint32_t r_l = r ^ a16_swz(g % 2), r_h = r ^ a16_swz(2 + g % 2);
    for (uint32_t step = 0; step < nstep; step++) {
        const uint32_t sb = step % NSB;
        Q4Sb16 ng = cg, nu = cu;
        if (step + 1 < nstep) {  // the next superblock's loads go out before this one's math
            const uint8_t *rg, *ru;
            rows_of(step + 1, rg, ru);
            load_q4sb16(rg, (step + 1) % NSB, lpc, ng);
            load_q4sb16(ru, (step + 1) % NSB, lpc, nu);
        }
        // (dd, mm) of sub-blocks 2 lpc, 2 lpc + 1 of the loaded row, gate then up
        wave_sync();
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            const uint32_t j = 2 * lpc + jj;
            dmw[lrow * DM_GU + j] = q4k_dm_rt(cg.hdr, j);
            dmw[(16 + lrow) * DM_GU + j] = q4k_dm_rt(cu.hdr, j);
        }
        const v4i_t qg[2] = {to_mfma(cg.q[0]), to_mfma(cg.q[1])}, qu[2] = {to_mfma(cu.q[0]), to_mfma(cu.q[1])};
        wave_sync();
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            // this lane's activation halves: sub-blocks 4pp + 2 (g / 2) (low nibbles) and the next
            const uint32_t bl = sb * 8 + 4 * pp + (first ? 0u : 2u);
            const v4i_t al = As[(bl * 2 + g % 2) * 16 + r_l], ah = As[((bl + 1) * 2 + g % 2) * 16 + r_h];
            const v4i_t wgl = qg[pp] & 0x0f0f0f0f, wgh = (qg[pp] >> 4) & 0x0f0f0f0f;
            const v4i_t wul = qu[pp] & 0x0f0f0f0f, wuh = (qu[pp] >> 4) & 0x0f0f0f0f;
            v4i dgv[4], duv[4];  // sub-blocks 4pp + 0..3
            {
                const v4i_t a0 = first ? al : zero4, a2 = first ? zero4 : al;
                const v4i_t a1 = first ? ah : zero4, a3 = first ? zero4 : ah;
                dgv[0] = mfma_i8_64(a0, wgl);
                duv[0] = mfma_i8_64(a0, wul);
                dgv[1] = mfma_i8_64(a1, wgh);
                duv[1] = mfma_i8_64(a1, wuh);
                dgv[2] = mfma_i8_64(a2, wgl);
                duv[2] = mfma_i8_64(a2, wul);
                dgv[3] = mfma_i8_64(a3, wgh);
                duv[3] = mfma_i8_64(a3, wuh);
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int j = 4 * pp + jj;
                const uint32_t B = sb * 8 + j;
                const v4i dg = dgv[jj], du = duv[jj];
                const float2 mg = dmw[r * DM_GU + j], mu = dmw[(16 + r) * DM_GU + j];
                gateup_block(accg, accu, dg, du, mg, mu, Sx[B * 16 + tl], Su[B * 16 + tl]);
            }
        }
        cg = ng;
        cu = nu;
        if (sb == NSB - 1) {
            // SwiGLU (elem.rs:173) and per-16 quantisation across the 16 lanes holding one entry's
            // strip (lanes 16g .. 16g+15, one DPP row)
            const uint32_t strip = bx * strips + wv + 4 * (step / NSB);
            // the item's first output row, opaque to the compiler (as in gateup_strips)
            uint32_t arow0 = shared ? n_ent + item.row0 : item.row0;
            asm volatile("" : "+v"(arow0));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t row = 4 * g + i;
                const float v = silu512(accg[i]) * accu[i];
                const float amax =
                        row16_allreduce(__builtin_fabsf(v), [](float x, float y) { return mx_ps(x, y); });
                const float s = amax / 127.0f;
                const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
                const int32_t qi = cvt_rne(v * inv);
                const int32_t sum = row16_allreduce(qi, [](int32_t x, int32_t y) { return x + y; });
                if (row < item.nrows) {
                    const uint32_t arow = arow0 + row;
                    ws.actq[(size_t)arow * F + strip * 16 + r] = sat_i8(qi);
                    if (r == 0) {
                        const float sf = s * wgt[i];  // exec_batch.rs:1533-1535
                        ws.acts[(size_t)arow * nbf + strip] = sf;
                        ws.actsum[(size_t)arow * nbf + strip] = sum;
                        ws.actu[(size_t)arow * nbf + strip] = sf * (float)sum;
                    }
                }
                accg[i] = 0.0f;
                accu[i] = 0.0f;
            }
        }
    }
}

typedef int v16i __attribute__((ext_vector_type(16)));
__device__ __forceinline__ v16i mfma_i8_32x32(v4i_t a, v4i_t b) {
    const v16i z = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

// The f32 epilogue of one 32-block on a 32 x 32 tile (gemv.rs:141-148 per output, blocks in
// order): lane (h, c) holds weight row c at tile rows 8q + 4h + u, u = 0 .. 3, in element u of
// acc[q].  sx4 / su4 hold the scales of tile rows 8q + 4h + (lane % 4), q = 0 .. 3: the rank-1
// MFMA's a operand for output u of this lane comes from lane 4 (lane / 4) + u.
__device__ __forceinline__ void block32(v4f (&acc)[4], const v16i& d, float2 dm, float4 sx4, float4 su4) {
    const float sx[4] = {sx4.x, sx4.y, sx4.z, sx4.w}, su[4] = {su4.x, su4.y, su4.z, su4.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const v4f ds = rank1(sx[q], dm.x, neg_zero4());
        acc[q] = rank1(su[q], dm.y, acc[q]);
#pragma unroll
        for (int u = 0; u < 4; u++) acc[q][u] = __builtin_fmaf((float)d[4 * q + u], ds[u], acc[q][u]);
    }
}

// (dd, mm) of sub-blocks 2 ch and 2 ch + 1 of this lane's row: lane (h, c) decodes sub-block
// 2 ch + h and permlane32_swap hands each half the other's (result 0 holds lanes 0-31's value in
// both halves, result 1 lanes 32-63's).
__device__ __forceinline__ void q4k_dm_pair(uint4 hdr, uint32_t ch, uint32_t h, float2& d0, float2& d1) {
    const float2 v = q4k_dm_rt(hdr, 2 * ch + h);
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v.x), __float_as_uint(v.x), false, false);
    const auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(v.y), __float_as_uint(v.y), false, false);
    d0 = make_float2(__uint_as_float(x[0]), __uint_as_float(y[0]));
    d1 = make_float2(__uint_as_float(x[1]), __uint_as_float(y[1]));
}

// gate/up of item pairs (large batches: an expert with more than 16 rows has several items; the
// dispatch lists its items as pairs of parts 2j, 2j + 1 in ws.pairs).  A pair is one 32-row tile of
// activation rows on v_mfma_i32_32x32x32_i8: rows 0-15 the first item's, 16-31 the second's.  A wave
// takes a strip of 16 features at a time with its 16 gate rows and 16 up rows as the 32 B-operand
// rows: lane (h, c) = (lane / 32, lane % 32) feeds A = tile row c's activations and B = gate row c
// (c < 16) or up row c - 16 of the strip, k = 16h .. 16h + 15 of a 32-block, and gets back that
// weight row at tile rows 8q + 4h + u in element 4q + u.  A 16-byte qs piece holds 16 values of
// sub-block 2ch in its low nibbles and of 2ch + 1 in its high ones, so each nibble half is one
// MFMA with nothing masked, and every weight load, unpack and (dd, mm) decode serves 32 activation
// rows.  Eight waves share the staged activations (32 rows: 40 H bytes of LDS, two workgroups per
// CU) and hold few registers (four waves per SIMD).  The per-block f32 chain, SwiGLU, quantisation
// and fold are those of the 16-row path, output by output.
template <int NSB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void batch_gateup_pairs_kernel(
        Mat gate, Mat up, Mat shg, Mat shu, Workspace ws) {
    constexpr uint32_t H = NSB * 256, nb = NSB * 8;
    extern __shared__ __align__(16) uint8_t smem[];
    uint32_t bx, pu;  // column block and pair, in XCD order
    if (!xcd_order(ws.n_groups[4], bx, pu)) return;
    const uint32_t i0 = ws.pairs[pu];
    const Item it0 = ws.items[i0], it1 = ws.items[i0 + 1];
    const bool shared = it0.expert == NO_EXPERT;
    const Mat& G = shared ? shg : gate;
    const Mat& U = shared ? shu : up;
    const uint32_t e = shared ? 0u : it0.expert;
    const uint32_t F = G.rows, nbf = F / 16, n_ent = ws.n_groups[1];
    const uint32_t tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
    const uint32_t h = lane / 32, c = lane % 32;
    v4i_t* As = reinterpret_cast<v4i_t*>(smem);                   // [nb][2 halves][32 rows]
    float4* SxT = reinterpret_cast<float4*>(smem + nb * 1024);     // [nb][8 (h, u)]: rows 8q + 4h + u
    float4* SuT = SxT + nb * 8;

    // tile row c's token and routing weight (exec_batch.rs:1533-1535; shared: the gate)
    const Item& itc = c < 16 ? it0 : it1;
    const uint32_t rc = c % 16 < itc.nrows ? c % 16 : 0u;
    const uint32_t tok = item_token(ws, itc, shared, c % 16);
    const float wgt_c = shared ? sigmoid_libm(ws.shl[itc.row0 + rc]) : ws.ent_w[itc.row0 + rc];

    // activations: 16-byte piece p of tile row r at As[p * 32 + (r ^ a16_swz(p))]; four lanes read
    // 64 contiguous bytes of one row, and the 16 lanes of a quarter-wave store to 16 bank groups
    {
        constexpr uint32_t lim = 32 * 2 * nb;
        for (uint32_t i0 = 0; i0 < lim; i0 += 4096) {
            v4i_t v[8];
            uint32_t dst[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t idx = i0 + tid + 512 * k, ic = idx < lim ? idx : lim - 1;
                const uint32_t row = (ic / 4) % 32, pc = 4 * (ic / 128) + ic % 4;
                const uint32_t t = (uint32_t)__shfl((int)tok, (int)row);
                v[k] = *reinterpret_cast<const v4i_t*>(ws.xq + (size_t)t * H + pc * 16);
                dst[k] = pc * 32 + (row ^ a16_swz(pc));
            }
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (i0 + tid + 512 * k < lim) As[dst[k]] = v[k];
        }
        constexpr uint32_t lims = 32 * nb;
        float* sx = reinterpret_cast<float*>(SxT);
        float* su = reinterpret_cast<float*>(SuT);
        for (uint32_t i0 = 0; i0 < lims; i0 += 2048) {
            float a[4], b[4];
            uint32_t dst[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t idx = i0 + tid + 512 * k, ic = idx < lims ? idx : lims - 1;
                const uint32_t row = (ic / 4) % 32, B = 4 * (ic / 128) + ic % 4;
                const uint32_t t = (uint32_t)__shfl((int)tok, (int)row);
                a[k] = ws.xs[(size_t)t * nb + B];
                b[k] = ws.xu[(size_t)t * nb + B];
                dst[k] = B * 32 + (row % 8) * 4 + row / 8;
            }
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (i0 + tid + 512 * k < lims) {
                    sx[dst[k]] = a[k];
                    su[dst[k]] = b[k];
                }
        }
    }
    __syncthreads();

    // Weight rows: lane (h, c) loads the header of B-operand row c; lane l loads the 16-byte qs
    // pieces 2 ch + ((l % 2) ^ (l / 32)) (ch = 0 .. 3) of B-operand row l / 2 (gate rows in lanes
    // 0-31, up rows in 32-63; two lanes read one 32-byte chunk), and MFMA lane (h, c) takes its piece
    // from lane 2c + (h ^ (c / 16)).
    // Gate and up have one shape and format, so one stride and row size serve both.
    const uint32_t strips = F / 16 / gridDim.x;  // of this workgroup; wave wv takes wv, wv + 8, ..
    const uint32_t nstep = (strips / 8) * NSB;   // (strip, superblock) steps of this wave
    const size_t rb = G.row_bytes;
    const uint8_t* hbase = (c < 16 ? G.ptr : U.ptr) + (size_t)e * G.stride + (size_t)(c % 16) * rb;
    const uint8_t* qbase =
            (lane < 32 ? G.ptr : U.ptr) + (size_t)e * G.stride + (size_t)((lane / 2) % 16) * rb + 16 +
            16 * ((lane % 2) ^ (lane / 32));
    // lanes 32-63 hold the two pieces of a chunk the other way round, so that MFMA lane (h, c) takes
    // its piece from lane 2c + (h ^ (c / 16)) and any 32 consecutive lanes read 32 sources distinct
    // modulo 32
    const int paddr = (int)(2 * c + (h ^ (c / 16))) * 4;
    auto strip_of = [&](uint32_t step) { return bx * strips + wv + 8 * (step / NSB); };
    struct Raw {
        uint4 hdr;
        v4i_t q[4];
    };
    auto load = [&](uint32_t step, Raw& w) {
        const size_t off = (size_t)strip_of(step) * 16 * rb + (step % NSB) * 144;
        w.hdr = *reinterpret_cast<const uint4*>(hbase + off);
#pragma unroll
        for (int ch = 0; ch < 4; ch++) w.q[ch] = *reinterpret_cast<const v4i_t*>(qbase + off + 32 * ch);
    };
    auto to_mfma = [&](const v4i_t& v) -> v4i_t {
        v4i_t o;
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = __builtin_amdgcn_ds_bpermute(paddr, v[i]);
        return o;
    };
    v4f acc[4];
#pragma unroll
    for (int q = 0; q < 4; q++) acc[q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t sl = 4 * h + (lane & 3);  // this lane's (h, u) slot of the scale tables
    const bool odd = c >= 16;                // this lane's row of the strip: up (odd DPP row) or gate
    // tile row c's staged slot in piece 2B + h: B % 2 = nib, so piece % 4 = 2 nib + h
    const uint32_t cs[2] = {c ^ a16_swz(h), c ^ a16_swz(2 + h)};
    // one (strip, superblock) step on the words in cur, the next step's loads going out into nxt first
    auto step_on = [&](uint32_t step, const Raw& cur, Raw& nxt) {
        const uint32_t sb = step % NSB;
        if (step + 1 < nstep) load(step + 1, nxt);
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            const v4i_t qv = to_mfma(cur.q[ch]);
            float2 dm[2];
            q4k_dm_pair(cur.hdr, ch, h, dm[0], dm[1]);
#pragma unroll
            for (int nib = 0; nib < 2; nib++) {
                const uint32_t B = sb * 8 + 2 * ch + nib;
                const v4i_t a = As[(B * 2 + h) * 32 + cs[nib]];
                const v4i_t w = nib ? (qv >> 4) & 0x0f0f0f0f : qv & 0x0f0f0f0f;
                block32(acc, mfma_i8_32x32(a, w), dm[nib], SxT[B * 8 + sl], SuT[B * 8 + sl]);
            }
        }
        if (sb != NSB - 1) return;
        // SwiGLU (elem.rs:173) and per-16 quantisation.  Gate rows sit in DPP rows 0 and 2 of the
        // wave, up rows in 1 and 3; one permlane16_swap per two outputs gives a gate lane the up
        // value of its tile row 8q + 4h + u (q = 0, 1) and an up lane the gate value of tile row
        // 8(q + 2) + 4h + u, so each lane finishes one output and the 16 lanes of a DPP row
        // quantise one tile row's strip.
        const uint32_t strip = strip_of(step);
        const Item& it = odd ? it1 : it0;
        // the first output row of this lane's item, opaque to the compiler: otherwise it hoists the
        // 16 row addresses below out of the strip loop and keeps them in scratch memory (spill
        // traffic through HBM on every strip)
        uint32_t arow0 = shared ? n_ent + it.row0 : it.row0;
        asm volatile("" : "+v"(arow0));
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float send = odd ? acc[qq][u] : acc[qq + 2][u];
                const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(send), __float_as_uint(send), false,
                                                                false);
                const float g = odd ? __uint_as_float(x[0]) : acc[qq][u];
                const float up_v = odd ? acc[qq + 2][u] : __uint_as_float(x[1]);
                const uint32_t row = 8 * qq + 4 * h + u, t = odd ? 16 + row : row;
                const float v = silu512(g) * up_v;
                const float amax = row16_allreduce(__builtin_fabsf(v), [](float x, float y) { return mx_ps(x, y); });
                const float s = amax / 127.0f;
                const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
                const int32_t qi = cvt_rne(v * inv);
                const int32_t sum = row16_allreduce(qi, [](int32_t x, int32_t y) { return x + y; });
                const float w = __shfl(wgt_c, (int)t);
                if (row < it.nrows) {
                    const uint32_t arow = arow0 + row;
                    ws.actq[(size_t)arow * F + strip * 16 + c % 16] = sat_i8(qi);
                    if (c % 16 == 0) {
                        const float sf = s * w;  // exec_batch.rs:1533-1535
                        ws.acts[(size_t)arow * nbf + strip] = sf;
                        ws.actsum[(size_t)arow * nbf + strip] = sum;
                        ws.actu[(size_t)arow * nbf + strip] = sf * (float)sum;
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 4; q++) acc[q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    };
    // two buffers of raw words, alternating (the loop runs two steps per turn, so no copies)
    Raw ra, rb2;
    load(0, ra);
    for (uint32_t step = 0; step < nstep; step += 2) {
        step_on(step, ra, rb2);
        if (step + 1 < nstep) step_on(step + 1, rb2, ra);
    }
}

// gate/up + SwiGLU + per-16 requantisation + weight fold (tasks A and B of moe_batch).
// Grid (F / 256, items): a workgroup covers 16 strips of F, each wave 4 of them.  Registers are
// held to three waves per SIMD (the LDS fits three workgroups per CU): at config 4 that took the
// kernel from 540 to 487 us against two waves, the few spilled words being on the small-item path.
// LIST: the items in no pair (ws.single), after batch_gateup_pairs_kernel has run the pairs.
template <int NSB, int LIST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void batch_gateup_kernel(
        Mat gate, Mat up, Mat shg, Mat shu, Workspace ws, uint32_t skip_rows) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint32_t bx, itn;  // column block and item, in XCD order
    // the unpaired items walk each XCD's run backwards: its first items then belong to the experts
    // the pairs launch read last on that XCD, whose weights may still sit in the caches
    if (!xcd_order(ws.n_groups[LIST ? 5 : 2], bx, itn, LIST != 0)) return;
    if (LIST) itn = ws.single[itn];
    gateup_item<NSB>(gate, up, shg, shu, ws, skip_rows, bx, itn, smem);
}

hipError_t launch_batch_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up,
                               const Workspace& ws, uint32_t m, uint32_t skip_rows, hipStream_t st) {
    const uint32_t H = gate.k, F = gate.rows, nb = H / 32;
    const size_t lds = (size_t)nb * 64 * 8 + (size_t)nb * 16 * 8 + 4 * 2 * 16 * DM_GU * 8 + 32 * 4;
    // a workgroup per (item, 16 strips) once the items fill the GPU; otherwise per (item, 4 strips)
    // so that a wave's chain of dependent weight loads stays short
    const uint32_t cols = geo::mfma_gateup_cols(m, F), rows = grouped_item_rows(ws, m);
    // item pairs of one expert as 32-row tiles where experts have several items (config 4: ~4
    // each), when no item streams and gate and up share one layout
    const bool pairs = geo::gateup_pairs(m, H) && skip_rows == 0 && geo::gateup_pair_strips(m, F) % 8 == 0 &&
                       gate.stride == up.stride && gate.row_bytes == up.row_bytes &&
                       sh_gate.row_bytes == gate.row_bytes && sh_up.row_bytes == gate.row_bytes;
    // the unpaired items (an expert's last when its count is odd) are one round of workgroups: a
    // strip per wave keeps their chains short
    const dim3 grid(cols, rows), pgrid(geo::gateup_pair_cols(m, F), rows / 2 + 1), sgrid(F % 64 == 0 ? F / 64 : cols, rows);
    const size_t plds = (size_t)geo::gateup_pair_lds(H);
    switch (H / 256 * 2 + (pairs ? 1 : 0)) {
#define GU_CASE(n) \
    case n * 2: batch_gateup_kernel<n, 0><<<grid, 256, lds, st>>>(gate, up, sh_gate, sh_up, ws, skip_rows); break;
#define GU_CASE2(n)                                                                                     \
    GU_CASE(n)                                                                                          \
    case n * 2 + 1:                                                                                     \
        batch_gateup_pairs_kernel<n><<<pgrid, 512, plds, st>>>(gate, up, sh_gate, sh_up, ws);           \
        batch_gateup_kernel<n, 1><<<sgrid, 256, lds, st>>>(gate, up, sh_gate, sh_up, ws, skip_rows);     \
        break;
        GU_CASE2(1) GU_CASE2(2) GU_CASE2(3) GU_CASE2(4) GU_CASE2(5) GU_CASE2(6) GU_CASE2(7) GU_CASE2(8) GU_CASE(9)
        GU_CASE(10) GU_CASE(11) GU_CASE(12) GU_CASE(13) GU_CASE(14) GU_CASE(15) GU_CASE(16)
#undef GU_CASE2
#undef GU_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- down ---------------------------------------------------------------------------------------
//
// Grid (H / 256, items): a workgroup covers 256 rows of H, each wave 4 strips of 16.  The down
// input is quantised per 16, so each 32-byte activation chunk feeds two MFMAs with the other
// half of its k-groups zeroed, giving the exact dot of each 16-block.

// Q6_K operands of one superblock for lane (g, r) (superblocks are only 2-byte aligned, so each
// piece comes from an aligned load and byte alignment): ql bytes 64n + 32s + 8g (n, s in {0, 1}),
// qh bytes 128 + 32n + 8g, the scales of blocks 4g .. 4g+3 (this lane decodes them) and d.
// Q6Raw holds the loaded words as they arrive; q6_settle aligns them when the superblock's math
// starts, so that the next superblock's loads, issued before, stay in flight meanwhile (work on
// a loaded value at load time would make the wave wait for it there).
typedef uint32_t v3u __attribute__((ext_vector_type(3)));
struct Q6Raw {
    v3u ql[4], qh[2];  // 12-byte loads at the 4-byte boundary at or below each 8-byte piece
    uint2 sv;          // the 8 bytes holding the 4 scale bytes 192 + 4g
    uint32_t sh;       // the superblock's misalignment in bytes (0 or 2)
    uint16_t d;
};
struct Q6Sb {
    uint2 ql[4], qh[2];
    uint32_t sc;  // int8 scales of blocks 4g .. 4g+3
    uint16_t d;
};
// The 12-byte load for the 8 bytes at p + o (p 2-byte aligned) stays inside the superblock when
// 2 <= o + 12 - shift <= 210 and o >= shift, as for every ql / qh piece.
__device__ __forceinline__ void load_q6sb(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t g, Q6Raw& w) {
    const uint8_t* p = rowp + sb * 210;
    const uint32_t sh = (uint32_t)reinterpret_cast<uintptr_t>(p) & 3u;  // 0 or 2
    const uint8_t* pa = p - sh;
#pragma unroll
    for (int i = 0; i < 4; i++) w.ql[i] = *reinterpret_cast<const v3u*>(pa + 64 * (i / 2) + 32 * (i % 2) + 8 * g);
#pragma unroll
    for (int n = 0; n < 2; n++) w.qh[n] = *reinterpret_cast<const v3u*>(pa + 128 + 32 * n + 8 * g);
    // the 4 scale bytes 192 + 4g: one 8-byte load that stays inside the superblock (at 188 + 4g
    // when p is 4-byte aligned, else at the 4-byte boundary 2 below 192 + 4g)
    w.sv = *reinterpret_cast<const uint2*>(sh ? pa + 192 + 4 * g : p + 188 + 4 * g);
    w.sh = sh;
    w.d = *reinterpret_cast<const uint16_t*>(p + 208);
}
__device__ __forceinline__ uint2 align64(const v3u& v, uint32_t sh) {
    return make_uint2(__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh));
}
__device__ __forceinline__ Q6Sb settle(const Q6Raw& r) {
    Q6Sb w;
#pragma unroll
    for (int i = 0; i < 4; i++) w.ql[i] = align64(r.ql[i], r.sh);
#pragma unroll
    for (int n = 0; n < 2; n++) w.qh[n] = align64(r.qh[n], r.sh);
    w.sc = r.sh ? __builtin_amdgcn_alignbyte(r.sv.y, r.sv.x, 2) : r.sv.y;
    w.d = r.d;
    return w;
}
// 8 consecutive 6-bit values e = 32*q8 + 8g .. +7 of the superblock (q8 compile-time)
__device__ __forceinline__ long q6_operand(const Q6Sb& w, int q8) {
    const int n = q8 / 4, g6 = q8 % 4;
    const uint2 lo = w.ql[2 * n + (g6 & 1)], hi = w.qh[n];
    const int sh = (g6 >> 1) ? 4 : 0;
    const uint32_t l0 = (lo.x >> sh) & 0x0f0f0f0fu, l1 = (lo.y >> sh) & 0x0f0f0f0fu;
    const uint32_t h0 = (hi.x >> (2 * g6)) & 0x03030303u, h1 = (hi.y >> (2 * g6)) & 0x03030303u;
    return (long)(((unsigned long long)(l1 | (h1 << 4)) << 32) | (l0 | (h0 << 4)));
}

__device__ __forceinline__ v4i mfma_i8_acc(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

// The f32 epilogue of one 32-wide chunk of the down input = two 16-blocks (gemv.rs:141-148, blocks in
// order): acc = fma(mm, u, acc), then acc = fma(dot, dd * sx, acc), per block.  The products
// dd * sx run as rank-1 MFMAs off the accumulation chain (the same bits as v_mul_f32); the chain
// stays on the VALU, since one chain per lane would otherwise wait on an MFMA every block.  sx
// points at this lane's row of the first block's scales, su4 at the four rows 4g .. of its u; the
// second block's are 16 floats on.
__device__ __forceinline__ void down_blocks(v4f& acc, const v4i& c0, const v4i& c1, float2 d0, float2 d1,
                                            const float* sx, const float* su4) {
    const v4f ds0 = rank1(sx[0], d0.x, neg_zero4()), ds1 = rank1(sx[16], d1.x, neg_zero4());
    const float4 u0 = *reinterpret_cast<const float4*>(su4), u1 = *reinterpret_cast<const float4*>(su4 + 16);
    const float u0a[4] = {u0.x, u0.y, u0.z, u0.w}, u1a[4] = {u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        acc[i] = __builtin_fmaf(d0.y, u0a[i], acc[i]);
        acc[i] = __builtin_fmaf((float)c0[i], ds0[i], acc[i]);
        acc[i] = __builtin_fmaf(d1.y, u1a[i], acc[i]);
        acc[i] = __builtin_fmaf((float)c1[i], ds1[i], acc[i]);
    }
}

// The whole block on the matrix cores but the dot's fma: acc = fma(mm, u, acc) as a rank-1 MFMA
// too (su: this lane's row's u), so the chain alternates MFMA and VALU
__device__ __forceinline__ void down_blocks_mc(v4f& acc, const v4i& c0, const v4i& c1, float2 d0, float2 d1,
                                               const float* sx, const float* su) {
    const v4f ds0 = rank1(sx[0], d0.x, neg_zero4()), ds1 = rank1(sx[16], d1.x, neg_zero4());
    acc = rank1(su[0], d0.y, acc);
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf((float)c0[i], ds0[i], acc[i]);
    acc = rank1(su[16], d1.y, acc);
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf((float)c1[i], ds1[i], acc[i]);
}

// The same chain with the products on the VALU too (fewer registers, for the small-item paths
// whose register count sets the kernel's)
__device__ __forceinline__ void down_blocks_valu(v4f& acc, const v4i& c0, const v4i& c1, float2 dm, const float* sx4,
                                                 const float* su4) {
    const float4 s0 = *reinterpret_cast<const float4*>(sx4), s1 = *reinterpret_cast<const float4*>(sx4 + 16);
    const float4 u0 = *reinterpret_cast<const float4*>(su4), u1 = *reinterpret_cast<const float4*>(su4 + 16);
    const float s0a[4] = {s0.x, s0.y, s0.z, s0.w}, u0a[4] = {u0.x, u0.y, u0.z, u0.w};
    const float s1a[4] = {s1.x, s1.y, s1.z, s1.w}, u1a[4] = {u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        acc[i] = __builtin_fmaf(dm.y, u0a[i], acc[i]);
        acc[i] = __builtin_fmaf((float)c0[i], dm.x * s0a[i], acc[i]);
        acc[i] = __builtin_fmaf(dm.y, u1a[i], acc[i]);
        acc[i] = __builtin_fmaf((float)c1[i], dm.x * s1a[i], acc[i]);
    }
}

// Q4_K down for items of at most 16 / S rows: S strips share one 16x16 MFMA output.  The rows of
// A are split into S slots of R = 16 / S; strip s's MFMA sees the item's activation rows in slot s
// and zeros elsewhere, and the S products of a chunk accumulate into one output.  Output row
// 4g + i then holds strip 4g / R (of the S) at activation row (4g + i) % R, so lane (g, r) ends
// with R-row strip g * S / 4 of weight row r, and the f32 epilogue (the VALU bound of this
// kernel) runs once for S strips instead of once per strip.  Each lane streams the k-group g
// pieces of its row in all S strips and the header of its own strip, whose (dd, mm) it decodes
// itself, chunk by chunk.
template <int NSB, int S>
__device__ __forceinline__ void down_strips_q4(const Mat& D, uint32_t e, const Item& item, uint32_t arow0, uint32_t H,
                                               const long* As, const float* Sx, const float* Su, const Workspace& ws,
                                               uint32_t wv, uint32_t lane, uint32_t strips, uint32_t bx) {
    constexpr uint32_t R = 16 / S;
    const uint32_t g = lane / 16, r = lane % 16;
    const uint32_t own = g * S / 4, orow = (4 * g) % R;  // output strip (of the S) and first act row
    const uint32_t arl = r % R, sel = r / R;             // act row this lane feeds A, and for which strip
    const uint32_t nstep = (strips / 4 / S) * NSB;
    auto row_of = [&](uint32_t step, uint32_t s) -> const uint8_t* {
        const uint32_t strip = bx * strips + wv + 4 * ((step / NSB) * S + s);
        return D.ptr + (size_t)e * D.stride + (size_t)(strip * 16 + r) * D.row_bytes;
    };
    struct W {
        uint4 hdr;
        uint2 qs[S][4];
    };
    auto load = [&](uint32_t step, W& w) {
        const uint32_t sb = step % NSB;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const uint8_t* p = row_of(step, s) + sb * 144;
#pragma unroll
            for (int c = 0; c < 4; c++) w.qs[s][c] = *reinterpret_cast<const uint2*>(p + 16 + 32 * c + 8 * g);
        }
        w.hdr = *reinterpret_cast<const uint4*>(row_of(step, own) + sb * 144);
    };
    W cw;
    load(0, cw);
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const v4i z = {0, 0, 0, 0};
    for (uint32_t step = 0; step < nstep; step++) {
        const uint32_t sb = step % NSB;
        W nw = cw;
        if (step + 1 < nstep) load(step + 1, nw);
#pragma unroll
        for (int q8 = 0; q8 < 8; q8++) {
            const uint32_t q = sb * 8 + q8;
            const long af = As[q * 64 + g * 16 + arl];
            const long alo = g < 2 ? af : 0l, ahi = g < 2 ? 0l : af;
            v4i c0 = z, c1 = z;
#pragma unroll
            for (int s = 0; s < S; s++) {
                const long bw = unpack8(cw.qs[s][q8 / 2], q8 % 2);
                c0 = mfma_i8_acc(sel == (uint32_t)s ? alo : 0l, bw, c0);
                c1 = mfma_i8_acc(sel == (uint32_t)s ? ahi : 0l, bw, c1);
            }
            const float2 dm = q4k_dm_rt(cw.hdr, q8);  // sub-block q8 = 16-blocks 2 q8, 2 q8 + 1
            down_blocks_valu(acc, c0, c1, dm, Sx + (2 * q) * 16 + orow, Su + (2 * q) * 16 + orow);
        }
        cw = nw;
        if (sb == NSB - 1) {
            const uint32_t strip = bx * strips + wv + 4 * ((step / NSB) * S + own);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t row = orow + i;
                if (row < item.nrows) ws.yent[(size_t)(arow0 + row) * H + strip * 16 + r] = acc[i];
                acc[i] = 0.0f;
            }
        }
    }
}

// Q8_0 operands of one unit of 8 blocks (272 bytes, 16-byte aligned) for lane (g, r): per block c
// the 8 value bytes 8g .. 8g + 7 (unit bytes 34c + 2 + 8g: 4-byte aligned for odd c, 2 past it for
// even c, read by an aligned 12-byte load and alignbyte), and the words holding d of blocks 2g
// (low half of the word at 68g) and 2g + 1 (high half of the word at 68g + 32).
struct Q8Raw {
    v3u ev[4];   // even blocks c = 2i: 12 bytes at the 4-byte boundary 2 below the 8 value bytes
    uint2 od[4];  // odd blocks c = 2i + 1: the 8 value bytes
    uint32_t d0, d1;
};
struct Q8Sb {
    uint2 q[8];
    uint32_t d0, d1;
};
__device__ __forceinline__ void load_q8sb(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t g, Q8Raw& w) {
    const uint8_t* p = rowp + sb * 272;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        w.ev[i] = *reinterpret_cast<const v3u*>(p + 34 * (2 * i) + 8 * g);
        w.od[i] = *reinterpret_cast<const uint2*>(p + 34 * (2 * i + 1) + 2 + 8 * g);
    }
    w.d0 = *reinterpret_cast<const uint32_t*>(p + 68 * g);
    w.d1 = *reinterpret_cast<const uint32_t*>(p + 68 * g + 32);
}
__device__ __forceinline__ Q8Sb settle(const Q8Raw& r) {
    Q8Sb w;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        w.q[2 * i] = align64(r.ev[i], 2);
        w.q[2 * i + 1] = r.od[i];
    }
    w.d0 = r.d0;
    w.d1 = r.d1;
    return w;
}

// Q5_1 operands of one unit of 8 blocks (192 bytes, 16-byte aligned) for lane (g, r): per block c
// one 16-byte load, at block byte 4 for even g (qh, qs 0-11) and 8 for odd g (qs 0-15), so a lane
// holds the qs bytes whose low (g < 2) or high (g >= 2) nibbles are elements 8g .. 8g + 7; an odd
// lane takes qh from its even partner 16 lanes away (permlane16 swap) when the operand is built,
// not at load time, so the loads stay in flight.  Plus the (d, m) words of blocks 2g and 2g + 1.
struct Q51Sb {
    uint4 v[8];
    uint32_t dm0, dm1;
};
__device__ __forceinline__ void load_q51sb(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t g, Q51Sb& w) {
    const uint8_t* p = rowp + sb * 192;
#pragma unroll
    for (int c = 0; c < 8; c++) w.v[c] = *reinterpret_cast<const uint4*>(p + 24 * c + (g % 2 ? 8 : 4));
    w.dm0 = *reinterpret_cast<const uint32_t*>(p + 48 * g);
    w.dm1 = *reinterpret_cast<const uint32_t*>(p + 48 * g + 24);
}
__device__ __forceinline__ const Q51Sb& settle(const Q51Sb& w) { return w; }
// elements 8g .. 8g + 7 of block q8 as 8 bytes (q5_1_rows, blocks.py:57-68); q5_hi4 puts four qh
// bits at bit 4 of four bytes.  The swap pairs lane groups 0/1 and 2/3 and leaves, in an odd
// group's lanes, their own first word in one result and the partner's (qh) in the other: the
// partner's is the one that differs (if they are equal, either is qh).
__device__ __forceinline__ long q51_operand(const Q51Sb& w, int q8, uint32_t g) {
    const uint4 v = w.v[q8];
    const bool odd = g % 2;
    const auto sw = __builtin_amdgcn_permlane16_swap(v.x, v.x, false, false);
    const uint32_t other = sw[0] == v.x ? sw[1] : sw[0];
    const uint32_t qh = odd ? other : v.x;
    const uint32_t qlo = odd ? v.z : v.y, qhi = odd ? v.w : v.z;
    const uint32_t sh = g < 2 ? 0u : 4u, h8 = (qh >> (8 * g)) & 0xffu;
    const uint32_t lo = ((qlo >> sh) & 0x0f0f0f0fu) | q5_hi4(h8 & 0xfu);
    const uint32_t hi = ((qhi >> sh) & 0x0f0f0f0fu) | q5_hi4(h8 >> 4);
    return (long)(((unsigned long long)hi << 32) | lo);
}

// One or two items of one expert (NI): their activation rows staged side by side, every weight
// load, unpack and (dd, mm) decode shared by both (at config 4 an expert's ~60 rows make ~4 items,
// each of which otherwise re-reads and re-unpacks the expert's weights).
template <int NSB, int FK, int NI, int NS = 1>
__device__ __forceinline__ void down_items(const Mat& D, uint32_t e, const Item (&its)[NI], const uint32_t (&arow0)[NI],
                                           const Workspace& ws, uint32_t H, uint32_t strips, uint32_t bx,
                                           uint8_t* smem) {
    constexpr bool Q6 = FK == 1;
    constexpr uint32_t F = NSB * 256, nbf = NSB * 16, NQ = NSB * 8;  // NQ 32-wide chunks
    const uint32_t tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
    long* As = reinterpret_cast<long*>(smem);                          // [NI][NQ][64]
    float* Sx = reinterpret_cast<float*>(smem + NI * NQ * 64 * 8);     // [NI][nbf][16] folded scales
    float* Su = Sx + NI * nbf * 16;                                    // [NI][nbf][16] scale * sum
    static_assert(NS == 1 || NI == 1, "two strips per wave for one item");
    // (dd, mm) per row: Q6_K's 16 blocks; the other formats' 8 (a 32-block's two 16-blocks share it)
    constexpr uint32_t DS = Q6 ? DM_STRIDE : 9;
    float2* Dm = reinterpret_cast<float2*>(Su + NI * nbf * 16);        // [4 waves][NS][16][DS]
    int32_t* Ss = reinterpret_cast<int32_t*>(Dm + 4 * NS * 16 * DS);   // [NI][nbf][16] sums (Q8_0)
    long* Zr = reinterpret_cast<long*>(Ss + (FK == 2 ? NI * nbf * 16 : 0));  // [DN_ZERO] zeros

    // small Q4_K items: several strips per MFMA output (a wave owns strips / 4 strips)
    const uint32_t small = FK != 0 || NI != 1 || NS != 1 ? 0u : (its[0].nrows <= 4 && strips % 16 == 0) ? 4u
                                                   : (its[0].nrows <= 8 && strips % 8 == 0) ? 2u : 0u;
    const uint32_t g = lane / 16, r = lane % 16;
    const uint32_t nstep = (strips / 4 / NS) * NSB;
    auto strip_of = [&](uint32_t step, int s) { return bx * strips + wv + 4 * ((step / NSB) * NS + s); };
    auto row_of = [&](uint32_t step, int s) -> const uint8_t* {
        return D.ptr + (size_t)e * D.stride + (size_t)(strip_of(step, s) * 16 + r) * D.row_bytes;
    };
    using W = typename std::conditional<
            Q6, Q6Raw,
            typename std::conditional<FK == 2, Q8Raw, typename std::conditional<FK == 3, Q51Sb, Q4Sb>::type>::type>::type;
    auto load = [&](uint32_t step, int s, W& w) {
        if constexpr (Q6)
            load_q6sb(row_of(step, s), step % NSB, g, w);
        else if constexpr (FK == 2)
            load_q8sb(row_of(step, s), step % NSB, g, w);
        else if constexpr (FK == 3)
            load_q51sb(row_of(step, s), step % NSB, g, w);
        else
            load_q4sb(row_of(step, s), step % NSB, g, w);
    };
    // The items' activation rows and their scales go out together.  Entry rows are consecutive
    // from arow0; rows past an item repeat its first row.  Thread j takes row j % 16, so
    // consecutive threads fill consecutive LDS words (no bank conflicts on the stores).
#pragma unroll
    for (int it = 0; it < NI; it++) {
        uint4 av[NSB];  // 16 rows x F / 16 pieces = 256 NSB pieces of 16 bytes
        float sv[NSB], uv[NSB];
        int32_t tv[NSB];
#pragma unroll
        for (int c = 0; c < NSB; c++) {
            const uint32_t j = tid + 256 * c, t = j % 16, o = j / 16;
            const size_t row = arow0[it] + (t < its[it].nrows ? t : 0u);
            av[c] = *reinterpret_cast<const uint4*>(ws.actq + row * F + o * 16);
            sv[c] = ws.acts[row * nbf + o];  // o < nbf = 16 NSB: block o of row t
            uv[c] = ws.actu[row * nbf + o];
            if constexpr (FK == 2) tv[c] = ws.actsum[row * nbf + o];
        }
        long* A = As + it * NQ * 64;
#pragma unroll
        for (int c = 0; c < NSB; c++) {
            const uint32_t j = tid + 256 * c, t = j % 16, o = j / 16;
            // piece o = k-groups 2 (o % 2), +1 of 32-wide chunk o / 2 (MFMA operand order)
            A[(o / 2) * 64 + (o % 2) * 32 + t] = (long)(((unsigned long long)av[c].y << 32) | av[c].x);
            A[(o / 2) * 64 + (o % 2) * 32 + 16 + t] = (long)(((unsigned long long)av[c].w << 32) | av[c].z);
            Sx[(it * nbf + o) * 16 + t] = sv[c];
            Su[(it * nbf + o) * 16 + t] = uv[c];
            if constexpr (FK == 2) Ss[(it * nbf + o) * 16 + t] = tv[c];
        }
    }
    for (uint32_t i = tid; i < DN_ZERO; i += 256) Zr[i] = 0;
    __syncthreads();

    if constexpr (FK == 0 && NI == 1) {
        if (small == 4) {
            down_strips_q4<NSB, 4>(D, e, its[0], arow0[0], H, As, Sx, Su, ws, wv, lane, strips, bx);
            return;
        }
        if (small == 2) {
            down_strips_q4<NSB, 2>(D, e, its[0], arow0[0], H, As, Sx, Su, ws, wv, lane, strips, bx);
            return;
        }
    }
    W lw[NS];  // issued here rather than before the staging: held across it, it cost the Q4_K kernel a wave per SIMD
#pragma unroll
    for (int s = 0; s < NS; s++) load(0, s, lw[s]);
    float2* dmw = Dm + wv * NS * 16 * DS;
    v4f acc[NI * NS];
#pragma unroll
    for (int it = 0; it < NI * NS; it++) acc[it] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t tl = 4 * g + (r & 3);  // the row whose scales this lane feeds the rank-1 MFMAs
    for (uint32_t step = 0; step < nstep; step++) {
        const uint32_t sb = step % NSB;
        // The two MFMAs of a 32-wide chunk take its activations with the other 16-block's k-groups
        // zeroed: lanes of the other half read a zero region instead (one pointer choice per step
        // and item rather than two selects per chunk and register).
        const long* alo[NI];
        const long* ahi[NI];
#pragma unroll
        for (int it = 0; it < NI; it++) {
            const long* a = As + (it * NQ + sb * 8) * 64 + lane;
            alo[it] = g < 2 ? a : Zr;
            ahi[it] = g < 2 ? Zr : a;
        }
        typename std::decay<decltype(settle(lw[0]))>::type cws[NS];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            cws[s] = settle(lw[s]);  // this superblock's words (loaded during the previous step)
            if (step + 1 < nstep) load(step + 1, s, lw[s]);  // the next superblock's loads go out now
        }
        // (dd, mm) of the superblock's 16 blocks of row r: this lane decodes blocks 4g .. 4g+3
        wave_sync();
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const auto& cw = cws[s];
            float2* dm_s = dmw + s * 16 * DS;
            if constexpr (Q6) {
                const float d = h2f(cw.d);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float dd = f16_round(d * (float)(int8_t)((cw.sc >> (8 * i)) & 0xffu));
                    dm_s[r * DS + 4 * g + i] = make_float2(dd, f16_round(-32.0f * dd));
                }
            } else if constexpr (FK == 3) {
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {  // block 2g + jj covers 16-blocks 4g + 2jj, +1
                    const uint32_t dm = jj ? cw.dm1 : cw.dm0;
                    dm_s[r * DS + 2 * g + jj] = make_float2(h2f((uint16_t)(dm & 0xffffu)), h2f((uint16_t)(dm >> 16)));
                }
            } else if constexpr (FK == 2) {
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {  // block 2g + jj covers 16-blocks 4g + 2jj, +1
                    const float dd = h2f((uint16_t)(jj ? cw.d1 >> 16 : cw.d0 & 0xffffu));
                    dm_s[r * DS + 2 * g + jj] = make_float2(dd, f16_round(-128.0f * dd));
                }
            } else {
#pragma unroll
                for (int jj = 0; jj < 2; jj++)  // sub-block 2g + jj covers blocks 4g + 2jj, +1
                    dm_s[r * DS + 2 * g + jj] = q4k_dm_rt(cw.hdr, 2 * g + jj);
            }
        }
        wave_sync();
#pragma unroll
        for (int q8 = 0; q8 < 8; q8++) {  // 32-wide chunks of the superblock = block pairs
            const uint32_t q = sb * 8 + q8;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const auto& cw = cws[s];
                long bw;
                if constexpr (Q6)
                    bw = q6_operand(cw, q8);
                else if constexpr (FK == 2)
                    bw = (long)(((unsigned long long)cw.q[q8].y << 32) | cw.q[q8].x);
                else if constexpr (FK == 3)
                    bw = q51_operand(cw, q8, g);
                else
                    bw = unpack8(cw.qs[q8 / 2], q8 % 2);
                const float2* dm_s = dmw + s * 16 * DS;
                const float2 d0 = Q6 ? dm_s[r * DS + 2 * q8] : dm_s[r * DS + q8];
                const float2 d1 = Q6 ? dm_s[r * DS + 2 * q8 + 1] : d0;
#pragma unroll
                for (int it = 0; it < NI; it++) {
                    v4i c0 = mfma_i8(alo[it][q8 * 64], bw), c1 = mfma_i8(ahi[it][q8 * 64], bw);
                    const float* sx = Sx + (it * nbf + 2 * q) * 16;
                    const float* su = Su + (it * nbf + 2 * q) * 16;
                    if constexpr (FK == 2) {
                        const int4 t0 = *reinterpret_cast<const int4*>(Ss + (it * nbf + 2 * q) * 16 + 4 * g);
                        const int4 t1 = *reinterpret_cast<const int4*>(Ss + (it * nbf + 2 * q + 1) * 16 + 4 * g);
                        c0 += v4i{t0.x, t0.y, t0.z, t0.w} * 128;
                        c1 += v4i{t1.x, t1.y, t1.z, t1.w} * 128;
                    }
                    // Q6_K and Q4_K: the chain's fma with mm on the matrix cores too, where other waves'
                    // VALU work overlaps it (config 4 Q6_K down 379-386 -> 371-372 us, M = 512 Q4_K
                    // 114.5 -> 112.5 us at four waves per SIMD); Q8_0 / Q5_1 keep it on the VALU
                    if constexpr (Q6 || FK == 0)
                        down_blocks_mc(acc[s * NI + it], c0, c1, d0, d1, sx + tl, su + tl);
                    else
                        down_blocks(acc[s * NI + it], c0, c1, d0, d1, sx + tl, su + 4 * g);
                }
            }
        }
        if (sb == NSB - 1) {
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const uint32_t strip = strip_of(step, s);
#pragma unroll
                for (int it = 0; it < NI; it++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t row = 4 * g + i;
                        if (row < its[it].nrows)
                            ws.yent[(size_t)(arow0[it] + row) * H + strip * 16 + r] = acc[s * NI + it][i];
                        acc[s * NI + it][i] = 0.0f;
                    }
            }
        }
    }
}

// FK: 0 Q4_K, 1 Q6_K, 2 Q8_0, 3 Q5_1.  Q8_0's MFMA runs on the signed bytes; the unsigned dot of
// q8_0_rows' form (blocks.py:71-78) adds 128 times the activation block's sum, in int32.
// PR = 2 (large batches): the items of one expert pair up as (part 2j, 2j + 1); a pair runs in the
// first item's workgroup as one group sharing the weights (the second's exits at once), other
// items alone.  Config 4's Q6_K down 416 -> 400 us against pairs by item index (2p, 2p + 1).
//
// Q6_K's registers are held to four waves per SIMD (config 4's down 461 -> 450 us); the other
// formats keep the compiler's allocation (held to four, the Q4_K small-item paths spill and the
// M = 512 down slows from 125.7 to 128-130 us).
template <int NSB, int FK, int PR>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(FK <= 1 ? 4 : 1))) void batch_down_kernel(
        Mat down, Mat shd, Workspace ws, uint32_t skip_rows) {
    const uint32_t H = down.rows, n_items = ws.n_groups[2], n_ent = ws.n_groups[1];
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t strips = H / 16 / gridDim.x;
    uint32_t bx, grp;  // column block and item, in XCD order
    if (!xcd_order(n_items, bx, grp)) return;
    auto item_args = [&](const Item& it, uint32_t& e, uint32_t& arow0) -> const Mat& {
        const bool shared = it.expert == NO_EXPERT;
        e = shared ? 0u : it.expert;
        arow0 = shared ? n_ent + it.row0 : it.row0;
        return shared ? shd : down;
    };
#ifndef TRK_DN_NS
#define TRK_DN_NS 2
#endif
    auto one = [&](uint32_t itn) {
        const Item its[1] = {ws.items[itn]};
        if (its[0].nrows <= skip_rows) return;  // a streaming-GEMV item (k_stream.hip)
        uint32_t e, a0[1];
        const Mat& D = item_args(its[0], e, a0[0]);
        // a wave walks two of its strips at once (two chains) unless the item takes a small-item
        // path (Q4_K, <= 8 rows); Q6_K stays at one: its four waves per SIMD leave no registers
        // for a second chain
        const bool small = FK == 0 && its[0].nrows <= 8;
        if constexpr (TRK_DN_NS == 2 && FK != 1) {
            if (!small && strips % 8 == 0) {
                down_items<NSB, FK, 1, 2>(D, e, its, a0, ws, H, strips, bx, smem);
                return;
            }
        }
        down_items<NSB, FK, 1, 1>(D, e, its, a0, ws, H, strips, bx, smem);
    };
    auto pair = [&](const Item& a, const Item& b) {  // consecutive items a, b that run as a pair
        return b.expert == a.expert && a.nrows > skip_rows && b.nrows > skip_rows &&
               (FK != 0 || (a.nrows > 8 && b.nrows > 8));
    };
    if constexpr (PR == 1) {
        one(grp);
    } else {
        // the items of one expert pair up as (part 2j, 2j + 1), run by the first item's workgroup
        const Item it = ws.items[grp];
        if (it.part % 2) {
            const Item pv = ws.items[grp - 1];
            if (pv.part + 1 == it.part && pair(pv, it)) return;
        } else if (grp + 1 < n_items) {
            const Item nx = ws.items[grp + 1];
            if (nx.part == it.part + 1 && pair(it, nx)) {
                const Item its[2] = {it, nx};
                uint32_t e, a0[2], e1;
                const Mat& D = item_args(it, e, a0[0]);
                item_args(nx, e1, a0[1]);
                down_items<NSB, FK, 2>(D, e, its, a0, ws, H, strips, bx, smem);
                return;
            }
        }
        one(grp);
    }
}

hipError_t launch_batch_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m, uint32_t skip_rows,
                             hipStream_t st) {
    const uint32_t H = down.rows, F = down.k, nbf = F / 16, NQ = F / 32;
    // item pairs sharing the weights where an expert has several items (config 4: ~4 per expert)
    const int pr = geo::down_pairs(m) ? 2 : 1;
    const int fk = down.fmt == TRK_FMT_Q6_K ? 1 : down.fmt == TRK_FMT_Q8_0 ? 2 : down.fmt == TRK_FMT_Q5_1 ? 3 : 0;
    // per item: activations, scales, scale * sum and (Q8_0) the sums; the (dd, mm) tables of four
    // waves for two strips each (one for Q6_K, which walks one strip at a time); the zero region.
    // Q6_K: 36.5 KB at F = 512, four workgroups per CU (the four waves per SIMD it is held to)
    const size_t lds = (size_t)pr * ((size_t)NQ * 64 * 8 + (size_t)nbf * 16 * (fk == 2 ? 12 : 8)) +
                       4 * (fk == 1 ? 1 : 2) * 16 * (fk == 1 ? DM_STRIDE : 9) * 8 + DN_ZERO * 8;
    const uint32_t rows = grouped_item_rows(ws, m);
    const dim3 grid(geo::mfma_down_cols(m, H), rows);
    if (down.fmt != sh_down.fmt) return hipErrorInvalidValue;  // one format per layer
    switch ((F / 256 * 4 + fk) * 2 + pr - 1) {
#define DN_CASE(n, f)                                                                                          \
    case (n * 4 + f) * 2: batch_down_kernel<n, f, 1><<<grid, 256, lds, st>>>(down, sh_down, ws, skip_rows); break; \
    case (n * 4 + f) * 2 + 1: batch_down_kernel<n, f, 2><<<grid, 256, lds, st>>>(down, sh_down, ws, skip_rows); break;
#define DN_F(n) DN_CASE(n, 0) DN_CASE(n, 1) DN_CASE(n, 2) DN_CASE(n, 3)
        DN_F(1) DN_F(2) DN_F(3) DN_F(4) DN_F(5) DN_F(6) DN_F(7) DN_F(8)
#undef DN_F
#undef DN_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- combine ----------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void batch_combine_kernel(Workspace ws, uint32_t m, float* __restrict__ out,
                                                           int residual) {
    const uint32_t t = blockIdx.x, H = ws.H, tid = threadIdx.x;
    __shared__ uint32_t pos[K_MAX];
    const uint32_t ns = ws.n_sel[t];
    const uint32_t n_ent = ws.n_groups[1];
    if (tid < 64) {
        // the token's entry positions (distinct), ranked: entries are sorted by (expert, token), so
        // ascending position = ascending expert
        const uint32_t v = tid < ns ? ws.ent_of[(size_t)t * K_MAX + tid] : 0xffffffffu;
        uint32_t rank = 0;
        for (uint32_t s2 = 0; s2 < ns; s2++) rank += (uint32_t)__builtin_amdgcn_readlane((int)v, (int)s2) < v ? 1u : 0u;
        if (tid < ns) pos[rank] = v;
    }
    __syncthreads();
    const uint32_t H4 = H / 4;
    for (uint32_t c = tid; c < H4; c += blockDim.x) {
        // a pack written for T tiles: each tile's sum is its partial, the partials summed in tile
        // order (exec_batch.rs:821-849)
        float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t tl = 0; tl < ws.tiles; tl++) {
            const float4* y4 = reinterpret_cast<const float4*>(ws.yent + (size_t)tl * ws.yent_tile);
            float4 p = y4[(size_t)(n_ent + t) * H4 + c];
#pragma unroll 4
            for (uint32_t j = 0; j < ns; j++) {
                const float4 v = y4[(size_t)pos[j] * H4 + c];
                p.x = p.x + v.x;
                p.y = p.y + v.y;
                p.z = p.z + v.z;
                p.w = p.w + v.w;
            }
            if (tl == 0)
                y = p;
            else
                y = make_float4(y.x + p.x, y.y + p.y, y.z + p.z, y.w + p.w);
        }
        float4* o = reinterpret_cast<float4*>(out + (size_t)t * H) + c;
        if (residual) {
            const float4 h = *o;
            y = make_float4(h.x + y.x, h.y + y.y, h.z + y.z, h.w + y.w);
        }
        *o = y;
    }
}

hipError_t launch_batch_combine(const Workspace& ws, uint32_t m, float* out, int residual, hipStream_t st) {
    batch_combine_kernel<<<m, 256, 0, st>>>(ws, m, out, residual);
    return hipGetLastError();
}

}  // namespace trk
