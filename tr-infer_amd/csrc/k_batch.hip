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

namespace trk {

constexpr uint32_t BR = 64;  // entry rows per work item: 4 waves x one 16-row MFMA tile
constexpr uint32_t DISPATCH_WAVES = 8;
constexpr uint32_t NO_EXPERT = 0xffffffffu;

__device__ __forceinline__ uint32_t popc64(unsigned long long v) { return (uint32_t)__popcll(v); }

// single workgroup (DISPATCH_WAVES waves)
__global__ __launch_bounds__(DISPATCH_WAVES * 64) void dispatch_kernel(Workspace ws, uint32_t m) {
    const uint32_t E = ws.E, tid = threadIdx.x, nt = blockDim.x;
    const uint32_t wv = tid / 64, lane = tid % 64;
    extern __shared__ __align__(16) uint8_t smem[];
    uint32_t* cnt = (uint32_t*)smem;                  // [E]
    uint32_t* start = cnt + E;                        // [E]
    uint32_t* run = start + E;                        // [E]
    uint32_t* gidx = run + E;                         // [E]
    uint32_t* off = gidx + E;                         // [W][E]
    uint32_t* scan_tmp = off + DISPATCH_WAVES * E;    // [2][E]
    uint32_t* masks = scan_tmp + 2 * E;               // [W][E][2] (64-bit token masks as 2 words)

    for (uint32_t e = tid; e < E; e += nt) cnt[e] = 0;
    __syncthreads();
    for (uint32_t t = tid; t < m; t += nt) {
        const uint32_t ns = ws.n_sel[t];
        for (uint32_t s = 0; s < ns; s++) atomicAdd(&cnt[ws.ids[(size_t)t * K_MAX + s]], 1u);
    }
    __syncthreads();
    // exclusive scans over experts: entry starts, and group index of each non-empty expert
    // (Hillis-Steele in LDS; E <= 1024)
    for (uint32_t e = tid; e < E; e += nt) {
        scan_tmp[e] = cnt[e];
        scan_tmp[E + e] = cnt[e] ? 1u : 0u;
    }
    __syncthreads();
    for (uint32_t d = 1; d < E; d <<= 1) {
        uint32_t a[4], b[4];
        uint32_t j = 0;
        for (uint32_t e = tid; e < E; e += nt, j++) {
            a[j] = scan_tmp[e] + (e >= d ? scan_tmp[e - d] : 0u);
            b[j] = scan_tmp[E + e] + (e >= d ? scan_tmp[E + e - d] : 0u);
        }
        __syncthreads();
        j = 0;
        for (uint32_t e = tid; e < E; e += nt, j++) {
            scan_tmp[e] = a[j];
            scan_tmp[E + e] = b[j];
        }
        __syncthreads();
    }
    for (uint32_t e = tid; e < E; e += nt) {
        start[e] = scan_tmp[e] - cnt[e];
        run[e] = start[e];
        gidx[e] = scan_tmp[E + e] - (cnt[e] ? 1u : 0u);
    }
    const uint32_t n_ent = scan_tmp[E - 1];
    const uint32_t ng = scan_tmp[2 * E - 1];
    __syncthreads();

    // rank-within-expert scatter, 64 tokens per wave, DISPATCH_WAVES chunks per round
    const uint32_t nchunks = (m + 63) / 64;
    for (uint32_t c0 = 0; c0 < nchunks; c0 += DISPATCH_WAVES) {
        for (uint32_t i = tid; i < DISPATCH_WAVES * E * 2; i += nt) masks[i] = 0;
        __syncthreads();
        const uint32_t c = c0 + wv, t = c * 64 + lane;
        const bool live = c < nchunks && t < m;
        const uint32_t ns = live ? ws.n_sel[t] : 0u;
        for (uint32_t s = 0; s < ns; s++) {
            const uint32_t e = ws.ids[(size_t)t * K_MAX + s];
            atomicOr(&masks[(wv * E + e) * 2 + (lane >> 5)], 1u << (lane & 31));
        }
        __syncthreads();
        for (uint32_t e = tid; e < E; e += nt) {
            uint32_t r = run[e];
            for (uint32_t w = 0; w < DISPATCH_WAVES; w++) {
                off[w * E + e] = r;
                r += __popc(masks[(w * E + e) * 2]) + __popc(masks[(w * E + e) * 2 + 1]);
            }
            run[e] = r;
        }
        __syncthreads();
        const unsigned long long below = lane ? ((1ull << lane) - 1ull) : 0ull;
        for (uint32_t s = 0; s < ns; s++) {
            const uint32_t e = ws.ids[(size_t)t * K_MAX + s];
            const unsigned long long mk = (unsigned long long)masks[(wv * E + e) * 2] |
                                          ((unsigned long long)masks[(wv * E + e) * 2 + 1] << 32);
            const uint32_t pos = off[wv * E + e] + popc64(mk & below);
            ws.ent_tok[pos] = t;
            ws.ent_w[pos] = ws.w[(size_t)t * K_MAX + s];
            ws.ent_exp[pos] = e;
            ws.ent_of[(size_t)t * K_MAX + s] = pos;
        }
        __syncthreads();
    }
    // group table (only non-empty experts, ascending) and work items
    for (uint32_t e = tid; e < E; e += nt)
        if (cnt[e]) {
            ws.grp_start[gidx[e]] = start[e];
            ws.grp_exp[gidx[e]] = e;
        }
    // items: chunks of BR rows per group, then the shared expert over the tokens
    for (uint32_t e = tid; e < E; e += nt) scan_tmp[e] = (cnt[e] + BR - 1) / BR;
    __syncthreads();
    for (uint32_t d = 1; d < E; d <<= 1) {
        uint32_t a[4];
        uint32_t j = 0;
        for (uint32_t e = tid; e < E; e += nt, j++) a[j] = scan_tmp[e] + (e >= d ? scan_tmp[e - d] : 0u);
        __syncthreads();
        j = 0;
        for (uint32_t e = tid; e < E; e += nt, j++) scan_tmp[e] = a[j];
        __syncthreads();
    }
    const uint32_t n_routed_items = scan_tmp[E - 1];
    for (uint32_t e = tid; e < E; e += nt) {
        const uint32_t nc = (cnt[e] + BR - 1) / BR;
        uint32_t o = scan_tmp[e] - nc;
        for (uint32_t c = 0; c < nc; c++) {
            const uint32_t r0 = start[e] + c * BR;
            const uint32_t nr = cnt[e] - c * BR < BR ? cnt[e] - c * BR : BR;
            ws.items[o + c] = Item{e, r0, nr, 0};
        }
    }
    const uint32_t n_sh = (m + BR - 1) / BR;
    for (uint32_t c = tid; c < n_sh; c += nt) {
        const uint32_t r0 = c * BR;
        ws.items[n_routed_items + c] = Item{NO_EXPERT, r0, m - r0 < BR ? m - r0 : BR, 0};
    }
    if (tid == 0) {
        ws.grp_start[ng] = n_ent;
        ws.n_groups[0] = ng;
        ws.n_groups[1] = n_ent;
        ws.n_groups[2] = n_routed_items + n_sh;
    }
}

hipError_t launch_dispatch(const Workspace& ws, uint32_t m, hipStream_t st) {
    const size_t E = ws.E;
    size_t lds = (4 * E + DISPATCH_WAVES * E + 2 * E + DISPATCH_WAVES * E * 2) * 4;
    dispatch_kernel<<<1, DISPATCH_WAVES * 64, lds, st>>>(ws, m);
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

// Token (activation row) of entry row `row` of an item; rows past the item reuse its first row
// (their outputs are never stored).
__device__ __forceinline__ uint32_t item_token(const Workspace& ws, const Item& it, bool shared, uint32_t row) {
    const uint32_t r = row < it.nrows ? row : 0u;
    return shared ? it.row0 + r : ws.ent_tok[it.row0 + r];
}

// gate/up + SwiGLU + per-16 requantisation + weight fold (tasks A and B of moe_batch).
// Workgroup: one item (<= 64 entry rows, a 16-row tile per wave) x one 16-row strip of F (16 gate
// rows and 16 up rows staged in LDS).  NSB = H / 256 superblocks per weight row.
template <int NSB>
__global__ __launch_bounds__(256) void batch_gateup_kernel(Mat gate, Mat up, Mat shg, Mat shu, Workspace ws) {
    constexpr uint32_t H = NSB * 256, nb = NSB * 8, rb = NSB * 144, rbp = rb + 16;  // padded LDS row
    constexpr uint32_t PER = rb;  // uint4 per 16-row strip of one matrix (contiguous rows)
    constexpr uint32_t NL = (2 * PER + 255) / 256;
    const uint32_t F = gate.rows, nbf = F / 16;
    const uint32_t strip = blockIdx.x, itn = blockIdx.y, tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
    if (itn >= ws.n_groups[2]) return;
    const Item item = ws.items[itn];
    const bool shared = item.expert == NO_EXPERT;
    const uint32_t n_ent = ws.n_groups[1];
    const Mat& G = shared ? shg : gate;
    const Mat& U = shared ? shu : up;
    const uint32_t e = shared ? 0u : item.expert;

    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t* wts = smem;                              // [32][rbp]: 16 gate rows, then 16 up rows
    float2* dm = (float2*)(smem + 32 * rbp);          // [32][nb] (dd, mm)

    {
        const uint8_t* src0 = G.ptr + (size_t)e * G.stride + (size_t)strip * 16 * rb;
        const uint8_t* src1 = U.ptr + (size_t)e * U.stride + (size_t)strip * 16 * rb;
        uint4 t[NL];
#pragma unroll
        for (uint32_t l = 0; l < NL; l++) {
            const uint32_t i = tid + 256 * l < 2 * PER ? tid + 256 * l : 0u;  // clamped: always a valid load
            t[l] = *reinterpret_cast<const uint4*>((i < PER ? src0 : src1) + (i % PER) * 16);
        }
#pragma unroll
        for (uint32_t l = 0; l < NL; l++) {
            const uint32_t i = tid + 256 * l;
            if (i < 2 * PER) {
                const uint32_t mat = i / PER, o = (i % PER) * 16;
                *reinterpret_cast<uint4*>(wts + (mat * 16 + o / rb) * rbp + o % rb) = t[l];
            }
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < 32 * NSB; i += blockDim.x) {
        const uint32_t r = i / NSB, sb = i % NSB;
        const uint8_t* hb = wts + r * rbp + sb * 144;
        const float d = h2f(ld16(hb)), dmin = h2f(ld16(hb + 2));
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            q4k_scale_min(hb + 4, j, sc, mn);
            float a, b;
            q4k_dm(d, dmin, sc, mn, a, b);
            dm[r * nb + sb * 8 + j] = make_float2(a, b);
        }
    }
    __syncthreads();

    // Per-superblock entry scales (sx and u = sx * sum of the item's 64 entry rows) pass through a
    // double-buffered LDS stage: every thread moves one float4 per superblock.
    float* scl = reinterpret_cast<float*>(dm + 32 * nb);  // [2][64 entries][16]: sx[8] | u[8]
    const uint32_t le = tid / 4, lp = tid % 4;
    const float* lsrc = (lp < 2 ? ws.xs : ws.xu) + (size_t)item_token(ws, item, shared, le) * nb + (lp & 1) * 4;
    auto scl_load = [&](uint32_t sb) { return *reinterpret_cast<const float4*>(lsrc + sb * 8); };
    auto scl_store = [&](uint32_t buf, float4 v) {
        *reinterpret_cast<float4*>(scl + buf * 1024 + le * 16 + lp * 4) = v;
    };

    const uint32_t t0 = wv * 16;
    const bool active = t0 < item.nrows;  // waves past the item still stage scales
    const uint32_t g = lane / 16, f = lane % 16;
    const int8_t* xa = ws.xq + (size_t)item_token(ws, item, shared, t0 + f) * H + 8 * g;
    float accg[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accu[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint8_t* wg = wts + f * rbp + 16 + 8 * g;
    const uint8_t* wu = wts + (16 + f) * rbp + 16 + 8 * g;
    long a0[8], a1[8];  // A operands of a superblock (8 chunks), one superblock ahead
    auto fetch_a = [&](uint32_t sb, long* a) {
#pragma unroll
        for (int j = 0; j < 8; j++) a[j] = *reinterpret_cast<const long*>(xa + sb * 256 + 32 * j);
    };
    auto step = [&](uint32_t sb, const long* a) {
        const float* sc = scl + (sb & 1) * 1024 + (t0 + 4 * g) * 16;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint2 pg = *reinterpret_cast<const uint2*>(wg + sb * 144 + 32 * c);
            const uint2 pu = *reinterpret_cast<const uint2*>(wu + sb * 144 + 32 * c);
            float2 sxv[4], suv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sxv[i] = *reinterpret_cast<const float2*>(sc + i * 16 + 2 * c);
                suv[i] = *reinterpret_cast<const float2*>(sc + i * 16 + 8 + 2 * c);
            }
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int j = 2 * c + h;
                const v4i cg = mfma_i8(a[j], unpack8(pg, h));
                const v4i cu = mfma_i8(a[j], unpack8(pu, h));
                const float2 dg = dm[f * nb + sb * 8 + j], du = dm[(16 + f) * nb + sb * 8 + j];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float sx = h ? sxv[i].y : sxv[i].x, u = h ? suv[i].y : suv[i].x;
                    const float tg = dg.x * sx, tu = du.x * sx;
                    accg[i] = __builtin_fmaf(dg.y, u, accg[i]);
                    accg[i] = __builtin_fmaf((float)cg[i], tg, accg[i]);
                    accu[i] = __builtin_fmaf(du.y, u, accu[i]);
                    accu[i] = __builtin_fmaf((float)cu[i], tu, accu[i]);
                }
            }
        }
    };
    scl_store(0, scl_load(0));
    if (active) fetch_a(0, a0);
    __syncthreads();
#pragma unroll 1
    for (uint32_t sb = 0; sb < NSB; sb += 2) {
        const float4 n1 = sb + 1 < NSB ? scl_load(sb + 1) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (active && sb + 1 < NSB) fetch_a(sb + 1, a1);
        if (active) step(sb, a0);
        if (sb + 1 < NSB) scl_store(1, n1);
        __syncthreads();
        if (sb + 1 < NSB) {
            const float4 n2 = sb + 2 < NSB ? scl_load(sb + 2) : make_float4(0.f, 0.f, 0.f, 0.f);
            if (active && sb + 2 < NSB) fetch_a(sb + 2, a0);
            if (active) step(sb + 1, a1);
            if (sb + 2 < NSB) scl_store(0, n2);
            __syncthreads();
        }
    }
    if (!active) return;
    // SwiGLU (elem.rs:173) and per-16 quantisation across the 16 lanes holding one entry's strip
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = t0 + 4 * g + i;
        const float v = silu512(accg[i]) * accu[i];
        // the 16 lanes of an entry's strip are one DPP row (lanes 16g .. 16g+15)
        const float amax = row16_allreduce(__builtin_fabsf(v), [](float a, float b) { return mx_ps(a, b); });
        const float s = amax / 127.0f;
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        const int32_t qi = cvt_rne(v * inv);
        const int32_t sum = row16_allreduce(qi, [](int32_t a, int32_t b) { return a + b; });
        if (row < item.nrows) {
            const uint32_t arow = shared ? n_ent + item.row0 + row : item.row0 + row;
            ws.actq[(size_t)arow * F + strip * 16 + f] = sat_i8(qi);
            if (f == 0) {
                const float wgt = shared ? sigmoid_libm(ws.shl[item.row0 + row]) : ws.ent_w[item.row0 + row];
                const float sf = s * wgt;  // exec_batch.rs:1533-1535
                ws.acts[(size_t)arow * nbf + strip] = sf;
                ws.actsum[(size_t)arow * nbf + strip] = sum;
                ws.actu[(size_t)arow * nbf + strip] = sf * (float)sum;
            }
        }
    }
}

hipError_t launch_batch_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up,
                               const Workspace& ws, uint32_t m, hipStream_t st) {
    const uint32_t H = gate.k, F = gate.rows, nb = H / 32;
    const size_t lds = 32 * (size_t)(gate.row_bytes + 16) + 32 * (size_t)nb * 8 + 2 * 64 * 16 * 4;
    const dim3 grid(F / 16, ws.item_cap);
    switch (H / 256) {
#define GU_CASE(n) \
    case n: batch_gateup_kernel<n><<<grid, 256, lds, st>>>(gate, up, sh_gate, sh_up, ws); break;
        GU_CASE(1) GU_CASE(2) GU_CASE(3) GU_CASE(4) GU_CASE(5) GU_CASE(6) GU_CASE(7) GU_CASE(8) GU_CASE(9)
        GU_CASE(10) GU_CASE(11) GU_CASE(12) GU_CASE(13) GU_CASE(14) GU_CASE(15) GU_CASE(16)
#undef GU_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- down ---------------------------------------------------------------------------------------
//
// Workgroup: one item x 64 rows of H (4 MFMA column tiles).  The down input is quantised per 16,
// so each 32-byte activation chunk feeds two MFMAs with the other half of its k-groups zeroed,
// giving the exact dot of each 16-block.  Q6_K superblocks are re-laid to 224 bytes in LDS so
// that every 8-byte operand read is aligned.

constexpr uint32_t DN_COLS = 64;

__device__ __forceinline__ long q6k_operand(const uint8_t* sbp, uint32_t q8, uint32_t g) {
    // 8 consecutive values e = 32*q8 + 8g .. +7 of a superblock: ql nibble, qh 2-bit field
    const uint32_t n = q8 / 4, g6 = q8 % 4;
    const uint2 lo = *reinterpret_cast<const uint2*>(sbp + 64 * n + 32 * (g6 & 1) + 8 * g);
    const uint2 hi = *reinterpret_cast<const uint2*>(sbp + 128 + 32 * n + 8 * g);
    const int sh = (g6 >> 1) ? 4 : 0;
    const uint32_t l0 = (lo.x >> sh) & 0x0f0f0f0fu, l1 = (lo.y >> sh) & 0x0f0f0f0fu;
    const uint32_t h0 = (hi.x >> (2 * g6)) & 0x03030303u, h1 = (hi.y >> (2 * g6)) & 0x03030303u;
    return (long)(((unsigned long long)(l1 | (h1 << 4)) << 32) | (l0 | (h0 << 4)));
}

template <int NSB>
__global__ __launch_bounds__(256) void batch_down_kernel(Mat down, Mat shd, Workspace ws) {
    constexpr uint32_t F = NSB * 256, nbf = NSB * 16, NQ = NSB * 8;  // NQ 32-wide chunks
    const uint32_t H = down.rows;
    const uint32_t strip = blockIdx.x, itn = blockIdx.y, tid = threadIdx.x, wv = tid / 64, lane = tid % 64;
    if (itn >= ws.n_groups[2]) return;
    const Item item = ws.items[itn];
    const bool shared = item.expert == NO_EXPERT;
    const uint32_t n_ent = ws.n_groups[1];
    const Mat& D = shared ? shd : down;
    const uint32_t e = shared ? 0u : item.expert;
    const bool q6 = D.fmt == TRK_FMT_Q6_K;
    const uint32_t sbb = q6 ? 224u : 144u;          // LDS bytes per superblock
    const uint32_t rbp = NSB * sbb + 16;            // padded LDS row stride
    const uint32_t arow0 = shared ? n_ent + item.row0 : item.row0;

    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t* wts = smem;                                  // [64][rbp]
    float2* dm = (float2*)(smem + DN_COLS * rbp);         // [64][nbf] (dd, mm)

    const uint8_t* src = D.ptr + (size_t)e * D.stride + (size_t)strip * DN_COLS * D.row_bytes;
    if (!q6) {
        constexpr uint32_t rb = NSB * 144, PER = DN_COLS * rb / 16;
#pragma unroll 8
        for (uint32_t i = tid; i < PER; i += 256)
            *reinterpret_cast<uint4*>(wts + (i * 16 / rb) * rbp + (i * 16) % rb) =
                reinterpret_cast<const uint4*>(src)[i];
    } else {
        const uint32_t per = DN_COLS * NSB * 105;  // 2-byte words
        for (uint32_t i = tid; i < per; i += blockDim.x) {
            const uint32_t r = i / (NSB * 105), rem = i % (NSB * 105), sb = rem / 105, w = rem % 105;
            reinterpret_cast<uint16_t*>(wts + r * rbp + sb * sbb)[w] =
                reinterpret_cast<const uint16_t*>(src + (size_t)r * D.row_bytes + sb * 210)[w];
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < DN_COLS * NSB; i += blockDim.x) {
        const uint32_t r = i / NSB, sb = i % NSB;
        const uint8_t* hb = wts + r * rbp + sb * sbb;
        if (!q6) {
            const float d = h2f(ld16(hb)), dmin = h2f(ld16(hb + 2));
#pragma unroll
            for (int j = 0; j < 8; j++) {
                int sc, mn;
                q4k_scale_min(hb + 4, j, sc, mn);
                float a, b;
                q4k_dm(d, dmin, sc, mn, a, b);
                dm[r * nbf + sb * 16 + 2 * j] = make_float2(a, b);
                dm[r * nbf + sb * 16 + 2 * j + 1] = make_float2(a, b);
            }
        } else {
            const float d = h2f(ld16(hb + 208));
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float a = f16_round(d * (float)(int8_t)hb[192 + j]);
                dm[r * nbf + sb * 16 + j] = make_float2(a, f16_round(-32.0f * a));
            }
        }
    }
    __syncthreads();

    // the item's activation scales (folded sx and u) for all nbf blocks, staged once
    float2* scl = reinterpret_cast<float2*>(dm + DN_COLS * nbf);  // [64 entries][nbf] (sx, u)
#pragma unroll 8
    for (uint32_t i = tid; i < 64 * nbf; i += 256) {
        const uint32_t r = i / nbf, b = i % nbf;
        const size_t row = (size_t)arow0 + (r < item.nrows ? r : 0u);
        scl[i] = make_float2(ws.acts[row * nbf + b], ws.actu[row * nbf + b]);
    }
    __syncthreads();

    const uint32_t t0 = wv * 16;
    if (t0 >= item.nrows) return;  // no barrier below
    const uint32_t g = lane / 16, f = lane % 16;
    const uint32_t ra = t0 + f < item.nrows ? t0 + f : 0u;  // A row (entry) of this lane
    const int8_t* xa = ws.actq + (size_t)(arow0 + ra) * F + 8 * g;
    const float2* sce = scl + (t0 + 4 * g) * nbf;  // this lane's 4 entries
    float acc[4][4];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[c][i] = 0.0f;
    auto step = [&](uint32_t q, long af) {
        const long alo = g < 2 ? af : 0l, ahi = g < 2 ? 0l : af;
        const uint32_t sb = q / 8, q8 = q % 8;
        float2 s0[4], s1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s0[i] = sce[i * nbf + 2 * q];
            s1[i] = sce[i * nbf + 2 * q + 1];
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint8_t* sbp = wts + (c * 16 + f) * rbp + sb * sbb;
            long b;
            if (!q6) {
                const uint2 p = *reinterpret_cast<const uint2*>(sbp + 16 + 32 * (q8 / 2) + 8 * g);
                b = unpack8(p, (int)(q8 % 2));
            } else {
                b = q6k_operand(sbp, q8, g);
            }
            const v4i c0 = mfma_i8(alo, b), c1 = mfma_i8(ahi, b);
            const float2 d0 = dm[(c * 16 + f) * nbf + 2 * q], d1 = dm[(c * 16 + f) * nbf + 2 * q + 1];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[c][i] = __builtin_fmaf(d0.y, s0[i].y, acc[c][i]);
                acc[c][i] = __builtin_fmaf((float)c0[i], d0.x * s0[i].x, acc[c][i]);
                acc[c][i] = __builtin_fmaf(d1.y, s1[i].y, acc[c][i]);
                acc[c][i] = __builtin_fmaf((float)c1[i], d1.x * s1[i].x, acc[c][i]);
            }
        }
    };
    long af0 = *reinterpret_cast<const long*>(xa), af1;
#pragma unroll 1
    for (uint32_t q = 0; q < NQ; q += 2) {  // 32-wide chunks = block pairs (2q, 2q+1); NQ is even
        af1 = *reinterpret_cast<const long*>(xa + 32 * (q + 1));
        step(q, af0);
        if (q + 2 < NQ) af0 = *reinterpret_cast<const long*>(xa + 32 * (q + 2));
        step(q + 1, af1);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t r = t0 + 4 * g + i;
        if (r < item.nrows) {
            float* y = ws.yent + (size_t)(arow0 + r) * H + strip * DN_COLS + f;
#pragma unroll
            for (int c = 0; c < 4; c++) y[c * 16] = acc[c][i];
        }
    }
}

hipError_t launch_batch_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m, hipStream_t st) {
    const uint32_t H = down.rows, F = down.k, nsb = F / 256, nbf = F / 16;
    const bool q6 = down.fmt == TRK_FMT_Q6_K || sh_down.fmt == TRK_FMT_Q6_K;
    const size_t rbp = nsb * (q6 ? 224 : 144) + 16;
    const size_t lds = DN_COLS * rbp + (size_t)DN_COLS * nbf * 8 + (size_t)64 * nbf * 8;
    const dim3 grid(H / DN_COLS, ws.item_cap);
    switch (nsb) {
#define DN_CASE(n) \
    case n: batch_down_kernel<n><<<grid, 256, lds, st>>>(down, sh_down, ws); break;
        DN_CASE(1) DN_CASE(2) DN_CASE(3) DN_CASE(4) DN_CASE(5) DN_CASE(6) DN_CASE(7) DN_CASE(8)
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
    __shared__ uint32_t np;
    if (tid == 0) {
        const uint32_t ns = ws.n_sel[t];
        // entries are sorted by (expert, token): ascending position = ascending expert
        for (uint32_t s = 0; s < ns; s++) {
            uint32_t v = ws.ent_of[(size_t)t * K_MAX + s];
            int j = (int)s - 1;
            while (j >= 0 && pos[j] > v) {
                pos[j + 1] = pos[j];
                j--;
            }
            pos[j + 1] = v;
        }
        np = ns;
    }
    __syncthreads();
    const uint32_t n_ent = ws.n_groups[1];
    for (uint32_t c = tid; c < H; c += blockDim.x) {
        float y = ws.yent[(size_t)(n_ent + t) * H + c];
        for (uint32_t j = 0; j < np; j++) y = y + ws.yent[(size_t)pos[j] * H + c];
        float* o = out + (size_t)t * H + c;
        *o = residual ? *o + y : y;
    }
}

hipError_t launch_batch_combine(const Workspace& ws, uint32_t m, float* out, int residual, hipStream_t st) {
    batch_combine_kernel<<<m, 256, 0, st>>>(ws, m, out, residual);
    return hipGetLastError();
}

}  // namespace trk
