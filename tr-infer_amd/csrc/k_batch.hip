// Batch path (M >= 2): Model::moe_batch (crates/tr-model/src/exec_batch.rs:1404-1580).
//
//   dispatch: the stable sort of (token, slot) entries by expert (exec_batch.rs:1428-1462) as a
//             histogram + exclusive scan + rank-within-expert scatter (ranks from per-wave token
//             bitmaps, so the order is the reference's token-major order), plus the compressed
//             group table and the grouped-GEMM work list.
//   gate/up:  per work item (an expert and up to BR of its entry rows, or up to BR tokens of the
//             shared expert) and 16-row strip of F: the 32 weight rows are staged in LDS once and
//             every (row, entry) thread runs the reference's sequential per-block epilogue; SwiGLU,
//             the per-16 requantisation and the weight fold follow in the same workgroup.
//   down:     per work item and 32-row strip of H: per-entry outputs into yent.
//   combine:  per token, shared row first, then its entries in ascending expert order (the
//             reference's overwrite-then-accumulate order, exec_batch.rs:1539-1561).
#include "common.hpp"

namespace trk {

constexpr uint32_t BR = 8;  // entry rows per work item
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

// ---- gate/up -----------------------------------------------------------------------------------

// 16 gate rows + 16 up rows of one strip staged in LDS; thread (row r, entry i) runs the
// per-block epilogue chain over the whole K for its row and entry.
__global__ __launch_bounds__(256) void batch_gateup_kernel(Mat gate, Mat up, Mat shg, Mat shu, Workspace ws,
                                                          uint32_t m) {
    const uint32_t H = gate.k, F = gate.rows, nsb = H / 256, nb = H / 32, nbf = F / 16;
    const uint32_t strip = blockIdx.x, itn = blockIdx.y, tid = threadIdx.x;
    if (itn >= ws.n_groups[2]) return;
    const Item item = ws.items[itn];
    const bool shared = item.expert == NO_EXPERT;
    const uint32_t n_ent = ws.n_groups[1];
    const Mat& G = shared ? shg : gate;
    const Mat& U = shared ? shu : up;
    const uint32_t e = shared ? 0u : item.expert;
    const uint32_t rb = G.row_bytes;  // 144 * nsb

    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t* wts = smem;                                   // [32][rb]
    int8_t* xq = (int8_t*)(smem + 32 * rb);                // [BR][H]
    float* xs = (float*)(xq + BR * H);                     // [BR][nb]
    int32_t* xsu = (int32_t*)(xs + BR * nb);               // [BR][nb]
    float* hres = (float*)(xsu + BR * nb);                 // [32][BR]
    float* act = hres + 32 * BR;                           // [BR][16]

    {
        const int4* gsrc = reinterpret_cast<const int4*>(G.ptr + (size_t)e * G.stride + (size_t)strip * 16 * rb);
        const int4* usrc = reinterpret_cast<const int4*>(U.ptr + (size_t)e * U.stride + (size_t)strip * 16 * rb);
        int4* dst = reinterpret_cast<int4*>(wts);
        const uint32_t n16 = 16 * rb / 16;
        for (uint32_t i = tid; i < n16; i += blockDim.x) {
            dst[i] = gsrc[i];
            dst[n16 + i] = usrc[i];
        }
        for (uint32_t i = 0; i < item.nrows; i++) {
            const uint32_t tok = shared ? item.row0 + i : ws.ent_tok[item.row0 + i];
            const int4* xsrc = reinterpret_cast<const int4*>(ws.xq + (size_t)tok * H);
            for (uint32_t j = tid; j < H / 16; j += blockDim.x) reinterpret_cast<int4*>(xq + i * H)[j] = xsrc[j];
            for (uint32_t j = tid; j < nb; j += blockDim.x) {
                xs[i * nb + j] = ws.xs[(size_t)tok * nb + j];
                xsu[i * nb + j] = ws.xsum[(size_t)tok * nb + j];
            }
        }
    }
    __syncthreads();

    const uint32_t r = tid / BR, i = tid % BR;  // 32 rows x 8 entries
    if (i < item.nrows) {
        const uint8_t* row = wts + (size_t)r * rb;
        const int* xw = reinterpret_cast<const int*>(xq + i * H);
        float acc = 0.0f;
        for (uint32_t sb = 0; sb < nsb; sb++) {
            const uint32_t* s4 = reinterpret_cast<const uint32_t*>(row + sb * 144);
            const uint8_t* hb = row + sb * 144;
            const float d = h2f(ld16(hb)), dmin = h2f(ld16(hb + 2));
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int c = j / 2, h = j % 2;
                int dot = 0;
#pragma unroll
                for (int w = 0; w < 8; w++) {
                    uint32_t q = (s4[4 + 8 * c + w] >> (4 * h)) & 0x0f0f0f0fu;
                    dot = sdot4((int)q, xw[(sb * 256 + j * 32) / 4 + w], dot);
                }
                int sc, mn;
                q4k_scale_min(hb + 4, j, sc, mn);
                float dd, mm;
                q4k_dm(d, dmin, sc, mn, dd, mm);
                const uint32_t b = sb * 8 + j;
                const float sx = xs[i * nb + b];
                const float u = sx * (float)xsu[i * nb + b];
                const float t = dd * sx;
                acc = __builtin_fmaf(mm, u, acc);
                acc = __builtin_fmaf((float)dot, t, acc);
            }
        }
        hres[r * BR + i] = acc;
    }
    __syncthreads();
    if (tid < 16 * BR) {
        const uint32_t ii = tid / 16, c = tid % 16;
        if (ii < item.nrows) act[ii * 16 + c] = silu512(hres[c * BR + ii]) * hres[(16 + c) * BR + ii];
    }
    __syncthreads();
    if (tid < item.nrows) {
        const uint32_t ii = tid;
        const uint32_t arow = shared ? n_ent + item.row0 + ii : item.row0 + ii;
        const float wgt = shared ? sigmoid_libm(ws.shl[item.row0 + ii]) : ws.ent_w[item.row0 + ii];
        float v[16];
        int8_t q[16];
        for (int j = 0; j < 16; j++) v[j] = act[ii * 16 + j];
        float s;
        int32_t su;
        quant_block_regs<16>(v, q, s, su, nullptr);
        int8_t* dq = ws.actq + (size_t)arow * F + strip * 16;
        for (int j = 0; j < 16; j++) dq[j] = q[j];
        ws.acts[(size_t)arow * nbf + strip] = s * wgt;
        ws.actsum[(size_t)arow * nbf + strip] = su;
    }
}

hipError_t launch_batch_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up,
                               const Workspace& ws, uint32_t m, hipStream_t st) {
    const uint32_t H = gate.k, F = gate.rows, nb = H / 32;
    size_t lds = 32 * (size_t)gate.row_bytes + BR * H + BR * nb * 8 + 32 * BR * 4 + BR * 16 * 4 + 64;
    dim3 g(F / 16, ws.item_cap);
    batch_gateup_kernel<<<g, 256, lds, st>>>(gate, up, sh_gate, sh_up, ws, m);
    return hipGetLastError();
}

// ---- down -------------------------------------------------------------------------------------

constexpr uint32_t DN_ROWS = 32;
__global__ __launch_bounds__(256) void batch_down_kernel(Mat down, Mat shd, Workspace ws, uint32_t m) {
    const uint32_t H = down.rows, F = down.k, nsb = F / 256, nbf = F / 16;
    const uint32_t strip = blockIdx.x, itn = blockIdx.y, tid = threadIdx.x;
    if (itn >= ws.n_groups[2]) return;
    const Item item = ws.items[itn];
    const bool shared = item.expert == NO_EXPERT;
    const uint32_t n_ent = ws.n_groups[1];
    const Mat& D = shared ? shd : down;
    const uint32_t e = shared ? 0u : item.expert;
    const uint32_t rb = D.row_bytes;
    const uint32_t arow0 = shared ? n_ent + item.row0 : item.row0;

    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t* wts = smem;                                    // [32][rb] (rb padded to 16)
    const uint32_t rbp = (rb + 15) / 16 * 16;
    int8_t* aq = (int8_t*)(smem + DN_ROWS * rbp);           // [BR][F]
    float* as = (float*)(aq + BR * F);                      // [BR][nbf]
    int32_t* asu = (int32_t*)(as + BR * nbf);

    {
        const uint8_t* src = D.ptr + (size_t)e * D.stride + (size_t)strip * DN_ROWS * rb;
        if ((rb & 15) == 0) {
            const int4* s16 = reinterpret_cast<const int4*>(src);
            for (uint32_t i = tid; i < DN_ROWS * rb / 16; i += blockDim.x) reinterpret_cast<int4*>(wts)[i] = s16[i];
        } else {  // Q6_K rows (210*nsb bytes): copy row by row with 2-byte loads
            for (uint32_t i = tid; i < DN_ROWS * (rb / 2); i += blockDim.x) {
                const uint32_t r = i / (rb / 2), o = i % (rb / 2);
                reinterpret_cast<uint16_t*>(wts + r * rbp)[o] = reinterpret_cast<const uint16_t*>(src + (size_t)r * rb)[o];
            }
        }
        for (uint32_t i = 0; i < item.nrows; i++) {
            const int4* s16 = reinterpret_cast<const int4*>(ws.actq + (size_t)(arow0 + i) * F);
            for (uint32_t j = tid; j < F / 16; j += blockDim.x) reinterpret_cast<int4*>(aq + i * F)[j] = s16[j];
            for (uint32_t j = tid; j < nbf; j += blockDim.x) {
                as[i * nbf + j] = ws.acts[(size_t)(arow0 + i) * nbf + j];
                asu[i * nbf + j] = ws.actsum[(size_t)(arow0 + i) * nbf + j];
            }
        }
    }
    __syncthreads();
    const uint32_t r = tid / BR, i = tid % BR;
    if (i >= item.nrows) return;
    const uint8_t* row = wts + (size_t)r * rbp;
    const int8_t* xr = aq + i * F;
    float acc = 0.0f;
    for (uint32_t sb = 0; sb < nsb; sb++) {
        int dl[16];
        float dd[16], mm[16];
        const int8_t* xp[1] = {xr + sb * 256};
        if (D.fmt == TRK_FMT_Q4_K) {
            const uint8_t* sp = row + sb * 144;
            const uint32_t* s4 = reinterpret_cast<const uint32_t*>(sp);
            const float d = h2f(ld16(sp)), dmin = h2f(ld16(sp + 2));
#pragma unroll
            for (int j = 0; j < 8; j++) {
                int sc, mn;
                q4k_scale_min(sp + 4, j, sc, mn);
                float a, b;
                q4k_dm(d, dmin, sc, mn, a, b);
                const int c = j / 2, h = j % 2;
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const int* xw = reinterpret_cast<const int*>(xp[0] + j * 32 + half * 16);
                    int dot = 0;
#pragma unroll
                    for (int w = 0; w < 4; w++)
                        dot = sdot4((int)((s4[4 + 8 * c + 4 * half + w] >> (4 * h)) & 0x0f0f0f0fu), xw[w], dot);
                    dl[2 * j + half] = dot;
                    dd[2 * j + half] = a;
                    mm[2 * j + half] = b;
                }
            }
        } else {
            const uint8_t* sp = row + sb * 210;
            const float d = h2f(ld16(sp + 208));
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float a = f16_round(d * (float)(int8_t)sp[192 + j]);
                dd[j] = a;
                mm[j] = f16_round(-32.0f * a);
                const int n = j / 8, g = (j % 8) / 2, l0 = 16 * (j % 2);
                const int* xw = reinterpret_cast<const int*>(xp[0] + j * 16);
                int dot = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint8_t* lp = sp + 64 * n + 32 * (g & 1) + l0 + 4 * t;
                    const uint8_t* hp = sp + 128 + 32 * n + l0 + 4 * t;
                    uint32_t lo = (uint32_t)lp[0] | ((uint32_t)lp[1] << 8) | ((uint32_t)lp[2] << 16) | ((uint32_t)lp[3] << 24);
                    uint32_t hi = (uint32_t)hp[0] | ((uint32_t)hp[1] << 8) | ((uint32_t)hp[2] << 16) | ((uint32_t)hp[3] << 24);
                    lo = (g >> 1) ? ((lo >> 4) & 0x0f0f0f0fu) : (lo & 0x0f0f0f0fu);
                    hi = (hi >> (2 * g)) & 0x03030303u;
                    dot = sdot4((int)(lo | (hi << 4)), xw[t], dot);
                }
                dl[j] = dot;
            }
        }
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t b = sb * 16 + j;
            const float sx = as[i * nbf + b];
            const float u = sx * (float)asu[i * nbf + b];
            const float t = dd[j] * sx;
            acc = __builtin_fmaf(mm[j], u, acc);
            acc = __builtin_fmaf((float)dl[j], t, acc);
        }
    }
    ws.yent[(size_t)(arow0 + i) * H + strip * DN_ROWS + r] = acc;
}

hipError_t launch_batch_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m, hipStream_t st) {
    const uint32_t H = down.rows, F = down.k, nbf = F / 16;
    const uint32_t rbp = (down.row_bytes + 15) / 16 * 16;
    const uint32_t rbp2 = (sh_down.row_bytes + 15) / 16 * 16;
    size_t lds = DN_ROWS * (size_t)(rbp > rbp2 ? rbp : rbp2) + BR * F + BR * nbf * 8 + 64;
    dim3 g(H / DN_ROWS, ws.item_cap);
    batch_down_kernel<<<g, 256, lds, st>>>(down, sh_down, ws, m);
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
