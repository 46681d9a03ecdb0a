// The MoE layer on the reference's own packed TQ experts (codec.rs:1-46): gate/up in a kb-32 codec
// (TQ4_32 in the reference's packs), down in a kb-16 codec (TQ5_16), any F that is a multiple of
// 16 (the real n_ff = 640).  Router, routing, dispatch and the batch combine are the layer's
// common kernels; the expert products are grouped TQ GEMVs:
//
//   tq_layer_kernel   one 16-row strip of one matrix for one work unit (a decode slot or a batch
//                     item) against that unit's activation rows: phase 1 forms every block's
//                     exact dot with a 16-lane group per TQ block (16-byte loads); phase 2 runs
//                     the per-(row, activation) f32 chain (gemv.rs:141-148) in block order.
//                       gate/up: h[row][0, F) = gate . x, h[row][F, 2F) = up . x
//                       down:    yent[row][0, H) = down . act
//   tq_act_kernel     SwiGLU of h (elem.rs:173), the per-16 quantisation of the result (two levels
//                     at M = 1 with TR_HIPREC, quant.rs:96-108) and the routing-weight fold into
//                     its scales (exec.rs:1584-1606, exec_batch.rs:1528-1536)
//   tq_combine_kernel decode: the slots' down rows summed in slot order, the shared expert last
//                     (exec.rs:1610-1621); batch: batch_combine_kernel
#include "tq.hpp"

namespace trk {

enum : int { TQ_DEC_GU = 0, TQ_BAT_GU = 1, TQ_DEC_DN = 2, TQ_BAT_DN = 3 };

struct TqArgs {
    Mat a, b, sha, shb;  // gate/up: gate, up, shared gate, shared up; down: down, -, shared down, -
    Workspace ws;
    float* h;            // [rows][2F] gate/up outputs
    int mode, pair;
};

constexpr uint32_t TQ_R = 16;  // rows per workgroup: one strip

// gv_terms_tq with a runtime slice length S (dl [NA][S][16], dm [S][16], xq [NA][S * KB], xs [NA][S])
template <int GK, int KB, int NA>
__device__ __forceinline__ void gv_terms_tq_rt(const GvTQ<GK, KB>& w, uint32_t l, uint32_t j, uint32_t na,
                                               const int8_t* xq, const float4* xs, float* dl, float2* dm, uint32_t S) {
    using T = GvTQ<GK, KB>;
    const uint32_t cl = l / 4, rq = l % 4;
    uint32_t lo[T::CPL][4], hi[T::CPL][4];
#pragma unroll
    for (uint32_t t = 0; t < T::CPL; t++) {
        const uint32_t qw[4] = {w.q[t].x, w.q[t].y, w.q[t].z, w.q[t].w};
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            if constexpr (T::BITS == 8) {
                lo[t][rr] = qw[rr] ^ 0x80808080u;  // q - 128
                hi[t][rr] = 0;
            } else {
                lo[t][rr] = qw[rr] & 0x0f0f0f0fu;
                hi[t][rr] = (qw[rr] >> 4) & 0x0f0f0f0fu;
                if constexpr (T::BITS == 5) {
                    const uint32_t r = 4 * rq + rr;
                    const uint32_t pl = r < 8 ? w.p[t].x : w.p[t].y, ph = r < 8 ? w.p[t].z : w.p[t].w;
                    lo[t][rr] |= q5_hi4((pl >> (4 * (r % 8))) & 0xfu);
                    hi[t][rr] |= q5_hi4((ph >> (4 * (r % 8))) & 0xfu);
                }
            }
        }
    }
#pragma unroll
    for (uint32_t a = 0; a < NA; a++) {
        if (a >= na) break;
        const int* x = reinterpret_cast<const int*>(xq + (size_t)a * S * KB + (size_t)j * KB);
        int dot[4] = {0, 0, 0, 0};
#pragma unroll
        for (uint32_t t = 0; t < T::CPL; t++) {
            const uint32_t c = cl + 4 * t;
            if (T::NCH % 4 == 0 || c < T::NCH) {
                const int xl = x[c];
                const int xh = T::BITS == 8 ? 0 : x[T::NCH + c];
#pragma unroll
                for (int rr = 0; rr < 4; rr++) {
                    dot[rr] = sdot4((int)lo[t][rr], xl, dot[rr]);
                    if constexpr (T::BITS != 8) dot[rr] = sdot4((int)hi[t][rr], xh, dot[rr]);
                }
            }
        }
        const int corr = T::BITS == 8 ? 128 * __float_as_int(xs[(size_t)a * S + j].z) : 0;
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const int v = dpp_ror8_add(dpp_ror4_add(dot[rr]));
            if (cl == 0) dl[((size_t)a * S + j) * TQ_R + 4 * rq + rr] = (float)(v + corr);
        }
    }
    if (cl == 0) {
        const uint16_t dv[4] = {(uint16_t)(w.d.x & 0xffff), (uint16_t)(w.d.x >> 16), (uint16_t)(w.d.y & 0xffff),
                                (uint16_t)(w.d.y >> 16)};
        const uint16_t mv[4] = {(uint16_t)(w.m.x & 0xffff), (uint16_t)(w.m.x >> 16), (uint16_t)(w.m.y & 0xffff),
                                (uint16_t)(w.m.y >> 16)};
#pragma unroll
        for (int rr = 0; rr < 4; rr++) dm[(size_t)j * TQ_R + 4 * rq + rr] = make_float2(h2f(dv[rr]), h2f(mv[rr]));
    }
}

// LDS of a workgroup with K slices of S blocks: staged activations, their (scale, u, byte sum),
// the block dots and the blocks' (d, m)
template <int KB, int NA>
constexpr size_t tq_lds_bytes(uint32_t S) {
    return (size_t)NA * S * KB + (size_t)NA * S * 16 + (size_t)NA * S * TQ_R * 4 + (size_t)S * TQ_R * 8;
}

// S: blocks per K slice (a multiple of 8, set by the launch from K so that the LDS, and with it
// the workgroups a CU holds, follows the shape)
template <int GK, int KB, int NA>
__global__ __launch_bounds__(256, 4) void tq_layer_kernel(TqArgs g, uint32_t S) {
    constexpr uint32_t R = TQ_R;
    // units whose loads a thread issues together: about 48 registers of weights (q chunks, the
    // 5-bit plane, d and m)
    using TW = GvTQ<GK, KB>;
    constexpr uint32_t UW = 4 * TW::CPL + (TW::BITS == 5 ? 4 * TW::CPL : 0) + 4;
    constexpr uint32_t UB = UW * 8 <= 32 ? 8 : (32 / UW > 2 ? 32 / UW : 2);
    constexpr bool XSUM = GK == GK_TQ8;
    extern __shared__ __align__(16) uint8_t tq_smem[];
    int8_t* xq_ = reinterpret_cast<int8_t*>(tq_smem);                             // [NA][S * KB]
    float4* xs_ = reinterpret_cast<float4*>(tq_smem + (size_t)NA * S * KB);       // [NA][S]
    float* dl_ = reinterpret_cast<float*>(xs_ + (size_t)NA * S);                  // [NA][S][R]
    float2* dm_ = reinterpret_cast<float2*>(dl_ + (size_t)NA * S * R);            // [S][R]
    auto XQ = [&](uint32_t a, uint32_t o) -> int8_t* { return xq_ + (size_t)a * S * KB + o; };
    auto XS = [&](uint32_t a, uint32_t j) -> float4& { return xs_[(size_t)a * S + j]; };
    auto DL = [&](uint32_t a, uint32_t j, uint32_t r) -> float& { return dl_[((size_t)a * S + j) * R + r]; };
    auto DM = [&](uint32_t j, uint32_t r) -> float2& { return dm_[(size_t)j * R + r]; };
    __shared__ uint32_t prow[2 * BR];  // physical activation rows of the unit
    __shared__ uint32_t orow[BR];      // output row of each logical row
    const Workspace& ws = g.ws;
    const uint32_t tid = threadIdx.x, l = tid % 16, gi = tid / 16, ca = tid / R, cr = tid % R;
    const bool gu = g.mode == TQ_DEC_GU || g.mode == TQ_BAT_GU, dec = g.mode == TQ_DEC_GU || g.mode == TQ_DEC_DN;
    const uint32_t F = ws.F, H = ws.H, t = blockIdx.x;

    // the work unit: a decode slot (routed slots in order, then the shared expert) or a batch item
    bool shared;
    uint32_t e, nr, P;
    Item item{};
    if (dec) {
        const uint32_t ns = ws.n_sel[0];
        if (blockIdx.y > ns) return;
        shared = blockIdx.y == ns;
        e = shared ? 0u : ws.ids[blockIdx.y];
        nr = 1;
        P = g.pair ? 2u : 1u;
    } else {
        if (blockIdx.y >= ws.n_groups[2]) return;
        item = ws.items[blockIdx.y];
        shared = item.expert == NO_EXPERT;
        e = shared ? 0u : item.expert;
        nr = item.nrows;
        P = 1;
    }
    const uint32_t n_ent = ws.n_groups[1];
    if (tid < nr * P) {
        const uint32_t i = tid / P, lv = tid % P;
        uint32_t pr, orr;
        if (g.mode == TQ_DEC_GU) {
            pr = lv;  // x's (coarse, residual) rows
            orr = blockIdx.y;
        } else if (g.mode == TQ_DEC_DN) {
            pr = 2 * blockIdx.y + lv;  // the slot's activation rows
            orr = blockIdx.y;
        } else if (g.mode == TQ_BAT_GU) {
            pr = item_token(ws, item, shared, i);
            orr = shared ? n_ent + item.row0 + i : item.row0 + i;
        } else {
            pr = orr = shared ? n_ent + item.row0 + i : item.row0 + i;
        }
        prow[tid] = pr;
        if (lv == 0) orow[i] = orr;
    }
    // the strip: gate/up tiles 0 .. F/16 - 1 are gate strips, the next F/16 up strips.  A pack
    // written for T tiles: a gate/up strip lives in tile strip / (F / T / 16) (mat_strip); the down
    // runs once per tile (grid.z) over the tile's columns [F / T z, F / T (z + 1)) of the activations,
    // each into its own block of yent (the tiles' partials, exec.rs:1035-1038)
    const Mat& M = gu ? (t < F / 16 ? (shared ? g.sha : g.a) : (shared ? g.shb : g.b)) : (shared ? g.sha : g.a);
    const uint32_t strip = gu && t >= F / 16 ? t - F / 16 : t;
    const uint32_t z = gu ? 0u : blockIdx.z, Kp = gu ? H : F, K = gu ? H : F / ws.tiles, nb = K / KB;
    const uint32_t k0 = z * K, nbp = Kp / KB;  // first column of this tile; blocks per activation row
    const uint8_t* sp = gu ? mat_strip(M, e, strip) : mat_tile(M, e, z) + (size_t)strip * M.row_bytes;
    const int8_t* q = gu ? ws.xq : ws.actq;
    const float* qs = gu ? ws.xs : ws.acts;
    const float* qu = gu ? ws.xu : ws.actu;
    float* out = gu ? g.h : ws.yent + (size_t)z * ws.yent_tile;
    const uint32_t opitch = gu ? 2 * F : H;
    const uint32_t np = nr * P, npass = (np + NA - 1) / NA;

    GvTQ<GK, KB> w[UB];
    auto n_items = [&](uint32_t sn) -> uint32_t { return (sn + 15 - gi) / 16; };
    auto load_batch = [&](uint32_t b0, uint32_t sn, uint32_t k0) {
        const uint32_t n = n_items(sn);
#pragma unroll
        for (uint32_t i = 0; i < UB; i++)
            if (k0 + i < n) gv_load_tq<GK, KB>(w[i], sp, b0 + gi + 16 * (k0 + i), l);
    };
    __syncthreads();  // prow / orow

    for (uint32_t pass = 0; pass < npass; pass++) {
        const uint32_t p0 = pass * NA, na = np - p0 < NA ? np - p0 : NA;
        float acc = 0.0f;
        uint32_t sn = nb < S ? nb : S;
        load_batch(0, sn, 0);  // in flight while the activations are staged
        for (uint32_t b0 = 0; b0 < nb;) {
            __syncthreads();
            const uint32_t pr = sn * KB / 16;
            for (uint32_t i = tid; i < NA * pr; i += 256) {
                const uint32_t a = i / pr, o = (i % pr) * 16;
                int4 v = make_int4(0, 0, 0, 0);
                if (a < na) v = *reinterpret_cast<const int4*>(q + (size_t)prow[p0 + a] * Kp + k0 + (size_t)b0 * KB + o);
                *reinterpret_cast<int4*>(XQ(a, o)) = v;
            }
            for (uint32_t i = tid; i < NA * S; i += 256) {
                const uint32_t a = i / S, j = i % S;
                float sx = 0.0f, u = 0.0f;
                int xsum = 0;
                if (a < na && j < sn) {
                    const size_t bi = (size_t)prow[p0 + a] * nbp + k0 / KB + b0 + j;
                    sx = qs[bi];
                    u = qu[bi];  // sx * (float)sum, formed where the row was quantised (gemv.rs:143)
                    if constexpr (XSUM) {
                        const int4* xp = reinterpret_cast<const int4*>(q + (size_t)prow[p0 + a] * Kp + k0 + (size_t)(b0 + j) * KB);
#pragma unroll
                        for (int c = 0; c < KB / 16; c++) {
                            const int4 v = xp[c];
                            xsum = sdot4(v.x, 0x01010101, xsum);
                            xsum = sdot4(v.y, 0x01010101, xsum);
                            xsum = sdot4(v.z, 0x01010101, xsum);
                            xsum = sdot4(v.w, 0x01010101, xsum);
                        }
                    }
                }
                XS(a, j) = make_float4(sx, u, __int_as_float(xsum), 0.0f);
            }
            __syncthreads();
            const uint32_t n = n_items(sn);
            for (uint32_t k0 = 0; k0 < n; k0 += UB) {
                if (k0) load_batch(b0, sn, k0);
#pragma unroll
                for (uint32_t i = 0; i < UB; i++)
                    if (k0 + i < n) gv_terms_tq_rt<GK, KB, NA>(w[i], l, gi + 16 * (k0 + i), na, XQ(0, 0), xs_, dl_, dm_, S);
            }
            const uint32_t b1 = b0 + sn, sn1 = nb - b1 < S ? nb - b1 : S;
            if (b1 < nb) load_batch(b1, sn1, 0);
            __syncthreads();
            if (ca < na) {
                uint32_t j = 0;
                for (; j + 4 <= sn; j += 4) {
                    float2 tt[4];
                    float4 x[4];
                    float d[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        tt[i] = DM(j + i, cr);
                        x[i] = XS(ca, j + i);
                        d[i] = DL(ca, j + i, cr);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc = __builtin_fmaf(tt[i].y, x[i].y, acc);
                        acc = __builtin_fmaf(d[i], tt[i].x * x[i].x, acc);
                    }
                }
                for (; j < sn; j++) {
                    const float2 tt = DM(j, cr);
                    const float4 x = XS(ca, j);
                    acc = __builtin_fmaf(tt.y, x.y, acc);
                    acc = __builtin_fmaf(DL(ca, j, cr), tt.x * x.x, acc);
                }
            }
            b0 = b1;
            sn = sn1;
        }
        __syncthreads();
        if (ca < na) DL(ca, 0, cr) = acc;
        __syncthreads();
        if (tid < R)
            for (uint32_t i = 0; i < na / P; i++) {
                // two-level rows: coarse + residual (gemv.rs:150-160)
                const float v = P == 2 ? DL(2 * i, 0, tid) + DL(2 * i + 1, 0, tid) : DL(i, 0, tid);
                out[(size_t)orow[p0 / P + i] * opitch + t * 16 + tid] = v;
            }
    }
}

// SwiGLU, quantisation per 16 and the weight fold: one thread per (row, 16-block).  Decode rows are
// slots (activation rows 2 s and 2 s + 1); batch rows are the entries, then one shared row per
// token.
__global__ __launch_bounds__(256) void tq_act_kernel(Workspace ws, const float* __restrict__ h, int dec, int pair,
                                                      uint32_t m, uint32_t rows_max) {
    const uint32_t F = ws.F, nbf = F / 16;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, row = i / nbf, b = i % nbf;
    if (row >= rows_max) return;
    float wgt;
    if (dec) {
        const uint32_t ns = ws.n_sel[0];
        if (row > ns) return;
        wgt = row < ns ? ws.w[row] : sigmoid_libm(ws.shl[0]);
    } else {
        const uint32_t n_ent = ws.n_groups[1];
        if (row >= n_ent + m) return;
        wgt = row < n_ent ? ws.ent_w[row] : sigmoid_libm(ws.shl[row - n_ent]);
    }
    const float4* hg = reinterpret_cast<const float4*>(h + (size_t)row * 2 * F + 16 * b);
    const float4* hu = reinterpret_cast<const float4*>(h + (size_t)row * 2 * F + F + 16 * b);
    float v[16];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float4 gg = hg[c], uu = hu[c];
        v[4 * c] = silu512(gg.x) * uu.x;
        v[4 * c + 1] = silu512(gg.y) * uu.y;
        v[4 * c + 2] = silu512(gg.z) * uu.z;
        v[4 * c + 3] = silu512(gg.w) * uu.w;
    }
    auto store = [&](uint32_t arow, const uint32_t (&qw)[4], float s, int32_t sum) {
        *reinterpret_cast<uint4*>(ws.actq + (size_t)arow * F + 16 * b) = make_uint4(qw[0], qw[1], qw[2], qw[3]);
        const float sf = s * wgt;
        ws.acts[(size_t)arow * nbf + b] = sf;
        ws.actsum[(size_t)arow * nbf + b] = sum;
        ws.actu[(size_t)arow * nbf + b] = sf * (float)sum;
    };
    uint32_t qw[4];
    float s;
    int32_t sum;
    if (dec && pair) {
        float r[16];
        quant_block_regs<16, true>(v, qw, s, sum, r);
        store(2 * row, qw, s, sum);
        quant_block_regs<16>(r, qw, s, sum);
        store(2 * row + 1, qw, s, sum);
    } else {
        quant_block_regs<16>(v, qw, s, sum);
        store(dec ? 2 * row : row, qw, s, sum);
    }
}

// decode: out (+)= the slots' down rows, summed in slot order (exec.rs:1610-1621); with T tiles each
// tile's slot sum is its partial, and the partials are summed in tile order (exchange.rs:122-136)
__global__ __launch_bounds__(256) void tq_combine_kernel(Workspace ws, float* __restrict__ out, int residual) {
    const uint32_t H4 = ws.H / 4, c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= H4) return;
    const uint32_t slots = ws.n_sel[0] + 1;
    float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t t = 0; t < ws.tiles; t++) {
        const float4* y4 = reinterpret_cast<const float4*>(ws.yent + (size_t)t * ws.yent_tile);
        float4 p = y4[c];
        for (uint32_t s = 1; s < slots; s++) {
            const float4 v = y4[(size_t)s * H4 + c];
            p = make_float4(p.x + v.x, p.y + v.y, p.z + v.z, p.w + v.w);
        }
        y = t == 0 ? p : make_float4(y.x + p.x, y.y + p.y, y.z + p.z, y.w + p.w);
    }
    float4* o = reinterpret_cast<float4*>(out) + c;
    if (residual) {
        const float4 hh = *o;
        y = make_float4(hh.x + y.x, hh.y + y.y, hh.z + y.z, hh.w + y.w);
    }
    *o = y;
}

// the K slice: all of K up to 128 blocks (64 with four activation rows per pass), rounded up to 8
template <int KB, int NA>
static hipError_t tq_go(const TqArgs& a, uint32_t fmt, uint32_t K, dim3 grid, hipStream_t st) {
    const uint32_t nb = K / KB, smax = NA <= 2 ? 128 : 64;
    const uint32_t S = nb < smax ? (nb + 7) / 8 * 8 : smax;
    const size_t lds = tq_lds_bytes<KB, NA>(S);
    switch (tq_bits(fmt)) {
        case 4: tq_layer_kernel<GK_TQ4, KB, NA><<<grid, 256, lds, st>>>(a, S); break;
        case 5: tq_layer_kernel<GK_TQ5, KB, NA><<<grid, 256, lds, st>>>(a, S); break;
        case 8: tq_layer_kernel<GK_TQ8, KB, NA><<<grid, 256, lds, st>>>(a, S); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_tq_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const Workspace& ws,
                            float* h, uint32_t m, uint32_t kcap, int pair, hipStream_t st) {
    if (tq_kb(gate.fmt) != 32) return hipErrorInvalidValue;
    const TqArgs a{gate, up, sh_gate, sh_up, ws, h, m == 1 ? TQ_DEC_GU : TQ_BAT_GU, pair};
    const dim3 grid(2 * ws.F / 16, m == 1 ? kcap + 1 : grouped_item_rows(ws, m));
    return m == 1 ? tq_go<32, 2>(a, gate.fmt, ws.H, grid, st) : tq_go<32, 4>(a, gate.fmt, ws.H, grid, st);
}

hipError_t launch_tq_act(const Workspace& ws, const float* h, uint32_t m, uint32_t kcap, int pair, hipStream_t st) {
    const uint32_t rows = m == 1 ? kcap + 1 : m * kcap + m;
    const uint32_t n = rows * (ws.F / 16);
    tq_act_kernel<<<(n + 255) / 256, 256, 0, st>>>(ws, h, m == 1, pair, m, rows);
    return hipGetLastError();
}

hipError_t launch_tq_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m, uint32_t kcap, int pair,
                          hipStream_t st) {
    if (tq_kb(down.fmt) != 16) return hipErrorInvalidValue;
    const TqArgs a{down, down, sh_down, sh_down, ws, nullptr, m == 1 ? TQ_DEC_DN : TQ_BAT_DN, pair};
    const dim3 grid(ws.H / 16, m == 1 ? kcap + 1 : grouped_item_rows(ws, m), ws.tiles);  // z: the tiles
    const uint32_t K = ws.F / ws.tiles;
    return m == 1 ? tq_go<16, 2>(a, down.fmt, K, grid, st) : tq_go<16, 4>(a, down.fmt, K, grid, st);
}

hipError_t launch_tq_combine(const Workspace& ws, float* out, int residual, hipStream_t st) {
    tq_combine_kernel<<<(ws.H / 4 + 255) / 256, 256, 0, st>>>(ws, out, residual);
    return hipGetLastError();
}

}  // namespace trk
