// Decode path (M = 1): Model::moe_block (crates/tr-model/src/exec.rs:1540-1623).
//
//   gate/up: one workgroup per (slot, 16-row strip of F).  Each thread issues the loads of one
//            (row, superblock) of the 16 gate + 16 up rows straight from their Q4_K superblocks,
//            and while they fly the first nb threads quantise x (two-level, per 32) into LDS —
//            every workgroup does this itself, so no separate quantisation launch.  The exact
//            int32 dot of every 32-block goes to LDS, one thread per (row, activation row) runs
//            the reference's sequential per-block f32 epilogue from b128 LDS reads, and since
//            the down input is quantised per 16, SwiGLU, the (pair) requantisation and the
//            routing-weight fold of the strip's 16-wide block finish in the same workgroup
//            (tasks A and B of moe_block).
//   down:    one workgroup per 8 output rows, all slots: a thread per (slot, row) streams the
//            row's superblocks, forms the per-16 block dots against the staged activations and
//            runs the chain in registers; slot 0 is stored and later slots (routing order,
//            shared last) are added — tasks C with the combine fused.
//   a few tokens (2 <= M <= 16): both launches take a token dimension (each token its own
//            routing, x row and activation slots, exactly a decode's), and the down adds a token's
//            rows in the batch combine's order (shared first, then ascending expert:
//            exec_batch.rs:1539-1578), so the grouped path's bits come out with no dispatch,
//            grouped items or combine launch.
#include "gemv.hpp"
#include "route.hpp"
#include "router.hpp"

namespace trk {

constexpr int DN_R = 4;      // output rows per down workgroup

// One gate/up unit (slot, strip) on a workgroup of at least GU_THREADS(NSB) threads.  Wave 0
// routes the token into LDS when `route` is set (always for routed slots).  `pre()` runs on every
// thread after the unit's first loads are issued (x; the shared expert's weights) and before the
// logits or the shared gate's logit are read (the pipelined layer waits there for the router
// workgroups).  `hook(r_ids, n)` runs on every thread once the routing is in LDS, before any
// weight of a routed slot is requested.  active = false: route and hook only.  pub: with publish,
// a counter raised once the published routing is visible device-wide (COH stores).
template <int P, int NSB, int NJ, bool COH, bool XPRE, typename Pre, typename Hook>
__device__ __forceinline__ void gateup_unit(const Mat& gate, const Mat& up, const Mat& shg, const Mat& shu,
                                            const float* __restrict__ x, const float* __restrict__ lg,
                                            const Workspace& ws, uint32_t k, const Policy& pol, uint32_t kcap,
                                            uint32_t slot, uint32_t strip, bool active, bool route, bool publish,
                                            uint8_t* smem, uint8_t* rsm, Pre&& pre, Hook&& hook,
                                            uint32_t* pub = nullptr) {
    constexpr uint32_t H = NSB * 256, nb = NSB * 8, XSB = 256 + 16, XP = NSB * XSB;
    const uint32_t F = gate.rows, E = ws.E;
    const uint32_t tid = threadIdx.x;
    const bool shared = active && slot == kcap;
    route = route || !shared;
    int8_t* xq = (int8_t*)smem;              // [P][NSB][XSB]: superblocks padded against bank conflicts
    float* xs = (float*)(smem + P * XP);     // [P][nb]  activation scales
    float* xu = xs + P * nb;                 // [P][nb]  sx * sum
    float* hres = xu + P * nb;               // [32][P]
    uint32_t* r_ids = (uint32_t*)rsm;              // [32] this token's routing
    float* r_w = (float*)(r_ids + K_MAX);          // [32]
    uint32_t* r_n = (uint32_t*)(r_w + K_MAX);      // [4]
    uint2* cand = (uint2*)(r_n + 4);               // [ROUTE_CAND] routing scratch
    float* ex = (float*)(cand + ROUTE_CAND);       // [E] (MassBasis::All only)

    // x first: its loads must not queue behind the (id-dependent) weight loads.  XPRE: x is
    // already quantised in ws.xq / xs / xu (the logits launch does it), one block per thread
    float4 xv[8];
    const bool qthread = active && tid >= 64 && tid < 64 + nb;
    if (qthread) {
        const uint32_t b = tid - 64;
        if constexpr (XPRE) {  // straight into LDS (the routing wave does not touch this area)
            uint4 pq[P][2];
            float ps[P], pu[P];
#pragma unroll
            for (int p = 0; p < P; p++) {
                const uint4* src = reinterpret_cast<const uint4*>(ws.xq + (size_t)p * H + b * 32);
                pq[p][0] = src[0];
                pq[p][1] = src[1];
                ps[p] = ws.xs[p * nb + b];
                pu[p] = ws.xu[p * nb + b];
            }
            const uint32_t xo = (b / 8) * XSB + (b % 8) * 32;
#pragma unroll
            for (int p = 0; p < P; p++) {
                *reinterpret_cast<uint4*>(xq + p * XP + xo) = pq[p][0];
                *reinterpret_cast<uint4*>(xq + p * XP + xo + 16) = pq[p][1];
                xs[p * nb + b] = ps[p];
                xu[p * nb + b] = pu[p];
            }
        } else {
            const float4* src = reinterpret_cast<const float4*>(x + (size_t)b * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) xv[i] = src[i];
        }
    }
    // lane (row r, superblock sb); rows never straddle a wave (the chain hands over lane to lane)
    constexpr uint32_t RPW = 64 / NSB;
    const uint32_t ln = tid % 64, sb = ln % NSB;
    const uint32_t r = ln < RPW * NSB ? (tid / 64) * RPW + ln / NSB : 32u;
    const bool wthread = r < 32;
    auto load_rows = [&](const Mat& G, const Mat& U, uint32_t e, uint4* wq) {
        const uint32_t rr = wthread ? r : 0u;
        const uint8_t* rowp = (rr < 16 ? G.ptr + (size_t)e * G.stride + (size_t)(strip * 16 + rr) * G.row_bytes
                                       : U.ptr + (size_t)e * U.stride + (size_t)(strip * 16 + rr - 16) * U.row_bytes) +
                              sb * 144;
        const uint4* s4 = reinterpret_cast<const uint4*>(rowp);
#pragma unroll
        for (int i = 0; i < 9; i++) wq[i] = s4[i];
    };
    uint4 wq[9];
    float shl = 0.0f;
    if (shared) load_rows(shg, shu, 0u, wq);  // the shared expert does not wait for the routing
    pre();
    if (shared) shl = COH ? ld_devf(ws.shl) : ws.shl[0];
    // route this token (wave 0): every routed workgroup repeats it, so no separate launch and no
    // round trip through memory sits between the logits and the expert weights.  Without a mass
    // policy the selection alone fixes every slot's expert: the workgroup then requests its slot's
    // weights before wave 0 works out the routing weights
    const bool early = route && !pol.enabled && !pol.packed;  // workgroup-uniform (a subset pack folds the ids after)
    uint32_t my_key = 0, my_idx = 0, ksel = 0;
    if (route && tid < 64) {
        ksel = route_select<NJ, COH>(lg, E, k, pol, tid, cand, my_key, my_idx);
        if (early) {
            if (tid < ksel) r_ids[tid] = my_idx;
            if (tid == 0) r_n[0] = ksel;  // top-k: the count is the selection's size
        }
    }
    bool loaded = false;
    if (early) {
        __syncthreads();
        if (active && !shared && slot < r_n[0]) {
            load_rows(gate, up, r_ids[slot], wq);
            loaded = true;
        }
    }
    if (route && tid < 64) {
        const uint32_t n = route_weights<COH>(lg, E, k, pol, tid, ex, ksel, my_key, my_idx, r_ids, r_w);
        if (tid == 0) r_n[0] = n;
        if (publish) {  // one workgroup publishes it (down kernel, introspection)
            wave_sync();
            if (tid < n) {
                if constexpr (COH) {
                    st_dev(ws.ids + tid, r_ids[tid]);
                    st_devf(ws.w + tid, r_w[tid]);
                } else {
                    ws.ids[tid] = r_ids[tid];
                    ws.w[tid] = r_w[tid];
                }
            }
            if (tid == 0) {
                if constexpr (COH)
                    st_dev(ws.n_sel, n);
                else
                    ws.n_sel[0] = n;
                if (ws.stats) {
                    atomicAdd(&ws.stats[0], 1ull);
                    atomicAdd(&ws.stats[1], (unsigned long long)n);
                }
            }
            if (pub) {  // this wave's stores are complete before the counter moves
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_s_waitcnt(0);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                if (tid == 0) __hip_atomic_fetch_add(pub, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    // quantise x per 32 (quantize_pair_blocks, quant.rs:96-108, or QAct::quantize) into LDS
    if (!XPRE && qthread) {
        const uint32_t b = tid - 64;
        float v[32], rs[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[4 * i] = xv[i].x; v[4 * i + 1] = xv[i].y; v[4 * i + 2] = xv[i].z; v[4 * i + 3] = xv[i].w;
        }
        uint32_t q[8];
        float s;
        int32_t su;
        quant_block_regs<32, P == 2>(v, q, s, su, rs);
        const uint32_t xo = (b / 8) * XSB + (b % 8) * 32;  // LDS offset of block b
        *reinterpret_cast<uint4*>(xq + xo) = make_uint4(q[0], q[1], q[2], q[3]);
        *reinterpret_cast<uint4*>(xq + xo + 16) = make_uint4(q[4], q[5], q[6], q[7]);
        xs[b] = s;
        xu[b] = s * (float)su;  // gemv.rs:144
        if (shared && strip == 0) {  // one workgroup publishes the quantised input (introspection)
            *reinterpret_cast<uint4*>(ws.xq + b * 32) = make_uint4(q[0], q[1], q[2], q[3]);
            *reinterpret_cast<uint4*>(ws.xq + b * 32 + 16) = make_uint4(q[4], q[5], q[6], q[7]);
            ws.xs[b] = s;
            ws.xsum[b] = su;
        }
        if (P == 2) {
            quant_block_regs<32>(rs, q, s, su);
            *reinterpret_cast<uint4*>(xq + XP + xo) = make_uint4(q[0], q[1], q[2], q[3]);
            *reinterpret_cast<uint4*>(xq + XP + xo + 16) = make_uint4(q[4], q[5], q[6], q[7]);
            xs[nb + b] = s;
            xu[nb + b] = s * (float)su;
            if (shared && strip == 0) {
                *reinterpret_cast<uint4*>(ws.xq + H + b * 32) = make_uint4(q[0], q[1], q[2], q[3]);
                *reinterpret_cast<uint4*>(ws.xq + H + b * 32 + 16) = make_uint4(q[4], q[5], q[6], q[7]);
                ws.xs[nb + b] = s;
                ws.xsum[nb + b] = su;
            }
        }
    }
    __syncthreads();
    hook(r_ids, route ? r_n[0] : 0u);
    if (!active) return;
    float wgt = 0.0f;
    if (!shared) {
        if (slot >= r_n[0]) return;  // workgroup-uniform
        if (!loaded) load_rows(gate, up, r_ids[slot], wq);
        wgt = r_w[slot];
    }

    // this lane's 8 blocks: exact dots, (dd, mm), t = dd * sx and u from LDS
    const uint32_t* w32 = reinterpret_cast<const uint32_t*>(wq);  // [0..3] header, [4..35] qs
    const float d = h2f((uint16_t)(wq[0].x & 0xffff)), dmin = h2f((uint16_t)(wq[0].x >> 16));
    float mmv[8], tv[P][8], uv[P][8], dotv[P][8];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const float4* sp = reinterpret_cast<const float4*>(xs + p * nb + sb * 8);
        const float4* up4 = reinterpret_cast<const float4*>(xu + p * nb + sb * 8);
        const float4 s0 = sp[0], s1 = sp[1], u0 = up4[0], u1 = up4[1];
        const float sxa[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        const float ua[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            tv[p][j] = sxa[j];
            uv[p][j] = ua[j];
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int sc, mn;
        q4k_scale_min_w(wq[0].y, wq[0].z, wq[0].w, j, sc, mn);
        float ddv;
        q4k_dm(d, dmin, sc, mn, ddv, mmv[j]);
#pragma unroll
        for (int p = 0; p < P; p++) tv[p][j] = ddv * tv[p][j];  // t = d * sx (gemv.rs:145)
    }
    // sub-block pairs (2c, 2c+1): the nibbles once for both levels
#pragma unroll
    for (int c = 0; c < 4; c++) {
        int4 xa[P][4];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int4* src = reinterpret_cast<const int4*>(xq + p * XP + sb * XSB + 64 * c);
#pragma unroll
            for (int i = 0; i < 4; i++) xa[p][i] = src[i];
        }
        int d0[P], d1[P];
#pragma unroll
        for (int p = 0; p < P; p++) d0[p] = d1[p] = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t qw = w32[4 + 8 * c + w];
            const int lo = (int)nib(qw, 0), hi = (int)nib(qw, 1);
#pragma unroll
            for (int p = 0; p < P; p++) {
                const int xl = w < 4 ? (&xa[p][0].x)[w] : (&xa[p][1].x)[w - 4];
                const int xh = w < 4 ? (&xa[p][2].x)[w] : (&xa[p][3].x)[w - 4];
                d0[p] = sdot4(lo, xl, d0[p]);
                d1[p] = sdot4(hi, xh, d1[p]);
            }
        }
#pragma unroll
        for (int p = 0; p < P; p++) {
            dotv[p][2 * c] = (float)d0[p];
            dotv[p][2 * c + 1] = (float)d1[p];
        }
    }
    // the chain (gemv.rs:141-148) in block order: superblock sb continues where sb-1 stopped
    float acc[P];
#pragma unroll
    for (int p = 0; p < P; p++) acc[p] = 0.0f;
#pragma unroll
    for (int st = 0; st < NSB; st++) {
        float in[P];
#pragma unroll
        for (int p = 0; p < P; p++) in[p] = st > 0 ? lane_up<NSB>(acc[p]) : 0.0f;
        if (sb == (uint32_t)st) {
#pragma unroll
            for (int p = 0; p < P; p++) {
                float a = in[p];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    a = __builtin_fmaf(mmv[j], uv[p][j], a);
                    a = __builtin_fmaf(dotv[p][j], tv[p][j], a);
                }
                acc[p] = a;
            }
        }
    }
    if (wthread && sb == NSB - 1)
#pragma unroll
        for (int p = 0; p < P; p++) hres[r * P + p] = acc[p];
    __syncthreads();
    if (tid < 16) {
        // pair rows: coarse + residual (gemv.rs:154); act = silu512(g) * u (elem.rs:173); then
        // quantise the 16-block (kb = down.kb = 16) across these 16 lanes and fold the weight
        // into the scales (exec.rs:1590-1605)
        const float g = P == 2 ? hres[tid * P] + hres[tid * P + 1] : hres[tid * P];
        const float u = P == 2 ? hres[(16 + tid) * P] + hres[(16 + tid) * P + 1] : hres[(16 + tid) * P];
        const float av = silu512(g) * u;
        if (shared) wgt = sigmoid_libm(shl);  // exec.rs:1606
        const uint32_t aslot = shared ? kcap : slot;
        const uint32_t nbf = F / 16;
        int8_t* dq = ws.actq + (size_t)aslot * P * F + strip * 16;
        float* ds = ws.acts + (size_t)aslot * P * nbf + strip;
        int32_t* dsu = ws.actsum + (size_t)aslot * P * nbf + strip;
        float* dsx = ws.actu + (size_t)aslot * P * nbf + strip;  // folded scale * sum (gemv.rs:144)
        float v = av;
#pragma unroll
        for (int p = 0; p < P; p++) {
            const float amax = row16_allreduce(__builtin_fabsf(v), [](float a, float b) { return mx_ps(a, b); });
            const float sc = amax / 127.0f;
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            const int32_t qi = cvt_rne(v * inv);
            const int32_t sum = row16_allreduce(qi, [](int32_t a, int32_t b) { return a + b; });
            if constexpr (COH) {  // 4 lanes' bytes in one device-coherent word (quad_perm gathers)
                const uint32_t b0 = (uint8_t)sat_i8(qi);
                const uint32_t b1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)b0, 0xF9, 0xf, 0xf, false);
                const uint32_t b2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)b0, 0xFE, 0xf, 0xf, false);
                const uint32_t b3 = (uint32_t)__builtin_amdgcn_mov_dpp((int)b0, 0xFF, 0xf, 0xf, false);
                if (tid % 4 == 0)
                    st_dev(reinterpret_cast<uint32_t*>(dq + p * F + tid), b0 | (b1 << 8) | (b2 << 16) | (b3 << 24));
                if (tid == 0) {
                    st_devf(ds + p * nbf, sc * wgt);
                    st_dev(reinterpret_cast<uint32_t*>(dsu + p * nbf), (uint32_t)sum);
                    st_devf(dsx + p * nbf, (sc * wgt) * (float)sum);
                }
            } else {
                dq[p * F + tid] = sat_i8(qi);
                if (tid == 0) {
                    ds[p * nbf] = sc * wgt;
                    dsu[p * nbf] = sum;
                    dsx[p * nbf] = (sc * wgt) * (float)sum;
                }
            }
            v = __builtin_fmaf(-(float)qi, sc, v);  // residual for the second level (quant.rs:132)
        }
    }
}

// LDS of a gate/up unit: x (padded superblocks), scales, row results; then the routing area
template <int P, int NSB>
constexpr uint32_t gu_lds_x() { return P * NSB * (256 + 16) + P * NSB * 8 * 8 + 32 * P * 4; }
constexpr uint32_t ROUTE_LDS = K_MAX * 8 + 16 + ROUTE_CAND * 8;  // + E floats for MassBasis::All

struct NoHook {
    __device__ void operator()(const uint32_t*, uint32_t) const {}
};
struct NoPre {
    __device__ void operator()() const {}
};

// Token t's view of the workspace for a batch run as per-token decode units (P = 1): its x row,
// shared-gate logit, routing row and (kcap + 1) activation slots.  t = 0 is the decode layout.
__device__ __forceinline__ Workspace ws_token(const Workspace& ws, uint32_t t, uint32_t kcap, uint32_t P) {
    Workspace w = ws;
    const uint32_t nb = ws.H / 32, nbf = ws.F / 16;
    const size_t ar = (size_t)t * (kcap + 1) * P;
    w.xq += (size_t)t * ws.H;
    w.xs += (size_t)t * nb;
    w.xsum += (size_t)t * nb;
    w.xu += (size_t)t * nb;
    w.shl += t;
    w.ids += (size_t)t * K_MAX;
    w.w += (size_t)t * K_MAX;
    w.n_sel += t;
    w.actq += ar * ws.F;
    w.acts += ar * nbf;
    w.actsum += ar * nbf;
    w.actu += ar * nbf;
    return w;
}

// Grid (F / 16 strips, kcap + 1 slots, tokens): token blockIdx.z's unit (slot, strip).
template <int P, int NSB, int NJ>
__global__ __launch_bounds__(GU_THREADS(NSB)) void decode_gateup_kernel(
        Mat gate, Mat up, Mat shg, Mat shu, const float* __restrict__ x, const float* __restrict__ lg, Workspace ws,
        uint32_t k, Policy pol, uint32_t kcap) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t t = blockIdx.z;
    const Workspace wt = ws_token(ws, t, kcap, P);
    gateup_unit<P, NSB, NJ, false, true>(gate, up, shg, shu, x + (size_t)t * ws.H, lg + (size_t)t * ws.E, wt, k, pol,
                                         kcap, blockIdx.y, blockIdx.x, true, false, blockIdx.x == 0 && blockIdx.y == 0,
                                         smem, smem + gu_lds_x<P, NSB>(), NoPre{}, NoHook{});
}

hipError_t launch_decode_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const float* x,
                                const float* lg, const Workspace& ws, uint32_t k, Policy pol, int pair, uint32_t kcap,
                                hipStream_t st, uint32_t m) {
    if (m > 1 && pair) return hipErrorInvalidValue;  // a batch's activations are single-level
    const uint32_t H = gate.k, F = gate.rows, nb = H / 32, nsb = H / 256;
    const int P = pair ? 2 : 1;
    size_t lds = (size_t)P * nsb * 272 + (size_t)P * nb * 8 + 32 * P * 4 + ROUTE_LDS;
    if (pol.enabled && pol.basis == TRK_BASIS_ALL) lds += (size_t)ws.E * 4;
    const dim3 g(F / 16, kcap + 1, m);
    const uint32_t threads = GU_THREADS(nsb);
    const bool nj16 = route_nj(ws.E) == 16;
    switch ((nsb * 2 + (pair ? 1 : 0)) * 2 + (nj16 ? 1 : 0)) {
#define GU_CASE2(ns, p, nj)                                                                                      \
    case (ns * 2 + p - 1) * 2 + (nj == 16 ? 1 : 0):                                                              \
        decode_gateup_kernel<p, ns, nj><<<g, threads, lds, st>>>(gate, up, sh_gate, sh_up, x, lg, ws, k, pol, kcap); \
        break;
#define GU_CASE(ns) GU_CASE2(ns, 1, 8) GU_CASE2(ns, 1, 16) GU_CASE2(ns, 2, 8) GU_CASE2(ns, 2, 16)
        GU_CASE(1) GU_CASE(2) GU_CASE(3) GU_CASE(4) GU_CASE(5) GU_CASE(6) GU_CASE(7) GU_CASE(8)
#undef GU_CASE
#undef GU_CASE2
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- down ------------------------------------------------------------------------------------

// A unit is one (slot, output row) of a down workgroup; its 16-blocks are split over DN_L = 2*NSB
// lanes, half a superblock (8 blocks) each, in chain order.  The lanes of a unit sit side by side
// in one wave and never straddle a wave.
template <int NSB>
struct DownLanes {
    static constexpr int L = 2 * NSB;        // lanes per unit
    static constexpr int UPW = 64 / L;       // units per wave
    static constexpr int UPP = 4 * UPW;      // units per pass of the 256-thread workgroup
};


// Work unit u = slot * DN_R + row of a workgroup; slots 0..kcap-1 are the routed slots (those at
// or past n idle), slot kcap is the shared expert.  Activation rows are staged in LDS with slot
// stride P*F + 16 bytes (fewer bank conflicts between slots).  `ids` / `n` are the routing (in
// global memory for the standalone kernel, in LDS for the fused layer kernel).

// A lane's first unit, with its weights requested ahead of everything else.
struct DownFirst {
    bool live;
    const uint8_t* rowp;
    uint4 hdr, qs[4];
};

template <int NSB>
__device__ __forceinline__ const uint8_t* down_unit_row(const Mat& down, const Mat& shd, uint32_t kcap, uint32_t n,
                                                        uint32_t eid, uint32_t row0, uint32_t u, bool& live) {
    using DL = DownLanes<NSB>;
    const uint32_t ln = threadIdx.x % 64;
    const uint32_t s = u / DN_R, r = u % DN_R;
    const bool sh = s == kcap;
    live = ln < (uint32_t)(DL::UPW * DL::L) && u < (kcap + 1) * DN_R && (sh || s < n);
    // per-lane choice of matrix: select the fields (a per-lane reference would put both in scratch)
    const uint8_t* base = sh ? shd.ptr : down.ptr;
    const uint64_t stride = sh ? shd.stride : down.stride;
    const uint32_t rb = sh ? shd.row_bytes : down.row_bytes;
    const uint32_t e = (sh || !live) ? 0u : eid;
    return base + (size_t)e * stride + (size_t)(row0 + r) * rb;
}

// The slot id a lane's first unit reads (requested ahead of the activations, so that the weight
// requests wait only for it).
template <int NSB>
__device__ __forceinline__ uint32_t down_first_id(const uint32_t* ids, uint32_t kcap) {
    using DL = DownLanes<NSB>;
    const uint32_t s = (threadIdx.x / 64 * DL::UPW + threadIdx.x % 64 / DL::L) / DN_R;
    return ids[s < kcap ? s : 0u];
}

// Q4: 1 the down format is Q4_K, 0 another, -1 known only at run time.  Known at compile time the
// requests need no branch around them (a branch makes the wait before the activation stores cover
// the weights too).
template <int NSB, int Q4 = -1>
__device__ __forceinline__ void down_first(const Mat& down, const Mat& shd, uint32_t kcap, uint32_t n,
                                           uint32_t eid0, uint32_t row0, DownFirst& f) {
    using DL = DownLanes<NSB>;
    const uint32_t wv = threadIdx.x / 64, ln = threadIdx.x % 64, q = ln % DL::L;
    const uint32_t u0 = wv * DL::UPW + ln / DL::L;
    f.rowp = down_unit_row<NSB>(down, shd, kcap, n, eid0, row0, u0, f.live);
    f.hdr = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) f.qs[i] = f.hdr;
    // lanes without a unit read expert 0 (a valid row): no per-lane branch around the requests
    if (Q4 == 1 || (Q4 < 0 && down.fmt == TRK_FMT_Q4_K)) load_half_q4k(f.rowp, q / 2, q % 2, f.hdr, f.qs);
}

// The slots' activation rows, scales and sums, staged in LDS: one piece (16 bytes of a row, its
// 16-block's scale and sum) per entry, a round of 4 entries per thread (1024 per round).
typedef int v4i32 __attribute__((ext_vector_type(4)));  // (HIP's int4 arrays went to scratch here)
struct DownStage {
    v4i32 t[4];
    float sc[4], u[4];  // folded scale, scale * sum (written by the gate/up launch)
};

template <int P, int NSB, bool COH>
__device__ __forceinline__ void down_stage_load(const Workspace& ws, uint32_t kcap, uint32_t i0, DownStage& st) {
    constexpr uint32_t F = NSB * 256, QP = P * F / 16;  // int4 pieces of a slot = its scales = its sums
    const uint32_t tid = threadIdx.x, nq = (kcap + 1) * QP;
    // clamped indices, so no per-lane branch separates the loads
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t i = i0 + tid + 256 * c, ic = i < nq ? i : nq - 1;
        const uint32_t a = ic / QP;  // slot (the shared expert's at kcap)
        const int4* src = reinterpret_cast<const int4*>(ws.actq + (size_t)a * P * F) + ic % QP;
        const size_t o = (size_t)a * QP + ic % QP;
        if constexpr (COH) {
            const unsigned long long* w2 = reinterpret_cast<const unsigned long long*>(src);
            const unsigned long long lo = ld_dev(w2), hi = ld_dev(w2 + 1);
            st.t[c] = v4i32{(int)(uint32_t)lo, (int)(uint32_t)(lo >> 32), (int)(uint32_t)hi, (int)(uint32_t)(hi >> 32)};
            st.sc[c] = ld_devf(ws.acts + o);
            st.u[c] = ld_devf(ws.actu + o);
        } else {
            st.t[c] = *reinterpret_cast<const v4i32*>(src);
            st.sc[c] = ws.acts[o];
            st.u[c] = ws.actu[o];
        }
    }
}

template <int P, int NSB>
__device__ __forceinline__ void down_stage_store(uint8_t* smem, uint32_t kcap, uint32_t i0, const DownStage& st) {
    constexpr uint32_t F = NSB * 256, nbf = NSB * 16, SQ = P * F + 16, QP = P * F / 16;
    static_assert(QP == P * nbf, "a 16-byte piece per 16-block");
    const uint32_t slots = kcap + 1, nq = slots * QP, tid = threadIdx.x;
    int8_t* aq = (int8_t*)smem;                       // [slots][SQ]
    float* as = (float*)(smem + (size_t)slots * SQ);  // [slots][P][nbf] folded scale
    float* au = as + slots * P * nbf;                 // [slots][P][nbf] scale * sum
    // every thread stores (entries past the end repeat the last one with its own value): a
    // conditional store would let the compiler sink the loads behind the weight requests
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t i = i0 + tid + 256 * c, ic = i < nq ? i : nq - 1;
        *reinterpret_cast<v4i32*>(aq + (size_t)(ic / QP) * SQ + (ic % QP) * 16) = st.t[c];
        as[ic] = st.sc[c];
        au[ic] = st.u[c];
    }
}

// PRE: st holds the first staging round, already requested (the standalone kernel requests it ahead
// of the weights, so the activations' round trip overlaps the weights'); otherwise requested here
// BORDER: the batch combine's order (exec_batch.rs:1539-1578: the shared expert's row first, then
// the token's entries by ascending expert) instead of the decode's (slots in routing order, the
// shared expert last).
template <int P, int NSB, bool COH, bool PRE, bool BORDER = false>
__device__ __forceinline__ void down_unit(const Mat& down, const Mat& shd, const Workspace& ws, uint32_t kcap,
                                          uint32_t n, const uint32_t* ids, float* __restrict__ out, int residual,
                                          uint32_t row0, uint8_t* smem, const DownFirst& first, DownStage& st) {
    using DL = DownLanes<NSB>;
    constexpr uint32_t F = NSB * 256, nbf = NSB * 16, SQ = P * F + 16;
    const uint32_t tid = threadIdx.x;
    const uint32_t slots = kcap + 1, units = slots * DN_R;
    const uint32_t wv = tid / 64, ln = tid % 64, q = ln % DL::L;
    const uint32_t sb = q / 2, h2 = q % 2;
    const bool q4 = down.fmt == TRK_FMT_Q4_K, q8 = down.fmt == TRK_FMT_Q8_0, q5 = down.fmt == TRK_FMT_Q5_1;

    int8_t* aq = (int8_t*)smem;                                // [slots][SQ]
    float* as = (float*)(smem + (size_t)slots * SQ);           // [slots][P][nbf] folded scale
    float* au = as + slots * P * nbf;                          // [slots][P][nbf] scale * sum
    float* vres = au + slots * P * nbf;                        // [slots][DN_R]

    {
        // one memory round trip per round of 4 (int4 piece, scale, sum) per thread
        const uint32_t nq = slots * (P * F / 16);
        if (!PRE) down_stage_load<P, NSB, COH>(ws, kcap, 0, st);
        down_stage_store<P, NSB>(smem, kcap, 0, st);
        for (uint32_t i0 = 1024; i0 < nq; i0 += 1024) {
            DownStage sn;
            down_stage_load<P, NSB, COH>(ws, kcap, i0, sn);
            down_stage_store<P, NSB>(smem, kcap, i0, sn);
        }
    }
    __syncthreads();
    const uint32_t u0 = wv * DL::UPW + ln / DL::L;
    uint4 hdr = first.hdr, qs[4] = {first.qs[0], first.qs[1], first.qs[2], first.qs[3]};
    for (uint32_t pass = 0; pass * DL::UPP < units; pass++) {
        const uint32_t u = pass * DL::UPP + u0;
        bool live = first.live;
        const uint8_t* rowp = first.rowp;
        if (pass > 0) {
            const uint32_t su = u / DN_R;
            rowp = down_unit_row<NSB>(down, shd, kcap, n, su < kcap ? ids[su] : 0u, row0, u, live);
            if (live && q4) load_half_q4k(rowp, sb, h2, hdr, qs);
        }
        const uint32_t s = live ? u / DN_R : 0u;
        float dotv[P][8], tv[P][8], mmv[8], uv[P][8];
        const uint32_t b0 = 8 * q;  // first block of this lane within the row
        const int8_t* a = aq + (size_t)s * SQ + b0 * 16;
        const float* sa = as + s * P * nbf + b0;
        const float* ua = au + s * P * nbf + b0;
        if (q4)
            half_terms_q4k<P>(hdr, qs, h2, a, F, sa, ua, nbf, dotv, tv, mmv, uv);
        else if (q8)
            half_terms_q80<P>(rowp, sb, h2, a, F, sa, ua, nbf, dotv, tv, mmv, uv);
        else if (q5)
            half_terms_q51<P>(rowp, sb, h2, a, F, sa, ua, nbf, dotv, tv, mmv, uv);
        else
            half_terms_q6k<P>(rowp, sb, h2, a, F, sa, ua, nbf, dotv, tv, mmv, uv);
        // the chain (gemv.rs:141-148) over the unit's lanes in block order
        float acc[P];
#pragma unroll
        for (int p = 0; p < P; p++) acc[p] = 0.0f;
#pragma unroll
        for (int st = 0; st < DL::L; st++) {
            float in[P];
#pragma unroll
            for (int p = 0; p < P; p++) in[p] = st > 0 ? unit_up<DL::L>(acc[p]) : 0.0f;
            if (q == (uint32_t)st) {
#pragma unroll
                for (int p = 0; p < P; p++) {
                    float v = in[p];
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        v = __builtin_fmaf(mmv[i], uv[p][i], v);
                        v = __builtin_fmaf(dotv[p][i], tv[p][i], v);
                    }
                    acc[p] = v;
                }
            }
        }
        if (live && q == (uint32_t)DL::L - 1)
            vres[s * DN_R + u % DN_R] = P == 2 ? acc[0] + acc[1] : acc[0];  // gemv.rs:154
    }
    uint32_t* perm = reinterpret_cast<uint32_t*>(vres + slots * DN_R);  // [32] BORDER: slots by expert
    if constexpr (BORDER) {
        if (tid < n) {  // the token's experts are distinct: rank = how many are smaller
            const uint32_t e = ids[tid];
            uint32_t rank = 0;
            for (uint32_t j = 0; j < n; j++) rank += ids[j] < e ? 1u : 0u;
            perm[rank] = tid;
        }
    }
    __syncthreads();
    if (tid < DN_R) {
        float y;
        if constexpr (BORDER) {
            y = vres[kcap * DN_R + tid];
            for (uint32_t j = 0; j < n; j++) y = y + vres[perm[j] * DN_R + tid];
        } else {
            // slot 0 stores, later slots accumulate, the shared expert last (gemv.rs:150-160 with
            // accumulate = slot > 0; exec.rs:1607-1620)
            y = n > 0 ? vres[tid] : vres[kcap * DN_R + tid];
            for (uint32_t s = 1; s < n; s++) y = y + vres[s * DN_R + tid];
            if (n > 0) y = y + vres[kcap * DN_R + tid];
        }
        float* o = out + row0 + tid;
        *o = residual ? *o + y : y;
    }
}

// Grid (H / DN_R, tokens): token blockIdx.y's output rows; BORDER for a batch (the batch combine's
// order), the decode's order otherwise.
template <int P, int NSB, int Q4, bool BORDER>
__global__ __launch_bounds__(256) void decode_down_kernel(Mat down, Mat shd, Workspace ws, uint32_t kcap,
                                                         float* __restrict__ out, int residual) {
    extern __shared__ __align__(16) uint8_t smem[];
    const Workspace wt = ws_token(ws, blockIdx.y, kcap, P);
    out += (size_t)blockIdx.y * ws.H;
    // the count and the first unit's expert id are requested together (slots below kcap are inside
    // the id row; a slot past the count is never used), then the activations, whose round trip runs
    // beside the weights' once the id is in
    const uint32_t row0 = blockIdx.x * DN_R, n = wt.n_sel[0], eid0 = down_first_id<NSB>(wt.ids, kcap);
    DownStage st;
    down_stage_load<P, NSB, false>(wt, kcap, 0, st);
    __builtin_amdgcn_sched_barrier(0);  // keep those requests ahead of the weights'
    DownFirst first;
    down_first<NSB, Q4>(down, shd, kcap, n, eid0, row0, first);
    down_unit<P, NSB, false, true, BORDER>(down, shd, wt, kcap, n, wt.ids, out, residual, row0, smem, first, st);
}

// ---- the whole decode layer in one launch ----------------------------------------------------
//
// One grid, four roles by workgroup index, in dependency order:
//   [0, nA)              router logits (attn::dot order, exec.rs:1003-1011) and the shared gate's
//                        logit, a wave per router row;
//   next S = F / 16      the shared expert's gate/up strips: they need no routing, so their weights
//                        are requested at once (only the sigmoid fold waits for the gate's logit);
//   next kcap * S        the routed gate/up units (slot, strip): each waits for the router
//                        workgroups, routes the token itself (no round trip through memory between
//                        the logits and the expert weights) and runs its unit; unit (0, 0) also
//                        publishes the routing;
//   last H / DN_R        down + combine for DN_R output rows each: waits for the published routing,
//                        requests its down weights at once, then waits for every gate/up unit.
// A workgroup only waits on workgroups of lower index, which the dispatcher places first, so the
// grid need not be resident at once.  The waits are counters in ws.counters, raised by the waited-on
// workgroups once their device-coherent stores (st_dev: past the per-XCD L2s) are complete; the last
// workgroup to finish zeroes them for the next launch.  Every wait is bounded: on time-out it raises
// the flag at ws.counters[2] (trk_get_stats reports it) and carries on.

constexpr uint32_t PIPE_A = BAR_LINE, PIPE_R = 2 * BAR_LINE, PIPE_B = 3 * BAR_LINE, PIPE_D = 4 * BAR_LINE;
constexpr uint32_t PIPE_SPIN = 1u << 16;  // polls before a wait gives up (tens of ms)

__device__ __forceinline__ void pipe_wait(uint32_t* words, uint32_t which, uint32_t target) {
    if (threadIdx.x == 0) {
        uint32_t spins = 0;
        while (ld_dev(words + which) < target) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins == PIPE_SPIN) {
                __hip_atomic_fetch_or(words + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
}

// raise counter `which` once every thread's stores of this workgroup are complete
__device__ __forceinline__ void pipe_signal(uint32_t* words, uint32_t which) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(words + which, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int P, int NSB, int NJ, int NSBF>
__global__ __launch_bounds__(256) void decode_pipe_kernel(const float* __restrict__ router,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ shgv, Mat gate, Mat up, Mat down,
                                                         Mat shg, Mat shu, Mat shd, const float* __restrict__ x,
                                                         const float* __restrict__ lg_in, Workspace ws, uint32_t k,
                                                         Policy pol, uint32_t kcap, float* __restrict__ out,
                                                         int residual, uint32_t rsm_bytes, uint32_t nA) {
    constexpr uint32_t H = NSB * 256;
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t* rsm = smem;              // routing
    uint8_t* usm = smem + rsm_bytes;  // unit area: gate/up or down
    const uint32_t E = ws.E, nwg = gridDim.x, wg = blockIdx.x, tid = threadIdx.x;
    const uint32_t S = gate.rows / 16, gu = S * (kcap + 1);
    uint32_t* cw = ws.counters;

    if (wg < nA) {
        const uint32_t wv = tid / 64, lane = tid % 64;
        for (uint32_t row = wg * 4 + wv; row <= E; row += nA * 4) {
            if (lg_in && row < E) continue;
            const float* wr = row < E ? router + (size_t)row * H : shgv;
            float res[DOT_MR];
            dot_rows(wr, x, 0, 1, H, lane, res);
            if (lane == 0) {
                if (row < E)
                    st_devf(ws.rlog + row, bias ? res[0] + bias[row] : res[0]);
                else
                    st_devf(ws.shl, res[0]);
            }
        }
        pipe_signal(cw, PIPE_A);
    } else if (wg < nA + gu) {
        const uint32_t u = wg - nA;
        const uint32_t slot = u < S ? kcap : u / S - 1, strip = u % S;  // the shared strips first
        const float* lg = lg_in ? lg_in : ws.rlog;
        gateup_unit<P, NSB, NJ, true, false>(gate, up, shg, shu, x, lg, ws, k, pol, kcap, slot, strip, true, false,
                                             slot == 0 && strip == 0, usm, rsm,
                                             [&]() { pipe_wait(cw, PIPE_A, nA); }, NoHook{}, cw + PIPE_R);
        pipe_signal(cw, PIPE_B);
    } else {
        const uint32_t row0 = (wg - nA - gu) * DN_R;
        uint32_t* r_ids = reinterpret_cast<uint32_t*>(rsm);  // [K_MAX] ids, then n
        pipe_wait(cw, PIPE_R, 1);
        if (tid < kcap) r_ids[tid] = ld_dev(ws.ids + tid);
        if (tid == 0) r_ids[K_MAX] = ld_dev(ws.n_sel);
        __syncthreads();
        const uint32_t n = r_ids[K_MAX];
        DownFirst first;
        down_first<NSBF>(down, shd, kcap, n, down_first_id<NSBF>(r_ids, kcap), row0, first);  // in flight during the wait
        pipe_wait(cw, PIPE_B, gu);
        DownStage st;
        down_unit<P, NSBF, true, false>(down, shd, ws, kcap, n, r_ids, out, residual, row0, usm, first, st);
    }
    __syncthreads();
    if (tid == 0) {  // the last workgroup out zeroes the counters for the next launch
        const uint32_t done = __hip_atomic_fetch_add(cw + PIPE_D, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == nwg - 1) {
            st_dev(cw + PIPE_A, 0u);
            st_dev(cw + PIPE_R, 0u);
            st_dev(cw + PIPE_B, 0u);
            st_dev(cw + PIPE_D, 0u);
        }
    }
}

template <int P, int NSB, int NSBF>
static size_t pipe_lds(uint32_t E, uint32_t kcap, bool mass_all, uint32_t& rsm) {
    rsm = (ROUTE_LDS + (mass_all ? E * 4 : 0) + 15) / 16 * 16;
    const size_t gu = gu_lds_x<P, NSB>();
    const size_t slots = kcap + 1, F = NSBF * 256, nbf = F / 16;
    const size_t dn = slots * (P * F + 16) + slots * P * nbf * 8 + slots * DN_R * 4 + 64;
    return rsm + (gu > dn ? gu : dn);
}

// The shapes the one-launch layer is instantiated for (H / 256, F / 256): BASELINE's layer
// (2048, 512) and the test shapes (512, 256), (768, 768).
static int pipe_shape(uint32_t H, uint32_t F) {
    if (H == 2048 && F == 512) return 0;
    if (H == 512 && F == 256) return 1;
    if (H == 768 && F == 768) return 2;
    return -1;
}

bool decode_layer_supported(const Mat& gate, const Mat& down, const Mat& sh_down, uint32_t E, int pair,
                            uint32_t kcap) {
    (void)pair;
    (void)kcap;
    return pipe_shape(gate.k, gate.rows) >= 0 && E <= 1024 && down.fmt == sh_down.fmt && gate.k % DN_R == 0;
}

template <int P, int NSB, int NJ, int NSBF>
static hipError_t launch_pipe(const float* router, const float* bias, const float* shexp_gate, const Mat& gate,
                              const Mat& up, const Mat& down, const Mat& sh_gate, const Mat& sh_up, const Mat& sh_down,
                              const float* x, const float* rlog, const Workspace& ws, uint32_t k, Policy pol,
                              uint32_t kcap, float* out, int residual, hipStream_t st) {
    const uint32_t H = gate.k, F = gate.rows, E = ws.E;
    const bool mass_all = pol.enabled && pol.basis == TRK_BASIS_ALL;
    uint32_t rsm = 0;
    const size_t lds = pipe_lds<P, NSB, NSBF>(E, kcap, mass_all, rsm);
    const uint32_t nA = rlog ? 1u : (E + 1 + 3) / 4;
    const uint32_t nwg = nA + (F / 16) * (kcap + 1) + H / DN_R;
    decode_pipe_kernel<P, NSB, NJ, NSBF><<<nwg, 256, lds, st>>>(router, bias, shexp_gate, gate, up, down, sh_gate,
                                                                sh_up, sh_down, x, rlog, ws, k, pol, kcap, out,
                                                                residual, rsm, nA);
    return hipGetLastError();
}

// The whole layer in one launch: hipErrorNotSupported when the shape has no instantiation (the
// caller then runs the three separate launches).  check_only: answer that without launching.
hipError_t launch_decode_layer(const float* router, const float* bias, const float* shexp_gate, const Mat& gate,
                               const Mat& up, const Mat& down, const Mat& sh_gate, const Mat& sh_up,
                               const Mat& sh_down, const float* x, const float* rlog, const Workspace& ws, uint32_t k,
                               Policy pol, int pair, uint32_t kcap, float* out, int residual, bool check_only,
                               hipStream_t st) {
    const int shp = pipe_shape(gate.k, gate.rows);
    if (!decode_layer_supported(gate, down, sh_down, ws.E, pair, kcap) || !ws.counters || shp < 0 ||
        (!router && !rlog))
        return hipErrorNotSupported;
    if (check_only) return hipSuccess;
    const bool nj16 = route_nj(ws.E) == 16;
#define PIPE_ARGS router, bias, shexp_gate, gate, up, down, sh_gate, sh_up, sh_down, x, rlog, ws, k, pol, kcap, out, residual, st
#define PIPE_SHAPE(P, NSB, NSBF) \
    return nj16 ? launch_pipe<P, NSB, 16, NSBF>(PIPE_ARGS) : launch_pipe<P, NSB, 8, NSBF>(PIPE_ARGS);
    if (pair) {
        if (shp == 0) PIPE_SHAPE(2, 8, 2)
        if (shp == 1) PIPE_SHAPE(2, 2, 1)
        PIPE_SHAPE(2, 3, 3)
    } else {
        if (shp == 0) PIPE_SHAPE(1, 8, 2)
        if (shp == 1) PIPE_SHAPE(1, 2, 1)
        PIPE_SHAPE(1, 3, 3)
    }
#undef PIPE_SHAPE
#undef PIPE_ARGS
}

hipError_t launch_decode_down(const Mat& down, const Mat& sh_down, const Workspace& ws, int pair, uint32_t kcap,
                              float* out, int residual, hipStream_t st, uint32_t m) {
    const uint32_t H = down.rows, F = down.k, nbf = F / 16;
    const int P = pair ? 2 : 1;
    if (m > 1 && pair) return hipErrorInvalidValue;  // a batch's activations are single-level
    const size_t slots = kcap + 1;
    const size_t lds = slots * ((size_t)P * F + 16) + slots * P * nbf * 8 + slots * DN_R * 4 + K_MAX * 4 + 64;
    const bool q4 = down.fmt == TRK_FMT_Q4_K;
    const dim3 grid(H / DN_R, m);
    switch ((F / 256 * 2 + (pair ? 1 : 0)) * 2 + (q4 ? 1 : 0)) {
#define DN_CASE2(ns, p, q)                                                                                          \
    case (ns * 2 + p - 1) * 2 + q:                                                                                  \
        if (m > 1)                                                                                                  \
            decode_down_kernel<p, ns, q, true><<<grid, 256, lds, st>>>(down, sh_down, ws, kcap, out, residual);     \
        else                                                                                                        \
            decode_down_kernel<p, ns, q, false><<<grid, 256, lds, st>>>(down, sh_down, ws, kcap, out, residual);    \
        break;
#define DN_CASE(ns) DN_CASE2(ns, 1, 0) DN_CASE2(ns, 1, 1) DN_CASE2(ns, 2, 0) DN_CASE2(ns, 2, 1)
        DN_CASE(1) DN_CASE(2) DN_CASE(3) DN_CASE(4) DN_CASE(5) DN_CASE(6) DN_CASE(7) DN_CASE(8)
#undef DN_CASE
#undef DN_CASE2
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace trk
