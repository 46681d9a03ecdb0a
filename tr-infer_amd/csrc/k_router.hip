// Router logits and routing.
//
//   router_dot:   attn::dot order (attn.rs:329-357), one wave per weight row: lane L = 16c + j is
//                 lane j of accumulator chain c, so the wave holds exactly the reference's four
//                 16-lane FMA chains (64-wide steps), the 16-wide tail goes to chain 0, then
//                 (c0 + c1) + (c2 + c3) lanewise and the halving tree of _mm512_reduce_add_ps.
//   router_gemm:  smallgemm::gemm_f32_nt order (smallgemm.rs:8-59): per output, 16 lane chains
//                 over 16-wide steps, then the halving tree; LDS-staged register tiles.
//   route:        one wave per token runs route_row (route.hpp).  The decode path (M = 1) routes
//                 inside its gate/up kernel instead (k_decode.hip).
#include "route.hpp"
#include "router.hpp"

namespace trk {

// Quantise a 32-block held by the 4 lanes of a quad (lane q: values 8q..8q+7) as quant_block_regs<32>
// does (quant.rs:112-166): the block maximum and the integer sum do not depend on the order, so
// quad all-reduces give the same scale and sum.  qw: this lane's 8 bytes.
template <bool RESID>
__device__ __forceinline__ void quant_block_quad(const float (&v)[8], uint32_t (&qw)[2], float& scale, int32_t& sum,
                                                 float (&resid)[8]) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = mx_ps(amax, __builtin_fabsf(v[i]));
    amax = mx_ps(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0xB1, 0xf, 0xf, false)));
    amax = mx_ps(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x4E, 0xf, 0xf, false)));
    const float s = amax / 127.0f;
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    int32_t su = 0;
#pragma unroll
    for (int w = 0; w < 2; w++) {
        uint32_t packed = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int i = 4 * w + b;
            const int32_t qi = cvt_rne(v[i] * inv);
            su += qi;
            packed |= (uint32_t)(uint8_t)sat_i8(qi) << (8 * b);
            if (RESID) resid[i] = __builtin_fmaf(-(float)qi, s, v[i]);
        }
        qw[w] = packed;
    }
    su += __builtin_amdgcn_mov_dpp(su, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    su += __builtin_amdgcn_mov_dpp(su, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    scale = s;
    sum = su;
}

// x quantised per 32 by the workgroups after the logit rows, four lanes per block: one row in
// pair mode (quantize_pair_blocks, quant.rs:96-108: level 1 at +H / +H/32), else m rows single
// level (QAct::quantize, quant.rs:76-92, as moe_batch's quant_rows).
// NORM: x is rmsnorm's input; the workgroup's waves first compute the factors of the rows its
// blocks fall in (rinv: LDS, one per row, at most blockDim.x / 4 / (H / 32) + 2 rows).
template <bool NORM = false>
__device__ __forceinline__ void quantize_x_rows(const float* __restrict__ x, uint32_t m, uint32_t H,
                                                const XQuant& xq, uint32_t qwg, const XNorm& nrm = XNorm{},
                                                float* rinv = nullptr) {
    const uint32_t nb = H / 32, t = qwg * blockDim.x + threadIdx.x, id = t / 4, qd = t % 4;
    const uint32_t idc = id < m * nb ? id : m * nb - 1;
    const uint32_t row = idc / nb, b = idc % nb;
    const bool live = id < m * nb;
    const float4* src = reinterpret_cast<const float4*>(x + (size_t)row * H + (size_t)b * 32 + 8 * qd);
    const float4 a = src[0], c = src[1];  // in flight while the factors are computed
    float rr = 1.0f;
    if constexpr (NORM) {
        const uint32_t i0 = qwg * blockDim.x / 4, i1 = i0 + blockDim.x / 4 - 1;
        const uint32_t r0 = (i0 < m * nb ? i0 : m * nb - 1) / nb, r1 = (i1 < m * nb ? i1 : m * nb - 1) / nb;
        for (uint32_t rw = r0 + threadIdx.x / WAVE; rw <= r1; rw += blockDim.x / WAVE) {
            const float v = row_rms_inv(x + (size_t)rw * H, H, nrm.eps, threadIdx.x % WAVE);
            if (threadIdx.x % WAVE == 0) rinv[rw - r0] = v;
        }
        __syncthreads();
        rr = rinv[row - r0];
    }
    float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
    if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = rms_apply(v[i], rr, nrm.w, b * 32 + 8 * qd + i);
    }
    float r[8], r2[8];
    uint32_t qw[2];
    float s;
    int32_t su;
    quant_block_quad<true>(v, qw, s, su, r);
    const size_t qo = (size_t)row * H + (size_t)b * 32 + 8 * qd, so = (size_t)row * nb + b;
    if (live) {
        *reinterpret_cast<uint2*>(xq.q + qo) = make_uint2(qw[0], qw[1]);
        if (qd == 0) {
            xq.s[so] = s;
            xq.sum[so] = su;
            xq.u[so] = s * (float)su;  // gemv.rs:144
        }
    }
    if (xq.pair) {  // m == 1
        quant_block_quad<false>(r, qw, s, su, r2);
        if (live) {
            *reinterpret_cast<uint2*>(xq.q + H + qo) = make_uint2(qw[0], qw[1]);
            if (qd == 0) {
                xq.s[nb + so] = s;
                xq.sum[nb + so] = su;
                xq.u[nb + so] = s * (float)su;
            }
        }
    }
}

// grid.x: waves over weight rows ([0, E) router rows + bias, row E = shared gate if shg), then
// (xquant) the workgroups that quantise x; grid.y: chunks of DOT_MR activation rows.
// NORM: x is rmsnorm's input (the config-5 layer), normalised where it is read: each dot wave
// computes its rows' factors, each quantising workgroup those of its rows.
template <bool NORM>
__global__ __launch_bounds__(128) void router_dot_kernel(const float* __restrict__ router,
                                                        const float* __restrict__ bias,
                                                        const float* __restrict__ shg,
                                                        const float* __restrict__ x, uint32_t m, uint32_t E,
                                                        uint32_t H, float* __restrict__ rlog, float* __restrict__ sh,
                                                        XQuant xquant, uint32_t qwg0, XNorm nrm) {
    if (xquant.q && blockIdx.x >= qwg0) {  // workgroup-uniform
        if constexpr (NORM) {  // LDS only in this instantiation
            __shared__ float rq[128 / 4 + 2];
            if (blockIdx.y == 0) quantize_x_rows<true>(x, m, H, xquant, blockIdx.x - qwg0, nrm, rq);
        } else {
            if (blockIdx.y == 0) quantize_x_rows(x, m, H, xquant, blockIdx.x - qwg0);
        }
        return;
    }
    const uint32_t wave = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (wave >= E + (shg ? 1u : 0u)) return;
    const float* wr = wave < E ? router + (size_t)wave * H : shg;
    const uint32_t m0 = blockIdx.y * DOT_MR;
    const uint32_t mr = m - m0 < (uint32_t)DOT_MR ? m - m0 : (uint32_t)DOT_MR;
    float res[DOT_MR];
    if constexpr (NORM) {
        if (mr == 1 && H % 64 == 0 && H <= 64 * 32) {  // decode: one pass over the row
            res[0] = dot_row_norm(wr, x + (size_t)m0 * H, H, lane, nrm.w, nrm.eps);
        } else {  // the factors first, then the dots normalising as they read
            float rinv[DOT_MR];
#pragma unroll
            for (int r = 0; r < DOT_MR; r++)
                rinv[r] = (uint32_t)r < mr ? row_rms_inv(x + (size_t)(m0 + r) * H, H, nrm.eps, lane) : 1.0f;
            dot_rows<true>(wr, x, m0, mr, H, lane, res, rinv, nrm.w);
        }
    } else {
        dot_rows(wr, x, m0, mr, H, lane, res);
    }
    if (lane == 0)
        for (uint32_t r = 0; r < mr; r++) {
            if (wave < E)
                rlog[(size_t)(m0 + r) * E + wave] = bias ? res[r] + bias[wave] : res[r];
            else
                sh[m0 + r] = res[r];
        }
}

// gemm_f32_nt order: output (m, e) has 16 lane chains j, chain j = fma over the steps s of
// x[m][16s + j] * w[e][16s + j], then the halving tree.  Thread (j, q) of a 256-thread workgroup
// carries chain j of an RM x RE block of outputs (q = qm * QE + qe); the workgroup tile is
// (QM*RM) rows x (QE*RE) experts.  x and router chunks of KC columns are staged in LDS row-major
// (float4 global loads, 8-byte LDS stores), and lane j reads column 16s + j of each of its rows.
// Row pitches are padded so that the four 16-lane groups of a wave that read different rows fall
// on different bank halves.  The global loads of a chunk are issued two chunks before its math
// (two register stages); DB: two LDS buffers (one barrier per chunk) instead of one (two).
__host__ __device__ constexpr int gemm_pad(int d, int kc) {  // floats of padding for row distance d
    for (int p = 2; p <= 32; p += 2)
        if (d == 0 || (d * (kc + p)) % 32 == 16) return p;
    return 4;
}
// The first n_aux workgroups of the grid do the launch's other work, so that it needs no launch of
// its own: workgroups < n_dot compute the shared gate's logit (always in dot order,
// exec_batch.rs:1520), a wave per DOT_MR rows; the rest quantise x for the grouped kernels.
__device__ __forceinline__ void router_aux(const float* __restrict__ x, uint32_t m, uint32_t H,
                                           const float* __restrict__ shg, float* __restrict__ sh, const XQuant& xquant,
                                           uint32_t n_dot, uint32_t aux) {
    if (aux < n_dot) {
        const uint32_t lane = threadIdx.x % WAVE, m0 = (aux * 4 + threadIdx.x / WAVE) * DOT_MR;
        if (m0 < m) {
            const uint32_t mr = m - m0 < (uint32_t)DOT_MR ? m - m0 : (uint32_t)DOT_MR;
            float res[DOT_MR];
            dot_rows(shg, x, m0, mr, H, lane, res);
            if (lane == 0)
                for (uint32_t r = 0; r < mr; r++) sh[m0 + r] = res[r];
        }
    } else {
        quantize_x_rows(x, m, H, xquant, aux - n_dot);
    }
}
template <int RM, int RE, int QM, int KC, bool DB>
__global__ __launch_bounds__(256) void router_gemm_kernel(const float* __restrict__ router,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ x, uint32_t m, uint32_t E,
                                                         uint32_t H, float* __restrict__ rlog,
                                                         const float* __restrict__ shg, float* __restrict__ sh,
                                                         XQuant xquant, uint32_t n_dot, uint32_t n_aux) {
    constexpr int QE = 16 / QM, TM = QM * RM, TE = QE * RE;
    if (blockIdx.x < n_aux) {  // workgroup-uniform
        router_aux(x, m, H, shg, sh, xquant, n_dot, blockIdx.x);
        return;
    }
    // rows between the 16-lane groups of one wave (q = 0..3): x rows differ when qm does
    constexpr int DX = QE >= 4 ? 0 : RM * (QE == 1 ? 1 : 0) + (QE == 2 ? RM : 0);
    constexpr int DW = QE == 1 ? 0 : RE;
    constexpr int XK = KC + gemm_pad(DX, KC), WK = KC + gemm_pad(DW, KC);
    constexpr int NB = DB ? 2 : 1;
    __shared__ __align__(16) float xs[NB][TM][XK];
    __shared__ __align__(16) float wsm[NB][TE][WK];
    const uint32_t tid = threadIdx.x, j = tid % 16, q = tid / 16, qm = q / QE, qe = q % QE;
    const uint32_t tiles_e = (E + TE - 1) / TE, bx = blockIdx.x - n_aux;
    const uint32_t m0 = (bx / tiles_e) * TM, e0 = (bx % tiles_e) * TE;

    // staging: TM rows of x and TE rows of the router, KC columns each, as float4 along k
    constexpr int XV = TM * KC / 4, WV = TE * KC / 4;  // float4 per chunk
    constexpr int NV = (XV + WV + 255) / 256;
    float4 sa[NV], sb[NV];
    auto fetch = [&](uint32_t ck, float4 (&st)[NV]) {
        const uint32_t k0 = ck * KC;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint32_t v = tid + 256 * i;
            if (v < (uint32_t)XV) {
                const uint32_t r = v / (KC / 4), c4 = v % (KC / 4);
                const uint32_t row = m0 + r < m ? m0 + r : m - 1;
                st[i] = *reinterpret_cast<const float4*>(x + (size_t)row * H + k0 + 4 * c4);
            } else if (v < (uint32_t)(XV + WV)) {
                const uint32_t u = v - XV, r = u / (KC / 4), c4 = u % (KC / 4);
                const uint32_t ex = e0 + r < E ? e0 + r : E - 1;
                st[i] = *reinterpret_cast<const float4*>(router + (size_t)ex * H + k0 + 4 * c4);
            }
        }
    };
    auto store = [&](int buf, const float4 (&st)[NV]) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint32_t v = tid + 256 * i;
            float* dst = nullptr;
            if (v < (uint32_t)XV)
                dst = &xs[buf][v / (KC / 4)][4 * (v % (KC / 4))];
            else if (v < (uint32_t)(XV + WV))
                dst = &wsm[buf][(v - XV) / (KC / 4)][4 * ((v - XV) % (KC / 4))];
            if (dst) {
                reinterpret_cast<float2*>(dst)[0] = make_float2(st[i].x, st[i].y);
                reinterpret_cast<float2*>(dst)[1] = make_float2(st[i].z, st[i].w);
            }
        }
    };
    float acc[RM][RE];
#pragma unroll
    for (int a = 0; a < RM; a++)
#pragma unroll
        for (int b = 0; b < RE; b++) acc[a][b] = 0.0f;
    auto compute = [&](int buf) {
#pragma unroll 4
        for (int s4 = 0; s4 < KC / 16; s4++) {
            const uint32_t c = 16 * s4 + j;
            float xv[RM], wv[RE];
#pragma unroll
            for (int a = 0; a < RM; a++) xv[a] = xs[buf][qm * RM + a][c];
#pragma unroll
            for (int b = 0; b < RE; b++) wv[b] = wsm[buf][qe * RE + b][c];
#pragma unroll
            for (int a = 0; a < RM; a++)
#pragma unroll
                for (int b = 0; b < RE; b++) acc[a][b] = __builtin_fmaf(xv[a], wv[b], acc[a][b]);
        }
    };
    // chunk c: register stage sa (c even) / sb (c odd), filled two chunks ahead; LDS buffer c % NB
    const uint32_t nchunk = H / KC;
    fetch(0, sa);
    if (nchunk > 1) fetch(1, sb);
    store(0, sa);
    __syncthreads();
    for (uint32_t ck = 0; ck < nchunk; ck += 2) {
        if (ck + 2 < nchunk) fetch(ck + 2, sa);
        if constexpr (DB) {
            if (ck + 1 < nchunk) store(1, sb);  // the other buffer: nobody reads it now
            compute(0);
            __syncthreads();
        } else {
            compute(0);
            __syncthreads();
            if (ck + 1 < nchunk) {
                store(0, sb);
                __syncthreads();
            }
        }
        if (ck + 1 >= nchunk) break;
        if (ck + 3 < nchunk) fetch(ck + 3, sb);
        if constexpr (DB) {
            if (ck + 2 < nchunk) store(0, sa);
            compute(1);
            __syncthreads();
        } else {
            compute(0);
            __syncthreads();
            if (ck + 2 < nchunk) {
                store(0, sa);
                __syncthreads();
            }
        }
    }
    // halving trees (all lanes of the 16-lane row get each sum); lane j stores every 16th output
#pragma unroll
    for (int a = 0; a < RM; a++)
#pragma unroll
        for (int b = 0; b < RE; b++) {
            const float sum = reduce16_lanes(acc[a][b]);
            const uint32_t row = m0 + qm * RM + a, ex = e0 + qe * RE + b;
            if (((uint32_t)(a * RE + b) % 16u) == j && row < m && ex < E)
                rlog[(size_t)row * E + ex] = bias ? sum + bias[ex] : sum;
        }
}

// The same gemm_f32_nt order on the matrix cores.  v_mfma_f32_4x4x1f32 is 16 independent 4x4 outer
// products with accumulate, each element one fma rounded once (the same bits as v_fma_f32): block
// j of the instruction is chain j of a 4-token x 4-expert tile, its k = 16s + j.  Lane l = 4j + u
// gives the A value x[token u][k] and the B value w[expert u][k], and gets back acc[token v][expert
// u] of chain j, v = 0..3.  A wave holds a 16 x 16 tile as 4 x 4 such accumulators (64 VGPRs): per
// 16-wide step it reads 8 floats from LDS for 16 instructions = 4096 fmas, twice the VALU's fma
// rate with a quarter of the register tile's LDS reads per fma.  The chains are reduced at the end
// by the same halving tree (chain j ^ 8, ^ 4, ^ 2, ^ 1: lanes 32, 16, 8, 4 apart).
// Workgroup tile TM x TE = 32 x 32 (waves 2 x 2), x and router staged in LDS row-major in KC-wide
// chunks, double-buffered, the global loads two chunks ahead (as in router_gemm_kernel).
__device__ __forceinline__ float chains_sum(float v) {  // lanes 4j + u, over j: the halving tree
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);  // chains j, j ^ 8
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(b[0]) + __uint_as_float(b[1]);  // j ^ 4
    v = v + dpp_f<0x128>(v);                            // row_ror:8: j ^ 2
    v = v + dpp_f<0x124>(v);                            // row_ror:4: j +- 1, equal after the step before
    return v;
}
template <int KC, int NB>
__global__ __launch_bounds__(256) void router_mfma_kernel(const float* __restrict__ router,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ x, uint32_t m, uint32_t E,
                                                         uint32_t H, float* __restrict__ rlog,
                                                         const float* __restrict__ shg, float* __restrict__ sh,
                                                         XQuant xquant, uint32_t n_dot) {
    // row pitch 8 mod 32 words: the 4 rows x 8 columns each half-wave reads fall in 32 distinct banks
    // NB = 4: a wave holds 16 tokens x 16 experts (32 x 32 per workgroup); NB = 2: 16 x 8 (twice
    // the workgroups for the same rows, where one 32 x 32 tile per CU left a wave per SIMD)
    constexpr int TM = 32, TE = 8 * NB, XK = KC + 8;
    // tiles first, the aux workgroups after them; the tiles in XCD order (xcd_order): an XCD takes
    // a contiguous run of tiles, so the expert tiles of one token tile share its L2's copy of x
    const uint32_t tiles_e = (E + TE - 1) / TE, tiles = tiles_e * ((m + TM - 1) / TM);
    if (blockIdx.x >= tiles) {  // workgroup-uniform
        router_aux(x, m, H, shg, sh, xquant, n_dot, blockIdx.x - tiles);
        return;
    }
    uint32_t bx;
    if (!xcd_order_1d(tiles, bx)) return;
    __shared__ __align__(16) float xs[2][TM][XK];
    __shared__ __align__(16) float wsm[2][TE][XK];
    const uint32_t tid = threadIdx.x, wv = tid / WAVE, lane = tid % WAVE, j = lane / 4, u = lane % 4;
    const uint32_t wm = wv / 2, we = wv % 2;  // the wave's 16 x 16 quadrant
    const uint32_t m0 = (bx / tiles_e) * TM, e0 = (bx % tiles_e) * TE;

    constexpr int XV = TM * KC / 4, WV = TE * KC / 4;  // float4 per chunk
    constexpr int NV = (XV + WV) / 256;
    static_assert((XV + WV) % 256 == 0, "every thread stages the same number of float4");
    float4 sa[NV], sb[NV];
    auto fetch = [&](uint32_t ck, float4 (&st)[NV]) {
        const uint32_t k0 = ck * KC;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint32_t v = tid + 256 * i;
            if (v < (uint32_t)XV) {
                const uint32_t r = v / (KC / 4), c4 = v % (KC / 4);
                const uint32_t row = m0 + r < m ? m0 + r : m - 1;
                st[i] = *reinterpret_cast<const float4*>(x + (size_t)row * H + k0 + 4 * c4);
            } else {
                const uint32_t w = v - XV, r = w / (KC / 4), c4 = w % (KC / 4);
                const uint32_t ex = e0 + r < E ? e0 + r : E - 1;
                st[i] = *reinterpret_cast<const float4*>(router + (size_t)ex * H + k0 + 4 * c4);
            }
        }
    };
    auto store = [&](int buf, const float4 (&st)[NV]) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint32_t v = tid + 256 * i;
            float* dst = v < (uint32_t)XV ? &xs[buf][v / (KC / 4)][4 * (v % (KC / 4))]
                                          : &wsm[buf][(v - XV) / (KC / 4)][4 * ((v - XV) % (KC / 4))];
            reinterpret_cast<float2*>(dst)[0] = make_float2(st[i].x, st[i].y);
            reinterpret_cast<float2*>(dst)[1] = make_float2(st[i].z, st[i].w);
        }
    };
    v4f acc[4][NB];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[a][b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf) {
#pragma unroll
        for (int s = 0; s < KC / 16; s++) {
            const uint32_t c = 16 * s + j;
            float xv[4], wvv[NB];
#pragma unroll
            for (int a = 0; a < 4; a++) xv[a] = xs[buf][16 * wm + 4 * a + u][c];
#pragma unroll
            for (int b = 0; b < NB; b++) wvv[b] = wsm[buf][4 * NB * we + 4 * b + u][c];
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < NB; b++) acc[a][b] = rank1(xv[a], wvv[b], acc[a][b]);
        }
    };
    const uint32_t nchunk = H / KC;
    fetch(0, sa);
    if (nchunk > 1) fetch(1, sb);
    store(0, sa);
    __syncthreads();
    for (uint32_t ck = 0; ck < nchunk; ck += 2) {
        if (ck + 2 < nchunk) fetch(ck + 2, sa);
        if (ck + 1 < nchunk) store(1, sb);  // the other buffer: nobody reads it now
        compute(0);
        __syncthreads();
        if (ck + 1 >= nchunk) break;
        if (ck + 3 < nchunk) fetch(ck + 3, sb);
        if (ck + 2 < nchunk) store(0, sa);
        compute(1);
        __syncthreads();
    }
    // every lane ends with all 4 NB (a, b) sums; lane (j, u), j < 4 NB, stores tile (a, b) =
    // (j / NB, j % NB): tokens 4a + v, expert 4b + u
    float outv[4];
#pragma unroll
    for (int v = 0; v < 4; v++) outv[v] = 0.0f;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float t = chains_sum(acc[a][b][v]);
                outv[v] = j == (uint32_t)(NB * a + b) ? t : outv[v];
            }
    const uint32_t ex = e0 + 4 * NB * we + 4 * (j % NB) + u;
    if (j < 4 * NB && ex < E) {
        const float bb = bias ? bias[ex] : 0.0f;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const uint32_t row = m0 + 16 * wm + 4 * (j / NB) + v;
            if (row < m) rlog[(size_t)row * E + ex] = bias ? outv[v] + bb : outv[v];
        }
    }
}

// workgroup tiles of the router gemm by batch size (the first entry whose min_m <= m and whose
// chunk divides H)
struct GemmCfg {
    uint32_t min_m, kc;
    int id;
};
// (a chunk must divide H: the kernel walks H / KC whole chunks; 64- and 16-wide chunks take the
// K-split slices of a tiled router, e.g. 2560 / 8 = 320 columns)
static const GemmCfg kGemmCfg[] = {{256, 128, 1}, {64, 256, 5}, {0, 512, 2}, {0, 128, 3}, {0, 64, 6}, {0, 16, 7}};

template <int RM, int RE, int QM, int KC, bool DB>
static void launch_gemm_cfg(const float* router, const float* bias, const float* x, uint32_t m, uint32_t E,
                            uint32_t H, float* rlog, const float* shg, float* sh, const XQuant& xq,
                            uint32_t n_dot, uint32_t n_aux, hipStream_t st) {
    constexpr uint32_t TM = QM * RM, TE = (16 / QM) * RE;
    const uint32_t tiles = ((E + TE - 1) / TE) * ((m + TM - 1) / TM);
    router_gemm_kernel<RM, RE, QM, KC, DB><<<n_aux + tiles, 256, 0, st>>>(router, bias, x, m, E, H, rlog, shg, sh, xq,
                                                                         n_dot, n_aux);
}

hipError_t launch_router_logits(const float* router, const float* bias, const float* shexp_gate, const float* x,
                                uint32_t m, uint32_t E, uint32_t H, int gemm_order, float* rlog, float* sh,
                                hipStream_t st, const XQuant* xquant, const XNorm* norm) {
    const uint32_t chunks = (m + DOT_MR - 1) / DOT_MR;
    const XQuant none{};
    if (xquant && (H % 32 || (xquant->pair && m != 1))) return hipErrorInvalidValue;  // pair: one decode row
    if (norm && gemm_order) return hipErrorInvalidValue;  // rmsnorm is fused into the dot-order launch only
    if (!gemm_order) {
        const uint32_t nrow = E + (shexp_gate ? 1 : 0), wgs = (nrow + 1) / 2;
        const uint32_t qwgs = xquant ? (m * (H / 32) * 4 + 127) / 128 : 0;  // four lanes per 32-block
        const dim3 grid(wgs + qwgs, chunks);
        if (norm)
            router_dot_kernel<true><<<grid, 128, 0, st>>>(router, bias, shexp_gate, x, m, E, H, rlog, sh,
                                                          xquant ? *xquant : none, wgs, *norm);
        else
            router_dot_kernel<false><<<grid, 128, 0, st>>>(router, bias, shexp_gate, x, m, E, H, rlog, sh,
                                                           xquant ? *xquant : none, wgs, XNorm{});
    } else {
        if (H % 16) return hipErrorInvalidValue;
        int id = 3;
        for (const GemmCfg& c : kGemmCfg)
            if (m >= c.min_m && H % c.kc == 0) {
                id = c.id;
                break;
            }
        // ahead of the tiles: the shared gate's logit (a wave per DOT_MR rows) and x's quantisation
        const uint32_t n_dot = shexp_gate ? (chunks + 3) / 4 : 0u;
        const uint32_t n_aux = n_dot + (xquant ? (m * (H / 32) * 4 + 255) / 256 : 0u);
        const XQuant& xq = xquant ? *xquant : none;
        // the matrix-core gemm from 512 rows (config 4: 160 -> 91 us; M = 512: 35 -> 31 us, its 256
        // workgroups one per CU).  64-wide chunks: 32 and 128 were no faster, nor chunks stored
        // transposed so that a lane reads its four steps as one float4
        if (m >= 512 && H % 64 == 0 && m < 1024) {  // 16 x 8 per wave: two waves per SIMD at M = 512
            const uint32_t tiles = ((E + 15) / 16) * ((m + 31) / 32);
            router_mfma_kernel<64, 2><<<tiles + n_aux, 256, 0, st>>>(router, bias, x, m, E, H, rlog, shexp_gate, sh, xq,
                                                                    n_dot);
            return hipGetLastError();
        } else if (m >= 512 && H % 64 == 0) {
            const uint32_t tiles = ((E + 31) / 32) * ((m + 31) / 32);
            router_mfma_kernel<64, 4><<<tiles + n_aux, 256, 0, st>>>(router, bias, x, m, E, H, rlog, shexp_gate, sh, xq,
                                                                  n_dot);
            return hipGetLastError();
        }
        switch (id) {
#define GEMM_ARGS router, bias, x, m, E, H, rlog, shexp_gate, sh, xq, n_dot, n_aux, st
            case 1: launch_gemm_cfg<4, 4, 4, 128, true>(GEMM_ARGS); break;
            case 2: launch_gemm_cfg<1, 2, 16, 512, false>(GEMM_ARGS); break;
            case 5: launch_gemm_cfg<4, 2, 4, 256, true>(GEMM_ARGS); break;
            case 6: launch_gemm_cfg<1, 2, 16, 64, true>(GEMM_ARGS); break;
            case 7: launch_gemm_cfg<1, 2, 16, 16, true>(GEMM_ARGS); break;
            default: launch_gemm_cfg<1, 2, 16, 128, true>(GEMM_ARGS); break;
#undef GEMM_ARGS
        }
    }
    return hipGetLastError();
}

// ---- routing -----------------------------------------------------------------------------------

template <int NJ>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, uint32_t m, uint32_t E, uint32_t k,
                                                   Policy pol, uint32_t* __restrict__ ids, float* __restrict__ wout,
                                                   uint32_t* __restrict__ n_sel, unsigned long long* __restrict__ stats) {
    __shared__ uint2 cand[4][ROUTE_CAND];
    extern __shared__ float ex_all[];  // [4][E] for MassBasis::All
    const uint32_t wv = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint32_t row = blockIdx.x * 4 + wv;
    if (row >= m) return;
    const uint32_t n = route_row<NJ>(logits + (size_t)row * E, E, k, pol, lane, cand[wv], ex_all + (size_t)wv * E,
                                     ids + (size_t)row * K_MAX, wout + (size_t)row * K_MAX);
    if (lane == 0) {
        n_sel[row] = n;
        if (stats) {
            atomicAdd(&stats[0], 1ull);
            atomicAdd(&stats[1], (unsigned long long)n);
        }
    }
}

hipError_t launch_route(const float* logits, uint32_t m, uint32_t E, uint32_t k, Policy pol, uint32_t* ids,
                        float* w, uint32_t* n_sel, unsigned long long* stats, hipStream_t st) {
    const size_t lds = (pol.enabled && pol.basis == TRK_BASIS_ALL) ? (size_t)4 * E * sizeof(float) : 0;
    if (E <= 512)
        route_kernel<8><<<(m + 3) / 4, 256, lds, st>>>(logits, m, E, k, pol, ids, w, n_sel, stats);
    else
        route_kernel<16><<<(m + 3) / 4, 256, lds, st>>>(logits, m, E, k, pol, ids, w, n_sel, stats);
    return hipGetLastError();
}

// router::mass_profile (router.rs:152-166) of each logit row, added to MoeStats's fixed-point sums
// as MoeStats::profile_row does (exec.rs:582-592): prof[j] += (u64)(cum[j] * 1e6) for j < 32,
// prof[32] += 1.  One wave per row: the top-32 come from route_row's selection (the insertion
// order of topk_sorted), the denominator over all logits is summed in index order by one lane.
template <int NJ>
__global__ __launch_bounds__(256) void mass_profile_kernel(const float* __restrict__ logits, uint32_t m, uint32_t E,
                                                          unsigned long long* __restrict__ prof) {
    __shared__ uint2 cand[4][ROUTE_CAND];
    __shared__ uint32_t top_i[4][K_MAX];
    __shared__ float top_w[4][K_MAX];
    extern __shared__ float ex_all[];  // [4][E]
    const uint32_t wv = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint32_t row = blockIdx.x * 4 + wv;
    if (row >= m) return;
    const float* lg = logits + (size_t)row * E;
    const uint32_t kk = E < (uint32_t)K_MAX ? E : (uint32_t)K_MAX;
    const Policy none{0, 0, 0, 0, 0.0f};
    const uint32_t n = route_row<NJ>(lg, E, kk, none, lane, cand[wv], nullptr, top_i[wv], top_w[wv]);
    wave_sync();
    // topk_sorted's values in order; slots it leaves unfilled stay -inf (router.rs:155-158)
    const float tv = lane < n ? lg[top_i[wv][lane]] : -__builtin_inff();
    const float mx = rdl(tv, 0);
    float* ex = ex_all + (size_t)wv * E;
    for (uint32_t i = lane; i < E; i += WAVE) ex[i] = expf_libm(lg[i] - mx);
    wave_sync();
    float denom = 0.0f;
    if (lane == 0)
        for (uint32_t i = 0; i < E; i++) denom += ex[i];
    denom = rdl(denom, 0);
    const float e = lane < kk ? expf_libm(tv - mx) / denom : 0.0f;
    float mass = 0.0f, mine = 0.0f;
    for (uint32_t j = 0; j < (uint32_t)K_MAX; j++) {  // cum[j] = mass of the best j + 1
        if (j < kk) mass += rdl(e, j);
        if (lane == j) mine = mass;
    }
    if (lane < (uint32_t)K_MAX) {
        // (m as f64 * 1e6) as u64: truncation, NaN and negatives to 0, saturating
        const double d = (double)mine * 1e6;
        const unsigned long long fx =
                !(d > 0.0) ? 0ull : (d >= 18446744073709551615.0 ? ~0ull : (unsigned long long)d);
        atomicAdd(&prof[lane], fx);
    }
    if (lane == 0) atomicAdd(&prof[K_MAX], 1ull);
}

hipError_t launch_mass_profile(const float* logits, uint32_t m, uint32_t E, unsigned long long* prof, hipStream_t st) {
    const size_t lds = (size_t)4 * E * sizeof(float);
    if (E <= 512)
        mass_profile_kernel<8><<<(m + 3) / 4, 256, lds, st>>>(logits, m, E, prof);
    else
        mass_profile_kernel<16><<<(m + 3) / 4, 256, lds, st>>>(logits, m, E, prof);
    return hipGetLastError();
}

}  // namespace trk
