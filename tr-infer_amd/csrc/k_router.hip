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

// x of one row (decode) quantised per 32 by the workgroups after the logit rows: four lanes per
// block; pair = quantize_pair_blocks (quant.rs:96-108), else QAct::quantize.
__device__ __forceinline__ void quantize_x_row(const float* __restrict__ x, uint32_t H, const XQuant& xq,
                                               uint32_t qwg) {
    const uint32_t nb = H / 32, t = qwg * blockDim.x + threadIdx.x, b = t / 4, qd = t % 4;
    const uint32_t bc = b < nb ? b : nb - 1;
    const float4* src = reinterpret_cast<const float4*>(x + (size_t)bc * 32 + 8 * qd);
    const float4 a = src[0], c = src[1];
    const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
    float r[8], r2[8];
    uint32_t qw[2];
    float s;
    int32_t su;
    quant_block_quad<true>(v, qw, s, su, r);
    if (b < nb) {
        *reinterpret_cast<uint2*>(xq.q + (size_t)b * 32 + 8 * qd) = make_uint2(qw[0], qw[1]);
        if (qd == 0) {
            xq.s[b] = s;
            xq.sum[b] = su;
            xq.u[b] = s * (float)su;  // gemv.rs:144
        }
    }
    if (xq.pair) {
        quant_block_quad<false>(r, qw, s, su, r2);
        if (b < nb) {
            *reinterpret_cast<uint2*>(xq.q + (size_t)H + (size_t)b * 32 + 8 * qd) = make_uint2(qw[0], qw[1]);
            if (qd == 0) {
                xq.s[nb + b] = s;
                xq.sum[nb + b] = su;
                xq.u[nb + b] = s * (float)su;
            }
        }
    }
}

// grid.x: waves over weight rows ([0, E) router rows + bias, row E = shared gate if shg), then
// (xquant) the workgroups that quantise x; grid.y: chunks of DOT_MR activation rows.
__global__ __launch_bounds__(128) void router_dot_kernel(const float* __restrict__ router,
                                                        const float* __restrict__ bias,
                                                        const float* __restrict__ shg,
                                                        const float* __restrict__ x, uint32_t m, uint32_t E,
                                                        uint32_t H, float* __restrict__ rlog, float* __restrict__ sh,
                                                        XQuant xquant, uint32_t qwg0) {
    if (xquant.q && blockIdx.x >= qwg0) {  // workgroup-uniform
        quantize_x_row(x, H, xquant, blockIdx.x - qwg0);
        return;
    }
    const uint32_t wave = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (wave >= E + (shg ? 1u : 0u)) return;
    const float* wr = wave < E ? router + (size_t)wave * H : shg;
    const uint32_t m0 = blockIdx.y * DOT_MR;
    const uint32_t mr = m - m0 < (uint32_t)DOT_MR ? m - m0 : (uint32_t)DOT_MR;
    float res[DOT_MR];
    dot_rows(wr, x, m0, mr, H, lane, res);
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
// (QM*RM) rows x (QE*RE) experts.  x and router chunks of KC columns go through LDS transposed
// ([k][row]), double-buffered, so a thread reads its RM rows / RE experts at column 16s + j with
// vector LDS reads.
template <int RM, int RE, int QM>
__global__ __launch_bounds__(256) void router_gemm_kernel(const float* __restrict__ router,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ x, uint32_t m, uint32_t E,
                                                         uint32_t H, float* __restrict__ rlog) {
    constexpr int QE = 16 / QM, TM = QM * RM, TE = QE * RE, KC = 64;
    constexpr int XP = TM + 4, WP = TE + 4;  // padded LDS rows (keep 16-byte alignment)
    __shared__ __align__(16) float xs[2][KC][XP];
    __shared__ __align__(16) float wsm[2][KC][WP];
    const uint32_t tid = threadIdx.x, j = tid % 16, q = tid / 16, qm = q / QE, qe = q % QE;
    const uint32_t m0 = blockIdx.y * TM, e0 = blockIdx.x * TE;

    // staging: TM rows of x and TE rows of the router, KC columns each, as float4 along k
    constexpr int XV = TM * KC / 4, WV = TE * KC / 4;  // float4 per chunk
    constexpr int NV = (XV + WV + 255) / 256;
    float4 st[NV];
    auto fetch = [&](uint32_t k0) {
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
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint32_t v = tid + 256 * i;
            if (v < (uint32_t)XV) {
                const uint32_t r = v / (KC / 4), c4 = v % (KC / 4);
                xs[buf][4 * c4 + 0][r] = st[i].x;
                xs[buf][4 * c4 + 1][r] = st[i].y;
                xs[buf][4 * c4 + 2][r] = st[i].z;
                xs[buf][4 * c4 + 3][r] = st[i].w;
            } else if (v < (uint32_t)(XV + WV)) {
                const uint32_t u = v - XV, r = u / (KC / 4), c4 = u % (KC / 4);
                wsm[buf][4 * c4 + 0][r] = st[i].x;
                wsm[buf][4 * c4 + 1][r] = st[i].y;
                wsm[buf][4 * c4 + 2][r] = st[i].z;
                wsm[buf][4 * c4 + 3][r] = st[i].w;
            }
        }
    };
    float acc[RM][RE];
#pragma unroll
    for (int a = 0; a < RM; a++)
#pragma unroll
        for (int b = 0; b < RE; b++) acc[a][b] = 0.0f;
    fetch(0);
    store(0);
    __syncthreads();
    const uint32_t nchunk = H / KC;
    for (uint32_t ck = 0; ck < nchunk; ck++) {
        const int buf = ck & 1;
        if (ck + 1 < nchunk) fetch((ck + 1) * KC);
#pragma unroll
        for (int s4 = 0; s4 < KC / 16; s4++) {
            const uint32_t c = 16 * s4 + j;
            float xv[RM], wv[RE];
#pragma unroll
            for (int a = 0; a < RM; a += 4) {
                const float4 t = *reinterpret_cast<const float4*>(&xs[buf][c][qm * RM + a]);
                xv[a] = t.x; xv[a + 1] = t.y; xv[a + 2] = t.z; xv[a + 3] = t.w;
            }
#pragma unroll
            for (int b = 0; b < RE; b += 2) {
                const float2 t = *reinterpret_cast<const float2*>(&wsm[buf][c][qe * RE + b]);
                wv[b] = t.x; wv[b + 1] = t.y;
            }
#pragma unroll
            for (int a = 0; a < RM; a++)
#pragma unroll
                for (int b = 0; b < RE; b++) acc[a][b] = __builtin_fmaf(xv[a], wv[b], acc[a][b]);
        }
        if (ck + 1 < nchunk) {
            store(buf ^ 1);
            __syncthreads();
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

hipError_t launch_router_logits(const float* router, const float* bias, const float* shexp_gate, const float* x,
                                uint32_t m, uint32_t E, uint32_t H, int gemm_order, float* rlog, float* sh,
                                hipStream_t st, const XQuant* xquant) {
    const uint32_t chunks = (m + DOT_MR - 1) / DOT_MR;
    const XQuant none{};
    if (xquant && (m != 1 || gemm_order || H % 32)) return hipErrorInvalidValue;  // one decode row
    if (!gemm_order) {
        const uint32_t nrow = E + (shexp_gate ? 1 : 0), wgs = (nrow + 1) / 2;
        const uint32_t qwgs = xquant ? (H / 32 * 4 + 127) / 128 : 0;  // four lanes per 32-block
        router_dot_kernel<<<dim3(wgs + qwgs, chunks), 128, 0, st>>>(router, bias, shexp_gate, x, m, E, H, rlog, sh,
                                                                    xquant ? *xquant : none, wgs);
    } else {
        if (m >= 256)
            router_gemm_kernel<8, 8, 4><<<dim3((E + 31) / 32, (m + 31) / 32), 256, 0, st>>>(router, bias, x, m, E,
                                                                                         H, rlog);
        else if (m >= 64)
            router_gemm_kernel<4, 4, 4><<<dim3((E + 15) / 16, (m + 15) / 16), 256, 0, st>>>(router, bias, x, m, E,
                                                                                         H, rlog);
        else
            router_gemm_kernel<4, 2, 4><<<dim3((E + 7) / 8, (m + 15) / 16), 256, 0, st>>>(router, bias, x, m, E, H,
                                                                                       rlog);
        if (shexp_gate)  // the shared gate always uses dot (exec_batch.rs:1520)
            router_dot_kernel<<<dim3(1, chunks), 64, 0, st>>>(router, nullptr, shexp_gate, x, m, 0, H, rlog, sh,
                                                              none, 1);
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

}  // namespace trk
