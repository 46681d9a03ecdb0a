// Router logits and routing.
//
//   router_dot:   attn::dot order (attn.rs:329-357), one wave per weight row: lane L = 16c + j is
//                 lane j of accumulator chain c, so the wave holds exactly the reference's four
//                 16-lane FMA chains (64-wide steps), the 16-wide tail goes to chain 0, then
//                 (c0 + c1) + (c2 + c3) lanewise and the halving tree of _mm512_reduce_add_ps.
//   router_gemm:  smallgemm::gemm_f32_nt order (smallgemm.rs:8-59): per output, 16 lane chains
//                 over 16-wide steps, then the halving tree.
//   route:        one wave per token runs route_row (route.hpp).  The decode path (M = 1) routes
//                 inside its gate/up kernel instead (k_decode.hip).
#include "route.hpp"

namespace trk {

constexpr int DOT_MR = 8;  // activation rows per pass of a router_dot wave

// ---- router logits ---------------------------------------------------------------------------

__device__ __forceinline__ void dot_rows(const float* __restrict__ wr, const float* __restrict__ x, uint32_t m0,
                                         uint32_t mr, uint32_t H, uint32_t lane, float* res /*[DOT_MR], all lanes*/) {
    float acc[DOT_MR];
#pragma unroll
    for (int r = 0; r < DOT_MR; r++) acc[r] = 0.0f;
    constexpr int U = 32;  // 64-wide steps whose loads are issued together (all of H = 2048)
    uint32_t i = 0;
    for (; i + 64 * U <= H; i += 64 * U) {
        float a[U];
#pragma unroll
        for (int u = 0; u < U; u++) a[u] = wr[i + 64 * u + lane];
#pragma unroll
        for (int r = 0; r < DOT_MR; r++) {
            if ((uint32_t)r >= mr) break;
            float b[U];
            const float* xr = x + (size_t)(m0 + r) * H + i + lane;
#pragma unroll
            for (int u = 0; u < U; u++) b[u] = xr[64 * u];
#pragma unroll
            for (int u = 0; u < U; u++) acc[r] = __builtin_fmaf(a[u], b[u], acc[r]);
        }
    }
    for (; i + 64 <= H; i += 64) {
        const float a = wr[i + lane];
#pragma unroll
        for (int r = 0; r < DOT_MR; r++)
            if ((uint32_t)r < mr) acc[r] = __builtin_fmaf(a, x[(size_t)(m0 + r) * H + i + lane], acc[r]);
    }
    for (; i + 16 <= H; i += 16)
        if (lane < 16) {
            const float a = wr[i + lane];
#pragma unroll
            for (int r = 0; r < DOT_MR; r++)
                if ((uint32_t)r < mr) acc[r] = __builtin_fmaf(a, x[(size_t)(m0 + r) * H + i + lane], acc[r]);
        }
#pragma unroll
    for (int r = 0; r < DOT_MR; r++) {
        if ((uint32_t)r >= mr) break;
        res[r] = reduce16_lanes(rows4_sum(acc[r]));  // H % 16 == 0: no scalar tail
    }
}

// grid.x: waves over weight rows ([0, E) router rows + bias, row E = shared gate if shg);
// grid.y: chunks of DOT_MR activation rows.
__global__ __launch_bounds__(128) void router_dot_kernel(const float* __restrict__ router,
                                                        const float* __restrict__ bias,
                                                        const float* __restrict__ shg,
                                                        const float* __restrict__ x, uint32_t m, uint32_t E,
                                                        uint32_t H, float* __restrict__ rlog, float* __restrict__ sh) {
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

// Each 16-lane group plays the 16 lanes of one AVX-512 register; each thread carries 4 rows x 4
// experts of the 16 x 16 output tile.
__global__ __launch_bounds__(256) void router_gemm_kernel(const float* __restrict__ router,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ x, uint32_t m, uint32_t E,
                                                         uint32_t H, float* __restrict__ rlog) {
    const uint32_t l = threadIdx.x & 15, g = threadIdx.x >> 4;
    const uint32_t rg = g >> 2, eg = g & 3;
    const uint32_t row0 = blockIdx.y * 16 + rg * 4, e0 = blockIdx.x * 16 + eg * 4;
    const float* xr[4];
    const float* wr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) xr[r] = x + (size_t)(row0 + r < m ? row0 + r : m - 1) * H + l;
#pragma unroll
    for (int e = 0; e < 4; e++) wr[e] = router + (size_t)(e0 + e < E ? e0 + e : E - 1) * H + l;
    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[r][e] = 0.0f;
    for (uint32_t kk = 0; kk < H; kk += 16) {
        float xv[4], wv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) xv[r] = xr[r][kk];
#pragma unroll
        for (int e = 0; e < 4; e++) wv[e] = wr[e][kk];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[r][e] = __builtin_fmaf(xv[r], wv[e], acc[r][e]);
    }
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float s = reduce16_lanes(acc[r][e]);
            if (l == (uint32_t)(r * 4 + e) && row0 + r < m && e0 + e < E)
                rlog[(size_t)(row0 + r) * E + e0 + e] = bias ? s + bias[e0 + e] : s;
        }
}

hipError_t launch_router_logits(const float* router, const float* bias, const float* shexp_gate, const float* x,
                                uint32_t m, uint32_t E, uint32_t H, int gemm_order, float* rlog, float* sh,
                                hipStream_t st) {
    const uint32_t chunks = (m + DOT_MR - 1) / DOT_MR;
    if (!gemm_order) {
        const uint32_t nrow = E + (shexp_gate ? 1 : 0);
        router_dot_kernel<<<dim3((nrow + 1) / 2, chunks), 128, 0, st>>>(router, bias, shexp_gate, x, m, E, H, rlog, sh);
    } else {
        router_gemm_kernel<<<dim3((E + 15) / 16, (m + 15) / 16), 256, 0, st>>>(router, bias, x, m, E, H, rlog);
        if (shexp_gate)  // the shared gate always uses dot (exec_batch.rs:1520)
            router_dot_kernel<<<dim3(1, chunks), 64, 0, st>>>(router, nullptr, shexp_gate, x, m, 0, H, rlog, sh);
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
