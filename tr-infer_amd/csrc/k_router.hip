// Router logits and routing.
//
//   router_dot:   attn::dot order (attn.rs:329-357), one wave per weight row: lane L = 16c + j is
//                 lane j of accumulator chain c, so the wave holds exactly the reference's four
//                 16-lane FMA chains (64-wide steps), the 16-wide tail goes to chain 0, then
//                 (c0 + c1) + (c2 + c3) lanewise and the halving tree of _mm512_reduce_add_ps.
//   router_gemm:  smallgemm::gemm_f32_nt order (smallgemm.rs:8-59): per output, 16 lane chains
//                 over 16-wide steps, then the halving tree.
//   route_row:    route_topk / route_mass (router.rs:70-148) for one token on one wave: lanes
//                 sort their logits, then k rounds of a DPP wave arg-max over the lane heads.
//   router_route: the decode path's logits and routing in one launch — the last workgroup to
//                 finish its logits (device-scope counter) routes.
#include "common.hpp"

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
        const float c1 = __shfl(acc[r], (lane + 16) & 63);
        const float c2 = __shfl(acc[r], (lane + 32) & 63);
        const float c3 = __shfl(acc[r], (lane + 48) & 63);
        res[r] = reduce16_lanes((acc[r] + c1) + (c2 + c3));  // H % 16 == 0: no scalar tail
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

constexpr int ROUTE_NJ = 16;  // E <= 1024: 16 logits per lane

// order-preserving key of a logit (-0 and +0 share one key, as they compare equal); 0 for values
// that never enter the top-k (nan, -inf: router.rs:75-76)
__device__ __forceinline__ uint32_t fkey(float v) {
    if (!(v > -__builtin_inff())) return 0u;
    const uint32_t u = __float_as_uint(v + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ float rdl(float v, uint32_t l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)l));
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One token on one (whole) wave.  Writes the first `count` ids / weights and returns count.
// Each lane sorts its NJ logits (value desc, index asc); then k rounds of a wave-wide arg-max over
// the lanes' heads — exactly the order of the reference's insertion sort (router.rs:70-89).
// `ex` (E floats of LDS) is used only for MassBasis::All.
template <int NJ>
__device__ uint32_t route_row(const float* __restrict__ lg, uint32_t E, uint32_t k, const Policy& pol, uint32_t lane,
                              float* ex, uint32_t* __restrict__ ids_out, float* __restrict__ w_out) {
    uint32_t key[NJ], jj[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t i = lane + 64u * j;
        key[j] = i < E ? fkey(lg[i]) : 0u;
        jj[j] = (uint32_t)j;
    }
    // odd-even transposition sort, descending key; equal keys keep ascending j (stable)
#pragma unroll
    for (int pass = 0; pass < NJ; pass++)
#pragma unroll
        for (int j = pass & 1; j + 1 < NJ; j += 2)
            if (key[j + 1] > key[j]) {
                const uint32_t tk = key[j], tj = jj[j];
                key[j] = key[j + 1];
                jj[j] = jj[j + 1];
                key[j + 1] = tk;
                jj[j + 1] = tj;
            }
    const uint32_t kk = pol.enabled ? pol.max : k;
    uint32_t my_key = 0, my_idx = 0xffffffffu, ksel = 0;
    for (uint32_t rd = 0; rd < kk; rd++) {
        const uint32_t wmax = wave_max_u32(key[0]);
        if (wmax == 0u) break;  // no selectable logit left
        const uint32_t widx = wave_min_u32(key[0] == wmax ? lane + 64u * jj[0] : 0xffffffffu);
        if (lane == widx % 64u) {  // pop this lane's head
#pragma unroll
            for (int j = 0; j + 1 < NJ; j++) {
                key[j] = key[j + 1];
                jj[j] = jj[j + 1];
            }
            key[NJ - 1] = 0u;
        }
        if (lane == rd) {
            my_key = wmax;
            my_idx = widx;
        }
        ksel = rd + 1;
    }
    if (ksel == 0) return 0;  // nothing selectable (the reference would index u32::MAX)
    const float my_tv = lane < ksel ? fkey_inv(my_key) : -__builtin_inff();
    const float mx = rdl(my_tv, 0);
    const float e = lane < kk ? expf_libm(my_tv - mx) : 0.0f;  // slots past ksel: exp(-inf) = 0
    uint32_t count = kk;
    if (pol.enabled) {  // route_mass (router.rs:118-148)
        float denom = 0.0f;
        if (pol.basis == TRK_BASIS_ALL) {
            for (uint32_t i = lane; i < E; i += 64u) ex[i] = expf_libm(lg[i] - mx);
            wave_sync();
            if (lane == 0)
                for (uint32_t i = 0; i < E; i++) denom += ex[i];
            denom = rdl(denom, 0);
        } else {
            for (uint32_t j = 0; j < kk; j++) denom += rdl(e, j);
        }
        float mass = 0.0f;
        count = 0;
        while (count < kk) {
            mass += rdl(e, count) / denom;
            count++;
            if (count >= pol.min && mass >= pol.mass) break;
        }
    }
    if (count > ksel) count = ksel;
    float sum = 0.0f;  // renorm (router.rs:93-104)
    for (uint32_t j = 0; j < count; j++) sum += rdl(e, j);
    if (lane < count) {
        ids_out[lane] = my_idx;
        w_out[lane] = e / sum;
    }
    return count;
}

template <int NJ>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, uint32_t m, uint32_t E, uint32_t k,
                                                   Policy pol, uint32_t* __restrict__ ids, float* __restrict__ wout,
                                                   uint32_t* __restrict__ n_sel, unsigned long long* __restrict__ stats) {
    extern __shared__ float ex_all[];  // [4][E] for MassBasis::All
    const uint32_t wv = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint32_t row = blockIdx.x * 4 + wv;
    if (row >= m) return;
    const uint32_t n = route_row<NJ>(logits + (size_t)row * E, E, k, pol, lane, ex_all + (size_t)wv * E,
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
        route_kernel<ROUTE_NJ><<<(m + 3) / 4, 256, lds, st>>>(logits, m, E, k, pol, ids, w, n_sel, stats);
    return hipGetLastError();
}

// ---- decode: logits + routing in one launch ------------------------------------------------------

// Two waves per workgroup compute router rows (dot order) for all m <= ROUTER_ROUTE_MAX_M rows;
// the workgroup that finishes last (device-scope counter; its fence makes every workgroup's
// logits visible) routes every row and re-arms the counter for the next launch.
template <int NJ>
__global__ __launch_bounds__(128) void router_route_kernel(const float* __restrict__ router,
                                                          const float* __restrict__ bias,
                                                          const float* __restrict__ shg,
                                                          const float* __restrict__ x, uint32_t m, uint32_t E,
                                                          uint32_t H, float* __restrict__ rlog, float* __restrict__ sh,
                                                          uint32_t k, Policy pol, uint32_t* __restrict__ ids,
                                                          float* __restrict__ wout, uint32_t* __restrict__ n_sel,
                                                          unsigned long long* __restrict__ stats,
                                                          uint32_t* __restrict__ counter) {
    __shared__ uint32_t last;
    extern __shared__ float ex_all[];  // [2][E] for MassBasis::All
    const uint32_t wv = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const uint32_t wave = blockIdx.x * 2 + wv;
    if (wave < E + 1) {
        const float* wr = wave < E ? router + (size_t)wave * H : shg;
        for (uint32_t m0 = 0; m0 < m; m0 += DOT_MR) {
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
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(counter, 1u) == gridDim.x - 1 ? 1u : 0u;
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (uint32_t row = wv; row < m; row += 2) {
        const uint32_t n = route_row<NJ>(rlog + (size_t)row * E, E, k, pol, lane, ex_all + (size_t)wv * E,
                                         ids + (size_t)row * K_MAX, wout + (size_t)row * K_MAX);
        if (lane == 0) {
            n_sel[row] = n;
            if (stats) {
                atomicAdd(&stats[0], 1ull);
                atomicAdd(&stats[1], (unsigned long long)n);
            }
        }
    }
    if (threadIdx.x == 0) *counter = 0u;
}

hipError_t launch_router_route(const float* router, const float* bias, const float* shexp_gate, const float* x,
                               uint32_t m, uint32_t E, uint32_t H, float* rlog, float* sh, uint32_t k, Policy pol,
                               uint32_t* ids, float* w, uint32_t* n_sel, unsigned long long* stats, uint32_t* counter,
                               hipStream_t st) {
    const size_t lds = (pol.enabled && pol.basis == TRK_BASIS_ALL) ? (size_t)2 * E * sizeof(float) : 0;
    if (E <= 512)
        router_route_kernel<8><<<(E + 2) / 2, 128, lds, st>>>(router, bias, shexp_gate, x, m, E, H, rlog, sh, k, pol,
                                                              ids, w, n_sel, stats, counter);
    else
        router_route_kernel<ROUTE_NJ><<<(E + 2) / 2, 128, lds, st>>>(router, bias, shexp_gate, x, m, E, H, rlog, sh, k,
                                                                     pol, ids, w, n_sel, stats, counter);
    return hipGetLastError();
}

}  // namespace trk
