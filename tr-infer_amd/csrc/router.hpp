// Router dot products in attn::dot order (crates/tr-kernels/src/attn.rs:329-357), shared by the
// router kernels and the fused decode layer kernel.
#pragma once

#include "common.hpp"

namespace trk {

constexpr int DOT_MR = 8;  // activation rows per pass of a router_dot wave

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

}  // namespace trk
