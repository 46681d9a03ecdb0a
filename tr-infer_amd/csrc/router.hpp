// Router dot products in attn::dot order (crates/tr-kernels/src/attn.rs:329-357), shared by the
// router kernels and the fused decode layer kernel.
#pragma once

#include "common.hpp"

namespace trk {

constexpr int DOT_MR = 8;  // activation rows per pass of a router_dot wave

// One row's dot in the same order as dot_rows, on rmsnorm(x) with x unnormalised: the row's
// router weights, x and norm weights are requested together, the sumsq (row_rms_inv's order for
// H % 64 == 0) is taken from the x registers, then the normalised values feed the chain
// (H % 64 == 0, H <= 2048).
__device__ __forceinline__ float dot_row_norm(const float* __restrict__ wr, const float* __restrict__ xr, uint32_t H,
                                              uint32_t lane, const float* __restrict__ nw, float eps) {
    constexpr int U = 32;
    const uint32_t nu = H / 64;
    float a[U], b[U], c[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if ((uint32_t)u < nu) {
            a[u] = wr[64 * u + lane];
            b[u] = xr[64 * u + lane];
            c[u] = nw ? nw[64 * u + lane] : 1.0f;
        }
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < U; u++)
        if ((uint32_t)u < nu) acc = __builtin_fmaf(b[u], b[u], acc);
    const float s = reduce16_lanes(rows4_sum(acc));
    const float r = 1.0f / __builtin_sqrtf(s / (float)H + eps);
    float d = 0.0f;
#pragma unroll
    for (int u = 0; u < U; u++)
        if ((uint32_t)u < nu) d = __builtin_fmaf(a[u], nw ? (b[u] * r) * c[u] : b[u] * r, d);
    return reduce16_lanes(rows4_sum(d));
}

template <bool NORM>
__device__ __forceinline__ float xat(const float* __restrict__ x, uint32_t row, uint32_t H, uint32_t j,
                                     const float* rinv, int r, const float* __restrict__ nw) {
    const float v = x[(size_t)row * H + j];
    if constexpr (NORM) return rms_apply(v, rinv[r], nw, j);
    return v;
}

// NORM: x holds the rows before rmsnorm, and each element is normalised as it is read with the
// row's factor rinv[r] and the weights nw, giving the same floats as a normalised copy.
template <bool NORM = false>
__device__ __forceinline__ void dot_rows(const float* __restrict__ wr, const float* __restrict__ x, uint32_t m0,
                                         uint32_t mr, uint32_t H, uint32_t lane, float* res /*[DOT_MR], all lanes*/,
                                         const float* rinv = nullptr, const float* __restrict__ nw = nullptr) {
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
            if constexpr (NORM) {
#pragma unroll
                for (int u = 0; u < U; u++) b[u] = rms_apply(b[u], rinv[r], nw, i + 64 * u + lane);
            }
#pragma unroll
            for (int u = 0; u < U; u++) acc[r] = __builtin_fmaf(a[u], b[u], acc[r]);
        }
    }
    // the rest of the 64-wide steps, 8 at a time with their loads issued together (H = 2560 leaves
    // 8 steps after the 32 above); the chain order is the same step order
    constexpr int U2 = 8;
    for (; i + 64 * U2 <= H; i += 64 * U2) {
        float a[U2];
#pragma unroll
        for (int u = 0; u < U2; u++) a[u] = wr[i + 64 * u + lane];
#pragma unroll
        for (int r = 0; r < DOT_MR; r++) {
            if ((uint32_t)r >= mr) break;
            float b[U2];
#pragma unroll
            for (int u = 0; u < U2; u++) b[u] = xat<NORM>(x, m0 + r, H, i + 64 * u + lane, rinv, r, nw);
#pragma unroll
            for (int u = 0; u < U2; u++) acc[r] = __builtin_fmaf(a[u], b[u], acc[r]);
        }
    }
    for (; i + 64 <= H; i += 64) {
        const float a = wr[i + lane];
#pragma unroll
        for (int r = 0; r < DOT_MR; r++)
            if ((uint32_t)r < mr) acc[r] = __builtin_fmaf(a, xat<NORM>(x, m0 + r, H, i + lane, rinv, r, nw), acc[r]);
    }
    for (; i + 16 <= H; i += 16)
        if (lane < 16) {
            const float a = wr[i + lane];
#pragma unroll
            for (int r = 0; r < DOT_MR; r++)
                if ((uint32_t)r < mr)
                    acc[r] = __builtin_fmaf(a, xat<NORM>(x, m0 + r, H, i + lane, rinv, r, nw), acc[r]);
        }
#pragma unroll
    for (int r = 0; r < DOT_MR; r++) {
        if ((uint32_t)r >= mr) break;
        res[r] = reduce16_lanes(rows4_sum(acc[r]));  // H % 16 == 0: no scalar tail
    }
}

}  // namespace trk
