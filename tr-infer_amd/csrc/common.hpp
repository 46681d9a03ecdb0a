// Device-side building blocks shared by the MoE kernels (gfx950, wave64).
//
// Arithmetic follows the reference's CPU path bit for bit: products and sums round on their own
// (the library is built with -ffp-contract=off), and every FMA of the reference is an explicit
// __builtin_fmaf here.  Citations are to tokenring-ai/tr-infer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "trmoe_internal.h"

namespace trk {

constexpr int WAVE = 64;

// ---- half precision ------------------------------------------------------------------------
// f16 bits -> f32 (exact) and f32 -> f16 with round-to-nearest-even (v_cvt_f16_f32).
__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, h);
    return (float)v;
}
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float f16_round(float f) { return (float)(_Float16)f; }

__device__ __forceinline__ uint16_t ld16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// ---- x86 min/max semantics (maxps(a, b) = a > b ? a : b) --------------------------------------
__device__ __forceinline__ float mx_ps(float a, float b) { return a > b ? a : b; }
__device__ __forceinline__ float mn_ps(float a, float b) { return a < b ? a : b; }

// ---- exp / sigmoid / SiLU ------------------------------------------------------------------
// elem.rs:7-25: clamped degree-6 polynomial exp with a two-part ln2 (tr-infer's own constants).
__device__ __forceinline__ float exp512(float x) {
    x = mn_ps(mx_ps(x, -87.3f), 88.3f);
    float fx = __builtin_rintf(x * 1.442695041f);
    float r = __builtin_fmaf(-fx, 0.693145752f, x);
    r = __builtin_fmaf(-fx, 1.42860677e-6f, r);
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    float r2 = r * r;
    p = __builtin_fmaf(p, r2, r);
    p = p + 1.0f;
    return __builtin_ldexpf(p, (int)fx);
}
// elem.rs:27-38
__device__ __forceinline__ float sigmoid512(float x) { return 1.0f / (1.0f + exp512(0.0f - x)); }
__device__ __forceinline__ float silu512(float x) { return x * sigmoid512(x); }

// Rust f32::exp (libm expf): evaluated in double and rounded once to f32.  This is the correctly
// rounded value except in rare near-tie cases, where libm's expf may land one ulp away.
__device__ __forceinline__ float expf_libm(float x) { return (float)::exp((double)x); }
// elem.rs:57-59
__device__ __forceinline__ float sigmoid_libm(float x) { return 1.0f / (1.0f + expf_libm(-x)); }

// ---- activation quantisation (quant.rs:112-166) --------------------------------------------
__device__ __forceinline__ int32_t cvt_rne(float v) { return (int32_t)__builtin_rintf(v); }
__device__ __forceinline__ int8_t sat_i8(int32_t v) { return (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v)); }

// Quantise N (16 or 32) values in registers; q comes back packed 4 per word (little-endian bytes);
// optionally produce the fnmadd residual.
template <int N, bool RESID = false>
__device__ __forceinline__ void quant_block_regs(const float* x, uint32_t* qw, float& scale, int32_t& sum,
                                                 float* resid = nullptr) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < N; i++) amax = mx_ps(amax, __builtin_fabsf(x[i]));
    const float s = amax / 127.0f;
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    int32_t su = 0;
#pragma unroll
    for (int w = 0; w < N / 4; w++) {
        uint32_t packed = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int i = 4 * w + b;
            const int32_t qi = cvt_rne(x[i] * inv);
            su += qi;
            packed |= (uint32_t)(uint8_t)sat_i8(qi) << (8 * b);
            if (RESID) resid[i] = __builtin_fmaf(-(float)qi, s, x[i]);
        }
        qw[w] = packed;
    }
    scale = s;
    sum = su;
}

// ---- _mm512_reduce_add_ps halving tree over 16 lanes ------------------------------------------
__device__ __forceinline__ float reduce16(const float* v) {
    float a[8], b[4], c[2];
#pragma unroll
    for (int i = 0; i < 8; i++) a[i] = v[i] + v[i + 8];
#pragma unroll
    for (int i = 0; i < 4; i++) b[i] = a[i] + a[i + 4];
#pragma unroll
    for (int i = 0; i < 2; i++) c[i] = b[i] + b[i + 2];
    return c[0] + c[1];
}

// Cross-lane version for a value held by lanes j of a 16-lane row (lane j holds element j):
// returns the tree sum in every lane of the row.  The partners come from DPP row rotations by 8,
// 4, 2, 1: after the step with distance d every lane's value equals that of lane j ^ d', d' >= d,
// so the rotation partner holds the same value as the xor partner and lane 0 computes exactly
// a[0] = v0 + v8, b[0] = a0 + a4, c[0] = b0 + b2, c0 + c1 (other lanes: the same sums commuted).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float reduce16_lanes(float v) {
    v = v + dpp_f<0x128>(v);  // row_ror:8
    v = v + dpp_f<0x124>(v);  // row_ror:4
    v = v + dpp_f<0x122>(v);  // row_ror:2
    v = v + dpp_f<0x121>(v);  // row_ror:1
    return v;
}

// (row0 + row1) + (row2 + row3) of a wave, lanewise (lane j of every row gets the sum over
// lanes j, j+16, j+32, j+48 in that bracketing): permlane16_swap pairs rows 0/1 and 2/3,
// permlane32_swap the two halves.  Both swaps are symmetric, so the sum of their two results
// does not depend on which of the pair carries which half.
__device__ __forceinline__ float rows4_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 1 / sqrt(mean(x^2) + eps) of one row of n floats, in every lane of the wave (elem.rs:255-262):
// sumsq (elem.rs:224-252) in the dot order, lane j carrying the chain over elements j + 64 i, the
// 16-wide tail on lanes 0-15, the scalar tail after the reduction.
__device__ __forceinline__ float row_rms_inv(const float* __restrict__ xr, uint32_t n, float eps, uint32_t lane) {
    float acc = 0.0f;
    uint32_t i = 0;
    constexpr int U = 16;  // 64-wide steps whose loads are issued together
    for (; i + 64 * U <= n; i += 64 * U) {
        float a[U];
#pragma unroll
        for (int u = 0; u < U; u++) a[u] = xr[i + 64 * u + lane];
#pragma unroll
        for (int u = 0; u < U; u++) acc = __builtin_fmaf(a[u], a[u], acc);
    }
    for (; i + 64 <= n; i += 64) {
        float a = xr[i + lane];
        acc = __builtin_fmaf(a, a, acc);
    }
    for (; i + 16 <= n; i += 16)
        if (lane < 16) {
            float a = xr[i + lane];
            acc = __builtin_fmaf(a, a, acc);
        }
    float s = reduce16_lanes(rows4_sum(acc));  // the same value in every lane
    for (; i < n; i++) s += xr[i] * xr[i];
    return 1.0f / __builtin_sqrtf(s / (float)n + eps);
}
// one element of rmsnorm's output: (x * r) * w, or x * r without weights (elem.rs:259-261)
__device__ __forceinline__ float rms_apply(float x, float r, const float* __restrict__ w, uint32_t j) {
    return w ? (x * r) * w[j] : x * r;
}

// ---- Q4_K / Q6_K superblock decoding ------------------------------------------------------------
// blocks.py:16-22 (_scale_min_k)
__device__ __forceinline__ void q4k_scale_min(const uint8_t* s, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[4 + j] & 63;
    } else {
        sc = (s[8 + j - 4] & 15) | ((s[j - 4] >> 6) << 4);
        mn = (s[8 + j - 4] >> 4) | ((s[4 + j - 4] >> 6) << 4);
    }
}

// The same from the header words of a superblock held in registers: bytes 4..15 of the header
// are words w1, w2, w3 (little-endian); j must be a compile-time constant after unrolling.
__device__ __forceinline__ void q4k_scale_min_w(uint32_t w1, uint32_t w2, uint32_t w3, int j, int& sc, int& mn) {
    auto byte = [&](int i) -> int {
        const uint32_t w = i < 4 ? w1 : (i < 8 ? w2 : w3);
        return (int)((w >> (8 * (i & 3))) & 0xffu);
    };
    if (j < 4) {
        sc = byte(j) & 63;
        mn = byte(4 + j) & 63;
    } else {
        sc = (byte(8 + j - 4) & 15) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(8 + j - 4) >> 4) | ((byte(4 + j - 4) >> 6) << 4);
    }
}

// blocks.py:35-36: dd = f16(d*sc), mm = f16(-(dmin*mn)), then widened back to f32 (gemv.rs:104-105)
__device__ __forceinline__ void q4k_dm(float d, float dmin, int sc, int mn, float& dd, float& mm) {
    dd = f16_round(d * (float)sc);
    mm = f16_round(-(dmin * (float)mn));
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// ---- rank-1 f32 terms on the matrix cores ---------------------------------------------------------
// v_mfma_f32_4x4x1f32 (16 blocks of 4x4x1): lane l = 16g + r returns, for v = 0..3,
//   c[v] + a_{16g + 4(r / 4) + v} * b_l
// with one rounding: v_fma_f32's result bit for bit, and with c = -0 the rounded product,
// v_mul_f32's result, signed zeros included (checked on gfx950 over random bit patterns,
// denormals and infinities).  With a_l taken from token 4g + (l % 4) and b_l from output r this is
// the per-block fma(m, u, acc) / d * sx of the MFMA epilogues, in the layout of a 16x16 MFMA's
// output (lane (g, r) holds rows 4g .. 4g + 3 of column r).
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4f rank1(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f neg_zero4() { return v4f{-0.0f, -0.0f, -0.0f, -0.0f}; }

// Device-coherent word access for data exchanged between workgroups inside one launch:
// agent-scope atomic loads and stores go to memory directly, past the per-XCD L2, so neither
// side needs a whole-cache write-back or invalidate.
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_dev(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_devf(const float* p) {
    return __uint_as_float(ld_dev(reinterpret_cast<const uint32_t*>(p)));
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_devf(float* p, float v) { st_dev(reinterpret_cast<uint32_t*>(p), __float_as_uint(v)); }

// LDS writes of this wave visible to its own later reads (no workgroup barrier)
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- wave-wide reductions with DPP (row shifts, then row broadcasts 15 / 31) ----------------------
// The result of the running scan sits in lane 63; it is returned in every lane (readlane).
template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v) {
    auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    // lanes without a source keep their own value (old = v), the identity of max / min
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x113, 0xf, 0xf, false));  // row_shr:3
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x114, 0xf, 0xe, false));  // row_shr:4
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x118, 0xf, 0xc, false));  // row_shr:8
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return wave_reduce_u32<true>(v); }

// Inclusive prefix sum over the 64 lanes (Kogge-Stone within each row of 16, then the row
// broadcasts 15 / 31); lanes without a source add 0.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

// All-reduce within each 16-lane row with DPP: quad_perm [1,0,3,2], quad_perm [2,3,0,1], half-row
// mirror, row mirror.  The pairing differs from an xor butterfly, so it is only for operations
// whose result does not depend on the order (max of non-NaN values, integer sums).
template <typename T, typename Op>
__device__ __forceinline__ T row16_allreduce(T v, Op op) {
    static_assert(sizeof(T) == 4, "32-bit values");
    auto mv = [](T x, auto ctrl) -> T {
        return __builtin_bit_cast(T, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), decltype(ctrl)::value, 0xf,
                                                              0xf, false));
    };
    v = op(v, mv(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
    v = op(v, mv(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
    v = op(v, mv(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
    v = op(v, mv(v, std::integral_constant<int, 0x140>{}));  // row_mirror
    return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return wave_reduce_u32<false>(v); }

// Token (activation row) of entry row `row` of a grouped work item; rows past the item reuse its
// first row (their outputs are never stored).
// XCD-aware order of a grouped launch's (column block, item) workgroups.  The dispatcher deals
// workgroup ids round robin to the 8 XCDs (id % 8), each with its own L2.  Here XCD x takes a
// contiguous run of the live ids [0, gridDim.x * n_items) in dispatch order, so the consecutive
// items of one expert (each re-reads that expert's weights) run on one XCD close in time and
// share its L2.  A bijection on the live ids; false for the ids past them.
// reverse: each XCD walks its run from the end (the last items first).
__device__ __forceinline__ bool xcd_order(uint32_t n_items, uint32_t& col, uint32_t& itn, bool reverse = false) {
    const uint32_t gx = gridDim.x, id = blockIdx.x + gx * blockIdx.y, T = gx * n_items;
    if (id >= T) return false;
    const uint32_t x = id % 8, slot = id / 8, base = T / 8, rem = T % 8;
    const uint32_t cnt = base + (x < rem ? 1u : 0u);  // ids of this XCD: slot < cnt
    const uint32_t nid = x * base + (x < rem ? x : rem) + (reverse ? cnt - 1 - slot : slot);
    col = nid % gx;
    itn = nid / gx;
    return true;
}

// The same for a 1-D grid whose first n workgroups are live: id -> its place in XCD order.
__device__ __forceinline__ bool xcd_order_1d(uint32_t n, uint32_t& idx) {
    const uint32_t id = blockIdx.x;
    if (id >= n) return false;
    const uint32_t x = id % 8, slot = id / 8, base = n / 8, rem = n % 8;
    idx = x * base + (x < rem ? x : rem) + slot;
    return true;
}

__device__ __forceinline__ uint32_t item_token(const Workspace& ws, const Item& it, bool shared, uint32_t row) {
    const uint32_t r = row < it.nrows ? row : 0u;
    return shared ? it.row0 + r : ws.ent_tok[it.row0 + r];
}

}  // namespace trk
