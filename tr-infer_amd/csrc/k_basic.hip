// Activation quantisation, the kernel-level GEMV mirror, elementwise kernels and the
// synthetic-data generators.
#include "common.hpp"

namespace trk {

// ============================================================================================
// activation quantisation (quant.rs:36-53, 96-166)
// ============================================================================================

template <int KB>
__global__ void quantize_rows_kernel(const float* __restrict__ x, uint32_t m, uint32_t k, int8_t* __restrict__ q,
                                     float* __restrict__ s, int32_t* __restrict__ su, float* __restrict__ u) {
    uint32_t nb = k / KB;
    uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= m * nb) return;
    uint32_t r = idx / nb, b = idx % nb;
    const float* src = x + (size_t)r * k + (size_t)b * KB;
    float v[KB];
#pragma unroll
    for (int i = 0; i < KB; i += 4) {
        float4 t = *reinterpret_cast<const float4*>(src + i);
        v[i] = t.x; v[i + 1] = t.y; v[i + 2] = t.z; v[i + 3] = t.w;
    }
    uint32_t qq[KB / 4];
    float sc;
    int32_t sm;
    quant_block_regs<KB>(v, qq, sc, sm);
    uint4* dst = reinterpret_cast<uint4*>(q + (size_t)r * k + (size_t)b * KB);
#pragma unroll
    for (int i = 0; i < KB / 16; i++) dst[i] = make_uint4(qq[4 * i], qq[4 * i + 1], qq[4 * i + 2], qq[4 * i + 3]);
    s[idx] = sc;
    su[idx] = sm;
    if (u) u[idx] = sc * (float)sm;  // gemv.rs:144
}

// quantize_pair_blocks (quant.rs:96-108): row 0 = coarse, row 1 = quantised fnmadd residual
template <int KB>
__global__ void quantize_pair_kernel(const float* __restrict__ x, uint32_t k, int8_t* __restrict__ q,
                                     float* __restrict__ s, int32_t* __restrict__ su) {
    uint32_t nb = k / KB;
    uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nb) return;
    const float* src = x + (size_t)b * KB;
    float v[KB], r[KB];
#pragma unroll
    for (int i = 0; i < KB; i += 4) {
        float4 t = *reinterpret_cast<const float4*>(src + i);
        v[i] = t.x; v[i + 1] = t.y; v[i + 2] = t.z; v[i + 3] = t.w;
    }
    uint32_t q0[KB / 4], q1[KB / 4];
    float s0, s1;
    int32_t m0, m1;
    quant_block_regs<KB, true>(v, q0, s0, m0, r);
    quant_block_regs<KB>(r, q1, s1, m1);
    uint4* d0 = reinterpret_cast<uint4*>(q + (size_t)b * KB);
    uint4* d1 = reinterpret_cast<uint4*>(q + (size_t)k + (size_t)b * KB);
#pragma unroll
    for (int i = 0; i < KB / 16; i++) {
        d0[i] = make_uint4(q0[4 * i], q0[4 * i + 1], q0[4 * i + 2], q0[4 * i + 3]);
        d1[i] = make_uint4(q1[4 * i], q1[4 * i + 1], q1[4 * i + 2], q1[4 * i + 3]);
    }
    s[b] = s0;
    su[b] = m0;
    s[nb + b] = s1;
    su[nb + b] = m1;
}

hipError_t launch_quantize(const float* x, uint32_t m, uint32_t k, uint32_t kb, int pair, int8_t* q, float* s,
                           int32_t* su, float* u, hipStream_t st) {
    uint32_t nb = k / kb;
    if (pair) {
        dim3 g((nb + 63) / 64);
        if (kb == 32)
            quantize_pair_kernel<32><<<g, 64, 0, st>>>(x, k, q, s, su);
        else
            quantize_pair_kernel<16><<<g, 64, 0, st>>>(x, k, q, s, su);
    } else {
        dim3 g((m * nb + 255) / 256);
        if (kb == 32)
            quantize_rows_kernel<32><<<g, 256, 0, st>>>(x, m, k, q, s, su, u);
        else
            quantize_rows_kernel<16><<<g, 256, 0, st>>>(x, m, k, q, s, su, u);
    }
    return hipGetLastError();
}

// ============================================================================================
// elementwise (elem.rs)
// ============================================================================================

// swiglu_vec via zip16 (elem.rs:173-175, 209-221): silu512 on full 16-blocks, scalar silu on the
// tail.
__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ y,
                              size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    size_t body = n / 16 * 16;
    float gv = g[i];
    y[i] = (i < body ? silu512(gv) : gv * sigmoid_libm(gv)) * u[i];
}

hipError_t launch_swiglu(const float* g, const float* u, float* y, size_t n, hipStream_t st) {
    swiglu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(g, u, y, n);
    return hipGetLastError();
}

// rmsnorm (elem.rs:255-262) with sumsq (elem.rs:224-252) in the dot order: one wave per row.
__global__ void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w, float eps, uint32_t m,
                               uint32_t n, float* __restrict__ y) {
    uint32_t row = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    uint32_t lane = threadIdx.x % WAVE;
    if (row >= m) return;
    const float* xr = x + (size_t)row * n;
    const float r = row_rms_inv(xr, n, eps, lane);
    constexpr int U = 16;
    uint32_t j = lane;
    for (; j + WAVE * (U - 1) < n; j += WAVE * U) {  // loads first, U per lane
        float a[U], b[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            a[u] = xr[j + WAVE * u];
            b[u] = w ? w[j + WAVE * u] : 1.0f;
        }
#pragma unroll
        for (int u = 0; u < U; u++) y[(size_t)row * n + j + WAVE * u] = w ? (a[u] * r) * b[u] : a[u] * r;
    }
    for (; j < n; j += WAVE) y[(size_t)row * n + j] = w ? (xr[j] * r) * w[j] : xr[j] * r;
}

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, uint32_t m, uint32_t n, float* y,
                          hipStream_t st) {
    rmsnorm_kernel<<<(m + 3) / 4, 256, 0, st>>>(x, w, eps, m, n, y);
    return hipGetLastError();
}

__global__ void add_kernel(float* __restrict__ y, const float* __restrict__ a, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = y[i] + a[i];
}

hipError_t launch_add(float* y, const float* a, size_t n, hipStream_t st) {
    add_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(y, a, n);
    return hipGetLastError();
}

// ============================================================================================
// synthetic data: the test oracle's counter-based generator, bit for bit
// ============================================================================================

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t rng_u64(uint64_t key, uint64_t idx) { return mix64(key + idx * 0xd1b54a32d192ed03ull); }
__device__ __forceinline__ float unif24(uint64_t r, float lo, float hi) {
    float u = (float)(uint32_t)(r & 0xffffffu) * (1.0f / 16777216.0f);
    float span = hi - lo;
    float p = u * span;
    return lo + p;
}

// one thread per 8-byte word of a superblock (18 words for Q4_K, 27 for Q6_K, 34 for a Q8_0 unit
// of 8 blocks); grid.y runs over the `count` matrices of a stack, matrix e drawing from stream
// stream0 + e * step
__global__ void gen_gguf_kernel(uint32_t fmt, uint64_t seed, uint64_t stream0, uint64_t step, size_t nsb,
                                uint64_t stride, float dlo, float dhi, uint8_t* out) {
    if (fmt == TRK_FMT_Q5_1) {  // as orc_gen_gguf: words at sb * 64 + wi, block c's d, m at sb * 64 + 48 + c
        const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (t >= nsb * 24) return;
        const uint64_t key = mix64(seed ^ mix64(stream0 + (uint64_t)blockIdx.y * step));
        const size_t sb = t / 24, wi = t % 24;
        uint8_t* b = out + (size_t)blockIdx.y * stride + sb * 192;
        const uint64_t r = rng_u64(key, sb * 64 + wi);
        for (int j = 0; j < 8; j++) {
            const size_t o = wi * 8 + j, c = o / 24;
            uint8_t v = (uint8_t)(r >> (8 * j));
            if (o % 24 < 4) {
                const uint64_t rd = rng_u64(key, sb * 64 + 48 + c);
                const uint16_t h = o % 24 < 2 ? f2h(unif24(rd, dlo, dhi)) : f2h(-16.0f * unif24(rd >> 24, dlo, dhi));
                v = (o % 2) ? (uint8_t)(h >> 8) : (uint8_t)(h & 0xff);
            }
            b[o] = v;
        }
        return;
    }
    if (fmt == TRK_FMT_Q8_0) {  // as orc_gen_gguf: words at sb * 64 + wi, block c's d at sb * 64 + 48 + c
        const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (t >= nsb * 34) return;
        const uint64_t key = mix64(seed ^ mix64(stream0 + (uint64_t)blockIdx.y * step));
        const size_t sb = t / 34, wi = t % 34;
        uint8_t* b = out + (size_t)blockIdx.y * stride + sb * 272;
        const uint64_t r = rng_u64(key, sb * 64 + wi);
        for (int j = 0; j < 8; j++) {
            const size_t o = wi * 8 + j, c = o / 34;
            uint8_t v = (uint8_t)(r >> (8 * j));
            if (o % 34 < 2) {
                const uint16_t d = f2h(unif24(rng_u64(key, sb * 64 + 48 + c), dlo, dhi));
                v = (o % 34) ? (uint8_t)(d >> 8) : (uint8_t)(d & 0xff);
            }
            b[o] = v;
        }
        return;
    }
    const size_t sbb = fmt == TRK_FMT_Q6_K ? 210 : 144;
    const size_t nw = (sbb + 7) / 8;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nsb * nw) return;
    const uint64_t key = mix64(seed ^ mix64(stream0 + (uint64_t)blockIdx.y * step));  // as orc_rng_u64
    const size_t sb = t / nw, wi = t % nw;
    uint8_t* b = out + (size_t)blockIdx.y * stride + sb * sbb;
    const uint64_t r = rng_u64(key, sb * 32 + wi);
    const uint64_t rd = rng_u64(key, sb * 32 + 31);
    for (int j = 0; j < 8; j++) {
        const size_t o = wi * 8 + j;
        if (o >= sbb) break;
        uint8_t v = (uint8_t)(r >> (8 * j));
        if (fmt == TRK_FMT_Q6_K) {
            if (o == 208 || o == 209) {
                const uint16_t d = f2h(unif24(rd, dlo, dhi));
                v = o == 208 ? (uint8_t)(d & 0xff) : (uint8_t)(d >> 8);
            }
        } else if (o < 4) {
            const uint16_t d = f2h(unif24(o < 2 ? rd : rd >> 24, dlo, dhi));
            v = (o & 1) ? (uint8_t)(d >> 8) : (uint8_t)(d & 0xff);
        }
        b[o] = v;
    }
}

hipError_t launch_gen_gguf(uint32_t fmt, uint64_t seed, uint64_t stream0, uint64_t step, uint32_t count,
                           uint32_t rows, uint32_t k, float dlo, float dhi, void* out, uint64_t stride,
                           hipStream_t st) {
    const size_t nsb = (size_t)rows * (k / 256);
    const size_t nw = fmt == TRK_FMT_Q6_K ? 27 : fmt == TRK_FMT_Q8_0 ? 34 : fmt == TRK_FMT_Q5_1 ? 24 : 18;
    const size_t n = nsb * nw;
    gen_gguf_kernel<<<dim3((unsigned)((n + 255) / 256), count), 256, 0, st>>>(fmt, seed, stream0, step, nsb, stride,
                                                                               dlo, dhi, (uint8_t*)out);
    return hipGetLastError();
}

__global__ void gen_normal_kernel(uint64_t key, size_t n, double sigma, float* out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint64_t a = rng_u64(key, 2 * i), b = rng_u64(key, 2 * i + 1);
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
    double z = ::sqrt(-2.0 * ::log(u1)) * ::cos(6.283185307179586 * u2);
    out[i] = (float)(z * sigma);
}

hipError_t launch_gen_normal(uint64_t seed, uint64_t stream_id, size_t n, double sigma, float* out,
                             hipStream_t st) {
    auto hmix = [](uint64_t z) {
        z += 0x9e3779b97f4a7c15ull;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    };
    uint64_t key = hmix(seed ^ hmix(stream_id));
    gen_normal_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(key, n, sigma, out);
    return hipGetLastError();
}

// ---- the K-split router of a pack written for T tiles -------------------------------------------

// x [m][H] -> xt [T][m][H / T]: tile t's columns of every row, contiguous (the tile's router
// launch then reads rows of H / T)
__global__ __launch_bounds__(256) void tile_split_kernel(const float* __restrict__ x, uint32_t m, uint32_t H,
                                                         uint32_t T, float* __restrict__ xt) {
    const uint32_t hl = H / T, n4 = m * H / 4;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        const uint32_t row = 4 * i / H, col = 4 * i % H, t = col / hl, c = col % hl;  // hl % 16 == 0
        *reinterpret_cast<float4*>(xt + ((size_t)t * m + row) * hl + c) = reinterpret_cast<const float4*>(x)[i];
    }
}

// rlog[row][e] = the tiles' partials summed in tile order (Mailboxes::reduce, exchange.rs:122-136:
// the first copied, the others added), then the bias
__global__ __launch_bounds__(256) void tile_reduce_kernel(const float* __restrict__ plog, uint32_t m, uint32_t E,
                                                          uint32_t T, const float* __restrict__ bias,
                                                          float* __restrict__ rlog) {
    const size_t n = (size_t)m * E;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v = plog[i];
        for (uint32_t t = 1; t < T; t++) v = v + plog[(size_t)t * n + i];
        rlog[i] = bias ? v + bias[i % E] : v;
    }
}

hipError_t launch_tile_split(const float* x, uint32_t m, uint32_t H, uint32_t T, float* xt, hipStream_t st) {
    if (T == 0 || H % (16 * T)) return hipErrorInvalidValue;
    const uint32_t n4 = m * H / 4, wgs = (n4 + 255) / 256;
    tile_split_kernel<<<wgs < 2048 ? wgs : 2048, 256, 0, st>>>(x, m, H, T, xt);
    return hipGetLastError();
}

hipError_t launch_tile_reduce(const float* plog, uint32_t m, uint32_t E, uint32_t T, const float* bias, float* rlog,
                              hipStream_t st) {
    const size_t n = (size_t)m * E, wgs = (n + 255) / 256;
    tile_reduce_kernel<<<(uint32_t)(wgs < 2048 ? wgs : 2048), 256, 0, st>>>(plog, m, E, T, bias, rlog);
    return hipGetLastError();
}

}  // namespace trk
