// Streaming-GEMV building blocks shared by the decode kernels (k_decode.hip) and the small-item
// grouped kernels (k_stream.hip): per-lane Q4_K / Q6_K superblock pieces, their exact block dots
// against int8 activations, and the hand-over of the reference's per-block f32 chain
// (gemv.rs:141-148) from one lane to the next.
#pragma once

#include "common.hpp"

namespace trk {

// gate/up threads: a lane per (row, superblock) of a strip's 16 gate + 16 up rows, 64 / NSB rows
// per wave so that no row's lanes straddle two waves, at least two waves
#define GU_WAVES(nsb) ((32 + 64 / (nsb) - 1) / (64 / (nsb)))
#define GU_THREADS(nsb) (GU_WAVES(nsb) < 2 ? 128 : 64 * GU_WAVES(nsb))

__device__ __forceinline__ uint32_t nib(uint32_t w, int h) { return (w >> (4 * h)) & 0x0f0f0f0fu; }

// Lane (row r, superblock sb) of the workgroup: r = tid / NSB.  The per-row epilogue chain runs
// across the NSB lanes of a row in superblock order, the running f32 accumulators passed one lane
// up per step (DPP row shift when NSB divides 16).
template <int NSB>
__device__ __forceinline__ float lane_up(float v) {
    if constexpr (16 % NSB == 0)
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, false));  // row_shr:1
    else
        return __shfl_up(v, 1);
}

// the running accumulator one lane up (towards the next half-superblock of the unit)
template <int L>
__device__ __forceinline__ float unit_up(float v) {
    if constexpr (16 % L == 0)
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, false));  // row_shr:1
    else
        return __shfl_up(v, 1);
}

// Q4_K half superblock h2 of superblock sb: the 16-byte header and the 64 qs bytes of its four
// sub-blocks (sub-block j = 4*h2 + jj lives in nibble j%2 of qs[32*(j/2) + i]).
__device__ __forceinline__ void load_half_q4k(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t h2, uint4& hdr,
                                              uint4 (&qs)[4]) {
    const uint4* p = reinterpret_cast<const uint4*>(rowp + sb * 144);
    hdr = p[0];
    const uint4* q = reinterpret_cast<const uint4*>(rowp + sb * 144 + 16 + 64 * h2);
#pragma unroll
    for (int i = 0; i < 4; i++) qs[i] = q[i];
}

// per-block terms of a lane's 8 blocks (blocks 16*sb + 8*h2 + 0..7): exact int dot, t = dd*sx,
// mm and the activation's u = sx*sum, for P activation rows
template <int P>
__device__ __forceinline__ void half_terms_q4k(const uint4& hdr, const uint4 (&qs)[4], uint32_t h2,
                                               const int8_t* __restrict__ aq /*[P] rows, stride F, at block 0*/,
                                               uint32_t F, const float* __restrict__ as, const float* __restrict__ au,
                                               uint32_t nbf, float (&dotv)[P][8], float (&tv)[P][8], float (&mmv)[8],
                                               float (&uv)[P][8]) {
    const uint32_t* w32 = reinterpret_cast<const uint32_t*>(qs);
    const float d = h2f((uint16_t)(hdr.x & 0xffff)), dmin = h2f((uint16_t)(hdr.x >> 16));
#pragma unroll
    for (int p = 0; p < P; p++) {
        const float4* s4 = reinterpret_cast<const float4*>(as + p * nbf);
        const float4* u4 = reinterpret_cast<const float4*>(au + p * nbf);
        const float4 s0 = s4[0], s1 = s4[1], u0 = u4[0], u1 = u4[1];
        const float sa[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        const float ua[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            tv[p][i] = sa[i];
            uv[p][i] = ua[i];
        }
    }
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        int sc, mn;
        // h2 is 0 or 1: select the sub-block's scale/min without indexing by a runtime value
        int sc0, mn0, sc1, mn1;
        q4k_scale_min_w(hdr.y, hdr.z, hdr.w, jj, sc0, mn0);
        q4k_scale_min_w(hdr.y, hdr.z, hdr.w, 4 + jj, sc1, mn1);
        sc = h2 ? sc1 : sc0;
        mn = h2 ? mn1 : mn0;
        float ddv, mm;
        q4k_dm(d, dmin, sc, mn, ddv, mm);
        const int c = jj / 2, h = jj % 2;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int i = 2 * jj + hh;
            mmv[i] = mm;
#pragma unroll
            for (int p = 0; p < P; p++) {
                const int4 xv = *reinterpret_cast<const int4*>(aq + p * F + i * 16);
                int dot = sdot4((int)nib(w32[8 * c + 4 * hh + 0], h), xv.x, 0);
                dot = sdot4((int)nib(w32[8 * c + 4 * hh + 1], h), xv.y, dot);
                dot = sdot4((int)nib(w32[8 * c + 4 * hh + 2], h), xv.z, dot);
                dot = sdot4((int)nib(w32[8 * c + 4 * hh + 3], h), xv.w, dot);
                dotv[p][i] = (float)dot;
                tv[p][i] = ddv * tv[p][i];  // t = d * sx (gemv.rs:145)
            }
        }
    }
}

// Q6_K (210-byte superblocks, 2-byte aligned) half superblock h2: blocks j = 8*h2 + 0..7 use
// ql[64*h2 + ...], qh[32*h2 + ...], scales[8*h2 + ...] and d — the extension mapping: unsigned
// 6-bit q, dd = f16(d*sc), mm = f16(-32*dd), one block per scale.  In registers as 32-bit words
// (from 2-byte loads): ql bytes 64*h2 + 4j, qh bytes 128 + 32*h2 + 4j, the 8 int8 scales, d.
struct Q6Half {
    uint32_t ql[16], qh[8], sc[2];
    uint32_t d;
};
__device__ __forceinline__ void load_half_q6k(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t h2, Q6Half& w) {
    const uint16_t* s2 = reinterpret_cast<const uint16_t*>(rowp + sb * 210);
    auto w32 = [&](uint32_t o) -> uint32_t { return (uint32_t)s2[o] | ((uint32_t)s2[o + 1] << 16); };
#pragma unroll
    for (int j = 0; j < 16; j++) w.ql[j] = w32(32 * h2 + 2 * j);
#pragma unroll
    for (int j = 0; j < 8; j++) w.qh[j] = w32(64 + 16 * h2 + 2 * j);
#pragma unroll
    for (int j = 0; j < 2; j++) w.sc[j] = w32(96 + 4 * h2 + 2 * j);
    w.d = s2[104];
}

template <int P>
__device__ __forceinline__ void half_terms_q6k(const Q6Half& w, const int8_t* __restrict__ aq, uint32_t F,
                                               const float* __restrict__ as, const float* __restrict__ au,
                                               uint32_t nbf, float (&dotv)[P][8], float (&tv)[P][8], float (&mmv)[8],
                                               float (&uv)[P][8]) {
    const float d = h2f((uint16_t)w.d);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int8_t sc = (int8_t)((w.sc[i >> 2] >> (8 * (i & 3))) & 0xffu);
        const float ddv = f16_round(d * (float)sc);
        mmv[i] = f16_round(-32.0f * ddv);
        const int g = i / 2, l0 = 16 * (i % 2);
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int4 xv = *reinterpret_cast<const int4*>(aq + p * F + i * 16);
            const int xa[4] = {xv.x, xv.y, xv.z, xv.w};
            int dot = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                uint32_t lo = w.ql[8 * (g & 1) + l0 / 4 + t];
                lo = (g >> 1) ? ((lo >> 4) & 0x0f0f0f0fu) : (lo & 0x0f0f0f0fu);
                const uint32_t hi = (w.qh[l0 / 4 + t] >> (2 * g)) & 0x03030303u;
                dot = sdot4((int)(lo | (hi << 4)), xa[t], dot);
            }
            dotv[p][i] = (float)dot;
            tv[p][i] = ddv * as[p * nbf + i];
            uv[p][i] = au[p * nbf + i];
        }
    }
}

template <int P>
__device__ __forceinline__ void half_terms_q6k(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t h2,
                                               const int8_t* __restrict__ aq, uint32_t F,
                                               const float* __restrict__ as, const float* __restrict__ au,
                                               uint32_t nbf, float (&dotv)[P][8], float (&tv)[P][8], float (&mmv)[8],
                                               float (&uv)[P][8]) {
    Q6Half w;
    load_half_q6k(rowp, sb, h2, w);
    half_terms_q6k<P>(w, aq, F, as, au, nbf, dotv, tv, mmv, uv);
}

// Q8_0 (34-byte blocks: f16 d, 32 int8), read in units of 8 blocks (272 bytes, 16-byte aligned):
// half unit h2 = blocks 4 h2 .. 4 h2 + 3 = bytes 136 h2 .. +135, held as 34 words (8-byte loads).
// q8_0_rows' unsigned form (blocks.py:71-78): q = int8 + 128, dd = d, mm = f16(-128 d).  The
// unsigned dot is the signed one plus 128 times the activations' sum, both exact in int32.
struct Q8Half {
    uint32_t w[34];
};
__device__ __forceinline__ void load_half_q80(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t h2, Q8Half& w) {
    const uint2* p = reinterpret_cast<const uint2*>(rowp + sb * 272 + 136 * h2);
#pragma unroll
    for (int i = 0; i < 17; i++) {
        const uint2 v = p[i];
        w.w[2 * i] = v.x;
        w.w[2 * i + 1] = v.y;
    }
}
// the 4 bytes at byte o of the half (o a constant once unrolled)
__device__ __forceinline__ uint32_t q8_word(const Q8Half& w, uint32_t o) {
    return o % 4 ? __builtin_amdgcn_alignbyte(w.w[o / 4 + 1], w.w[o / 4], o % 4) : w.w[o / 4];
}

template <int P>
__device__ __forceinline__ void half_terms_q80(const Q8Half& w, const int8_t* __restrict__ aq, uint32_t F,
                                               const float* __restrict__ as, const float* __restrict__ au,
                                               uint32_t nbf, float (&dotv)[P][8], float (&tv)[P][8], float (&mmv)[8],
                                               float (&uv)[P][8]) {
#pragma unroll
    for (int i = 0; i < 8; i++) {  // 16-block i: half i % 2 of block j = i / 2
        const uint32_t j = i / 2, o = 34 * j;
        const float ddv = h2f((uint16_t)((w.w[o / 4] >> (8 * (o % 4))) & 0xffffu));
        mmv[i] = f16_round(-128.0f * ddv);
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int4 xv = *reinterpret_cast<const int4*>(aq + p * F + i * 16);
            const int xa[4] = {xv.x, xv.y, xv.z, xv.w};
            int dot = 0, sum = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                dot = sdot4((int)q8_word(w, o + 2 + 16 * (i % 2) + 4 * t), xa[t], dot);
                sum = sdot4(xa[t], 0x01010101, sum);
            }
            dotv[p][i] = (float)(dot + 128 * sum);
            tv[p][i] = ddv * as[p * nbf + i];
            uv[p][i] = au[p * nbf + i];
        }
    }
}

template <int P>
__device__ __forceinline__ void half_terms_q80(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t h2,
                                               const int8_t* __restrict__ aq, uint32_t F,
                                               const float* __restrict__ as, const float* __restrict__ au,
                                               uint32_t nbf, float (&dotv)[P][8], float (&tv)[P][8], float (&mmv)[8],
                                               float (&uv)[P][8]) {
    Q8Half w;
    load_half_q80(rowp, sb, h2, w);
    half_terms_q80<P>(w, aq, F, as, au, nbf, dotv, tv, mmv, uv);
}

// Q5_1 (24-byte blocks: f16 d, f16 m, u32 qh, 16 bytes qs), read in units of 8 blocks (192 bytes,
// 16-byte aligned): half unit h2 = blocks 4 h2 .. 4 h2 + 3 = 24 words.  q5_1_rows (blocks.py:57-68):
// element i is nibble i % 16 of qs (low for i < 16) with bit i of qh as its fifth bit; dd = d,
// mm = m as stored.
struct Q51Half {
    uint32_t w[24];
};
__device__ __forceinline__ void load_half_q51(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t h2, Q51Half& w) {
    const uint4* p = reinterpret_cast<const uint4*>(rowp + sb * 192 + 96 * h2);
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const uint4 v = p[i];
        w.w[4 * i] = v.x;
        w.w[4 * i + 1] = v.y;
        w.w[4 * i + 2] = v.z;
        w.w[4 * i + 3] = v.w;
    }
}
// four fifth bits (bits 0-3 of h4) moved to bit 4 of bytes 0-3: h4 * (1 + 2^7 + 2^14 + 2^21) puts
// bit b at bit 8b (the 16 partial products land on distinct bits, so nothing carries); both
// factors fit 24 bits, so the full-rate 24-bit multiply gives the product
__device__ __forceinline__ uint32_t q5_hi4(uint32_t h4) { return (__umul24(h4, 0x204081u) & 0x01010101u) << 4; }

template <int P>
__device__ __forceinline__ void half_terms_q51(const Q51Half& w, const int8_t* __restrict__ aq, uint32_t F,
                                               const float* __restrict__ as, const float* __restrict__ au,
                                               uint32_t nbf, float (&dotv)[P][8], float (&tv)[P][8], float (&mmv)[8],
                                               float (&uv)[P][8]) {
#pragma unroll
    for (int i = 0; i < 8; i++) {  // 16-block i: elements 16 (i % 2) .. +15 of block j = i / 2
        const int j = i / 2, hf = i % 2;
        const float ddv = h2f((uint16_t)(w.w[6 * j] & 0xffffu));
        mmv[i] = h2f((uint16_t)(w.w[6 * j] >> 16));
        const uint32_t qh = w.w[6 * j + 1];
        uint32_t qw[4];
#pragma unroll
        for (int t = 0; t < 4; t++)
            qw[t] = ((w.w[6 * j + 2 + t] >> (4 * hf)) & 0x0f0f0f0fu) | q5_hi4((qh >> (16 * hf + 4 * t)) & 0xfu);
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int4 xv = *reinterpret_cast<const int4*>(aq + p * F + i * 16);
            const int xa[4] = {xv.x, xv.y, xv.z, xv.w};
            int dot = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) dot = sdot4((int)qw[t], xa[t], dot);
            dotv[p][i] = (float)dot;
            tv[p][i] = ddv * as[p * nbf + i];
            uv[p][i] = au[p * nbf + i];
        }
    }
}

template <int P>
__device__ __forceinline__ void half_terms_q51(const uint8_t* __restrict__ rowp, uint32_t sb, uint32_t h2,
                                               const int8_t* __restrict__ aq, uint32_t F,
                                               const float* __restrict__ as, const float* __restrict__ au,
                                               uint32_t nbf, float (&dotv)[P][8], float (&tv)[P][8], float (&mmv)[8],
                                               float (&uv)[P][8]) {
    Q51Half w;
    load_half_q51(rowp, sb, h2, w);
    half_terms_q51<P>(w, aq, F, as, au, nbf, dotv, tv, mmv, uv);
}

}  // namespace trk
