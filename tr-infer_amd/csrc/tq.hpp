// The reference's packed TQ blocks (crates/tr-format/src/codec.rs:1-46) read on the GPU: the
// block loads of a 16-lane group and its exact block dots, shared by the kernel-level GEMV
// (k_gemv.hip) and the TQ layer kernels (k_tq.hip).
#pragma once

#include "gemv.hpp"

namespace trk {

enum : int { GK_Q4K = 0, GK_Q6K = 1, GK_Q80 = 2, GK_Q51 = 3, GK_TQ4 = 4, GK_TQ5 = 5, GK_TQ8 = 6 };

// TQ block (codec.rs:3-7): d[16] f16 | m[16] f16 | q chunks of 64 bytes (16 rows x 4 bytes) |
// 5-bit: the high-bit plane, per chunk 8 bytes (low half) then 8 bytes (high half), bit r*4+i.
// A block is read by a 16-lane group with 16-byte loads: lane l = 4 cl + rq holds chunks
// cl, cl + 4 of rows 4 rq .. 4 rq + 3 (and, at cl = 0, their d and m).
template <int GK, int KB>
struct GvTQ {
    static constexpr uint32_t BITS = GK == GK_TQ4 ? 4 : GK == GK_TQ5 ? 5 : 8;
    static constexpr uint32_t NCH = BITS == 8 ? KB / 4 : KB / 8;  // 64-byte q chunks per block
    static constexpr uint32_t CPL = (NCH + 3) / 4;                 // chunks per lane
    static constexpr uint32_t BB = 64 + (BITS == 8 ? 16 * KB : 8 * KB) + (BITS == 5 ? 2 * KB : 0);
    uint4 q[CPL];
    uint4 p[BITS == 5 ? CPL : 0];  // the 5-bit plane's chunks (none for 4- and 8-bit codecs)
    uint2 d, m;
};

// The lane's share of TQ block b of the strip at `strip` (lane l of its 16-lane group).
template <int GK, int KB>
__device__ __forceinline__ void gv_load_tq(GvTQ<GK, KB>& w, const uint8_t* __restrict__ strip, uint32_t b, uint32_t l) {
    using T = GvTQ<GK, KB>;
    const uint32_t cl = l / 4, rq = l % 4;
    const uint8_t* blk = strip + (size_t)b * T::BB;
#pragma unroll
    for (uint32_t t = 0; t < T::CPL; t++) {
        const uint32_t c = cl + 4 * t;
        if (c < T::NCH) {
            w.q[t] = *reinterpret_cast<const uint4*>(blk + 64 + 64 * c + 16 * rq);
            if constexpr (T::BITS == 5) w.p[t] = *reinterpret_cast<const uint4*>(blk + 64 + 64 * T::NCH + 16 * c);
        }
    }
    if (cl == 0) {
        w.d = *reinterpret_cast<const uint2*>(blk + 8 * rq);
        w.m = *reinterpret_cast<const uint2*>(blk + 32 + 8 * rq);
    }
}

__device__ __forceinline__ int dpp_ror4_add(int v) { return v + __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false); }
__device__ __forceinline__ int dpp_ror8_add(int v) { return v + __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false); }

// The block's 16 row dots against NA staged activation rows: partial dots over the lane's chunks,
// summed over the group's four chunk lanes (exact integer adds); lane cl = 0 writes its four rows'
// dots to dl[a][j][r0 + 4 rq + rr] and (d, m) to dm[j][...].
template <int GK, int KB, int NA, int R, int S>
__device__ __forceinline__ void gv_terms_tq(const GvTQ<GK, KB>& w, uint32_t l, uint32_t j, uint32_t r0, uint32_t na,
                                            const int8_t (*xq)[S * KB], const float4 (*xs)[S], float (*dl)[S][R],
                                            float2 (*dm)[R]) {
    using T = GvTQ<GK, KB>;
    const uint32_t cl = l / 4, rq = l % 4;
    // q words of row 4 rq + rr in chunk t, unpacked (4/5-bit: low and high nibble planes)
    uint32_t lo[T::CPL][4], hi[T::CPL][4];
#pragma unroll
    for (uint32_t t = 0; t < T::CPL; t++) {
        const uint32_t qw[4] = {w.q[t].x, w.q[t].y, w.q[t].z, w.q[t].w};
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            if constexpr (T::BITS == 8) {
                lo[t][rr] = qw[rr] ^ 0x80808080u;  // q - 128
                hi[t][rr] = 0;
            } else {
                lo[t][rr] = qw[rr] & 0x0f0f0f0fu;
                hi[t][rr] = (qw[rr] >> 4) & 0x0f0f0f0fu;
                if constexpr (T::BITS == 5) {
                    const uint32_t r = 4 * rq + rr;  // bits 4r .. 4r+3 of each 64-bit half
                    const uint32_t pl = r < 8 ? w.p[t].x : w.p[t].y, ph = r < 8 ? w.p[t].z : w.p[t].w;
                    lo[t][rr] |= q5_hi4((pl >> (4 * (r % 8))) & 0xfu);
                    hi[t][rr] |= q5_hi4((ph >> (4 * (r % 8))) & 0xfu);
                }
            }
        }
    }
#pragma unroll
    for (uint32_t a = 0; a < NA; a++) {
        if (a >= na) break;
        const int* x = reinterpret_cast<const int*>(&xq[a][j * KB]);
        int dot[4] = {0, 0, 0, 0};
#pragma unroll
        for (uint32_t t = 0; t < T::CPL; t++) {
            const uint32_t c = cl + 4 * t;
            if (T::NCH % 4 == 0 || c < T::NCH) {
                const int xl = x[c];
                const int xh = T::BITS == 8 ? 0 : x[T::NCH + c];
#pragma unroll
                for (int rr = 0; rr < 4; rr++) {
                    dot[rr] = sdot4((int)lo[t][rr], xl, dot[rr]);
                    if constexpr (T::BITS != 8) dot[rr] = sdot4((int)hi[t][rr], xh, dot[rr]);
                }
            }
        }
        const int corr = T::BITS == 8 ? 128 * __float_as_int(xs[a][j].z) : 0;
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            // the sum over the orbit {rq, rq + 4, rq + 8, rq + 12} (lanes without a chunk hold 0)
            const int v = dpp_ror8_add(dpp_ror4_add(dot[rr]));
            if (cl == 0) dl[a][j][r0 + 4 * rq + rr] = (float)(v + corr);
        }
    }
    if (cl == 0) {
        const uint16_t dv[4] = {(uint16_t)(w.d.x & 0xffff), (uint16_t)(w.d.x >> 16), (uint16_t)(w.d.y & 0xffff),
                                (uint16_t)(w.d.y >> 16)};
        const uint16_t mv[4] = {(uint16_t)(w.m.x & 0xffff), (uint16_t)(w.m.x >> 16), (uint16_t)(w.m.y & 0xffff),
                                (uint16_t)(w.m.y >> 16)};
#pragma unroll
        for (int rr = 0; rr < 4; rr++) dm[j][r0 + 4 * rq + rr] = make_float2(h2f(dv[rr]), h2f(mv[rr]));
    }
}

}  // namespace trk
