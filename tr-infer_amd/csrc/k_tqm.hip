// The MoE layer's expert products on the reference's packed TQ strips (codec.rs:1-46) with int8
// MFMA.  A TQ block is 16 weight rows x kb values, the shape of a v_mfma_i32_16x16x32_i8 operand:
// B[k 8g .. 8g+7][col r] for lane (g = l / 16, r = l % 16) is two 4-byte words of row r (chunks
// 2 (g % 2) and 2 (g % 2) + 1 at kb 32, low or high nibbles by g / 2), and A[row][k ..] holds up
// to 16 activation rows (a decode slot's one or two levels, or a batch item's entries).  One MFMA
// per block gives every (activation row, weight row) dot exactly; a kb-16 block pair shares one
// MFMA shape with the other block's activation lanes zeroed, so each 16-block's dot stays its own.
// Lane l then holds D[activation row 4 g + v][weight row r] and runs the reference's per-block
// f32 chain (gemv.rs:141-148) on its four outputs in block order.
//
//   tqm_gateup_kernel  a wave per (matrix, strip): waves 2 i and 2 i + 1 are the gate and up
//                      strips of strip pair i; then SwiGLU (elem.rs:173), the per-16 quantisation
//                      of the strip (two levels for a decode slot with TR_HIPREC, quant.rs:96-108)
//                      and the routing-weight fold (exec.rs:1584-1606, exec_batch.rs:1528-1536)
//   tqm_down_kernel    a wave per strip of H, the unit's down rows into yent
#include "route.hpp"
#include "tq.hpp"

namespace trk {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i tqm_mfma(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// B operand of lane (g, r) for the 32-wide unit at block b of a strip (kb 32: block b; kb 16:
// blocks 2b and 2b + 1, lanes g < 2 the first), plus the d / m of row r for the unit's block(s).
// The loads keep the raw words (no arithmetic on them), so a batch of units' loads stays in
// flight; tqm_operand decodes them when the unit is used.
template <int GK, int KB>
struct TqmB {
    static constexpr uint32_t NBL = KB == 16 ? 2 : 1;
    static constexpr uint32_t P5 = GvTQ<GK, KB>::BITS == 5 ? 1 : 0;
    static constexpr uint32_t REGS = 2 + 2 * P5 + 2 * NBL;  // VGPRs a unit holds
    uint32_t w0, w1;
    uint32_t p0[P5], p1[P5];
    uint32_t d[NBL], m[NBL];  // f16 bits, zero-extended by the loads (no packing, no wait)
};

template <int GK, int KB>
__device__ __forceinline__ void tqm_load(TqmB<GK, KB>& w, const uint8_t* __restrict__ strip, uint32_t b, uint32_t l) {
    using T = GvTQ<GK, KB>;
    const uint32_t g = l / 16, r = l % 16;
    auto ld32 = [](const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); };
    auto ld16 = [](const uint8_t* p) { return (uint32_t)*reinterpret_cast<const uint16_t*>(p); };
    if constexpr (KB == 32) {
        const uint8_t* blk = strip + (size_t)b * T::BB;
        // 8-bit: chunks 2g, 2g + 1 (k = 8g ..); 4/5-bit: chunks 2 (g % 2), +1 (nibble g / 2)
        const uint32_t c0 = T::BITS == 8 ? 2 * g : 2 * (g % 2);
        w.w0 = ld32(blk + 64 + 64 * c0 + 4 * r);
        w.w1 = ld32(blk + 64 + 64 * c0 + 64 + 4 * r);
        if constexpr (T::BITS == 5) {  // plane of chunk c: 8 bytes (low nibbles) then 8 (high)
            const uint8_t* pl = blk + 64 + 256 + 8 * (g / 2) + 4 * (r / 8);
            w.p0[0] = ld32(pl + 16 * c0);
            w.p1[0] = ld32(pl + 16 * (c0 + 1));
        }
        w.d[0] = ld16(blk + 2 * r);
        w.m[0] = ld16(blk + 32 + 2 * r);
    } else {
        // kb 16: lanes g < 2 take block 2b, g >= 2 block 2b + 1; within a block k 8 (g % 2) ..
        const uint8_t* blk = strip + (size_t)(2 * b + g / 2) * T::BB;
        const uint32_t gg = g % 2;
        if constexpr (T::BITS == 8) {  // 4 chunks: k = 4c ..; chunks 2gg, 2gg + 1
            w.w0 = ld32(blk + 64 + 128 * gg + 4 * r);
            w.w1 = ld32(blk + 64 + 128 * gg + 64 + 4 * r);
        } else {  // 2 chunks: low nibbles k = 4c .., high k = 8 + 4c ..; nibble gg
            w.w0 = ld32(blk + 64 + 4 * r);
            w.w1 = ld32(blk + 128 + 4 * r);
            if constexpr (T::BITS == 5) {
                const uint8_t* pl = blk + 64 + 128 + 8 * gg + 4 * (r / 8);
                w.p0[0] = ld32(pl);
                w.p1[0] = ld32(pl + 16);
            }
        }
        const uint8_t* b0 = strip + (size_t)(2 * b) * T::BB;
        w.d[0] = ld16(b0 + 2 * r);
        w.m[0] = ld16(b0 + 32 + 2 * r);
        w.d[1] = ld16(b0 + T::BB + 2 * r);
        w.m[1] = ld16(b0 + T::BB + 32 + 2 * r);
    }
}

// The 8 int8 B values of lane (g, r) from the raw words.
template <int GK, int KB>
__device__ __forceinline__ long tqm_operand(const TqmB<GK, KB>& w, uint32_t l) {
    using T = GvTQ<GK, KB>;
    const uint32_t g = l / 16, r = l % 16;
    uint32_t w0, w1;
    if constexpr (T::BITS == 8) {  // stored q + 128 unsigned
        w0 = w.w0 ^ 0x80808080u;
        w1 = w.w1 ^ 0x80808080u;
    } else {
        const uint32_t h = KB == 32 ? g / 2 : g % 2;  // the nibble
        w0 = (w.w0 >> (4 * h)) & 0x0f0f0f0fu;
        w1 = (w.w1 >> (4 * h)) & 0x0f0f0f0fu;
        if constexpr (T::BITS == 5) {
            w0 |= q5_hi4((w.p0[0] >> (4 * (r % 8))) & 0xfu);
            w1 |= q5_hi4((w.p1[0] >> (4 * (r % 8))) & 0xfu);
        }
    }
    return (long)(((unsigned long long)w1 << 32) | w0);
}

// The activation rows of a work unit: a decode slot's one or two levels (x at gate/up, the slot's
// SwiGLU rows at down) or a batch item's entry rows, staged in LDS once per workgroup in operand
// order with their per-block (scale, u, byte sum).
struct TqmArgs {
    Mat a, b, sha, shb;  // gate/up: gate, up, shared gate, shared up; down: down, -, shared down, -
    Workspace ws;
    int decode, pair;
    // decode gate/up with the routing inside (NJ > 0): every workgroup routes the logits row lg
    // itself (route_topk / route_mass, router.rs:106-148) and workgroup (0, 0) publishes the ids,
    // weights and count for the down and combine launches
    const float* lg;
    uint32_t k;
    Policy pol;
};

constexpr uint32_t TQM_PAIRS = 4;  // batch: strip pairs per workgroup (two passes of two; real shape: 5 per item)

// The unit of workgroup row y: returns false when there is none.  prow: physical activation rows;
// orow: output row of each logical row; nr logical rows, P physical per logical.
__device__ __forceinline__ bool tqm_unit(const Workspace& ws, bool gu, int decode, int pair, uint32_t y, bool& shared,
                                         uint32_t& e, uint32_t& nr, uint32_t& P, uint32_t* prow, uint32_t* orow,
                                         uint32_t tid, uint32_t ns, const uint32_t* ids) {
    Item item{};
    if (decode) {
        if (y > ns) return false;
        shared = y == ns;
        e = shared ? 0u : ids[y];
        nr = 1;
        P = pair ? 2u : 1u;
    } else {
        if (y >= ws.n_groups[2]) return false;
        item = ws.items[y];
        shared = item.expert == NO_EXPERT;
        e = shared ? 0u : item.expert;
        nr = item.nrows;
        P = 1;
    }
    const uint32_t n_ent = ws.n_groups[1];
    if (tid < nr * P) {
        const uint32_t i = tid / P, lv = tid % P;
        if (decode) {
            prow[tid] = gu ? lv : 2 * y + lv;
            if (lv == 0) orow[i] = y;
        } else {
            const uint32_t arow = shared ? n_ent + item.row0 + i : item.row0 + i;
            prow[tid] = gu ? item_token(ws, item, shared, i) : arow;
            orow[i] = arow;
        }
    }
    return true;
}

// Stage the unit's activation rows (K bytes each, int8) in operand order As[unit b][lane] (8 bytes:
// row l % 16, k 32b + 8 (l / 16) ..), zero for rows past np, and their per-block (scale, u) in
// Sc[block][row] (blocks of kbs values), with the byte sum as a third word for the 8-bit codecs
// (SC = 4 floats per entry; 2 otherwise).
template <int KBS, bool XSUM>
__device__ __forceinline__ void tqm_stage(const int8_t* __restrict__ q, const float* __restrict__ s,
                                          const float* __restrict__ u, const uint32_t* prow, uint32_t np, uint32_t K,
                                          long* As, float* Sc, uint32_t tid, uint32_t nthr) {
    const uint32_t nu = K / 32, nbs = K / KBS;
    // rows past np are zero in the operand (LDS stores only)
    if (np < 16)
        for (uint32_t i = tid; i < nu * 64; i += nthr)
            if (i % 16 >= np) As[i] = 0;
    // the live rows: 8-byte pieces (unit b, k-group g, row), 8 loads in flight per thread before
    // any is stored
    const uint32_t n = nu * 4 * np;
    for (uint32_t i0 = 0; i0 < n; i0 += 8 * nthr) {
        long v[8];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const uint32_t i = i0 + tid + nthr * c, ic = i < n ? i : n - 1;
            const uint32_t row = ic % np, bg = ic / np;  // bg = 4 b + g
            v[c] = *reinterpret_cast<const long*>(q + (size_t)prow[row] * K + 8 * bg);
        }
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const uint32_t i = i0 + tid + nthr * c;
            if (i < n) As[(i / np) * 16 + i % np] = v[c];  // As[b * 64 + g * 16 + row]
        }
    }
    // (scale, u, byte sum) per (block, row): zero rows past np, 4 blocks in flight per thread
    const uint32_t ns = nbs * 16;
    for (uint32_t i0 = 0; i0 < ns; i0 += 4 * nthr) {
        float4 v[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = i0 + tid + nthr * c, ic = i < ns ? i : ns - 1;
            const uint32_t b = ic / 16, row = ic % 16;
            v[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (row < np) {
                const size_t bi = (size_t)prow[row] * nbs + b;
                int xs = 0;
                if constexpr (XSUM) {  // 8-bit codecs: the block's byte sum corrects the q + 128 offset
                    const int4* xp = reinterpret_cast<const int4*>(q + (size_t)prow[row] * K + (size_t)KBS * b);
#pragma unroll
                    for (int t = 0; t < KBS / 16; t++) {
                        const int4 w = xp[t];
                        xs = sdot4(w.x, 0x01010101, xs);
                        xs = sdot4(w.y, 0x01010101, xs);
                        xs = sdot4(w.z, 0x01010101, xs);
                        xs = sdot4(w.w, 0x01010101, xs);
                    }
                }
                v[c] = make_float4(s[bi], u[bi], __int_as_float(xs), 0.0f);
            }
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = i0 + tid + nthr * c;
            if (i < ns) {
                if constexpr (XSUM)
                    reinterpret_cast<float4*>(Sc)[i] = v[c];
                else
                    reinterpret_cast<float2*>(Sc)[i] = make_float2(v[c].x, v[c].y);
            }
        }
    }
}

// The chain of one strip for lane l over all units: acc[v] for activation row 4 (l / 16) + v and
// weight row l % 16.  Loads run UB units ahead.  R1: the block's fma with mm and its products
// dd * sx as rank-1 MFMAs (rank1, the same bits), each lane reading only its own row's (s, u), with
// a quarter of the units in flight (the full window went to scratch memory).  The batch down takes
// it (real shape M = 512: 381 -> 347 us); the gate/up, whose waves each chain 5 strips, doubled in
// time with it (the MFMA latency on every block of the chain), and decode keeps the VALU form too.
template <int GK, int KB, bool R1>
__device__ __forceinline__ void tqm_strip(const uint8_t* __restrict__ strip, uint32_t K, const long* As,
                                          const float* Sc, uint32_t l, float (&acc)[4]) {
    // the walk over K is sequential per wave (the chain), so the loads run UB units ahead (about
    // 64 VGPRs of raw words: with about 4 loads per unit, near the 63 a wave's load counter tracks)
    constexpr uint32_t UB0 = 64 / TqmB<GK, KB>::REGS < 16 ? 64 / TqmB<GK, KB>::REGS : 16;
    constexpr uint32_t UB = R1 ? (UB0 / 4 > 0 ? UB0 / 4 : 1u) : UB0;
    constexpr bool U8 = GvTQ<GK, KB>::BITS == 8;
    constexpr uint32_t SC = U8 ? 4 : 2;  // floats per Sc entry
    const uint32_t nu = K / 32, g = l / 16, tl = 4 * g + (l & 3);
    for (int v = 0; v < 4; v++) acc[v] = 0.0f;
    v4f a4 = {0.0f, 0.0f, 0.0f, 0.0f};
    TqmB<GK, KB> w[UB];
#pragma unroll
    for (uint32_t i = 0; i < UB; i++)
        if (i < nu) tqm_load<GK, KB>(w[i], strip, i, l);
    for (uint32_t b0 = 0; b0 < nu; b0 += UB) {
#pragma unroll
        for (uint32_t i = 0; i < UB; i++) {
            const uint32_t b = b0 + i;
            if (b >= nu) break;
            const TqmB<GK, KB> cw = w[i];
            if (b + UB < nu) tqm_load<GK, KB>(w[i], strip, b + UB, l);  // the load UB units ahead
            const long a = As[b * 64 + l];
            const long bq = tqm_operand<GK, KB>(cw, l);
            constexpr uint32_t NBL = TqmB<GK, KB>::NBL;  // blocks of the unit
#pragma unroll
            for (uint32_t hb = 0; hb < NBL; hb++) {
                // kb 16: the activation lanes of the other block zeroed
                const long am = KB == 16 ? ((g / 2 == hb) ? a : 0) : a;
                const v4i d4 = tqm_mfma(am, bq);
                const uint32_t blk = NBL * b + hb;
                const float dd = h2f((uint16_t)cw.d[hb]), mm = h2f((uint16_t)cw.m[hb]);
                if constexpr (R1) {
                    const float2 su = *reinterpret_cast<const float2*>(&Sc[(blk * 16 + tl) * SC]);
                    a4 = rank1(su.y, mm, a4);
                    const v4f ds = rank1(su.x, dd, neg_zero4());
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int dot = U8 ? d4[v] + 128 * __float_as_int(Sc[(blk * 16 + 4 * g + v) * SC + 2]) : d4[v];
                        a4[v] = __builtin_fmaf((float)dot, ds[v], a4[v]);
                    }
                } else {
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const float* sx = Sc + (blk * 16 + 4 * g + v) * SC;
                        const int dot = U8 ? d4[v] + 128 * __float_as_int(sx[2]) : d4[v];
                        acc[v] = __builtin_fmaf(mm, sx[1], acc[v]);
                        acc[v] = __builtin_fmaf((float)dot, dd * sx[0], acc[v]);
                    }
                }
            }
        }
    }
    if constexpr (R1)
        for (int v = 0; v < 4; v++) acc[v] = a4[v];
}

// Two strips' chains in one wave (the batch gate/up): the same walk as tqm_strip's VALU form, with
// half the unit window per strip and each unit's activations and scales read once for both.  The
// waves of that kernel chain several strips each; two independent chains fill the latency of one.
template <int GK, int KB>
__device__ __forceinline__ void tqm_strip2(const uint8_t* __restrict__ s0, const uint8_t* __restrict__ s1, uint32_t K,
                                           const long* As, const float* Sc, uint32_t l, float (&acc0)[4],
                                           float (&acc1)[4]) {
    constexpr uint32_t UB0 = 64 / TqmB<GK, KB>::REGS < 16 ? 64 / TqmB<GK, KB>::REGS : 16;
    constexpr uint32_t UB = UB0 / 2 > 0 ? UB0 / 2 : 1u;
    constexpr bool U8 = GvTQ<GK, KB>::BITS == 8;
    constexpr uint32_t SC = U8 ? 4 : 2;  // floats per Sc entry
    const uint32_t nu = K / 32, g = l / 16;
    for (int v = 0; v < 4; v++) acc0[v] = acc1[v] = 0.0f;
    TqmB<GK, KB> w0[UB], w1[UB];
#pragma unroll
    for (uint32_t i = 0; i < UB; i++)
        if (i < nu) {
            tqm_load<GK, KB>(w0[i], s0, i, l);
            tqm_load<GK, KB>(w1[i], s1, i, l);
        }
    for (uint32_t b0 = 0; b0 < nu; b0 += UB) {
#pragma unroll
        for (uint32_t i = 0; i < UB; i++) {
            const uint32_t b = b0 + i;
            if (b >= nu) break;
            // the unit's operands and scales out of its registers first, then the loads UB units
            // ahead into the same registers, unconditionally (the strip's last unit again past its
            // end): no branch, so no copies of the window
            constexpr uint32_t NBL = TqmB<GK, KB>::NBL;  // blocks of the unit
            const long bq0 = tqm_operand<GK, KB>(w0[i], l), bq1 = tqm_operand<GK, KB>(w1[i], l);
            float dd0v[NBL], mm0v[NBL], dd1v[NBL], mm1v[NBL];
#pragma unroll
            for (uint32_t hb = 0; hb < NBL; hb++) {
                dd0v[hb] = h2f((uint16_t)w0[i].d[hb]);
                mm0v[hb] = h2f((uint16_t)w0[i].m[hb]);
                dd1v[hb] = h2f((uint16_t)w1[i].d[hb]);
                mm1v[hb] = h2f((uint16_t)w1[i].m[hb]);
            }
            const uint32_t bn = b + UB < nu ? b + UB : nu - 1;
            tqm_load<GK, KB>(w0[i], s0, bn, l);
            tqm_load<GK, KB>(w1[i], s1, bn, l);
            const long a = As[b * 64 + l];
#pragma unroll
            for (uint32_t hb = 0; hb < NBL; hb++) {
                const long am = KB == 16 ? ((g / 2 == hb) ? a : 0) : a;
                const v4i d40 = tqm_mfma(am, bq0), d41 = tqm_mfma(am, bq1);
                const uint32_t blk = NBL * b + hb;
                const float dd0 = dd0v[hb], mm0 = mm0v[hb], dd1 = dd1v[hb], mm1 = mm1v[hb];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const float* sx = Sc + (blk * 16 + 4 * g + v) * SC;
                    const int xs = U8 ? 128 * __float_as_int(sx[2]) : 0;
                    acc0[v] = __builtin_fmaf(mm0, sx[1], acc0[v]);
                    acc0[v] = __builtin_fmaf((float)(d40[v] + xs), dd0 * sx[0], acc0[v]);
                    acc1[v] = __builtin_fmaf(mm1, sx[1], acc1[v]);
                    acc1[v] = __builtin_fmaf((float)(d41[v] + xs), dd1 * sx[0], acc1[v]);
                }
            }
        }
    }
}

// SwiGLU and the per-16 quantisation of one strip's rows: the 16 lanes of lane group gq hold one
// activation row's 16 values (rows r of the strip); decode: levels 0 and 1 of the one logical
// row in lane group 0 (two-level quantisation with pair); batch: rows 4 gq + i of the item.
__device__ __forceinline__ void tqm_swiglu_store(const Workspace& ws, int decode, int pair, uint32_t P, uint32_t nr,
                                                 const uint32_t* orow, uint32_t n_ent, uint32_t F, uint32_t nbf,
                                                 uint32_t strip, uint32_t gq, uint32_t r, const float (&acc)[4],
                                                 const float* hu, uint32_t ns, const float* wsel) {
    auto quant16 = [&](float x, float& s, int32_t& sum, int8_t& q, float& res) {
        const float amax = row16_allreduce(__builtin_fabsf(x), [](float a, float b) { return mx_ps(a, b); });
        s = amax / 127.0f;
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        const int32_t qi = cvt_rne(x * inv);
        sum = row16_allreduce(qi, [](int32_t a, int32_t b) { return a + b; });
        q = sat_i8(qi);
        res = __builtin_fmaf(-(float)qi, s, x);
    };
    auto store = [&](uint32_t arow, int8_t q, float s, int32_t sum, float wgt) {
        ws.actq[(size_t)arow * F + strip * 16 + r] = q;
        if (r == 0) {
            const float sf = s * wgt;
            ws.acts[(size_t)arow * nbf + strip] = sf;
            ws.actsum[(size_t)arow * nbf + strip] = sum;
            ws.actu[(size_t)arow * nbf + strip] = sf * (float)sum;
        }
    };
    if (decode) {
        if (gq != 0) return;
        const float hg = P == 2 ? acc[0] + acc[1] : acc[0], hv = P == 2 ? hu[0] + hu[1] : hu[0];
        const float x = silu512(hg) * hv;
        const uint32_t y = orow[0];
        const float wgt = y < ns ? wsel[y] : sigmoid_libm(ws.shl[0]);
        float s, res, s2, res2;
        int32_t sum, sum2;
        int8_t q, q2;
        quant16(x, s, sum, q, res);
        store(2 * y, q, s, sum, wgt);
        if (pair) {
            quant16(res, s2, sum2, q2, res2);
            store(2 * y + 1, q2, s2, sum2, wgt);
        }
        return;
    }
    for (int i = 0; i < 4; i++) {
        const uint32_t row = 4 * gq + i;
        const float x = silu512(acc[i]) * hu[i];
        float s, res;
        int32_t sum;
        int8_t q;
        quant16(x, s, sum, q, res);
        if (row < nr) {
            const uint32_t arow = orow[row];
            const float wgt = arow < n_ent ? ws.ent_w[arow] : sigmoid_libm(ws.shl[arow - n_ent]);
            store(arow, q, s, sum, wgt);
        }
    }
}

// Grid (ceil(F / 16 / 2), units), 256 threads: waves 2i, 2i + 1 = gate and up of strip
// 2 blockIdx.x + i.
template <int GK, int NJ, bool DEC>
__global__ __launch_bounds__(256) void tqm_gateup_kernel(TqmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t prow[2 * BR], orow[BR];
    constexpr uint32_t SC = GK == GK_TQ8 ? 4 : 2;  // floats per Sc entry
    const Workspace& ws = g.ws;
    const uint32_t tid = threadIdx.x, wv = tid / 64, l = tid % 64, H = ws.H, F = ws.F, nbf = F / 16;
    long* As = reinterpret_cast<long*>(smem);                     // [H / 32][64]
    float* Sc = reinterpret_cast<float*>(As + (size_t)(H / 32) * 64);  // [H / 32][16][SC]
    // decode: MassBasis::All's exponentials during the routing, then the up accumulators
    float* tail = Sc + (size_t)(H / 32) * 16 * SC;
    uint32_t ns = 0;
    const uint32_t* ids = ws.ids;
    const float* wsel = ws.w;
    if constexpr (NJ > 0) {
        // the decode routing on wave 0 (the others wait at the barrier)
        __shared__ uint2 cand[ROUTE_CAND];
        __shared__ uint32_t r_ids[K_MAX];
        __shared__ float r_w[K_MAX];
        __shared__ uint32_t r_n;
        if (wv == 0) {
            const uint32_t n = route_row<NJ>(g.lg, ws.E, g.k, g.pol, l, cand, tail, r_ids, r_w);
            if (l == 0) r_n = n;
        }
        __syncthreads();
        ns = r_n;
        ids = r_ids;
        wsel = r_w;
        if (blockIdx.x == 0 && blockIdx.y == 0) {  // for the down and combine launches, MoeStats
            if (tid < ns) {
                ws.ids[tid] = r_ids[tid];
                ws.w[tid] = r_w[tid];
            }
            if (tid == 0) {
                ws.n_sel[0] = ns;
                if (ws.stats) {
                    atomicAdd(&ws.stats[0], 1ull);
                    atomicAdd(&ws.stats[1], (unsigned long long)ns);
                }
            }
        }
    } else if (DEC) {
        ns = ws.n_sel[0];
    }
    bool shared;
    uint32_t e, nr, P;
    if (!tqm_unit(ws, true, DEC, g.pair, blockIdx.y, shared, e, nr, P, prow, orow, tid, ns, ids)) return;
    __syncthreads();
    tqm_stage<32, GK == GK_TQ8>(ws.xq, ws.xs, ws.xu, prow, nr * P, H, As, Sc, tid, 256);
    __syncthreads();
    const uint32_t gq = l / 16, r = l % 16, n_ent = ws.n_groups[1];
    const Mat& Ga = shared ? g.sha : g.a;
    const Mat& Ub = shared ? g.shb : g.b;
    if constexpr (!DEC) {
        // Batch: four strips per pass (strip pairs blockIdx.x and blockIdx.x + gridDim.x, then every
        // 2 gridDim.x further); a wave takes one strip, its gate and up rows as two chains over the
        // staged activations (tqm_strip2), and finishes it with SwiGLU itself, so no accumulators
        // cross waves and the LDS holds only the activations (three workgroups per CU at the real
        // shape)
        for (uint32_t sp = blockIdx.x; 2 * sp < F / 16; sp += 2 * gridDim.x) {
            const uint32_t strip = wv < 2 ? 2 * sp + wv : 2 * (sp + gridDim.x) + wv - 2;
            if (strip >= F / 16) continue;  // wave-uniform
            float acc[4], accu[4];
            tqm_strip2<GK, 32>(Ga.ptr + (size_t)e * Ga.stride + (size_t)strip * Ga.row_bytes,
                               Ub.ptr + (size_t)e * Ub.stride + (size_t)strip * Ub.row_bytes, H, As, Sc, l, acc, accu);
            tqm_swiglu_store(ws, 0, 0, P, nr, orow, n_ent, F, nbf, strip, gq, r, acc, accu, ns, wsel);
        }
    } else {
    // decode: waves 2i, 2i + 1 = gate and up of strip 2 blockIdx.x + i; the up wave hands its
    // accumulators over in LDS
    float (*hu)[64][4] = reinterpret_cast<float (*)[64][4]>(tail);  // [2 strips][64][4]
    const bool up = wv % 2 == 1;
    for (uint32_t sp = blockIdx.x; 2 * sp < F / 16; sp += gridDim.x) {
        const uint32_t strip = 2 * sp + wv / 2;
        const bool live = strip < F / 16;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (live) {
            const Mat& M = up ? Ub : Ga;
            tqm_strip<GK, 32, false>(M.ptr + (size_t)e * M.stride + (size_t)strip * M.row_bytes, H, As, Sc, l, acc);
        }
        if (up)
            for (int v = 0; v < 4; v++) hu[wv / 2][l][v] = acc[v];
        __syncthreads();
        if (!up && live) tqm_swiglu_store(ws, 1, g.pair, P, nr, orow, n_ent, F, nbf, strip, gq, r, acc,
                                          hu[wv / 2][l], ns, wsel);
        __syncthreads();  // hu read before the next pass writes it
    }
    }
}

// Grid (H / 64, units), 256 threads: wave w takes strip 4 blockIdx.x + w of H.
template <int GK, bool R1>
__global__ __launch_bounds__(256) void tqm_down_kernel(TqmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t prow[2 * BR], orow[BR];
    const Workspace& ws = g.ws;
    const uint32_t tid = threadIdx.x, wv = tid / 64, l = tid % 64, H = ws.H, F = ws.F;
    bool shared;
    uint32_t e, nr, P;
    if (!tqm_unit(ws, false, g.decode, g.pair, blockIdx.y, shared, e, nr, P, prow, orow, tid,
                  g.decode ? ws.n_sel[0] : 0u, ws.ids))
        return;
    long* As = reinterpret_cast<long*>(smem);                        // [F / 32][64]
    float* Sc = reinterpret_cast<float*>(As + (size_t)(F / 32) * 64);  // [F / 16][16][SC]
    __syncthreads();
    tqm_stage<16, GK == GK_TQ8>(ws.actq, ws.acts, ws.actu, prow, nr * P, F, As, Sc, tid, 256);
    __syncthreads();
    const Mat& M = shared ? g.sha : g.a;
    const uint32_t gq = l / 16, r = l % 16;
    // strip groups blockIdx.x, + gridDim.x, ...: the staged activations serve them all
    for (uint32_t sg = blockIdx.x; 4 * sg < H / 16; sg += gridDim.x) {
        const uint32_t strip = 4 * sg + wv;
        float acc[4];
        tqm_strip<GK, 16, R1>(M.ptr + (size_t)e * M.stride + (size_t)strip * M.row_bytes, F, As, Sc, l, acc);
        if (g.decode) {
            if (gq == 0) ws.yent[(size_t)orow[0] * H + strip * 16 + r] = P == 2 ? acc[0] + acc[1] : acc[0];
            continue;
        }
        for (int i = 0; i < 4; i++) {
            const uint32_t row = 4 * gq + i;
            if (row < nr) ws.yent[(size_t)orow[row] * H + strip * 16 + r] = acc[i];
        }
    }
}

// ---- decode from LDS copies of the strips ----------------------------------------------------
//
// A decode wave chains one strip over its whole K.  Reading the strip unit by unit from global
// memory keeps at most ~60 loads (about 15 units) in flight per wave, so a real-shape gate/up strip
// (80 units, 25.6 KB) arrives in several memory round trips.  These kernels instead copy each
// strip into LDS with 16-byte loads (25 per lane for that strip, all in flight), then run the same
// operands and chain (tqm_load / tqm_operand from the LDS copy).  Only the P <= 2 live activation
// rows are staged: As_c [unit][k group g][2] (8 bytes), Sc_c [block][2] (scale, u, byte sum); the
// A operand's other rows are zero.

constexpr uint32_t TQD_NLD = 32;  // 16-byte loads per lane in flight per copy pass (a real-shape strip: one)
constexpr uint32_t TQD_LDS_MAX = 160 * 1024;  // gfx950's LDS; above 64 KB the launch opts in
constexpr uint32_t TQD_GU_SPW = 1;             // gate/up strips per workgroup (two waves each)

// The wave's copy of n16 16-byte pieces from src to the LDS at dst, in passes of TQD_NLD loads per
// lane; the loads of a pass are unconditional at a clamped index, so they stay in registers and in
// flight together.  issue() requests the first pass, finish() stores it and runs the rest, so the
// caller can request other data in between.
template <uint32_t NLD = TQD_NLD>
struct TqdCopy {
    v4i v[NLD];
    __device__ __forceinline__ void issue(const uint8_t* __restrict__ src, uint32_t n16, uint32_t l) {
        const v4i* s4 = reinterpret_cast<const v4i*>(src);
#pragma unroll
        for (uint32_t c = 0; c < NLD; c++) {
            const uint32_t i = l + 64 * c;
            if (64 * c < n16) v[c] = s4[i < n16 ? i : n16 - 1];  // wave-uniform: only the pass's live loads
        }
    }
    __device__ __forceinline__ void finish(const uint8_t* __restrict__ src, uint8_t* dst, uint32_t n16, uint32_t l) {
        const v4i* s4 = reinterpret_cast<const v4i*>(src);
        v4i* d4 = reinterpret_cast<v4i*>(dst);
        const uint32_t last = n16 ? n16 - 1 : 0;
        for (uint32_t i0 = 0;; i0 += NLD * 64) {
#pragma unroll
            for (uint32_t c = 0; c < NLD; c++) {
                const uint32_t i = i0 + l + 64 * c;
                if (i < n16) d4[i] = v[c];
            }
            if (i0 + NLD * 64 >= n16) break;
#pragma unroll
            for (uint32_t c = 0; c < NLD; c++) {
                const uint32_t i = i0 + NLD * 64 + l + 64 * c;
                if (i0 + NLD * 64 + 64 * c < n16) v[c] = s4[i < n16 ? i : last];
            }
        }
    }
};

// Stage P <= 2 activation rows (q rows r0, r0 + 1, K bytes each; scales and u per KBS-block) as
// As_c / Sc_c (byte sums for the 8-bit codecs), rows past P zero.  Every load of a pass is issued
// before the first store (row r0 + 1 exists in every caller's buffer; its values are dropped when
// P = 1).
template <int KBS, bool XSUM>
__device__ __forceinline__ void tqd_stage(const int8_t* __restrict__ q, const float* __restrict__ s,
                                          const float* __restrict__ u, uint32_t r0, uint32_t P, uint32_t K,
                                          long* As_c, float* Sc_c, uint32_t tid, uint32_t nthr) {
    constexpr uint32_t SC = XSUM ? 4 : 2, PA = 12, PE = 4, NX = XSUM ? KBS / 16 : 1;
    const uint32_t npc = K / 8, nbs = K / KBS, nA = 2 * npc, nE = 2 * nbs;
    for (uint32_t pa = 0, pe = 0; pa < nA || pe < nE; pa += PA * nthr, pe += PE * nthr) {
        long va[PA];
        float vs[PE], vu[PE];
        int4 vq[PE][NX];
#pragma unroll
        for (uint32_t c = 0; c < PA; c++) {  // piece i: row i % 2, 8-byte piece i / 2 (= 4 unit + g)
            const uint32_t i = pa + tid + nthr * c, ic = i < nA ? i : nA - 1;
            va[c] = *reinterpret_cast<const long*>(q + (size_t)(r0 + ic % 2) * K + 8 * (ic / 2));
        }
#pragma unroll
        for (uint32_t c = 0; c < PE; c++) {  // entry i: row i % 2, block i / 2
            const uint32_t i = pe + tid + nthr * c, ic = i < nE ? i : nE - 1;
            const size_t bi = (size_t)(r0 + ic % 2) * nbs + ic / 2;
            vs[c] = s[bi];
            vu[c] = u[bi];
            if constexpr (XSUM) {
                const int4* xp = reinterpret_cast<const int4*>(q + (size_t)(r0 + ic % 2) * K + (size_t)KBS * (ic / 2));
#pragma unroll
                for (uint32_t t = 0; t < NX; t++) vq[c][t] = xp[t];
            }
        }
#pragma unroll
        for (uint32_t c = 0; c < PA; c++) {
            const uint32_t i = pa + tid + nthr * c;
            if (i < nA) As_c[i] = i % 2 < P ? va[c] : 0;
        }
#pragma unroll
        for (uint32_t c = 0; c < PE; c++) {
            const uint32_t i = pe + tid + nthr * c;
            if (i >= nE) continue;
            const bool live = i % 2 < P;
            float* e = Sc_c + i * SC;
            e[0] = live ? vs[c] : 0.0f;
            e[1] = live ? vu[c] : 0.0f;
            if constexpr (XSUM) {
                int xs = 0;
#pragma unroll
                for (uint32_t t = 0; t < NX; t++) {
                    xs = sdot4(vq[c][t].x, 0x01010101, xs);
                    xs = sdot4(vq[c][t].y, 0x01010101, xs);
                    xs = sdot4(vq[c][t].z, 0x01010101, xs);
                    xs = sdot4(vq[c][t].w, 0x01010101, xs);
                }
                e[2] = live ? __int_as_float(xs) : 0.0f;
            }
        }
    }
}

// The chain of one strip (an LDS copy) over K for the live rows v < P (lanes of group 0 hold
// them: D[row v][weight row r]).  Units go in groups of G: their LDS reads, then their MFMAs back
// to back, then their epilogues in unit order.
// FULL: nu a multiple of G (no partial group).  Every lane reads A row r % 2 (rows past P are
// zero in As_c; the output rows past 1 are not used).
template <int GK, int KB, bool FULL>
__device__ __forceinline__ void tqd_chain(const uint8_t* strip, uint32_t u0, uint32_t nu, const long* As_c,
                                          const float* Sc_c, uint32_t l, float (&acc)[4]) {
    constexpr bool U8 = GvTQ<GK, KB>::BITS == 8;
    constexpr uint32_t SC = U8 ? 4 : 2, NBL = TqmB<GK, KB>::NBL, G = 8;
    const uint32_t g = l / 16, r = l % 16;
    constexpr uint32_t UBB = NBL * GvTQ<GK, KB>::BB;  // bytes of a unit
    for (uint32_t b0 = u0; b0 < nu; b0 += G) {
        TqmB<GK, KB> w[G];
        long a[G];
        // the group's bases, so a unit's reads take immediate offsets
        const uint8_t* sg = strip + (size_t)b0 * UBB;
        const long* ag = As_c + 8 * b0 + 2 * g + (r & 1);
#pragma unroll
        for (uint32_t i = 0; i < G; i++) {
            const uint32_t bi = FULL || b0 + i < nu ? i : nu - 1 - b0;
            tqm_load<GK, KB>(w[i], sg, bi, l);
            a[i] = ag[8 * bi];
        }
        v4i d[G][NBL];
#pragma unroll
        for (uint32_t i = 0; i < G; i++) {
            const long bq = tqm_operand<GK, KB>(w[i], l);
#pragma unroll
            for (uint32_t hb = 0; hb < NBL; hb++)
                d[i][hb] = tqm_mfma(KB == 16 ? ((g / 2 == hb) ? a[i] : 0) : a[i], bq);
        }
        const float* scg = Sc_c + (size_t)b0 * NBL * 2 * SC;
#pragma unroll
        for (uint32_t i = 0; i < G; i++) {
            const uint32_t b = b0 + i;
            if (!FULL && b >= nu) break;
#pragma unroll
            for (uint32_t hb = 0; hb < NBL; hb++) {
                const float dd = h2f((uint16_t)w[i].d[hb]), mm = h2f((uint16_t)w[i].m[hb]);
#pragma unroll
                for (uint32_t v = 0; v < 2; v++) {
                    const float* sx = scg + ((NBL * i + hb) * 2 + v) * SC;
                    const int dot = U8 ? d[i][hb][v] + 128 * __float_as_int(sx[2]) : d[i][hb][v];
                    acc[v] = __builtin_fmaf(mm, sx[1], acc[v]);
                    acc[v] = __builtin_fmaf((float)dot, dd * sx[0], acc[v]);
                }
            }
        }
    }
}

// Units [u0, u1) of the chain (acc carried in).
template <int GK, int KB>
__device__ __forceinline__ void tqd_chain_any(const uint8_t* strip, uint32_t u0, uint32_t u1, const long* As_c,
                                              const float* Sc_c, uint32_t l, float (&acc)[4]) {
    if ((u1 - u0) % 8 == 0)
        tqd_chain<GK, KB, true>(strip, u0, u1, As_c, Sc_c, l, acc);
    else
        tqd_chain<GK, KB, false>(strip, u0, u1, As_c, Sc_c, l, acc);
}

// Copy a strip of n16 16-byte pieces (NLD = ceil(n16 / 64): every lane's loads unconditional, so
// each store waits for its own load only) and chain it from LDS, the first half of the passes'
// units while the second half is still arriving.  issue() requests the pieces; run() stores and
// chains.
template <int GK, int KB, uint32_t NLD>
struct TqdStream {
    v4i v[NLD];
    __device__ __forceinline__ void issue(const uint8_t* __restrict__ src, uint32_t n16, uint32_t l) {
        const v4i* s4 = reinterpret_cast<const v4i*>(src);
#pragma unroll
        for (uint32_t c = 0; c < NLD; c++) v[c] = s4[l + 64 * c < n16 ? l + 64 * c : n16 - 1];
    }
    __device__ __forceinline__ void run(uint8_t* my, uint32_t n16, uint32_t K, const long* As_c, const float* Sc_c,
                                        uint32_t l, float (&acc)[4]) {
        constexpr uint32_t UBB = TqmB<GK, KB>::NBL * GvTQ<GK, KB>::BB, H1 = (NLD + 1) / 2;
        v4i* d4 = reinterpret_cast<v4i*>(my);
#pragma unroll
        for (uint32_t c = 0; c < H1; c++)
            if (l + 64 * c < n16) d4[l + 64 * c] = v[c];
        const uint32_t nu = K / 32, done = 64 * H1 < n16 ? 64 * H1 : n16;
        uint32_t um = done * 16 / UBB;  // units wholly copied, then whole groups of 8
        um = (um < nu ? um : nu) / 8 * 8;
        for (int q = 0; q < 4; q++) acc[q] = 0.0f;
        tqd_chain_any<GK, KB>(my, 0, um, As_c, Sc_c, l, acc);
#pragma unroll
        for (uint32_t c = H1; c < NLD; c++)
            if (l + 64 * c < n16) d4[l + 64 * c] = v[c];
        tqd_chain_any<GK, KB>(my, um, nu, As_c, Sc_c, l, acc);
    }
};

// Single-pass staging (every thread at most one piece and one entry of each kind), split so the
// caller can issue other loads between the staging loads and stores.
template <int KBS, bool XSUM>
struct TqdStage1 {
    static constexpr uint32_t NX = XSUM ? KBS / 16 : 1;
    long va;
    float vs, vu;
    int4 vq[NX];
    __device__ __forceinline__ static bool fits(uint32_t K, uint32_t nthr) { return 2 * (K / 8) <= nthr; }
    __device__ __forceinline__ void load(const int8_t* __restrict__ q, const float* __restrict__ s,
                                         const float* __restrict__ u, uint32_t r0, uint32_t K, uint32_t tid) {
        const uint32_t nA = 2 * (K / 8), nbs = K / KBS, nE = 2 * nbs;
        const uint32_t ia = tid < nA ? tid : nA - 1, ie = tid < nE ? tid : nE - 1;
        va = *reinterpret_cast<const long*>(q + (size_t)(r0 + ia % 2) * K + 8 * (ia / 2));
        const size_t bi = (size_t)(r0 + ie % 2) * nbs + ie / 2;
        vs = s[bi];
        vu = u[bi];
        if constexpr (XSUM) {
            const int4* xp = reinterpret_cast<const int4*>(q + (size_t)(r0 + ie % 2) * K + (size_t)KBS * (ie / 2));
#pragma unroll
            for (uint32_t t = 0; t < NX; t++) vq[t] = xp[t];
        }
    }
    __device__ __forceinline__ void store(uint32_t P, uint32_t K, long* As_c, float* Sc_c, uint32_t tid) {
        constexpr uint32_t SC = XSUM ? 4 : 2;
        const uint32_t nA = 2 * (K / 8), nE = 2 * (K / KBS);
        if (tid < nA) As_c[tid] = tid % 2 < P ? va : 0;
        if (tid < nE) {
            const bool live = tid % 2 < P;
            float* e = Sc_c + tid * SC;
            e[0] = live ? vs : 0.0f;
            e[1] = live ? vu : 0.0f;
            if constexpr (XSUM) {
                int xs = 0;
#pragma unroll
                for (uint32_t t = 0; t < NX; t++) {
                    xs = sdot4(vq[t].x, 0x01010101, xs);
                    xs = sdot4(vq[t].y, 0x01010101, xs);
                    xs = sdot4(vq[t].z, 0x01010101, xs);
                    xs = sdot4(vq[t].w, 0x01010101, xs);
                }
                e[2] = live ? __int_as_float(xs) : 0.0f;
            }
        }
    }
};

struct TqdLds {
    uint32_t strips, as, sc, hu, route, total;
};
// gate/up (spw strips per workgroup): [2 spw strips][row_bytes], As_c, Sc_c, hu [spw][64][2], the
// routing scratch (+ E floats for MassBasis::All); down: [4 strips][row_bytes], As_c, Sc_c
__host__ __device__ inline TqdLds tqd_lds(bool gu, uint32_t row_bytes, uint32_t K, uint32_t kbs, bool u8, uint32_t ex,
                                          uint32_t spw = 1) {
    TqdLds o;
    o.strips = 0;
    o.as = (gu ? 2 * spw : 4) * row_bytes;
    o.sc = o.as + K / 8 * 2 * 8;
    o.hu = o.sc + K / kbs * 2 * (u8 ? 16 : 8);
    o.route = o.hu + (gu ? spw * 64 * 2 * 4 : 0);
    o.total = o.route + (gu ? ROUTE_CAND * 8 + K_MAX * 8 + 16 + ex : 0);
    o.total = (o.total + 15) / 16 * 16;
    return o;
}

// Token t's view of the workspace for a batch run as per-token decode units: its x row (single
// level), shared-gate logit, routing row and kcap + 1 activation slots of two rows each (the
// decode layout, the second row unused).  t = 0 is the decode layout itself.
__device__ __forceinline__ Workspace tqd_token(const Workspace& ws, uint32_t t, uint32_t kcap) {
    Workspace w = ws;
    const uint32_t nb = ws.H / 32, nbf = ws.F / 16;
    const size_t ar = (size_t)t * (kcap + 1) * 2;
    w.xq += (size_t)t * ws.H;
    w.xs += (size_t)t * nb;
    w.xsum += (size_t)t * nb;
    w.xu += (size_t)t * nb;
    w.shl += t;
    w.ids += (size_t)t * K_MAX;
    w.w += (size_t)t * K_MAX;
    w.n_sel += t;
    w.actq += ar * ws.F;
    w.acts += ar * nbf;
    w.actsum += ar * nbf;
    w.actu += ar * nbf;
    return w;
}

// Decode gate/up: grid (F / 16, kcap + 1, tokens), 128 threads; wave 0 the gate strip, wave 1 the up strip
// of strip blockIdx.x for slot blockIdx.y.  Wave 0 routes (route_row, router.rs:106-148) while
// wave 1 stages x; the shared expert's row (slot ns) copies its strips before routing.  Row
// blockIdx.y = kcap is the shared expert's when ns = kcap (fixed top-k); with fewer selected, the
// shared expert is row ns and the rows between are idle, as in the generic decode.
template <int GK, int NJ, int SPW>
__global__ __launch_bounds__(128 * SPW) void tqd_gateup_kernel(TqmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool U8 = GK == GK_TQ8;
    const Workspace ws = tqd_token(g.ws, blockIdx.z, gridDim.y - 1);  // token blockIdx.z's
    const float* lg = g.lg + (size_t)blockIdx.z * ws.E;
    const uint32_t tid = threadIdx.x, wv = tid / 64, l = tid % 64, H = ws.H, F = ws.F, nbf = F / 16;
    const uint32_t strip = SPW * blockIdx.x + wv / 2, y = blockIdx.y, P = g.pair ? 2u : 1u;
    const TqdLds L = tqd_lds(true, g.a.row_bytes, H, 32, U8,
                             g.pol.enabled && g.pol.basis == TRK_BASIS_ALL ? ws.E * 4 : 0, SPW);
    uint8_t* my = smem + wv * g.a.row_bytes;
    long* As_c = reinterpret_cast<long*>(smem + L.as);
    float* Sc_c = reinterpret_cast<float*>(smem + L.sc);
    float* hu = reinterpret_cast<float*>(smem + L.hu);
    uint2* cand = reinterpret_cast<uint2*>(smem + L.route);
    uint32_t* r_ids = reinterpret_cast<uint32_t*>(cand + ROUTE_CAND);
    float* r_w = reinterpret_cast<float*>(r_ids + K_MAX);
    uint32_t* r_n = reinterpret_cast<uint32_t*>(r_w + K_MAX);
    float* ex = reinterpret_cast<float*>(r_n + 4);
    const bool last = y == gridDim.y - 1;  // the shared expert's row when ns = kcap
    // this wave's stacks by value (a reference chosen at run time would put the arguments in
    // scratch memory): routed (gate or up) and shared
    const bool isup = wv % 2 == 1;
    const uint8_t* rptr = isup ? g.b.ptr : g.a.ptr;
    const uint64_t rstride = isup ? g.b.stride : g.a.stride;
    const uint8_t* sptr = (isup ? g.shb.ptr : g.sha.ptr) + (size_t)strip * g.a.row_bytes;
    const uint32_t n16 = g.a.row_bytes / 16;
    if (last) {  // the shared expert's strips need no routing: copied first
        TqdCopy<> cp;
        cp.issue(sptr, n16, l);
        cp.finish(sptr, my, n16, l);
    }
    if (wv == 0) {
        const uint32_t n = route_row<NJ>(lg, ws.E, g.k, g.pol, l, cand, ex, r_ids, r_w);
        if (l == 0) r_n[0] = n;
    } else {
        tqd_stage<32, U8>(ws.xq, ws.xs, ws.xu, 0, P, H, As_c, Sc_c, tid - 64, 128 * SPW - 64);
    }
    __syncthreads();
    const uint32_t ns = r_n[0];
    if (blockIdx.x == 0 && y == 0) {  // for the down and combine launches, MoeStats
        if (tid < ns) {
            ws.ids[tid] = r_ids[tid];
            ws.w[tid] = r_w[tid];
        }
        if (tid == 0) {
            ws.n_sel[0] = ns;
            if (ws.stats) {
                atomicAdd(&ws.stats[0], 1ull);
                atomicAdd(&ws.stats[1], (unsigned long long)ns);
            }
        }
    }
    // the unit: routed slot y < ns; the shared expert at row ns (the last row when ns = kcap)
    const bool shared = last ? ns == gridDim.y - 1 : y == ns;
    if (!shared && y >= ns) return;
    if (last && !shared) return;  // ns < kcap: the last row is idle; row ns runs the shared expert
    float acc[4];
    const uint8_t* src = shared ? sptr : rptr + (size_t)r_ids[y] * rstride + (size_t)strip * g.a.row_bytes;
    if (!last && (n16 + 63) / 64 == 25) {
        // the real shape's strip (25 passes): the chain starts on the first half while the rest arrives
        TqdStream<GK, 32, 25> sm;
        sm.issue(src, n16, l);
        sm.run(my, n16, H, As_c, Sc_c, l, acc);
    } else {
        if (!last) {
            TqdCopy<> cp;
            cp.issue(src, n16, l);
            cp.finish(src, my, n16, l);
        }
        for (int q = 0; q < 4; q++) acc[q] = 0.0f;
        tqd_chain_any<GK, 32>(my, 0, H / 32, As_c, Sc_c, l, acc);
    }
    float* hs = hu + (wv / 2) * 128;  // this strip's up accumulators
    if (wv % 2 == 1) {
        hs[2 * l] = acc[0];
        hs[2 * l + 1] = acc[1];
    }
    __syncthreads();
    if (wv % 2 == 0) {
        const uint32_t orow[1] = {shared ? ns : y};
        const float hv[4] = {hs[2 * l], hs[2 * l + 1], 0.0f, 0.0f};
        tqm_swiglu_store(ws, 1, g.pair, P, 1, orow, 0, F, nbf, strip, l / 16, l % 16, acc, hv, ns, r_w);
    }
}

// Decode down: grid (H / 64, kcap + 1), 256 threads; wave w the strip 4 blockIdx.x + w of H for
// slot blockIdx.y (the routing from the gate/up launch: ids, n_sel; the shared expert at row ns).
template <int GK>
__global__ __launch_bounds__(256) void tqd_down_kernel(TqmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool U8 = GK == GK_TQ8;
    const Workspace& ws = g.ws;
    const uint32_t tid = threadIdx.x, wv = tid / 64, l = tid % 64, H = ws.H, F = ws.F;
    const uint32_t y = blockIdx.y, strip = 4 * blockIdx.x + wv, P = g.pair ? 2u : 1u;
    const uint32_t ns = ws.n_sel[0], id = ws.ids[y < K_MAX ? y : 0];  // both requested at once
    if (y > ns) return;
    const bool shared = y == ns;
    const TqdLds L = tqd_lds(false, g.a.row_bytes, F, 16, U8, 0);
    uint8_t* my = smem + wv * g.a.row_bytes;
    long* As_c = reinterpret_cast<long*>(smem + L.as);
    float* Sc_c = reinterpret_cast<float*>(smem + L.sc);
    const uint8_t* src = (shared ? g.sha.ptr : g.a.ptr + (size_t)id * g.a.stride) + (size_t)strip * g.a.row_bytes;
    const uint32_t n16 = g.a.row_bytes / 16;
    float acc[4];
    if ((n16 + 63) / 64 == 9 && TqdStage1<16, U8>::fits(F, 256)) {
        // the real shape's strip (9 passes): the activations' loads, the strip's, the activations
        // stored (a wait for their own loads only), then the streamed copy and chain
        TqdStage1<16, U8> sg;
        sg.load(ws.actq, ws.acts, ws.actu, 2 * y, F, tid);
        TqdStream<GK, 16, 9> sm;
        sm.issue(src, n16, l);
        sg.store(P, F, As_c, Sc_c, tid);
        __syncthreads();
        sm.run(my, n16, F, As_c, Sc_c, l, acc);
    } else {
        TqdCopy<16> cp;  // a strip of up to 16 KB per pass
        cp.issue(src, n16, l);  // the weights first, then the activations (one round trip for both)
        tqd_stage<16, U8>(ws.actq, ws.acts, ws.actu, 2 * y, P, F, As_c, Sc_c, tid, 256);
        cp.finish(src, my, n16, l);
        __syncthreads();
        for (int q = 0; q < 4; q++) acc[q] = 0.0f;
        tqd_chain_any<GK, 16>(my, 0, F / 32, As_c, Sc_c, l, acc);
    }
    if (l < 16) ws.yent[(size_t)y * H + strip * 16 + l] = P == 2 ? acc[0] + acc[1] : acc[0];
}

// Staging of P <= 2 activation rows by one wave in a single pass (PA pieces and PE entries per
// lane at most), split so the caller can issue other loads between the loads and the stores.
template <int KBS, bool XSUM, uint32_t PA, uint32_t PE>
struct TqdStageW {
    static constexpr uint32_t NX = XSUM ? KBS / 16 : 1;
    long va[PA];
    float vs[PE], vu[PE];
    int4 vq[PE][NX];
    __host__ __device__ static bool fits(uint32_t K) { return 2 * (K / 8) <= PA * 64 && 2 * (K / KBS) <= PE * 64; }
    __device__ __forceinline__ void load(const int8_t* __restrict__ q, const float* __restrict__ s,
                                         const float* __restrict__ u, uint32_t r0, uint32_t K, uint32_t l) {
        const uint32_t nA = 2 * (K / 8), nbs = K / KBS, nE = 2 * nbs;
#pragma unroll
        for (uint32_t c = 0; c < PA; c++) {
            const uint32_t i = l + 64 * c, ic = i < nA ? i : nA - 1;
            va[c] = *reinterpret_cast<const long*>(q + (size_t)(r0 + ic % 2) * K + 8 * (ic / 2));
        }
#pragma unroll
        for (uint32_t c = 0; c < PE; c++) {
            const uint32_t i = l + 64 * c, ic = i < nE ? i : nE - 1;
            const size_t bi = (size_t)(r0 + ic % 2) * nbs + ic / 2;
            vs[c] = s[bi];
            vu[c] = u[bi];
            if constexpr (XSUM) {
                const int4* xp = reinterpret_cast<const int4*>(q + (size_t)(r0 + ic % 2) * K + (size_t)KBS * (ic / 2));
#pragma unroll
                for (uint32_t t = 0; t < NX; t++) vq[c][t] = xp[t];
            }
        }
    }
    __device__ __forceinline__ void store(uint32_t P, uint32_t K, long* As_c, float* Sc_c, uint32_t l) {
        constexpr uint32_t SC = XSUM ? 4 : 2;
        const uint32_t nA = 2 * (K / 8), nE = 2 * (K / KBS);
#pragma unroll
        for (uint32_t c = 0; c < PA; c++) {
            const uint32_t i = l + 64 * c;
            if (i < nA) As_c[i] = i % 2 < P ? va[c] : 0;
        }
#pragma unroll
        for (uint32_t c = 0; c < PE; c++) {
            const uint32_t i = l + 64 * c;
            if (i >= nE) continue;
            const bool live = i % 2 < P;
            float* e = Sc_c + i * SC;
            e[0] = live ? vs[c] : 0.0f;
            e[1] = live ? vu[c] : 0.0f;
            if constexpr (XSUM) {
                int xs = 0;
#pragma unroll
                for (uint32_t t = 0; t < NX; t++) {
                    xs = sdot4(vq[c][t].x, 0x01010101, xs);
                    xs = sdot4(vq[c][t].y, 0x01010101, xs);
                    xs = sdot4(vq[c][t].z, 0x01010101, xs);
                    xs = sdot4(vq[c][t].w, 0x01010101, xs);
                }
                e[2] = live ? __int_as_float(xs) : 0.0f;
            }
        }
    }
};

// LDS of the fused decode down: nw strips, per wave its activations (As_c, Sc_c), the slots' rows,
// the slots in expert order (batch order)
__host__ __device__ inline size_t tqd_dc_lds(uint32_t nw, uint32_t row_bytes, uint32_t F, bool u8) {
    return (size_t)nw * row_bytes + (size_t)nw * (F / 8 * 2 * 8 + F / 16 * 2 * (u8 ? 16 : 8)) + (size_t)nw * 16 * 4 +
           K_MAX * 4;
}

// Decode down and combine in one launch: grid (H / 16, tokens), 64 (kcap + 1) threads.  Wave y
// chains strip blockIdx.x of H for slot y (the routed expert y < ns, the shared expert at y = ns:
// the routing of the gate/up launch), from a streamed LDS copy; then the strip's 16 outputs are the
// slots' rows added in slot order from slot 0, shared last (exec.rs:1610-1621), or for a batch run
// as per-token decodes (border) in the batch combine's order, the shared row first, then the
// token's entries by ascending expert (exec_batch.rs:1539-1578); plus out when residual.  This
// replaces the per-slot rows in yent and the combine launch.
template <int GK>
__global__ __launch_bounds__(1024) void tqd_down_combine_kernel(TqmArgs g, float* __restrict__ out, int residual,
                                                               int border) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool U8 = GK == GK_TQ8;
    constexpr uint32_t SC = U8 ? 4 : 2;
    const uint32_t tid = threadIdx.x, y = tid / 64, l = tid % 64, nw = blockDim.x / 64;
    const Workspace ws = tqd_token(g.ws, blockIdx.y, nw - 1);  // token blockIdx.y's
    out += (size_t)blockIdx.y * ws.H;
    const uint32_t F = ws.F, strip = blockIdx.x, P = g.pair ? 2u : 1u, rb = g.a.row_bytes;
    const uint32_t ns = ws.n_sel[0], id = ws.ids[y < K_MAX ? y : 0];  // both requested at once
    uint8_t* my = smem + (size_t)y * rb;
    const size_t act = (size_t)F / 8 * 2 * 8 + (size_t)F / 16 * 2 * SC * 4;
    long* As_c = reinterpret_cast<long*>(smem + (size_t)nw * rb + y * act);
    float* Sc_c = reinterpret_cast<float*>(smem + (size_t)nw * rb + y * act + (size_t)F / 8 * 2 * 8);
    float* res = reinterpret_cast<float*>(smem + (size_t)nw * (rb + act));
    uint32_t* perm = reinterpret_cast<uint32_t*>(res + nw * 16);  // [K_MAX] border: slots by expert
    if (border && y < ns && l == 0) {  // the token's experts are distinct: rank = how many are smaller
        uint32_t rank = 0;
        for (uint32_t j = 0; j < ns; j++) rank += ws.ids[j] < id ? 1u : 0u;
        perm[rank] = y;
    }
    if (y <= ns) {  // wave-uniform
        const uint8_t* src = (y == ns ? g.sha.ptr : g.a.ptr + (size_t)id * g.a.stride) + (size_t)strip * rb;
        const uint32_t n16 = rb / 16;
        float acc[4];
        // the activations' loads, the strip's, the activations stored, then the streamed chain
        TqdStageW<16, U8, 4, 2> sg;
        sg.load(ws.actq, ws.acts, ws.actu, 2 * y, F, l);
        TqdStream<GK, 16, 9> sm;
        sm.issue(src, n16, l);
        sg.store(P, F, As_c, Sc_c, l);
        sm.run(my, n16, F, As_c, Sc_c, l, acc);
        if (l < 16) res[y * 16 + l] = P == 2 ? acc[0] + acc[1] : acc[0];
    }
    __syncthreads();
    if (tid < 16) {
        float p;
        if (border) {
            p = res[ns * 16 + tid];
            for (uint32_t j = 0; j < ns; j++) p = p + res[perm[j] * 16 + tid];
        } else {
            p = res[tid];
            for (uint32_t s = 1; s <= ns; s++) p = p + res[s * 16 + tid];
        }
        float* o = out + (size_t)strip * 16 + tid;
        *o = residual ? *o + p : p;
    }
}

bool tqd_dc_ok(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t kcap) {
    const uint32_t F = ws.F, rb = down.row_bytes;
    auto al = [](const Mat& m) {
        return ((uintptr_t)m.ptr % 16 == 0) && m.stride % 16 == 0 && m.row_bytes % 16 == 0 && m.tile_stride == 0;
    };
    return tq_kb(down.fmt) == 16 && ws.tiles == 1 && al(down) && al(sh_down) && rb == sh_down.row_bytes &&
           (rb / 16 + 63) / 64 == 9 && TqdStageW<16, false, 4, 2>::fits(F) && kcap + 1 <= 16 && ws.H % 16 == 0 &&
           tqd_dc_lds(kcap + 1, rb, F, tq_bits(down.fmt) == 8) <= TQD_LDS_MAX;
}

hipError_t launch_tqd_down_combine(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t kcap, int pair,
                                   float* out, int residual, hipStream_t st, uint32_t m) {
    if (!tqd_dc_ok(down, sh_down, ws, kcap) || (m > 1 && (pair || !tqd_tokens_fit(ws, m, kcap))))
        return hipErrorInvalidValue;
    const TqmArgs a{down, down, sh_down, sh_down, ws, 1, pair, nullptr, 0, Policy{}};
    const uint32_t nw = kcap + 1;
    const size_t lds = tqd_dc_lds(nw, down.row_bytes, ws.F, tq_bits(down.fmt) == 8);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024) {
            const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        kern<<<dim3(ws.H / 16, m), 64 * nw, lds, st>>>(a, out, residual, m > 1 ? 1 : 0);
        return hipGetLastError();
    };
    switch (tq_bits(down.fmt)) {
        case 4: return go(tqd_down_combine_kernel<GK_TQ4>);
        case 5: return go(tqd_down_combine_kernel<GK_TQ5>);
        case 8: return go(tqd_down_combine_kernel<GK_TQ8>);
        default: return hipErrorInvalidValue;
    }
}

// The LDS decode kernels' shape conditions: 16-byte aligned strips and LDS within the limit.
static bool tqd_ok(const Mat& a, const Mat& b, const Mat& sa, const Mat& sb, size_t lds) {
    auto al = [](const Mat& m) {
        return ((uintptr_t)m.ptr % 16 == 0) && m.stride % 16 == 0 && m.row_bytes % 16 == 0 && m.tile_stride == 0;
    };
    return al(a) && al(b) && al(sa) && al(sb) && lds <= TQD_LDS_MAX;
}

bool tqd_gateup_ok(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const Workspace& ws,
                   const Policy& pol) {
    const uint32_t ex = pol.enabled && pol.basis == TRK_BASIS_ALL ? ws.E * 4 : 0;
    constexpr uint32_t SPW = TQD_GU_SPW;
    const size_t lds = tqd_lds(true, gate.row_bytes, ws.H, 32, tq_bits(gate.fmt) == 8, ex, SPW).total;
    return tq_kb(gate.fmt) == 32 && ws.H % 32 == 0 && tqd_ok(gate, up, sh_gate, sh_up, lds) &&
           gate.row_bytes == up.row_bytes && gate.row_bytes == sh_gate.row_bytes &&
           gate.row_bytes == sh_up.row_bytes && (ws.F / 16) % SPW == 0;
}

bool tqd_tokens_fit(const Workspace& ws, uint32_t m, uint32_t kcap) {
    return m <= ws.m_max && (uint64_t)m * (kcap + 1) * 2 <= ws.act_rows && ws.tiles == 1;
}

hipError_t launch_tqm_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const Workspace& ws,
                             uint32_t m, uint32_t kcap, int pair, const float* lg, uint32_t k, Policy pol,
                             hipStream_t st) {
    if (tq_kb(gate.fmt) != 32 || ws.H % 32) return hipErrorInvalidValue;
    // tokens: a batch of m rows as per-token decodes (grid z), routing inside, single-level
    const bool tokens = m > 1 && lg;
    if (tokens && (pair || !tqd_gateup_ok(gate, up, sh_gate, sh_up, ws, pol) || !tqd_tokens_fit(ws, m, kcap)))
        return hipErrorInvalidValue;
    const bool dec = m == 1 || tokens;
    const TqmArgs a{gate, up, sh_gate, sh_up, ws, dec ? 1 : 0, m == 1 && pair ? 1 : 0, lg, k, pol};
    const int nj = dec && lg ? (int)route_nj(ws.E) : 0;  // decode: routing inside
    // decode: a workgroup per strip pair; batch: a workgroup per TQM_PAIRS strip pairs of an item,
    // looping over them with the item's activations staged once (5 or 2 pairs per workgroup at the
    // real shape: 478 / 484 us against 460 for 4)
    if (dec && nj) {  // decode from LDS copies of the strips where they fit
        const uint32_t ex = pol.enabled && pol.basis == TRK_BASIS_ALL ? ws.E * 4 : 0;
        constexpr uint32_t SPW = TQD_GU_SPW;
        const size_t lds = tqd_lds(true, gate.row_bytes, ws.H, 32, tq_bits(gate.fmt) == 8, ex, SPW).total;
        if (tqd_gateup_ok(gate, up, sh_gate, sh_up, ws, pol)) {
            const dim3 grid(ws.F / 16 / SPW, kcap + 1, m);
            auto go = [&](auto kern) {
                if (lds > 64 * 1024) {
                    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                    if (e != hipSuccess) return e;
                }
                kern<<<grid, 128 * SPW, lds, st>>>(a);
                return hipGetLastError();
            };
            switch (tq_bits(gate.fmt) * 100 + nj) {
                case 408: return go(tqd_gateup_kernel<GK_TQ4, 8, SPW>);
                case 416: return go(tqd_gateup_kernel<GK_TQ4, 16, SPW>);
                case 508: return go(tqd_gateup_kernel<GK_TQ5, 8, SPW>);
                case 516: return go(tqd_gateup_kernel<GK_TQ5, 16, SPW>);
                case 808: return go(tqd_gateup_kernel<GK_TQ8, 8, SPW>);
                case 816: return go(tqd_gateup_kernel<GK_TQ8, 16, SPW>);
                default: return hipErrorInvalidValue;
            }
        }
    }
    const uint32_t pairs = (ws.F / 16 + 1) / 2;
    const dim3 grid(m == 1 ? pairs : (pairs + TQM_PAIRS - 1) / TQM_PAIRS, m == 1 ? kcap + 1 : grouped_item_rows(ws, m));
    const size_t sc = tq_bits(gate.fmt) == 8 ? 16 : 8;  // bytes per Sc entry
    size_t lds = (size_t)(ws.H / 32) * 64 * 8 + (size_t)(ws.H / 32) * 16 * sc;
    if (m == 1) {  // decode: the up accumulators of two strips; route_row's exponentials before them
        const size_t ex = nj && pol.enabled && pol.basis == TRK_BASIS_ALL ? (size_t)ws.E * 4 : 0;
        lds += ex > 2 * 64 * 4 * 4 ? ex : 2 * 64 * 4 * 4;
    }
    switch (tq_bits(gate.fmt) * 100 + nj + (m == 1 ? 1 : 0)) {
#define TQM_GU(b, gk)                                                                       \
    case b * 100: tqm_gateup_kernel<gk, 0, false><<<grid, 256, lds, st>>>(a); break;        \
    case b * 100 + 1: tqm_gateup_kernel<gk, 0, true><<<grid, 256, lds, st>>>(a); break;     \
    case b * 100 + 8 + 1: tqm_gateup_kernel<gk, 8, true><<<grid, 256, lds, st>>>(a); break; \
    case b * 100 + 16 + 1: tqm_gateup_kernel<gk, 16, true><<<grid, 256, lds, st>>>(a); break;
        TQM_GU(4, GK_TQ4) TQM_GU(5, GK_TQ5) TQM_GU(8, GK_TQ8)
#undef TQM_GU
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_tqm_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m, uint32_t kcap, int pair,
                           hipStream_t st) {
    if (tq_kb(down.fmt) != 16 || ws.F % 32 || ws.H % 64) return hipErrorInvalidValue;
    const TqmArgs a{down, down, sh_down, sh_down, ws, m == 1 ? 1 : 0, m == 1 && pair ? 1 : 0, nullptr, 0, Policy{}};
    if (m == 1) {  // decode from LDS copies of the strips where they fit
        const size_t lds = tqd_lds(false, down.row_bytes, ws.F, 16, tq_bits(down.fmt) == 8, 0).total;
        if (tqd_ok(down, down, sh_down, sh_down, lds) && down.row_bytes == sh_down.row_bytes) {
            const dim3 grid(ws.H / 64, kcap + 1);
            switch (tq_bits(down.fmt)) {
                case 4: tqd_down_kernel<GK_TQ4><<<grid, 256, lds, st>>>(a); break;
                case 5: tqd_down_kernel<GK_TQ5><<<grid, 256, lds, st>>>(a); break;
                case 8: tqd_down_kernel<GK_TQ8><<<grid, 256, lds, st>>>(a); break;
                default: return hipErrorInvalidValue;
            }
            return hipGetLastError();
        }
    }
    // decode: a workgroup per strip group; batch: per four strip groups of an item (each wave walks
    // four strips), so an item's activations are staged once per 256 output rows rather than per
    // 64 (real shape M = 512: 343 -> 301 us; per 128 rows 315, per 512 320)
    const uint32_t sg = m == 1 || (ws.H / 64) % 4 ? 1u : 4u;
    const dim3 grid(ws.H / 64 / sg, m == 1 ? kcap + 1 : grouped_item_rows(ws, m));
    const size_t lds = (size_t)(ws.F / 32) * 64 * 8 + (size_t)(ws.F / 16) * 16 * 16;
    // the batch kernels with the rank-1 MFMA epilogue, decode with the VALU one
    switch (tq_bits(down.fmt) * 2 + (m == 1 ? 0 : 1)) {
        case 8: tqm_down_kernel<GK_TQ4, false><<<grid, 256, lds, st>>>(a); break;
        case 9: tqm_down_kernel<GK_TQ4, true><<<grid, 256, lds, st>>>(a); break;
        case 10: tqm_down_kernel<GK_TQ5, false><<<grid, 256, lds, st>>>(a); break;
        case 11: tqm_down_kernel<GK_TQ5, true><<<grid, 256, lds, st>>>(a); break;
        case 16: tqm_down_kernel<GK_TQ8, false><<<grid, 256, lds, st>>>(a); break;
        case 17: tqm_down_kernel<GK_TQ8, true><<<grid, 256, lds, st>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}


// ---- hyper-connection mix, part B (the MoE layer's input stage) ----------------------------
//
// mixed [m][hh] from the normed streams xn [m][hc][hh] and the low-rank projection lo [m][lr]:
//   decode (m = 1, exec.rs:1196-1234): l = silu(lo / hc) (scalar silu), quantised per 32, in
//     pairs with hiprec; g = sigmoid(up . q) (scalar sigmoid); mixed[c] = (sum_s xn_s[c] g_s[c],
//     from 0, multiply then add) * (1 / hc)
//   batch (exec_batch.rs:929-968): l = silu(lo * (1 / hc)) (silu512 on 16-blocks), quantised per
//     32; g = sigmoid512(up . q); mixed = xn_0 g_0, then fma(xn_s, g_s, .) for s >= 1, then * (1/hc)
// The up rows s hh + c of the hc streams for a column c form one 16-row strip per stream, so a
// workgroup owns 16 columns c0 .. c0 + 15 and runs a wave per stream: wave s chains strip
// (s hh + c0) / 16 over the lr / 32 blocks in order (gemv.rs:141-148) with one MFMA per block and
// token tile, the q rows as the A operand (the expert products' layout above).  The batch rows are
// quantised once by hc_quant_kernel into the operand image below; decode quantises its one row
// inside every workgroup while the strip's weights are in flight.
constexpr uint32_t HC_MAXLR = 1024;  // most low-rank width

// The operand image of a tile of nr <= 16 tokens (nr = 16 but for a ragged last tile), 44 nu nr
// bytes for nu = lr / 32 blocks:
//   As [nu][4][nr]  8 bytes: q of (block b, k group g, token row): the MFMA's A operand
//   SU [nu][nr]     float2: the block's (scale, u = scale * sum) per token row
//   XC [nu][nr]     int: 128 x the block's byte sum (the 8-bit codecs' accumulator input)
// A full tile's image is the LDS image hc_mix_kernel chains from, so a workgroup stages its full
// tiles with one contiguous copy; tiles are 704 nu bytes apart in the batch's image.
__host__ __device__ constexpr uint32_t hc_img_as(uint32_t nu, uint32_t nr) { return 0; }
__host__ __device__ constexpr uint32_t hc_img_su(uint32_t nu, uint32_t nr) { return 32 * nu * nr; }
__host__ __device__ constexpr uint32_t hc_img_xc(uint32_t nu, uint32_t nr) { return 40 * nu * nr; }
__host__ __device__ constexpr uint32_t hc_img_tile(uint32_t nu) { return 704 * nu; }

struct HcArgs {
    Mat up;  // TQ [hc * hh][lr], kb 32
    const float* xn;
    const float* lo;
    const uint8_t* img;  // batch: the quantised rows' operand image (hc_quant_kernel)
    float* mixed;
    uint32_t hc, hh, lr, m;
    int pair;
};

// batch: silu(lo * (1 / hc)) of every row quantised per 32, once, into the operand image.  A
// thread per value and a half-wave per block (lr % 32 == 0: a block is 32 consecutive values of
// one row): the lanes reduce the block's |max| and sums with xor shuffles (max and integer sums:
// any order gives quant_block_regs' values for finite input), stage their q bytes in LDS, and
// four lanes write the block's 8-byte operand pieces.
__global__ __launch_bounds__(256) void hc_quant_kernel(const float* __restrict__ lo, uint32_t m, uint32_t lr,
                                                       uint32_t hc, uint8_t* __restrict__ img) {
    __shared__ __align__(16) int8_t qs[8][32];
    const uint32_t tid = threadIdx.x, j = blockIdx.x * 256u + tid, n = m * lr, k = tid % 32, hb = tid / 32;
    const bool live = j < n;  // a whole half-wave in or out
    const float inv = 1.0f / (float)hc;
    const uint32_t body = lr / 16 * 16;
    float x = 0.0f;
    if (live) {
        const float y = lo[j] * inv;
        x = j % lr < body ? silu512(y) : y * sigmoid_libm(y);
    }
    float amax = __builtin_fabsf(x);
#pragma unroll
    for (int o = 16; o >= 1; o /= 2) amax = mx_ps(amax, __shfl_xor(amax, o, 32));
    const float sc = amax / 127.0f;
    const float qinv = amax > 0.0f ? 127.0f / amax : 0.0f;
    const int32_t qi = cvt_rne(x * qinv);
    const int8_t qb = sat_i8(qi);
    int sum = qi, bs = qb;
#pragma unroll
    for (int o = 16; o >= 1; o /= 2) {
        sum += __shfl_xor(sum, o, 32);
        bs += __shfl_xor(bs, o, 32);
    }
    qs[hb][k] = qb;
    __syncthreads();
    if (!live || k >= 6) return;
    const uint32_t nu = lr / 32, bl = j / 32, tok = bl / nu, b = bl % nu, t = tok / 16, row = tok % 16;
    const uint32_t nr = m - 16 * t < 16 ? m - 16 * t : 16;
    uint8_t* ti = img + (size_t)t * hc_img_tile(nu);
    if (k < 4)
        reinterpret_cast<long*>(ti + hc_img_as(nu, nr))[(4 * b + k) * nr + row] =
            *reinterpret_cast<const long*>(&qs[hb][8 * k]);
    else if (k == 4)
        reinterpret_cast<float2*>(ti + hc_img_su(nu, nr))[b * nr + row] = make_float2(sc, sc * (float)sum);
    else
        reinterpret_cast<int*>(ti + hc_img_xc(nu, nr))[b * nr + row] = 128 * bs;
}

// LDS of hc_mix_kernel: NT tile images (16 rows each), reused for the mix's xn values [TT][hc][16]
// once the chains are done; the gates [hc][TT][16].
struct HcLds {
    size_t gate, total;
};
__host__ __device__ inline HcLds hc_lds(uint32_t nt, uint32_t nu, uint32_t hc) {
    HcLds o;
    const size_t ops = (size_t)nt * hc_img_tile(nu), xs = (size_t)16 * nt * hc * 16 * 4;
    o.gate = ops > xs ? ops : xs;
    o.total = o.gate + (size_t)hc * 16 * nt * 16 * 4;
    return o;
}

constexpr uint32_t HC_PC = 8;  // batch staging: 16-byte pieces per thread per pass (real shape: one pass)

// Grid (hh / 16, ceil(m / (16 NT))), 64 hc threads.  NT token tiles of 16 per workgroup share each
// weight unit: a unit's B operand feeds NT MFMAs, one per tile.  The first loads issued are the
// ones the first wait needs (batch: the tile images; decode: the lo row), then the strip's weights
// and the mix's xn values, so their latency runs under the staging (or the quantisation).  The
// block's f32 terms run as rank-1 MFMAs (rank1: fma(m, u, acc) and d * sx, the same bits), the
// 8-bit codecs' + 128 x byte-sum correction as the integer MFMA's accumulator input, leaving the
// VALU a conversion and one fma per output and block.
template <int GK, int NT, bool DEC>
__global__ __launch_bounds__(512) void hc_mix_kernel(HcArgs g) {
    using B = TqmB<GK, 32>;
    constexpr bool U8 = GvTQ<GK, 32>::BITS == 8;
    constexpr uint32_t TT = 16 * NT;  // tokens per workgroup
    constexpr uint32_t J = TT / 4;    // xn values per thread: TT hc 16 over 64 hc threads
    // units in flight: about 64 VGPRs of raw words
    constexpr uint32_t UB = 64 / B::REGS < 16 ? 64 / B::REGS : 16;
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t tid = threadIdx.x, nthr = blockDim.x, wv = tid / 64, l = tid % 64, gq = l / 16, r = l % 16;
    const uint32_t nu = g.lr / 32, c0 = blockIdx.x * 16, t0 = blockIdx.y * TT;
    const uint32_t nt = g.m - t0 < TT ? g.m - t0 : TT, ntl = (nt + 15) / 16;  // live tokens, tiles
    const HcLds L = hc_lds(NT, nu, g.hc);
    const uint32_t tile = hc_img_tile(nu), oSU = hc_img_su(nu, 16), oXC = hc_img_xc(nu, 16);
    float* xs = reinterpret_cast<float*>(smem);  // over the tile images after the chains
    float* gate = reinterpret_cast<float*>(smem + L.gate);
    const uint8_t* strip = g.up.ptr + (size_t)((wv * g.hh + c0) / 16) * g.up.row_bytes;
    B w[UB];
    float xv[DEC ? 1 : J];
    // the strip's first UB units; batch: xn (token tx + 4 j, stream sx / 16, column sx % 16) of the
    // workgroup's [TT][hc][16], a 64-byte run per 16 threads; decode: lane r < 16 of wave s holds xn
    // (s, c0 + r)
    auto issue_rest = [&]() {
#pragma unroll
        for (uint32_t i = 0; i < UB; i++)
            if (i < nu) tqm_load<GK, 32>(w[i], strip, i, l);
        if constexpr (DEC) {
            xv[0] = l < 16 ? g.xn[(size_t)wv * g.hh + c0 + l] : 0.0f;
        } else {
            const uint32_t tx = tid / (16 * g.hc), sx = tid % (16 * g.hc);
            const float* xp = g.xn + ((size_t)(t0 + tx) * g.hc + sx / 16) * g.hh + c0 + sx % 16;
            const size_t step = (size_t)4 * g.hc * g.hh;
#pragma unroll
            for (uint32_t j = 0; j < J; j++) xv[j] = tx + 4 * j < nt ? xp[step * j] : 0.0f;
        }
    };
    if constexpr (DEC) {
        // the one row's silu(lo / hc) and its per-32 quantisation (two levels with hiprec), a
        // value per lane: block b = j / 32 of value j = tid + nthr c is a half-wave, whose lanes
        // reduce the block's |max| and sums with xor shuffles (max and integer sums: any order
        // gives quant_block_regs' values for finite input) and write their q bytes in the 16-row
        // tile image, level lv as A row lv
        long* As = reinterpret_cast<long*>(smem);
        int8_t* Ab = reinterpret_cast<int8_t*>(smem);
        float2* SU = reinterpret_cast<float2*>(smem + oSU);
        int* XC = reinterpret_cast<int*>(smem + oXC);
        const uint32_t P = g.pair ? 2u : 1u;
        constexpr uint32_t NL = HC_MAXLR / 64;  // lo values per thread at most (64 threads)
        float lv[NL];
#pragma unroll
        for (uint32_t c = 0; c < NL; c++) {
            const uint32_t j = tid + nthr * c;
            lv[c] = j < g.lr ? g.lo[j] : 0.0f;
        }
        issue_rest();
        for (uint32_t i = tid; i < nu * 64; i += nthr)
            if (i % 16 >= P) As[i] = 0;
        for (uint32_t i = tid; i < nu * 16; i += nthr)
            if (i % 16 >= P) {
                SU[i] = make_float2(0.0f, 0.0f);
                XC[i] = 0;
            }
        const uint32_t k = tid % 32;  // the value's index in its block
#pragma unroll
        for (uint32_t c = 0; c < NL; c++) {
            const uint32_t j = tid + nthr * c, b = j / 32;
            if (j < g.lr) {  // a whole half-wave in or out (lr % 32 == 0)
                const float y = lv[c] / (float)g.hc;
                float x = y * sigmoid_libm(y);
                for (uint32_t lev = 0; lev < P; lev++) {
                    float amax = __builtin_fabsf(x);
#pragma unroll
                    for (int o = 16; o >= 1; o /= 2) amax = mx_ps(amax, __shfl_xor(amax, o, 32));
                    const float sc = amax / 127.0f;
                    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
                    const int32_t qi = cvt_rne(x * inv);
                    const int8_t qb = sat_i8(qi);
                    int sum = qi, bs = qb;
#pragma unroll
                    for (int o = 16; o >= 1; o /= 2) {
                        sum += __shfl_xor(sum, o, 32);
                        bs += __shfl_xor(bs, o, 32);
                    }
                    Ab[((b * 4 + k / 8) * 16 + lev) * 8 + k % 8] = qb;
                    if (k == 0) {
                        SU[b * 16 + lev] = make_float2(sc, sc * (float)sum);
                        XC[b * 16 + lev] = U8 ? 128 * bs : 0;
                    }
                    x = __builtin_fmaf(-(float)qi, sc, x);  // the residual, the second level's input
                }
            }
        }
    } else {
        // the full tiles: one contiguous copy of their images; a ragged last tile (nr < 16 rows,
        // compact in the batch image) spread to 16 rows with the rows past nr zero
        const uint32_t full = nt / 16, nr = nt % 16, nch = full * tile / 16;
        // (the loads unconditional at a clamped index, into a register vector: a conditional load
        // into an array of structs went to scratch memory, each behind its own wait)
        const v4i* src = reinterpret_cast<const v4i*>(g.img + (size_t)(t0 / 16) * tile);
        v4i* dst = reinterpret_cast<v4i*>(smem);
        const uint32_t last = nch ? nch - 1 : 0;
        v4i v[HC_PC];
#pragma unroll
        for (uint32_t c = 0; c < HC_PC; c++) {
            const uint32_t k = tid + nthr * c;
            v[c] = src[k < nch ? k : last];
        }
        issue_rest();
#pragma unroll
        for (uint32_t c = 0; c < HC_PC; c++) {
            const uint32_t k = tid + nthr * c;
            if (k < nch) dst[k] = v[c];
        }
        for (uint32_t k0 = HC_PC * nthr; k0 < nch; k0 += HC_PC * nthr) {
#pragma unroll
            for (uint32_t c = 0; c < HC_PC; c++) {
                const uint32_t k = k0 + tid + nthr * c;
                v[c] = src[k < nch ? k : last];
            }
#pragma unroll
            for (uint32_t c = 0; c < HC_PC; c++) {
                const uint32_t k = k0 + tid + nthr * c;
                if (k < nch) dst[k] = v[c];
            }
        }
        if (nr) {
            const uint8_t* ti = g.img + (size_t)(t0 / 16 + full) * tile;
            const long* sA = reinterpret_cast<const long*>(ti + hc_img_as(nu, nr));
            const float2* sS = reinterpret_cast<const float2*>(ti + hc_img_su(nu, nr));
            const int* sX = reinterpret_cast<const int*>(ti + hc_img_xc(nu, nr));
            uint8_t* di = smem + (size_t)full * tile;
            long* As = reinterpret_cast<long*>(di);
            float2* SU = reinterpret_cast<float2*>(di + oSU);
            int* XC = reinterpret_cast<int*>(di + oXC);
            for (uint32_t p = tid; p < nu * 64; p += nthr) As[p] = p % 16 < nr ? sA[(p / 16) * nr + p % 16] : 0;
            for (uint32_t p = tid; p < nu * 16; p += nthr) {
                const bool live = p % 16 < nr;
                SU[p] = live ? sS[(p / 16) * nr + p % 16] : make_float2(0.0f, 0.0f);
                XC[p] = live ? sX[(p / 16) * nr + p % 16] : 0;
            }
        }
    }
    __syncthreads();
    // the chain: acc[t][v] for token 16 t + 4 gq + v of the tile and weight row r (column c0 + r);
    // rank1's a operand is the (scale, u) of token 4 gq + l % 4
    const uint32_t tl = 4 * gq + (l & 3);
    v4f acc[NT];
#pragma unroll
    for (uint32_t t = 0; t < NT; t++) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t b0 = 0; b0 < nu; b0 += UB) {
#pragma unroll
        for (uint32_t i = 0; i < UB; i++) {
            const uint32_t b = b0 + i;
            if (b >= nu) break;
            const B cw = w[i];
            if (b + UB < nu) tqm_load<GK, 32>(w[i], strip, b + UB, l);  // the load UB units ahead
            const long bq = tqm_operand<GK, 32>(cw, l);
            const float dd = h2f((uint16_t)cw.d[0]), mm = h2f((uint16_t)cw.m[0]);
#pragma unroll
            for (uint32_t t = 0; t < NT; t++) {
                if (t >= ntl) break;
                const uint8_t* ti = smem + t * tile;
                const v4i c4 = U8 ? *reinterpret_cast<const v4i*>(ti + oXC + 4 * (b * 16 + 4 * gq)) : v4i{0, 0, 0, 0};
                const long a = *reinterpret_cast<const long*>(ti + 8 * (b * 64 + l));
                const v4i d4 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bq, c4, 0, 0, 0);
                const float2 su = *reinterpret_cast<const float2*>(ti + oSU + 8 * (b * 16 + tl));
                acc[t] = rank1(su.y, mm, acc[t]);
                const v4f ds = rank1(su.x, dd, neg_zero4());
#pragma unroll
                for (int v = 0; v < 4; v++) acc[t][v] = __builtin_fmaf((float)d4[v], ds[v], acc[t][v]);
            }
        }
    }
    const float inv = 1.0f / (float)g.hc;
    if constexpr (DEC) {
        // lane r of wave s: the product xn_s[c] g_s[c] (rounded, as the reference's multiply then
        // add); thread c then adds the hc products in stream order from 0
        if (gq == 0) gate[wv * 16 + r] = xv[0] * sigmoid_libm(g.pair ? acc[0][0] + acc[0][1] : acc[0][0]);
        __syncthreads();
        if (tid < 16) {
            float o = 0.0f;
            for (uint32_t s = 0; s < g.hc; s++) o = o + gate[s * 16 + tid];
            g.mixed[c0 + tid] = o * inv;
        }
    } else {
#pragma unroll
        for (uint32_t t = 0; t < NT; t++)
            if (t < ntl)
                for (int v = 0; v < 4; v++) gate[(wv * TT + 16 * t + 4 * gq + v) * 16 + r] = sigmoid512(acc[t][v]);
        __syncthreads();  // the tile images free
        {
            const uint32_t tx = tid / (16 * g.hc), sx = tid % (16 * g.hc);
#pragma unroll
            for (uint32_t j = 0; j < J; j++) xs[((tx + 4 * j) * g.hc + sx / 16) * 16 + sx % 16] = xv[j];
        }
        __syncthreads();
        for (uint32_t o = tid; o < TT * 16; o += nthr) {
            const uint32_t tok = o / 16, c = o % 16;
            if (tok >= nt) break;
            const float* x = xs + (size_t)tok * g.hc * 16 + c;
            float y = x[0] * gate[tok * 16 + c];
            for (uint32_t s = 1; s < g.hc; s++) y = __builtin_fmaf(x[16 * s], gate[(s * TT + tok) * 16 + c], y);
            g.mixed[(size_t)(t0 + tok) * g.hh + c0 + c] = y * inv;
        }
    }
}

hipError_t launch_hc_mix(const Mat& up, uint32_t hc, uint32_t hh, uint32_t lr, const float* xn, const float* lo,
                         uint32_t m, int pair, const Workspace& ws, float* mixed, hipStream_t st) {
    const uint32_t nu = lr / 32;
    // the batch image (44 bytes per token and block: 1.375 m lr) lives in the per-entry output rows,
    // free until the layer's down stage
    const size_t img_bytes = hc_image_bytes(m, lr);
    if (tq_kb(up.fmt) != 32 || hc == 0 || hc > 8 || lr == 0 || lr % 32 || lr > HC_MAXLR || hh % 16 ||
        (m > 1 && img_bytes > (size_t)ws.tiles * ws.yent_tile * 4))
        return hipErrorInvalidValue;
    const bool dec = m == 1;
    // batch: four (else two) token tiles per workgroup where the LDS allows and the grid keeps 1024
    // workgroups (4 per CU)
    uint32_t nt = 1;
    if (!dec)
        for (uint32_t c : {4u, 2u})
            if (hc_lds(c, nu, hc).total <= 64 * 1024 && (size_t)(hh / 16) * ((m + 16 * c - 1) / (16 * c)) >= 1024) {
                nt = c;
                break;
            }
    uint8_t* img = reinterpret_cast<uint8_t*>(ws.yent);
    const HcArgs a{up, xn, lo, img, mixed, hc, hh, lr, m, dec && pair ? 1 : 0};
    if (!dec) hc_quant_kernel<<<(m * lr + 255) / 256, 256, 0, st>>>(lo, m, lr, hc, img);
    const dim3 grid(hh / 16, (m + 16 * nt - 1) / (16 * nt));
    const size_t lds = hc_lds(nt, nu, hc).total;
    const uint32_t thr = 64 * hc;
    switch (tq_bits(up.fmt) * 10 + (dec ? 0 : nt)) {
#define HC_GO(bits, gk)                                                                \
    case bits * 10: hc_mix_kernel<gk, 1, true><<<grid, thr, lds, st>>>(a); break;      \
    case bits * 10 + 1: hc_mix_kernel<gk, 1, false><<<grid, thr, lds, st>>>(a); break; \
    case bits * 10 + 2: hc_mix_kernel<gk, 2, false><<<grid, thr, lds, st>>>(a); break; \
    case bits * 10 + 4: hc_mix_kernel<gk, 4, false><<<grid, thr, lds, st>>>(a); break;
        HC_GO(4, GK_TQ4) HC_GO(5, GK_TQ5) HC_GO(8, GK_TQ8)
#undef HC_GO
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace trk
