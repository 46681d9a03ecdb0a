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
    // 64 VGPRs of raw words)
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
            const TqmB<GK, KB> c0 = w0[i], c1 = w1[i];
            if (b + UB < nu) {  // the loads UB units ahead
                tqm_load<GK, KB>(w0[i], s0, b + UB, l);
                tqm_load<GK, KB>(w1[i], s1, b + UB, l);
            }
            const long a = As[b * 64 + l];
            const long bq0 = tqm_operand<GK, KB>(c0, l), bq1 = tqm_operand<GK, KB>(c1, l);
            constexpr uint32_t NBL = TqmB<GK, KB>::NBL;  // blocks of the unit
#pragma unroll
            for (uint32_t hb = 0; hb < NBL; hb++) {
                const long am = KB == 16 ? ((g / 2 == hb) ? a : 0) : a;
                const v4i d40 = tqm_mfma(am, bq0), d41 = tqm_mfma(am, bq1);
                const uint32_t blk = NBL * b + hb;
                const float dd0 = h2f((uint16_t)c0.d[hb]), mm0 = h2f((uint16_t)c0.m[hb]);
                const float dd1 = h2f((uint16_t)c1.d[hb]), mm1 = h2f((uint16_t)c1.m[hb]);
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
template <int GK, int NJ>
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
    } else if (g.decode) {
        ns = ws.n_sel[0];
    }
    bool shared;
    uint32_t e, nr, P;
    if (!tqm_unit(ws, true, g.decode, g.pair, blockIdx.y, shared, e, nr, P, prow, orow, tid, ns, ids)) return;
    __syncthreads();
    tqm_stage<32, GK == GK_TQ8>(ws.xq, ws.xs, ws.xu, prow, nr * P, H, As, Sc, tid, 256);
    __syncthreads();
    const uint32_t gq = l / 16, r = l % 16, n_ent = ws.n_groups[1];
    const Mat& Ga = shared ? g.sha : g.a;
    const Mat& Ub = shared ? g.shb : g.b;
    if (NJ == 0 && !g.decode) {
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
        return;
    }
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
        if (!up && live) tqm_swiglu_store(ws, g.decode, g.pair, P, nr, orow, n_ent, F, nbf, strip, gq, r, acc,
                                          hu[wv / 2][l], ns, wsel);
        __syncthreads();  // hu read before the next pass writes it
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

hipError_t launch_tqm_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const Workspace& ws,
                             uint32_t m, uint32_t kcap, int pair, const float* lg, uint32_t k, Policy pol,
                             hipStream_t st) {
    if (tq_kb(gate.fmt) != 32 || ws.H % 32) return hipErrorInvalidValue;
    const TqmArgs a{gate, up, sh_gate, sh_up, ws, m == 1 ? 1 : 0, m == 1 && pair ? 1 : 0, lg, k, pol};
    const int nj = m == 1 && lg ? (int)route_nj(ws.E) : 0;  // decode: routing inside
    // decode: a workgroup per strip pair; batch: a workgroup per TQM_PAIRS strip pairs of an item,
    // looping over them with the item's activations staged once (5 or 2 pairs per workgroup at the
    // real shape: 478 / 484 us against 460 for 4)
    const uint32_t pairs = (ws.F / 16 + 1) / 2;
    const dim3 grid(m == 1 ? pairs : (pairs + TQM_PAIRS - 1) / TQM_PAIRS, m == 1 ? kcap + 1 : grouped_item_rows(ws, m));
    const size_t sc = tq_bits(gate.fmt) == 8 ? 16 : 8;  // bytes per Sc entry
    size_t lds = (size_t)(ws.H / 32) * 64 * 8 + (size_t)(ws.H / 32) * 16 * sc;
    if (m == 1) {  // decode: the up accumulators of two strips; route_row's exponentials before them
        const size_t ex = nj && pol.enabled && pol.basis == TRK_BASIS_ALL ? (size_t)ws.E * 4 : 0;
        lds += ex > 2 * 64 * 4 * 4 ? ex : 2 * 64 * 4 * 4;
    }
    switch (tq_bits(gate.fmt) * 100 + nj) {
#define TQM_GU(b, gk)                                                                 \
    case b * 100: tqm_gateup_kernel<gk, 0><<<grid, 256, lds, st>>>(a); break;         \
    case b * 100 + 8: tqm_gateup_kernel<gk, 8><<<grid, 256, lds, st>>>(a); break;     \
    case b * 100 + 16: tqm_gateup_kernel<gk, 16><<<grid, 256, lds, st>>>(a); break;
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

}  // namespace trk
