// The kernel-level GEMV: y[map[i]][r] (+)= W[r] . x_i for r in 16-row strips [s0, s1) of one
// weight matrix and int8 activation rows x (gemv_tq_rows / gemm_tq_rows, gemv.rs:16-78), on GGUF
// superblocks (Q4_K, Q6_K, Q8_0, Q5_1) or on the reference's own TQ strips (codec.rs:1-46).
//
// Exactness fixes the shape of the work: each block's dot is an exact integer, so blocks may be
// reduced in any order and on any lane, but the per-(row, activation) f32 chain
//     acc = fma(m, sx * sum, acc); acc = fma(float(dot), d * sx, acc)          (gemv.rs:141-148)
// runs over the blocks in order.  A workgroup owns R rows (16 or 64) and walks K in slices:
//   phase 1  every lane decodes weight units of its row (a TQ block or half a GGUF superblock),
//            forms the block dots against the staged activations and writes (dot) and (d, m) to
//            LDS: K-parallel, four waves over the slice's units;
//   phase 2  lane (activation a, row r) runs the chain over the slice's blocks from LDS.
// After the last slice one lane per row writes the logical rows in order, so a row map with
// repeats accumulates in the reference's order (its store loop, gemv.rs:150-171).
#include "tq.hpp"

namespace trk {

constexpr uint32_t GV_NA = 4;  // most physical activation rows per pass

struct GemvArgs {
    const uint8_t* w;   // the matrix (item applied)
    uint64_t pitch;     // GGUF: bytes per row; TQ: bytes per 16-row strip
    uint32_t k, nb;     // k and blocks per row (k / KB)
    uint32_t r_lo, r_hi;  // output rows [r_lo, r_hi)
    const int8_t* q;    // [m][k]
    const float* s;     // [m][nb]
    const int32_t* su;  // [m][nb]
    uint32_t m;         // physical activation rows
    uint32_t npass;     // passes of NA physical rows
    int pair;
    float* y;
    uint32_t ldy;
    const uint32_t* map;  // logical row -> y row, or null (identity)
    int accumulate;
};


template <int GK, int KB>
struct GvUnit {
    // blocks per unit: a TQ block, or half a GGUF superblock (128 values)
    static constexpr int U = GK >= GK_TQ4 ? 1 : 128 / KB;
};

// One unit's weight bytes in registers.
template <int GK, int KB>
struct GvW;
template <int KB>
struct GvW<GK_Q4K, KB> {
    uint4 hdr, qs[4];
};
template <int KB>
struct GvW<GK_Q6K, KB> {
    Q6Half h;
};
template <int KB>
struct GvW<GK_Q80, KB> {
    Q8Half h;
};
template <int KB>
struct GvW<GK_Q51, KB> {
    Q51Half h;
};
template <int KB>
struct GvW<GK_TQ4, KB> : GvTQ<GK_TQ4, KB> {};
template <int KB>
struct GvW<GK_TQ5, KB> : GvTQ<GK_TQ5, KB> {};
template <int KB>
struct GvW<GK_TQ8, KB> : GvTQ<GK_TQ8, KB> {};
// Load the GGUF unit starting at block b of the row.
template <int GK, int KB>
__device__ __forceinline__ void gv_load(GvW<GK, KB>& w, const uint8_t* __restrict__ rowp, uint32_t b) {
    const uint32_t unit = b / GvUnit<GK, KB>::U, sb = unit / 2, h2 = unit % 2;
    if constexpr (GK == GK_Q4K)
        load_half_q4k(rowp, sb, h2, w.hdr, w.qs);
    else if constexpr (GK == GK_Q6K)
        load_half_q6k(rowp, sb, h2, w.h);
    else if constexpr (GK == GK_Q80)
        load_half_q80(rowp, sb, h2, w.h);
    else
        load_half_q51(rowp, sb, h2, w.h);
}

// Phase 1 for one loaded GGUF unit: its block dots against NA staged activation rows (xq: LDS,
// [NA][S * KB] bytes; the unit's first block at slice column j0) into dl[a][j0 + i][rl], and the
// blocks' (d, m) into dm[j0 + i][rl].  xs[a][j].z holds the activation block's byte sum (Q8_0's
// unsigned q is its int8 plus 128).  h2: the unit's half of its superblock.
template <int GK, int KB, int NA, int R, int S>
__device__ __forceinline__ void gv_terms(const GvW<GK, KB>& w, uint32_t h2, uint32_t j0, uint32_t na,
                                         const int8_t (*xq)[S * KB], const float4 (*xs)[S], float (*dl)[S][R],
                                         float2 (*dm)[R], uint32_t rl) {
    auto xw = [&](uint32_t a, uint32_t j, uint32_t word) -> int {
        return reinterpret_cast<const int*>(&xq[a][j * KB])[word];
    };
    if constexpr (GK == GK_Q4K) {
        const uint32_t* w32 = reinterpret_cast<const uint32_t*>(w.qs);
        const float d = h2f((uint16_t)(w.hdr.x & 0xffff)), dmin = h2f((uint16_t)(w.hdr.x >> 16));
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {  // sub-block 4 h2 + jj: nibble jj % 2 of qs words 8 (jj / 2) ..
            int sc0, mn0, sc1, mn1;
            q4k_scale_min_w(w.hdr.y, w.hdr.z, w.hdr.w, jj, sc0, mn0);
            q4k_scale_min_w(w.hdr.y, w.hdr.z, w.hdr.w, 4 + jj, sc1, mn1);
            float dd, mm;
            q4k_dm(d, dmin, h2 ? sc1 : sc0, h2 ? mn1 : mn0, dd, mm);
            const int c = jj / 2, h = jj % 2;
            if constexpr (KB == 32) {
                dm[j0 + jj][rl] = make_float2(dd, mm);
#pragma unroll
                for (uint32_t a = 0; a < NA; a++) {
                    if (a >= na) break;
                    int dot = 0;
#pragma unroll
                    for (int t = 0; t < 8; t++) dot = sdot4((int)nib(w32[8 * c + t], h), xw(a, j0 + jj, t), dot);
                    dl[a][j0 + jj][rl] = (float)dot;
                }
            } else {
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const uint32_t j = j0 + 2 * jj + hh;
                    dm[j][rl] = make_float2(dd, mm);
#pragma unroll
                    for (uint32_t a = 0; a < NA; a++) {
                        if (a >= na) break;
                        int dot = 0;
#pragma unroll
                        for (int t = 0; t < 4; t++) dot = sdot4((int)nib(w32[8 * c + 4 * hh + t], h), xw(a, j, t), dot);
                        dl[a][j][rl] = (float)dot;
                    }
                }
            }
        }
    } else if constexpr (GK == GK_Q6K) {  // kb 16: one block per scale
        const float d = h2f((uint16_t)w.h.d);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int8_t sc = (int8_t)((w.h.sc[i >> 2] >> (8 * (i & 3))) & 0xffu);
            const float ddv = f16_round(d * (float)sc);
            dm[j0 + i][rl] = make_float2(ddv, f16_round(-32.0f * ddv));
            const int g = i / 2, l0 = 16 * (i % 2);
            uint32_t qw[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                uint32_t lo = w.h.ql[8 * (g & 1) + l0 / 4 + t];
                lo = (g >> 1) ? ((lo >> 4) & 0x0f0f0f0fu) : (lo & 0x0f0f0f0fu);
                qw[t] = lo | (((w.h.qh[l0 / 4 + t] >> (2 * g)) & 0x03030303u) << 4);
            }
#pragma unroll
            for (uint32_t a = 0; a < NA; a++) {
                if (a >= na) break;
                int dot = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) dot = sdot4((int)qw[t], xw(a, j0 + i, t), dot);
                dl[a][j0 + i][rl] = (float)dot;
            }
        }
    } else if constexpr (GK == GK_Q80) {  // four 32-blocks: f16 d, 32 int8 (q + 128 unsigned)
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
            const uint32_t o = 34 * jb;
            const float dd = h2f((uint16_t)((w.h.w[o / 4] >> (8 * (o % 4))) & 0xffffu));
            const float mm = f16_round(-128.0f * dd);
            constexpr int NB = 32 / KB;  // activation blocks per Q8_0 block
#pragma unroll
            for (int hf = 0; hf < NB; hf++) {
                const uint32_t j = j0 + NB * jb + hf;
                dm[j][rl] = make_float2(dd, mm);
#pragma unroll
                for (uint32_t a = 0; a < NA; a++) {
                    if (a >= na) break;
                    int dot = 0;
#pragma unroll
                    for (int t = 0; t < KB / 4; t++) dot = sdot4((int)q8_word(w.h, o + 2 + KB * hf + 4 * t), xw(a, j, t), dot);
                    dl[a][j][rl] = (float)(dot + 128 * __float_as_int(xs[a][j].z));
                }
            }
        }
    } else {  // Q5_1: four 32-blocks: f16 d, f16 m, u32 qh, 16 bytes qs
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
            const float dd = h2f((uint16_t)(w.h.w[6 * jb] & 0xffffu)), mm = h2f((uint16_t)(w.h.w[6 * jb] >> 16));
            const uint32_t qh = w.h.w[6 * jb + 1];
            uint32_t qw[2][4];  // element 16 hf + 4 t + i
#pragma unroll
            for (int hf = 0; hf < 2; hf++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    qw[hf][t] = ((w.h.w[6 * jb + 2 + t] >> (4 * hf)) & 0x0f0f0f0fu) | q5_hi4((qh >> (16 * hf + 4 * t)) & 0xfu);
            constexpr int NB = 32 / KB;
#pragma unroll
            for (int hb = 0; hb < NB; hb++) {
                const uint32_t j = j0 + NB * jb + hb;
                dm[j][rl] = make_float2(dd, mm);
#pragma unroll
                for (uint32_t a = 0; a < NA; a++) {
                    if (a >= na) break;
                    int dot = 0;
#pragma unroll
                    for (int t = 0; t < KB / 4; t++) {
                        const int hf = NB == 2 ? hb : t / 4;
                        dot = sdot4((int)qw[hf][t % 4], xw(a, j, t), dot);
                    }
                    dl[a][j][rl] = (float)dot;
                }
            }
        }
    }
}

// R rows per workgroup (16 or 64), S blocks per K slice (S * R fixed by the LDS budget)
template <int GK, int KB, int NA, int R>
__global__ __launch_bounds__(256) void gemv_rows_kernel(GemvArgs g) {
    constexpr bool TQ = GK >= GK_TQ4;
    constexpr uint32_t U = GvUnit<GK, KB>::U;
    constexpr uint32_t S = (NA <= 2 ? 2048 : 1024) / R;
    // phase-1 units: GGUF: (row, unit column), the columns of a row on consecutive lanes (NCOL
    // columns, NRG rows at a time); TQ: (strip, block), one per 16-lane group (NSTR strips)
    constexpr uint32_t NCOL = TQ ? 16 : (R == 16 ? 16 : 4), NRG = 256 / NCOL, NSTR = R / 16;
    // units whose loads a thread issues together: about 48 registers of weights, 24 for TQ strips
    // (two units: more waves per SIMD beat more loads per wave, e.g. the LM head 165 -> 148 us)
    constexpr uint32_t UW = sizeof(GvW<GK, KB>) / 4, UREG = TQ ? 24 : 48;
    constexpr uint32_t UB = UW * 8 <= UREG ? 8 : (UREG / UW > 2 ? UREG / UW : 2);
    constexpr bool XSUM = GK == GK_Q80 || GK == GK_TQ8;
    __shared__ __align__(16) int8_t xq[NA][S * KB];
    __shared__ __align__(16) float4 xs[NA][S];  // sx, u = sx * sum, byte sum (int bits), -
    __shared__ float dl[NA][S][R];
    __shared__ float2 dm[S][R];
    const uint32_t tid = threadIdx.x, row0 = g.r_lo + blockIdx.x * R;
    // phase 1 (GGUF): rows gr, gr + NRG, ... (R / NRG of them) at unit column gc
    const uint32_t gc = tid % NCOL, gr = tid / NCOL;
    // phase 1 (TQ): lane l of group gi
    const uint32_t l = tid % 16, gi = tid / 16;
    // phase 2: thread (activation ca, row cr)
    const uint32_t ca = tid / R, cr = tid % R;
    const uint32_t per = g.pair ? 2u : 1u;
    constexpr uint32_t RPT = TQ ? 1 : (R + NRG - 1) / NRG;  // GGUF rows per thread
    const uint8_t* rowp[RPT];
#pragma unroll
    for (uint32_t i = 0; i < RPT; i++) {
        const uint32_t r = row0 + gr + i * NRG, rc = r < g.r_hi ? r : g.r_hi - 1;
        rowp[i] = g.w + (size_t)rc * g.pitch;
    }

    // the unit (loads) of a thread's k-th phase-1 work item of a slice of sn blocks at b0
    constexpr uint32_t NU_ROW = S / U;  // GGUF units per row per slice (at most)
    auto n_items = [&](uint32_t sn) -> uint32_t {
        return TQ ? (NSTR * sn + 15 - gi) / 16 : ((gr < R ? (R - gr + NRG - 1) / NRG : 0) * ((sn / U + NCOL - 1 - gc) / NCOL));
    };
    GvW<GK, KB> w[UB];
    auto load_item = [&](GvW<GK, KB>& wi, uint32_t b0, uint32_t sn, uint32_t k) {
        if constexpr (TQ) {
            const uint32_t u = gi + 16 * k, sl = u % NSTR, j = u / NSTR;
            const uint32_t st = row0 / 16 + sl, stc = st < g.r_hi / 16 ? st : g.r_hi / 16 - 1;
            gv_load_tq<GK, KB>(wi, g.w + (size_t)stc * g.pitch, b0 + j, l);
        } else {
            const uint32_t ncu = (sn / U + NCOL - 1 - gc) / NCOL;  // this thread's unit columns
            const uint32_t ri = k / ncu, uu = gc + NCOL * (k % ncu);
            const uint8_t* rp = rowp[0];
#pragma unroll
            for (uint32_t i = 1; i < RPT; i++)
                if (ri == i) rp = rowp[i];
            gv_load<GK, KB>(wi, rp, b0 + uu * U);
        }
    };
    auto terms_item = [&](const GvW<GK, KB>& wi, uint32_t b0, uint32_t sn, uint32_t k, uint32_t na) {
        if constexpr (TQ) {
            const uint32_t u = gi + 16 * k, sl = u % NSTR, j = u / NSTR;
            gv_terms_tq<GK, KB, NA, R, S>(wi, l, j, 16 * sl, na, xq, xs, dl, dm);
        } else {
            const uint32_t ncu = (sn / U + NCOL - 1 - gc) / NCOL;
            const uint32_t ri = k / ncu, uu = gc + NCOL * (k % ncu);
            gv_terms<GK, KB, NA, R, S>(wi, ((b0 + uu * U) / U) % 2, uu * U, na, xq, xs, dl, dm, gr + ri * NRG);
        }
    };
    auto load_batch = [&](uint32_t b0, uint32_t sn, uint32_t k0) {
        const uint32_t n = n_items(sn);
#pragma unroll
        for (uint32_t i = 0; i < UB; i++)
            if (k0 + i < n) load_item(w[i], b0, sn, k0 + i);
    };
    (void)NU_ROW;

    for (uint32_t pass = blockIdx.y; pass < g.npass; pass += gridDim.y) {
        const uint32_t p0 = pass * NA, na = g.m - p0 < NA ? g.m - p0 : NA;
        float acc = 0.0f;
        uint32_t sn = g.nb < S ? g.nb : S;
        load_batch(0, sn, 0);  // in flight while the activations are staged
        for (uint32_t b0 = 0; b0 < g.nb;) {
            __syncthreads();  // the previous slice's readers are done
            const uint32_t pr = sn * KB / 16;
            for (uint32_t i = tid; i < NA * pr; i += 256) {
                const uint32_t a = i / pr, o = (i % pr) * 16;
                int4 v = make_int4(0, 0, 0, 0);
                if (a < na) v = *reinterpret_cast<const int4*>(g.q + (size_t)(p0 + a) * g.k + (size_t)b0 * KB + o);
                *reinterpret_cast<int4*>(&xq[a][o]) = v;
            }
            for (uint32_t i = tid; i < NA * S; i += 256) {
                const uint32_t a = i / S, j = i % S;
                float sx = 0.0f, u = 0.0f;
                int xsum = 0;
                if (a < na && j < sn) {
                    const size_t bi = (size_t)(p0 + a) * g.nb + b0 + j;
                    sx = g.s[bi];
                    u = sx * (float)g.su[bi];  // gemv.rs:143
                    if constexpr (XSUM) {
                        const int4* xp = reinterpret_cast<const int4*>(g.q + (size_t)(p0 + a) * g.k + (size_t)(b0 + j) * KB);
#pragma unroll
                        for (int t = 0; t < KB / 16; t++) {
                            const int4 v = xp[t];
                            xsum = sdot4(v.x, 0x01010101, xsum);
                            xsum = sdot4(v.y, 0x01010101, xsum);
                            xsum = sdot4(v.z, 0x01010101, xsum);
                            xsum = sdot4(v.w, 0x01010101, xsum);
                        }
                    }
                }
                xs[a][j] = make_float4(sx, u, __int_as_float(xsum), 0.0f);
            }
            __syncthreads();
            // phase 1: the thread's work items, UB items' loads at a time
            const uint32_t n = n_items(sn);
            for (uint32_t k0 = 0; k0 < n; k0 += UB) {
                if (k0) load_batch(b0, sn, k0);
#pragma unroll
                for (uint32_t i = 0; i < UB; i++)
                    if (k0 + i < n) terms_item(w[i], b0, sn, k0 + i, na);
            }
            // the next slice's first batch, in flight during this slice's chain
            const uint32_t b1 = b0 + sn, sn1 = g.nb - b1 < S ? g.nb - b1 : S;
            if (b1 < g.nb) load_batch(b1, sn1, 0);
            __syncthreads();
            // phase 2: the chain in block order
            if (ca < na) {
                uint32_t j = 0;
                for (; j + 8 <= sn; j += 8) {
                    float2 t[8];
                    float4 x[8];
                    float d[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        t[i] = dm[j + i][cr];
                        x[i] = xs[ca][j + i];
                        d[i] = dl[ca][j + i][cr];
                    }
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        acc = __builtin_fmaf(t[i].y, x[i].y, acc);
                        acc = __builtin_fmaf(d[i], t[i].x * x[i].x, acc);
                    }
                }
                for (; j < sn; j++) {
                    const float2 t = dm[j][cr];
                    const float4 x = xs[ca][j];
                    acc = __builtin_fmaf(t.y, x.y, acc);
                    acc = __builtin_fmaf(dl[ca][j][cr], t.x * x.x, acc);
                }
            }
            b0 = b1;
            sn = sn1;
        }
        __syncthreads();
        if (ca < na) dl[ca][0][cr] = acc;
        __syncthreads();
        // the logical rows in order, one thread per output row (gemv.rs:150-171)
        const uint32_t row = row0 + tid;
        if (tid < R && row < g.r_hi) {
            for (uint32_t i = 0; i < na / per; i++) {
                const float v = g.pair ? dl[2 * i][0][tid] + dl[2 * i + 1][0][tid] : dl[i][0][tid];
                const uint32_t lg = p0 / per + i;
                float* yp = g.y + (size_t)(g.map ? g.map[lg] : lg) * g.ldy + row;
                *yp = g.accumulate ? *yp + v : v;
            }
        }
    }
}

template <int GK, int KB, int R>
static hipError_t gemv_go_r(const GemvArgs& g, uint32_t na, dim3 grid, hipStream_t st) {
    if (na <= 1)
        gemv_rows_kernel<GK, KB, 1, R><<<grid, 256, 0, st>>>(g);
    else if (na <= 2)
        gemv_rows_kernel<GK, KB, 2, R><<<grid, 256, 0, st>>>(g);
    else
        gemv_rows_kernel<GK, KB, 4, R><<<grid, 256, 0, st>>>(g);
    return hipGetLastError();
}

// 64 rows per workgroup when that still gives every CU a workgroup, else 16 (more workgroups,
// longer K slices)
template <int GK, int KB>
static hipError_t gemv_go(const GemvArgs& g, uint32_t na, uint32_t gy, hipStream_t st) {
    const uint32_t n = g.r_hi - g.r_lo;
    if (n >= 64 * 1024) return gemv_go_r<GK, KB, 64>(g, na, dim3((n + 63) / 64, gy), st);
    return gemv_go_r<GK, KB, 16>(g, na, dim3((n + 15) / 16, gy), st);
}

hipError_t launch_gemv(const Mat& w, uint32_t item, uint32_t s0, uint32_t s1, uint32_t kb, const int8_t* q,
                       const float* s, const int32_t* su, uint32_t m, int pair, float* y, uint32_t ldy,
                       const uint32_t* rows, int accumulate, hipStream_t st) {
    const bool tq = fmt_is_tq(w.fmt);
    GemvArgs g;
    g.w = w.ptr + (size_t)item * w.stride;
    g.pitch = w.row_bytes;
    g.k = w.k;
    g.nb = w.k / kb;
    g.r_lo = 16 * s0;
    g.r_hi = tq ? 16 * s1 : (16 * s1 < w.rows ? 16 * s1 : w.rows);
    g.q = q;
    g.s = s;
    g.su = su;
    g.m = m;
    g.pair = pair;
    g.y = y;
    g.ldy = ldy;
    g.map = rows;
    g.accumulate = accumulate;
    // physical rows per pass: the fewest of 1, 2, 4 that hold all rows (whole pairs), else 4
    const uint32_t na = m <= 1 ? 1 : m <= 2 ? 2 : GV_NA;
    g.npass = (m + na - 1) / na;
    // a row map may repeat a y row: then one workgroup runs every pass of its rows in order
    const uint32_t gy = rows ? 1u : (g.npass < 65535u ? g.npass : 65535u);
    switch (w.fmt) {
        case TRK_FMT_Q4_K: return kb == 32 ? gemv_go<GK_Q4K, 32>(g, na, gy, st) : gemv_go<GK_Q4K, 16>(g, na, gy, st);
        case TRK_FMT_Q6_K: return gemv_go<GK_Q6K, 16>(g, na, gy, st);
        case TRK_FMT_Q8_0: return kb == 32 ? gemv_go<GK_Q80, 32>(g, na, gy, st) : gemv_go<GK_Q80, 16>(g, na, gy, st);
        case TRK_FMT_Q5_1: return kb == 32 ? gemv_go<GK_Q51, 32>(g, na, gy, st) : gemv_go<GK_Q51, 16>(g, na, gy, st);
        case TRK_FMT_TQ4_32: return gemv_go<GK_TQ4, 32>(g, na, gy, st);
        case TRK_FMT_TQ4_16: return gemv_go<GK_TQ4, 16>(g, na, gy, st);
        case TRK_FMT_TQ5_32: return gemv_go<GK_TQ5, 32>(g, na, gy, st);
        case TRK_FMT_TQ5_16: return gemv_go<GK_TQ5, 16>(g, na, gy, st);
        case TRK_FMT_TQ8_32: return gemv_go<GK_TQ8, 32>(g, na, gy, st);
        case TRK_FMT_TQ8_16: return gemv_go<GK_TQ8, 16>(g, na, gy, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace trk
