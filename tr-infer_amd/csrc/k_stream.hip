// Grouped expert products for work items of few entry rows on the streaming GEMV:
// Model::moe_batch's tasks A/B (gate/up, SwiGLU, per-16 requantisation, weight fold) and task C
// (down, per-entry rows) for items of at most `max_rows` rows (exec_batch.rs:1404-1580).
//
// Every item of a batch of M <= 16 tokens runs here, as do the items of a few rows at larger M
// (the tail item of most experts); the int8 MFMA tiles of k_batch.hip take the rest.  A tile
// spends the same VALU epilogue on every one of its 16 rows, padding included, while a
// streaming unit reads each weight superblock once per item from HBM in 144-byte pieces and
// spends its epilogue only on the item's real rows.  Both give the same bits: every 32- (16-)
// block dot is an exact integer, and the f32 chain (gemv.rs:141-148) runs per (entry, row) in
// block order.
#include "gemv.hpp"

#include <type_traits>

namespace trk {

// The item of workgroup row y: the last item (the shared expert's, or the last 16-token piece of
// it) first, the routed items after it, so that the heaviest unit does not start last.  False
// when y is past the items or the item belongs to the MFMA kernels.
__device__ __forceinline__ bool stream_item(const Workspace& ws, uint32_t y, uint32_t max_rows, Item& it) {
    const uint32_t n = ws.n_groups[2];
    if (y >= n) return false;
    it = ws.items[y == 0 ? n - 1 : y - 1];
    return it.nrows <= max_rows;
}

// Stage `nr` rows of int8 activations (K bytes each, 16-byte pieces) into LDS rows of pitch
// `pitch` (a padded 272 bytes per 256 when `sbpad`), with their per-block scale and u terms
// (nbk blocks per row).  Every thread requests all of its pieces before it stores any.
template <bool SBPAD>
__device__ __forceinline__ void stage_rows(const int8_t* __restrict__ q, const float* __restrict__ s,
                                           const float* __restrict__ u, const uint32_t* __restrict__ rows,
                                           uint32_t nr, uint32_t K, uint32_t nbk, uint32_t pitch, int8_t* lq,
                                           float* ls, float* lu, uint32_t tid, uint32_t nthr) {
    const uint32_t pieces = K / 16, np = nr * pieces, ns = nr * nbk;
    for (uint32_t i0 = 0; i0 < np; i0 += 4 * nthr) {
        int4 v[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = i0 + tid + nthr * c, ic = i < np ? i : np - 1;
            v[c] = *reinterpret_cast<const int4*>(q + (size_t)rows[ic / pieces] * K + (ic % pieces) * 16);
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t i = i0 + tid + nthr * c;
            if (i < np) {
                const uint32_t o = (i % pieces) * 16;
                *reinterpret_cast<int4*>(lq + (i / pieces) * pitch + (SBPAD ? o + (o / 256) * 16 : o)) = v[c];
            }
        }
    }
    for (uint32_t i0 = 0; i0 < ns; i0 += 2 * nthr) {
        float a[2], b[2];
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const uint32_t i = i0 + tid + nthr * c, ic = i < ns ? i : ns - 1;
            a[c] = s[(size_t)rows[ic / nbk] * nbk + ic % nbk];
            b[c] = u[(size_t)rows[ic / nbk] * nbk + ic % nbk];
        }
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const uint32_t i = i0 + tid + nthr * c;
            if (i < ns) {
                ls[i] = a[c];
                lu[i] = b[c];
            }
        }
    }
}

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// ---- gate/up ----------------------------------------------------------------------------------
//
// Grid (F / 16 strips, items), GU_THREADS(NSB) threads: lane (row r of the strip's 16 gate and 16
// up rows, superblock sb) holds that superblock's 144 bytes and forms its 8 block dots against
// each entry's activations in turn (two entries at a time); the per-(entry, row) chain crosses
// the NSB lanes of the row in superblock order.  Then SwiGLU, the per-16 quantisation of each
// entry's strip and the weight fold, 16 lanes per entry.
template <int NSB>
__global__ __launch_bounds__(GU_THREADS(NSB)) void stream_gateup_kernel(Mat gate, Mat up, Mat shg, Mat shu,
                                                                       Workspace ws, uint32_t max_rows,
                                                                       uint32_t xall) {
    constexpr uint32_t H = NSB * 256, nb = NSB * 8, XSB = 256 + 16, XP = NSB * XSB, RPW = 64 / NSB, PPR = H / 16;
    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    // xall (a batch of xall <= 16 tokens): every token's x is staged, its loads issued before the
    // item is known (at most XV pieces and XS scales per thread, checked by the host)
    constexpr int XV = 8, XS = 4;
    constexpr uint32_t SCH = 4;  // entry rows staged per pass otherwise
    v4u xv[XV];
    float xsv[XS], xuv[XS];
    if (xall) {
        const uint32_t np = xall * PPR, ns = xall * nb;
#pragma unroll
        for (int c = 0; c < XV; c++) {
            const uint32_t i = tid + nthr * c, ic = i < np ? i : np - 1;
            xv[c] = *reinterpret_cast<const v4u*>(ws.xq + (size_t)(ic / PPR) * H + (ic % PPR) * 16);
        }
#pragma unroll
        for (int c = 0; c < XS; c++) {
            const uint32_t i = tid + nthr * c, ic = i < ns ? i : ns - 1;
            xsv[c] = ws.xs[ic];
            xuv[c] = ws.xu[ic];
        }
    }
    Item item;
    if (!stream_item(ws, blockIdx.y, max_rows, item)) return;
    const uint32_t F = gate.rows, nbf = F / 16, strip = blockIdx.x;
    const bool shared = item.expert == NO_EXPERT;
    const uint32_t nr = item.nrows, e = shared ? 0u : item.expert;

    // this lane's weights next: they depend on the item only
    const uint32_t ln = tid % 64, sb = ln % NSB;
    const uint32_t r = ln < RPW * NSB ? (tid / 64) * RPW + ln / NSB : 32u;
    const bool wthread = r < 32;
    const uint32_t rr = wthread ? r : 0u;
    const bool isg = rr < 16;
    const uint8_t* base = isg ? (shared ? shg.ptr : gate.ptr) : (shared ? shu.ptr : up.ptr);
    const uint64_t estride = isg ? (shared ? shg.stride : gate.stride) : (shared ? shu.stride : up.stride);
    const uint32_t rb = isg ? (shared ? shg.row_bytes : gate.row_bytes) : (shared ? shu.row_bytes : up.row_bytes);
    const v4u* wp = reinterpret_cast<const v4u*>(base + (size_t)e * estride +
                                                 (size_t)(strip * 16 + (isg ? rr : rr - 16)) * rb + sb * 144);
    v4u wq[9];
#pragma unroll
    for (int i = 0; i < 9; i++) wq[i] = wp[i];

    extern __shared__ __align__(16) uint8_t smem[];
    // staged activation rows: every token's (xall), else the item's entries SCH at a time
    const uint32_t R = xall ? xall : (nr < SCH ? nr : SCH);
    int8_t* xq = (int8_t*)smem;                   // [R][NSB][XSB]
    float* xs = (float*)(smem + R * XP);          // [R][nb]
    float* xu = xs + R * nb;                      // [R][nb]
    float* hres = xu + R * nb;                    // [nr][32]
    uint32_t* xrow = (uint32_t*)(hres + nr * 32);  // [nr] staged row of entry i
    uint32_t* xtok = xrow + nr;                    // [nr] its token
    if (tid < nr) {
        const uint32_t t = item_token(ws, item, shared, tid);
        xrow[tid] = xall ? t : tid;
        xtok[tid] = t;
    }
    if (xall) {
        const uint32_t np = xall * PPR, ns = xall * nb;
#pragma unroll
        for (int c = 0; c < XV; c++) {
            const uint32_t i = tid + nthr * c;
            if (i < np) {
                const uint32_t o = (i % PPR) * 16;
                *reinterpret_cast<v4u*>(xq + (i / PPR) * XP + o + (o / 256) * 16) = xv[c];
            }
        }
#pragma unroll
        for (int c = 0; c < XS; c++) {
            const uint32_t i = tid + nthr * c;
            if (i < ns) {
                xs[i] = xsv[c];
                xu[i] = xuv[c];
            }
        }
        __syncthreads();
    }

    // (dd, mm) of the superblock's 8 sub-blocks
    const float d = h2f((uint16_t)(wq[0].x & 0xffff)), dmin = h2f((uint16_t)(wq[0].x >> 16));
    float ddv[8], mmv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int sc, mn;
        q4k_scale_min_w(wq[0].y, wq[0].z, wq[0].w, j, sc, mn);
        q4k_dm(d, dmin, sc, mn, ddv[j], mmv[j]);
    }

    // entries i0 .. i0 + NE - 1 (clamped to nr - 1; a clamped entry's result is not stored)
    auto run = [&](auto ne_tag, uint32_t i0, uint32_t c0) {
        constexpr int NE = decltype(ne_tag)::value;
        // the nibbles are extracted per pass, not hoisted out of the entry loop (64 more registers)
#pragma unroll
        for (int i = 1; i < 9; i++) asm volatile("" : "+v"(wq[i]));
        float dotv[NE][8], tv[NE][8], uv[NE][8];
#pragma unroll
        for (int n = 0; n < NE; n++) {
            // staged row (read from LDS: an index the compiler cannot fold keeps it from hoisting
            // every entry's x reads ahead, and the registers with them)
            const uint32_t ie = i0 + n < nr ? i0 + n : i0, i = xrow[ie] - (xall ? 0u : c0);
            const float4* s4 = reinterpret_cast<const float4*>(xs + i * nb + sb * 8);
            const float4* u4 = reinterpret_cast<const float4*>(xu + i * nb + sb * 8);
            const float4 s0 = s4[0], s1 = s4[1], u0 = u4[0], u1 = u4[1];
            const float sa[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
            const float ua[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                tv[n][j] = ddv[j] * sa[j];  // t = d * sx (gemv.rs:145)
                uv[n][j] = ua[j];
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int4* xa = reinterpret_cast<const int4*>(xq + i * XP + sb * XSB + 64 * c);
                const int4 x0 = xa[0], x1 = xa[1], x2 = xa[2], x3 = xa[3];
                const int xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                const int xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
                int d0 = 0, d1 = 0;
#pragma unroll
                for (int w = 0; w < 8; w++) {
                    const uint32_t qw = wq[1 + 2 * c + w / 4][w % 4];
                    d0 = sdot4((int)nib(qw, 0), xl[w], d0);
                    d1 = sdot4((int)nib(qw, 1), xh[w], d1);
                }
                dotv[n][2 * c] = (float)d0;
                dotv[n][2 * c + 1] = (float)d1;
            }
        }
        // the chain (gemv.rs:141-148) in block order across the row's lanes
        float acc[NE];
#pragma unroll
        for (int n = 0; n < NE; n++) acc[n] = 0.0f;
#pragma unroll
        for (int st = 0; st < NSB; st++) {
            float in[NE];
#pragma unroll
            for (int n = 0; n < NE; n++) in[n] = st > 0 ? lane_up<NSB>(acc[n]) : 0.0f;
            if (sb == (uint32_t)st) {
#pragma unroll
                for (int n = 0; n < NE; n++) {
                    float a = in[n];
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        a = __builtin_fmaf(mmv[j], uv[n][j], a);
                        a = __builtin_fmaf(dotv[n][j], tv[n][j], a);
                    }
                    acc[n] = a;
                }
            }
        }
        if (wthread && sb == NSB - 1)
#pragma unroll
            for (int n = 0; n < NE; n++)
                if (i0 + n < nr) hres[(i0 + n) * 32 + r] = acc[n];
    };
#pragma nounroll
    for (uint32_t c0 = 0; c0 < nr; c0 += R) {  // one pass when xall or nr <= SCH
        const uint32_t c1 = nr - c0 < R ? nr : c0 + R;
        if (!xall) {
            __syncthreads();  // xtok written; the previous chunk's rows read
            stage_rows<true>(ws.xq, ws.xs, ws.xu, xtok + c0, c1 - c0, H, nb, XP, xq, xs, xu, tid, nthr);
            __syncthreads();
        }
        uint32_t i0 = c0;
#pragma nounroll
        for (; i0 + 1 < c1; i0 += 2) run(std::integral_constant<int, 2>{}, i0, c0);
        if (i0 < c1) run(std::integral_constant<int, 1>{}, i0, c0);
    }
    __syncthreads();

    // SwiGLU (elem.rs:173), per-16 quantisation of the strip (16 lanes = one DPP row per entry)
    // and the weight fold (exec_batch.rs:1528-1536)
    const uint32_t n_ent = ws.n_groups[1];
    for (uint32_t j0 = 0; j0 < nr; j0 += nthr / 16) {
        const uint32_t i = j0 + tid / 16, c16 = tid % 16;
        if (i < nr) {
            const float v = silu512(hres[i * 32 + c16]) * hres[i * 32 + 16 + c16];
            const float amax = row16_allreduce(__builtin_fabsf(v), [](float a, float b) { return mx_ps(a, b); });
            const float s = amax / 127.0f;
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            const int32_t qi = cvt_rne(v * inv);
            const int32_t sum = row16_allreduce(qi, [](int32_t a, int32_t b) { return a + b; });
            const uint32_t arow = shared ? n_ent + item.row0 + i : item.row0 + i;
            ws.actq[(size_t)arow * F + strip * 16 + c16] = sat_i8(qi);
            if (c16 == 0) {
                const float wgt = shared ? sigmoid_libm(ws.shl[item.row0 + i]) : ws.ent_w[item.row0 + i];
                const float sf = s * wgt;
                ws.acts[(size_t)arow * nbf + strip] = sf;
                ws.actsum[(size_t)arow * nbf + strip] = sum;
                ws.actu[(size_t)arow * nbf + strip] = sf * (float)sum;
            }
        }
    }
}

// ---- down -------------------------------------------------------------------------------------
//
// Grid (ceil(H / rows per workgroup), items), 256 threads: a row's 16-blocks are split over
// L = 2 * NSBF lanes, half a superblock each, in chain order (rows never straddle a wave); each
// lane holds its half superblock and runs every entry of the item against it, two at a time.
// Outputs are the per-entry rows of yent, combined later in the reference's order.
// FK: 0 Q4_K, 1 Q6_K, 2 Q8_0, 3 Q5_1
template <int NSBF, int FK>
__global__ __launch_bounds__(256) void stream_down_kernel(Mat down, Mat shd, Workspace ws, uint32_t max_rows) {
    constexpr uint32_t F = NSBF * 256, nbf = NSBF * 16, L = 2 * NSBF, RPW = 64 / L, RPB = 4 * RPW, SQ = F + 16;
    Item item;
    if (!stream_item(ws, blockIdx.y, max_rows, item)) return;
    const uint32_t H = down.rows, tid = threadIdx.x, ln = tid % 64, q = ln % L, sb = q / 2, h2 = q % 2;
    const bool shared = item.expert == NO_EXPERT;
    const uint32_t nr = item.nrows, e = shared ? 0u : item.expert;
    const uint32_t rloc = ln < RPW * L ? (tid / 64) * RPW + ln / L : RPB;
    const uint32_t row = blockIdx.x * RPB + (rloc < RPB ? rloc : 0u);
    const bool live = rloc < RPB && row < H;
    const uint32_t rowc = row < H ? row : H - 1;
    const uint8_t* rowp = (shared ? shd.ptr : down.ptr) + (size_t)e * (shared ? shd.stride : down.stride) +
                          (size_t)rowc * (shared ? shd.row_bytes : down.row_bytes);
    using W = typename std::conditional<
            FK == 1, Q6Half,
            typename std::conditional<FK == 2, Q8Half,
                                      typename std::conditional<FK == 3, Q51Half, v4u[5]>::type>::type>::type;
    W w;
    if constexpr (FK == 1) {
        load_half_q6k(rowp, sb, h2, w);
    } else if constexpr (FK == 2) {
        load_half_q80(rowp, sb, h2, w);
    } else if constexpr (FK == 3) {
        load_half_q51(rowp, sb, h2, w);
    } else {
        const v4u* p = reinterpret_cast<const v4u*>(rowp + sb * 144);
        w[0] = p[0];
#pragma unroll
        for (int i = 0; i < 4; i++) w[1 + i] = p[1 + 4 * h2 + i];
    }

    extern __shared__ __align__(16) uint8_t smem[];
    int8_t* aq = (int8_t*)smem;             // [nr][SQ]
    float* as = (float*)(smem + nr * SQ);   // [nr][nbf] folded scales
    float* au = as + nr * nbf;              // [nr][nbf] scale * sum
    uint32_t* arows = (uint32_t*)(au + nr * nbf);
    const uint32_t arow0 = shared ? ws.n_groups[1] + item.row0 : item.row0;
    if (tid < nr) arows[tid] = arow0 + tid;
    __syncthreads();
    stage_rows<false>(ws.actq, ws.acts, ws.actu, arows, nr, F, nbf, SQ, aq, as, au, tid, 256);
    __syncthreads();

    const uint32_t b0 = 8 * q;  // this lane's first 16-block
    auto run = [&](auto ne_tag, uint32_t i0) {
        constexpr int NE = decltype(ne_tag)::value;
        float dotv[NE][1][8], tv[NE][1][8], uv[NE][1][8], mmv[8];
#pragma unroll
        for (int n = 0; n < NE; n++) {
            const uint32_t i = i0 + n < nr ? i0 + n : nr - 1;
            const int8_t* a = aq + i * SQ + b0 * 16;
            if constexpr (FK == 1) {
                half_terms_q6k<1>(w, a, F, as + i * nbf + b0, au + i * nbf + b0, nbf, dotv[n], tv[n], mmv, uv[n]);
            } else if constexpr (FK == 2) {
                half_terms_q80<1>(w, a, F, as + i * nbf + b0, au + i * nbf + b0, nbf, dotv[n], tv[n], mmv, uv[n]);
            } else if constexpr (FK == 3) {
                half_terms_q51<1>(w, a, F, as + i * nbf + b0, au + i * nbf + b0, nbf, dotv[n], tv[n], mmv, uv[n]);
            } else {
                const uint4 hdr = make_uint4(w[0].x, w[0].y, w[0].z, w[0].w);
                const uint4 qs[4] = {make_uint4(w[1].x, w[1].y, w[1].z, w[1].w),
                                     make_uint4(w[2].x, w[2].y, w[2].z, w[2].w),
                                     make_uint4(w[3].x, w[3].y, w[3].z, w[3].w),
                                     make_uint4(w[4].x, w[4].y, w[4].z, w[4].w)};
                half_terms_q4k<1>(hdr, qs, h2, a, F, as + i * nbf + b0, au + i * nbf + b0, nbf, dotv[n], tv[n], mmv,
                                  uv[n]);
            }
        }
        float acc[NE];
#pragma unroll
        for (int n = 0; n < NE; n++) acc[n] = 0.0f;
#pragma unroll
        for (int st = 0; st < (int)L; st++) {
            float in[NE];
#pragma unroll
            for (int n = 0; n < NE; n++) in[n] = st > 0 ? unit_up<L>(acc[n]) : 0.0f;
            if (q == (uint32_t)st) {
#pragma unroll
                for (int n = 0; n < NE; n++) {
                    float v = in[n];
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        v = __builtin_fmaf(mmv[j], uv[n][0][j], v);
                        v = __builtin_fmaf(dotv[n][0][j], tv[n][0][j], v);
                    }
                    acc[n] = v;
                }
            }
        }
        if (live && q == L - 1)
#pragma unroll
            for (int n = 0; n < NE; n++)
                if (i0 + n < nr) ws.yent[(size_t)(arow0 + i0 + n) * H + row] = acc[n];
    };
    uint32_t i0 = 0;
    for (; i0 + 1 < nr; i0 += 2) run(std::integral_constant<int, 2>{}, i0);
    if (i0 < nr) run(std::integral_constant<int, 1>{}, i0);
}

// Work-item rows of a launch: every item has at least one entry row, so a batch of m tokens has
// at most m * k_cap routed items and ceil(m / 16) shared ones.
static uint32_t item_rows(const Workspace& ws, uint32_t m) {
    const uint64_t bound = (uint64_t)m * ws.k_cap + (m + BR - 1) / BR;
    return bound < ws.item_cap ? (uint32_t)bound : ws.item_cap;
}

uint32_t grouped_item_rows(const Workspace& ws, uint32_t m) { return item_rows(ws, m); }

hipError_t launch_stream_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up,
                                const Workspace& ws, uint32_t m, uint32_t max_rows, hipStream_t st) {
    const uint32_t H = gate.k, F = gate.rows, nsb = H / 256, nb = H / 32;
    const size_t cap = max_rows < BR ? max_rows : BR;  // rows of an item here
    // up to 4 tokens every token's x is staged up front (within the kernel's register budget for
    // it: 8 pieces and 4 scales per thread)
    uint32_t xall = m <= 4 ? m : 0u;
    const uint32_t threads = GU_THREADS(nsb);
    if ((size_t)xall * (H / 16) > 8u * threads || (size_t)xall * nb > 4u * threads) xall = 0;
    const size_t rows = xall ? xall : (cap < 4 ? cap : 4);  // staged rows (4 per pass: SCH)
    const size_t lds = rows * ((size_t)nsb * 272 + (size_t)nb * 8) + cap * (32 * 4 + 8);
    const dim3 grid(F / 16, item_rows(ws, m));
    switch (nsb) {
#define SG_CASE(n)                                                                                      \
    case n:                                                                                             \
        stream_gateup_kernel<n><<<grid, GU_THREADS(n), lds, st>>>(gate, up, sh_gate, sh_up, ws, max_rows, xall); \
        break;
        SG_CASE(1) SG_CASE(2) SG_CASE(3) SG_CASE(4) SG_CASE(5) SG_CASE(6) SG_CASE(7) SG_CASE(8)
#undef SG_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_stream_down(const Mat& down, const Mat& sh_down, const Workspace& ws, uint32_t m,
                              uint32_t max_rows, hipStream_t st) {
    const uint32_t H = down.rows, F = down.k, nsbf = F / 256, nbf = F / 16;
    if (down.fmt != sh_down.fmt) return hipErrorInvalidValue;  // one format per layer
    const int fk = down.fmt == TRK_FMT_Q6_K ? 1 : down.fmt == TRK_FMT_Q8_0 ? 2 : down.fmt == TRK_FMT_Q5_1 ? 3 : 0;
    const size_t cap = max_rows < BR ? max_rows : BR;
    const size_t lds = cap * ((size_t)F + 16 + (size_t)nbf * 8 + 4);
    const dim3 grid(geo::stream_down_cols(H, F), item_rows(ws, m));
    switch (nsbf * 4 + fk) {
#define SD_CASE(n)                                                                                        \
    case n * 4: stream_down_kernel<n, 0><<<grid, 256, lds, st>>>(down, sh_down, ws, max_rows); break;     \
    case n * 4 + 1: stream_down_kernel<n, 1><<<grid, 256, lds, st>>>(down, sh_down, ws, max_rows); break; \
    case n * 4 + 2: stream_down_kernel<n, 2><<<grid, 256, lds, st>>>(down, sh_down, ws, max_rows); break; \
    case n * 4 + 3: stream_down_kernel<n, 3><<<grid, 256, lds, st>>>(down, sh_down, ws, max_rows); break;
        SD_CASE(1) SD_CASE(2) SD_CASE(3) SD_CASE(4) SD_CASE(5) SD_CASE(6) SD_CASE(7) SD_CASE(8)
#undef SD_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace trk
