// Decode path (M = 1): Model::moe_block (crates/tr-model/src/exec.rs:1540-1623).
//
// Two kernels after routing:
//   gate/up: one workgroup per (slot, 16-row strip of F).  It streams the 16 gate rows and 16 up
//            rows of its expert straight from their Q4_K superblocks, forms the exact int32 dot of
//            every 32-block against the (two-level) int8 activations, runs the reference's
//            sequential per-block f32 epilogue per row, and — because the down input is quantised
//            per 16 — finishes SwiGLU, the (pair) requantisation and the routing-weight fold for
//            its 16-wide block on the spot (tasks A and B of moe_block).
//   down:    one workgroup per 4 output rows, all slots: per-slot chains as the reference's
//            gemv_tq, then slot 0 stored and later slots (routing order, shared last) added —
//            the combine of tasks C, fused.
#include "common.hpp"

namespace trk {

constexpr int GU_ROWS = 32;  // 16 gate + 16 up rows per workgroup
constexpr int DN_R = 4;      // output rows per down workgroup

// dot of 8 u4 lanes packed in a dword pair... helpers for a Q4_K superblock in registers:
// qs[32] dwords; sub-block j = 2c + h uses nibble h of dwords 8c .. 8c+7.
__device__ __forceinline__ uint32_t nib(uint32_t w, int h) { return (w >> (4 * h)) & 0x0f0f0f0fu; }

template <int P>
__global__ __launch_bounds__(256) void decode_gateup_kernel(Mat gate, Mat up, Mat shg, Mat shu, Workspace ws,
                                                           uint32_t kcap) {
    const uint32_t H = gate.k, nsb = H / 256, nb = H / 32;
    const uint32_t slot = blockIdx.y, strip = blockIdx.x, tid = threadIdx.x;
    const uint32_t n = ws.n_sel[0];
    const bool shared = slot == kcap;
    if (!shared && slot >= n) return;
    const uint32_t e = shared ? 0u : ws.ids[slot];
    const Mat& G = shared ? shg : gate;
    const Mat& U = shared ? shu : up;
    const uint8_t* gb = G.ptr + (size_t)e * G.stride + (size_t)strip * 16 * G.row_bytes;
    const uint8_t* ub = U.ptr + (size_t)e * U.stride + (size_t)strip * 16 * U.row_bytes;

    extern __shared__ __align__(16) uint8_t smem[];
    int8_t* xq = (int8_t*)smem;                       // [P][H]
    float* xs = (float*)(smem + P * H);               // [P][nb]
    int32_t* xsu = (int32_t*)(xs + P * nb);           // [P][nb]
    int32_t* dots = xsu + P * nb;                     // [32][nb][P]
    float* dd = (float*)(dots + GU_ROWS * nb * P);    // [32][nb]
    float* mm = dd + GU_ROWS * nb;                    // [32][nb]
    float* hres = mm + GU_ROWS * nb;                  // [32][P]
    float* act = hres + GU_ROWS * P;                  // [16]

    for (uint32_t i = tid; i < P * H / 16; i += blockDim.x)
        reinterpret_cast<int4*>(xq)[i] = reinterpret_cast<const int4*>(ws.xq)[i];
    for (uint32_t i = tid; i < P * nb; i += blockDim.x) {
        xs[i] = ws.xs[i];
        xsu[i] = ws.xsum[i];
    }
    __syncthreads();

    for (uint32_t it = tid; it < GU_ROWS * nsb; it += blockDim.x) {
        const uint32_t r = it / nsb, sb = it % nsb;
        const uint8_t* sp = (r < 16 ? gb + (size_t)r * G.row_bytes : ub + (size_t)(r - 16) * U.row_bytes) + sb * 144;
        const uint4* s4 = reinterpret_cast<const uint4*>(sp);
        uint4 hdr = s4[0];
        uint32_t qs[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint4 t = s4[1 + i];
            qs[4 * i] = t.x; qs[4 * i + 1] = t.y; qs[4 * i + 2] = t.z; qs[4 * i + 3] = t.w;
        }
        const uint8_t* hb = reinterpret_cast<const uint8_t*>(&hdr);
        float d = h2f((uint16_t)(hdr.x & 0xffff)), dmin = h2f((uint16_t)(hdr.x >> 16));
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            q4k_scale_min(hb + 4, j, sc, mn);
            float a, b;
            q4k_dm(d, dmin, sc, mn, a, b);
            dd[r * nb + sb * 8 + j] = a;
            mm[r * nb + sb * 8 + j] = b;
        }
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int* xw = reinterpret_cast<const int*>(xq + p * H + sb * 256);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                int d0 = 0, d1 = 0;
#pragma unroll
                for (int w = 0; w < 8; w++) {
                    uint32_t q = qs[8 * c + w];
                    d0 = sdot4((int)nib(q, 0), xw[(2 * c) * 8 + w], d0);
                    d1 = sdot4((int)nib(q, 1), xw[(2 * c + 1) * 8 + w], d1);
                }
                dots[(r * nb + sb * 8 + 2 * c) * P + p] = d0;
                dots[(r * nb + sb * 8 + 2 * c + 1) * P + p] = d1;
            }
        }
    }
    __syncthreads();

    // per-row sequential epilogue (gemv.rs:141-148), one thread per (row, activation row)
    if (tid < GU_ROWS * P) {
        const uint32_t r = tid / P, p = tid % P;
        float acc = 0.0f;
        for (uint32_t b = 0; b < nb; b++) {
            float sx = xs[p * nb + b];
            float u = sx * (float)xsu[p * nb + b];
            float t = dd[r * nb + b] * sx;
            acc = __builtin_fmaf(mm[r * nb + b], u, acc);
            acc = __builtin_fmaf((float)dots[(r * nb + b) * P + p], t, acc);
        }
        hres[r * P + p] = acc;
    }
    __syncthreads();
    if (tid < 16) {
        // pair rows: coarse + residual (gemv.rs:154); then act = silu512(g) * u (elem.rs:173)
        float g = P == 2 ? hres[tid * P] + hres[tid * P + 1] : hres[tid * P];
        float u = P == 2 ? hres[(16 + tid) * P] + hres[(16 + tid) * P + 1] : hres[(16 + tid) * P];
        act[tid] = silu512(g) * u;
    }
    __syncthreads();
    if (tid == 0) {
        // quantise the 16-block (kb = down.kb = 16) and fold the weight into the scales
        // (exec.rs:1590-1605)
        const float wgt = shared ? sigmoid_libm(ws.shl[0]) : ws.w[slot];
        const uint32_t aslot = shared ? (uint32_t)SH_SLOT : slot;
        const uint32_t F = gate.rows, nbf = F / 16;
        float v[16], res[16];
        int8_t q0[16], q1[16];
        for (int i = 0; i < 16; i++) v[i] = act[i];
        float s0, s1;
        int32_t m0, m1;
        quant_block_regs<16>(v, q0, s0, m0, P == 2 ? res : nullptr);
        int8_t* dq = ws.actq + (size_t)aslot * P * F;
        float* ds = ws.acts + (size_t)aslot * P * nbf;
        int32_t* dsu = ws.actsum + (size_t)aslot * P * nbf;
        for (int i = 0; i < 16; i++) dq[strip * 16 + i] = q0[i];
        ds[strip] = s0 * wgt;
        dsu[strip] = m0;
        if (P == 2) {
            quant_block_regs<16>(res, q1, s1, m1, nullptr);
            for (int i = 0; i < 16; i++) dq[F + strip * 16 + i] = q1[i];
            ds[nbf + strip] = s1 * wgt;
            dsu[nbf + strip] = m1;
        }
    }
}

hipError_t launch_decode_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up,
                                const Workspace& ws, int pair, uint32_t kcap, hipStream_t st) {
    const uint32_t H = gate.k, F = gate.rows, nb = H / 32;
    const int P = pair ? 2 : 1;
    size_t lds = (size_t)P * H + (size_t)P * nb * 8 + (size_t)GU_ROWS * nb * P * 4 + (size_t)GU_ROWS * nb * 8 +
                 GU_ROWS * P * 4 + 64;
    dim3 g(F / 16, kcap + 1);
    if (pair)
        decode_gateup_kernel<2><<<g, 256, lds, st>>>(gate, up, sh_gate, sh_up, ws, kcap);
    else
        decode_gateup_kernel<1><<<g, 256, lds, st>>>(gate, up, sh_gate, sh_up, ws, kcap);
    return hipGetLastError();
}

// ---- down ------------------------------------------------------------------------------------

// Q4_K superblock (144 B, 16-byte aligned) -> 16 blocks of 16: dot against x (int8, 256 values)
// and the block's (dd, mm); block j16 is half (j16 & 1) of sub-block j16 / 2.
template <int P>
__device__ __forceinline__ void q4k_sb_dots16(const uint8_t* sp, const int8_t* const* x, int* dots /*[16][P]*/,
                                              float* dd, float* mm) {
    const uint4* s4 = reinterpret_cast<const uint4*>(sp);
    uint4 hdr = s4[0];
    uint32_t qs[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint4 t = s4[1 + i];
        qs[4 * i] = t.x; qs[4 * i + 1] = t.y; qs[4 * i + 2] = t.z; qs[4 * i + 3] = t.w;
    }
    const uint8_t* hb = reinterpret_cast<const uint8_t*>(&hdr);
    float d = h2f((uint16_t)(hdr.x & 0xffff)), dmin = h2f((uint16_t)(hdr.x >> 16));
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int sc, mn;
        q4k_scale_min(hb + 4, j, sc, mn);
        float a, b;
        q4k_dm(d, dmin, sc, mn, a, b);
        dd[2 * j] = dd[2 * j + 1] = a;
        mm[2 * j] = mm[2 * j + 1] = b;
        const int c = j / 2, h = j % 2;
#pragma unroll
        for (int half = 0; half < 2; half++) {
#pragma unroll
            for (int p = 0; p < P; p++) {
                const int* xw = reinterpret_cast<const int*>(x[p] + j * 32 + half * 16);
                int acc = 0;
#pragma unroll
                for (int w = 0; w < 4; w++) acc = sdot4((int)nib(qs[8 * c + 4 * half + w], h), xw[w], acc);
                dots[(2 * j + half) * P + p] = acc;
            }
        }
    }
}

// Q6_K superblock (210 B, 2-byte aligned) -> 16 blocks of 16 (the extension mapping: unsigned
// 6-bit q, dd = f16(d*sc), mm = f16(-32*dd)).
template <int P>
__device__ __forceinline__ void q6k_sb_dots16(const uint8_t* sp, const int8_t* const* x, int* dots, float* dd,
                                              float* mm) {
    const uint16_t* s2 = reinterpret_cast<const uint16_t*>(sp);
    uint16_t w16[105];
#pragma unroll
    for (int i = 0; i < 105; i++) w16[i] = s2[i];
    auto dw = [&](int o) -> uint32_t { return (uint32_t)w16[o >> 1] | ((uint32_t)w16[(o >> 1) + 1] << 16); };
    float d = h2f(w16[104]);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int8_t sc = (int8_t)((w16[(192 + j) >> 1] >> (((192 + j) & 1) * 8)) & 0xff);
        float a = f16_round(d * (float)sc);
        dd[j] = a;
        mm[j] = f16_round(-32.0f * a);
        const int n = j / 8, g = (j % 8) / 2, l0 = 16 * (j % 2);
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int* xw = reinterpret_cast<const int*>(x[p] + j * 16);
            int acc = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                uint32_t lo = dw(64 * n + 32 * (g & 1) + l0 + 4 * t);
                lo = (g >> 1) ? ((lo >> 4) & 0x0f0f0f0fu) : (lo & 0x0f0f0f0fu);
                uint32_t hi = (dw(128 + 32 * n + l0 + 4 * t) >> (2 * g)) & 0x03030303u;
                acc = sdot4((int)(lo | (hi << 4)), xw[t], acc);
            }
            dots[j * P + p] = acc;
        }
    }
}

template <int P>
__global__ __launch_bounds__(256) void decode_down_kernel(Mat down, Mat shd, Workspace ws, float* __restrict__ out,
                                                         int residual) {
    const uint32_t F = down.k, nsb = F / 256, nbf = F / 16;
    const uint32_t tid = threadIdx.x, row0 = blockIdx.x * DN_R;
    const uint32_t n = ws.n_sel[0], slots = n + 1;

    extern __shared__ __align__(16) uint8_t smem[];
    int8_t* aq = (int8_t*)smem;                                // [slots][P][F]
    float* as = (float*)(smem + (size_t)slots * P * F);        // [slots][P][nbf]
    int32_t* asu = (int32_t*)(as + slots * P * nbf);           // [slots][P][nbf]
    int32_t* dots = asu + slots * P * nbf;                     // [slots][R][nbf][P]
    float* dd = (float*)(dots + slots * DN_R * nbf * P);       // [slots][R][nbf]
    float* mm = dd + slots * DN_R * nbf;                       // [slots][R][nbf]
    float* vres = mm + slots * DN_R * nbf;                     // [slots][R][P]

    for (uint32_t s = 0; s < slots; s++) {
        const uint32_t as_ = s < n ? s : (uint32_t)SH_SLOT;
        const int4* src = reinterpret_cast<const int4*>(ws.actq + (size_t)as_ * P * F);
        int4* dst = reinterpret_cast<int4*>(aq + (size_t)s * P * F);
        for (uint32_t i = tid; i < P * F / 16; i += blockDim.x) dst[i] = src[i];
        for (uint32_t i = tid; i < P * nbf; i += blockDim.x) {
            as[s * P * nbf + i] = ws.acts[(size_t)as_ * P * nbf + i];
            asu[s * P * nbf + i] = ws.actsum[(size_t)as_ * P * nbf + i];
        }
    }
    __syncthreads();

    const uint32_t items = slots * DN_R * nsb;
    for (uint32_t it = tid; it < items; it += blockDim.x) {
        const uint32_t s = it / (DN_R * nsb), r = (it / nsb) % DN_R, sb = it % nsb;
        const Mat& D = s < n ? down : shd;
        const uint32_t e = s < n ? ws.ids[s] : 0u;
        const uint8_t* rowp = D.ptr + (size_t)e * D.stride + (size_t)(row0 + r) * D.row_bytes;
        const int8_t* xp[P];
#pragma unroll
        for (int p = 0; p < P; p++) xp[p] = aq + ((size_t)s * P + p) * F + sb * 256;
        int dl[16 * P];
        float ddl[16], mml[16];
        if (D.fmt == TRK_FMT_Q4_K)
            q4k_sb_dots16<P>(rowp + sb * 144, xp, dl, ddl, mml);
        else
            q6k_sb_dots16<P>(rowp + sb * 210, xp, dl, ddl, mml);
        const uint32_t base = (s * DN_R + r) * nbf + sb * 16;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            dd[base + j] = ddl[j];
            mm[base + j] = mml[j];
#pragma unroll
            for (int p = 0; p < P; p++) dots[(base + j) * P + p] = dl[j * P + p];
        }
    }
    __syncthreads();

    for (uint32_t t = tid; t < slots * DN_R * P; t += blockDim.x) {
        const uint32_t s = t / (DN_R * P), r = (t / P) % DN_R, p = t % P;
        const uint32_t base = (s * DN_R + r) * nbf;
        float acc = 0.0f;
        for (uint32_t b = 0; b < nbf; b++) {
            float sx = as[(s * P + p) * nbf + b];
            float u = sx * (float)asu[(s * P + p) * nbf + b];
            float tt = dd[base + b] * sx;
            acc = __builtin_fmaf(mm[base + b], u, acc);
            acc = __builtin_fmaf((float)dots[(base + b) * P + p], tt, acc);
        }
        vres[(s * DN_R + r) * P + p] = acc;
    }
    __syncthreads();
    if (tid < DN_R) {
        // slot 0 stores, later slots accumulate (gemv.rs:150-160 with accumulate = slot > 0)
        const uint32_t r = tid;
        float y = 0.0f;
        for (uint32_t s = 0; s < slots; s++) {
            const float* v = vres + (s * DN_R + r) * P;
            float vs = P == 2 ? v[0] + v[1] : v[0];
            y = s == 0 ? vs : y + vs;
        }
        float* o = out + row0 + r;
        *o = residual ? *o + y : y;
    }
}

hipError_t launch_decode_down(const Mat& down, const Mat& sh_down, const Workspace& ws, int pair, uint32_t kcap,
                              float* out, int residual, hipStream_t st) {
    const uint32_t H = down.rows, F = down.k, nbf = F / 16;
    const int P = pair ? 2 : 1;
    const size_t slots = kcap + 1;
    size_t lds = slots * P * F + slots * P * nbf * 8 + slots * DN_R * nbf * P * 4 + slots * DN_R * nbf * 8 +
                 slots * DN_R * P * 4 + 64;
    if (pair)
        decode_down_kernel<2><<<H / DN_R, 256, lds, st>>>(down, sh_down, ws, out, residual);
    else
        decode_down_kernel<1><<<H / DN_R, 256, lds, st>>>(down, sh_down, ws, out, residual);
    return hipGetLastError();
}

}  // namespace trk
