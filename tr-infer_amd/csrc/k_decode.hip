// Decode path (M = 1): Model::moe_block (crates/tr-model/src/exec.rs:1540-1623).
//
//   gate/up: one workgroup per (slot, 16-row strip of F).  Each thread issues the loads of one
//            (row, superblock) of the 16 gate + 16 up rows straight from their Q4_K superblocks,
//            and while they fly the first nb threads quantise x (two-level, per 32) into LDS —
//            every workgroup does this itself, so no separate quantisation launch.  The exact
//            int32 dot of every 32-block goes to LDS, one thread per (row, activation row) runs
//            the reference's sequential per-block f32 epilogue from b128 LDS reads, and since
//            the down input is quantised per 16, SwiGLU, the (pair) requantisation and the
//            routing-weight fold of the strip's 16-wide block finish in the same workgroup
//            (tasks A and B of moe_block).
//   down:    one workgroup per 8 output rows, all slots: a thread per (slot, row) streams the
//            row's superblocks, forms the per-16 block dots against the staged activations and
//            runs the chain in registers; slot 0 is stored and later slots (routing order,
//            shared last) are added — tasks C with the combine fused.
#include "common.hpp"

namespace trk {

constexpr int GU_ROWS = 32;  // 16 gate + 16 up rows per workgroup
constexpr int DN_R = 8;      // output rows per down workgroup

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

template <int P, int NSB>
__global__ __launch_bounds__(32 * NSB < 64 ? 64 : 32 * NSB) void decode_gateup_kernel(
        Mat gate, Mat up, Mat shg, Mat shu, const float* __restrict__ x, Workspace ws, uint32_t kcap) {
    constexpr uint32_t H = NSB * 256, nb = NSB * 8;
    const uint32_t F = gate.rows;
    const uint32_t slot = blockIdx.y, strip = blockIdx.x, tid = threadIdx.x;
    const bool shared = slot == kcap;
    extern __shared__ __align__(16) uint8_t smem[];
    int8_t* xq = (int8_t*)smem;              // [P][H]
    float* xs = (float*)(smem + P * H);      // [P][nb]  activation scales
    float* xu = xs + P * nb;                 // [P][nb]  sx * sum
    float* hres = xu + P * nb;               // [32][P]
    float* act = hres + 32 * P;              // [16]

    // x first: its loads must not queue behind the (id-dependent) weight loads
    float4 xv[8];
    const bool qthread = tid < nb;
    if (qthread) {
        const float4* src = reinterpret_cast<const float4*>(x + (size_t)tid * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = src[i];
    }
    const uint32_t n = ws.n_sel[0];
    if (!shared && slot >= n) return;
    const uint32_t e = shared ? 0u : ws.ids[slot];
    const Mat& G = shared ? shg : gate;
    const Mat& U = shared ? shu : up;
    const uint32_t r = tid / NSB, sb = tid % NSB;
    const bool wthread = r < 32;
    uint4 wq[9];
    {
        const uint32_t rr = wthread ? r : 0u;
        const uint8_t* rowp = (rr < 16 ? G.ptr + (size_t)e * G.stride + (size_t)(strip * 16 + rr) * G.row_bytes
                                       : U.ptr + (size_t)e * U.stride + (size_t)(strip * 16 + rr - 16) * U.row_bytes) +
                              sb * 144;
        const uint4* s4 = reinterpret_cast<const uint4*>(rowp);
#pragma unroll
        for (int i = 0; i < 9; i++) wq[i] = s4[i];
    }
    // quantise x per 32 (quantize_pair_blocks, quant.rs:96-108, or QAct::quantize) into LDS
    if (qthread) {
        const uint32_t b = tid;
        float v[32], rs[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[4 * i] = xv[i].x; v[4 * i + 1] = xv[i].y; v[4 * i + 2] = xv[i].z; v[4 * i + 3] = xv[i].w;
        }
        uint32_t q[8];
        float s;
        int32_t su;
        quant_block_regs<32, P == 2>(v, q, s, su, rs);
        *reinterpret_cast<uint4*>(xq + b * 32) = make_uint4(q[0], q[1], q[2], q[3]);
        *reinterpret_cast<uint4*>(xq + b * 32 + 16) = make_uint4(q[4], q[5], q[6], q[7]);
        xs[b] = s;
        xu[b] = s * (float)su;  // gemv.rs:144
        if (shared && strip == 0) {  // one workgroup publishes the quantised input (introspection)
            *reinterpret_cast<uint4*>(ws.xq + b * 32) = make_uint4(q[0], q[1], q[2], q[3]);
            *reinterpret_cast<uint4*>(ws.xq + b * 32 + 16) = make_uint4(q[4], q[5], q[6], q[7]);
            ws.xs[b] = s;
            ws.xsum[b] = su;
        }
        if (P == 2) {
            quant_block_regs<32>(rs, q, s, su);
            *reinterpret_cast<uint4*>(xq + H + b * 32) = make_uint4(q[0], q[1], q[2], q[3]);
            *reinterpret_cast<uint4*>(xq + H + b * 32 + 16) = make_uint4(q[4], q[5], q[6], q[7]);
            xs[nb + b] = s;
            xu[nb + b] = s * (float)su;
            if (shared && strip == 0) {
                *reinterpret_cast<uint4*>(ws.xq + H + b * 32) = make_uint4(q[0], q[1], q[2], q[3]);
                *reinterpret_cast<uint4*>(ws.xq + H + b * 32 + 16) = make_uint4(q[4], q[5], q[6], q[7]);
                ws.xs[nb + b] = s;
                ws.xsum[nb + b] = su;
            }
        }
    }
    __syncthreads();

    // this lane's 8 blocks: exact dots, (dd, mm), t = dd * sx and u from LDS
    const uint32_t* w32 = reinterpret_cast<const uint32_t*>(wq);  // [0..3] header, [4..35] qs
    const float d = h2f((uint16_t)(wq[0].x & 0xffff)), dmin = h2f((uint16_t)(wq[0].x >> 16));
    float mmv[8], tv[P][8], uv[P][8], dotv[P][8];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const float4* sp = reinterpret_cast<const float4*>(xs + p * nb + sb * 8);
        const float4* up4 = reinterpret_cast<const float4*>(xu + p * nb + sb * 8);
        const float4 s0 = sp[0], s1 = sp[1], u0 = up4[0], u1 = up4[1];
        const float sxa[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        const float ua[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            tv[p][j] = sxa[j];
            uv[p][j] = ua[j];
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int sc, mn;
        q4k_scale_min_w(wq[0].y, wq[0].z, wq[0].w, j, sc, mn);
        float ddv;
        q4k_dm(d, dmin, sc, mn, ddv, mmv[j]);
#pragma unroll
        for (int p = 0; p < P; p++) tv[p][j] = ddv * tv[p][j];  // t = d * sx (gemv.rs:145)
    }
#pragma unroll
    for (int p = 0; p < P; p++) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int4* xa = reinterpret_cast<const int4*>(xq + p * H + sb * 256 + 64 * c);  // sub-blocks 2c, 2c+1
            const int4 x0 = xa[0], x1 = xa[1], x2 = xa[2], x3 = xa[3];
            const int xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const int xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
            int d0 = 0, d1 = 0;
#pragma unroll
            for (int w = 0; w < 8; w++) {
                const uint32_t qw = w32[4 + 8 * c + w];
                d0 = sdot4((int)nib(qw, 0), xl[w], d0);
                d1 = sdot4((int)nib(qw, 1), xh[w], d1);
            }
            dotv[p][2 * c] = (float)d0;
            dotv[p][2 * c + 1] = (float)d1;
        }
    }
    // the chain (gemv.rs:141-148) in block order: superblock sb continues where sb-1 stopped
    float acc[P];
#pragma unroll
    for (int p = 0; p < P; p++) acc[p] = 0.0f;
#pragma unroll
    for (int st = 0; st < NSB; st++) {
        float in[P];
#pragma unroll
        for (int p = 0; p < P; p++) in[p] = st > 0 ? lane_up<NSB>(acc[p]) : 0.0f;
        if (sb == (uint32_t)st) {
#pragma unroll
            for (int p = 0; p < P; p++) {
                float a = in[p];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    a = __builtin_fmaf(mmv[j], uv[p][j], a);
                    a = __builtin_fmaf(dotv[p][j], tv[p][j], a);
                }
                acc[p] = a;
            }
        }
    }
    if (wthread && sb == NSB - 1)
#pragma unroll
        for (int p = 0; p < P; p++) hres[r * P + p] = acc[p];
    __syncthreads();
    if (tid < 16) {
        // pair rows: coarse + residual (gemv.rs:154); act = silu512(g) * u (elem.rs:173); then
        // quantise the 16-block (kb = down.kb = 16) across these 16 lanes and fold the weight
        // into the scales (exec.rs:1590-1605)
        const float g = P == 2 ? hres[tid * P] + hres[tid * P + 1] : hres[tid * P];
        const float u = P == 2 ? hres[(16 + tid) * P] + hres[(16 + tid) * P + 1] : hres[(16 + tid) * P];
        const float av = silu512(g) * u;
        const float wgt = shared ? sigmoid_libm(ws.shl[0]) : ws.w[slot];
        const uint32_t aslot = shared ? (uint32_t)SH_SLOT : slot;
        const uint32_t nbf = F / 16;
        int8_t* dq = ws.actq + (size_t)aslot * P * F + strip * 16;
        float* ds = ws.acts + (size_t)aslot * P * nbf + strip;
        int32_t* dsu = ws.actsum + (size_t)aslot * P * nbf + strip;
        float v = av;
#pragma unroll
        for (int p = 0; p < P; p++) {
            float amax = __builtin_fabsf(v);
            amax = mx_ps(amax, __shfl_xor(amax, 1, 16));
            amax = mx_ps(amax, __shfl_xor(amax, 2, 16));
            amax = mx_ps(amax, __shfl_xor(amax, 4, 16));
            amax = mx_ps(amax, __shfl_xor(amax, 8, 16));
            const float sc = amax / 127.0f;
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            const int32_t qi = cvt_rne(v * inv);
            int32_t sum = qi;
            sum += __shfl_xor(sum, 1, 16);
            sum += __shfl_xor(sum, 2, 16);
            sum += __shfl_xor(sum, 4, 16);
            sum += __shfl_xor(sum, 8, 16);
            dq[p * F + tid] = sat_i8(qi);
            if (tid == 0) {
                ds[p * nbf] = sc * wgt;
                dsu[p * nbf] = sum;
            }
            v = __builtin_fmaf(-(float)qi, sc, v);  // residual for the second level (quant.rs:132)
        }
    }
}

hipError_t launch_decode_gateup(const Mat& gate, const Mat& up, const Mat& sh_gate, const Mat& sh_up, const float* x,
                                const Workspace& ws, int pair, uint32_t kcap, hipStream_t st) {
    const uint32_t H = gate.k, F = gate.rows, nb = H / 32, nsb = H / 256;
    const int P = pair ? 2 : 1;
    const size_t lds = (size_t)P * H + (size_t)P * nb * 8 + 32 * P * 4 + 64;
    const dim3 g(F / 16, kcap + 1);
    const uint32_t threads = 32 * nsb < 64 ? 64 : 32 * nsb;
    switch (nsb * 2 + (pair ? 1 : 0)) {
#define GU_CASE(ns) \
    case ns * 2: decode_gateup_kernel<1, ns><<<g, threads, lds, st>>>(gate, up, sh_gate, sh_up, x, ws, kcap); break; \
    case ns * 2 + 1: decode_gateup_kernel<2, ns><<<g, threads, lds, st>>>(gate, up, sh_gate, sh_up, x, ws, kcap); break;
        GU_CASE(1) GU_CASE(2) GU_CASE(3) GU_CASE(4) GU_CASE(5) GU_CASE(6) GU_CASE(7) GU_CASE(8)
#undef GU_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- down ------------------------------------------------------------------------------------

// One (slot, row) of the down projection: the row's superblocks in order, 16 blocks of 16 each,
// per-block epilogue chain for P activation rows kept in registers.  All NSB superblocks of the
// row are loaded before any is used.
template <int P, int NSB>
__device__ __forceinline__ void down_row_chain_q4k(const uint8_t* __restrict__ rowp,
                                                  const int8_t* __restrict__ aq /*[P][F]*/, uint32_t F,
                                                  const float* __restrict__ as, const float* __restrict__ au,
                                                  uint32_t nbf, float* acc) {
    uint4 wq[NSB][9];
#pragma unroll
    for (int sb = 0; sb < NSB; sb++)
#pragma unroll
        for (int i = 0; i < 9; i++) wq[sb][i] = reinterpret_cast<const uint4*>(rowp + sb * 144)[i];
#pragma unroll
    for (int sb = 0; sb < NSB; sb++) {
        const uint32_t* w32 = reinterpret_cast<const uint32_t*>(wq[sb]);
        const float d = h2f((uint16_t)(wq[sb][0].x & 0xffff)), dmin = h2f((uint16_t)(wq[sb][0].x >> 16));
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            q4k_scale_min_w(wq[sb][0].y, wq[sb][0].z, wq[sb][0].w, j, sc, mn);
            float ddv, mmv;
            q4k_dm(d, dmin, sc, mn, ddv, mmv);
            const int c = j / 2, h = j % 2;
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const uint32_t b = sb * 16 + 2 * j + half;
#pragma unroll
                for (int p = 0; p < P; p++) {
                    const int4 xv = *reinterpret_cast<const int4*>(aq + p * F + b * 16);
                    int dot = sdot4((int)nib(w32[4 + 8 * c + 4 * half + 0], h), xv.x, 0);
                    dot = sdot4((int)nib(w32[4 + 8 * c + 4 * half + 1], h), xv.y, dot);
                    dot = sdot4((int)nib(w32[4 + 8 * c + 4 * half + 2], h), xv.z, dot);
                    dot = sdot4((int)nib(w32[4 + 8 * c + 4 * half + 3], h), xv.w, dot);
                    const float sx = as[p * nbf + b];
                    const float t = ddv * sx;
                    acc[p] = __builtin_fmaf(mmv, au[p * nbf + b], acc[p]);
                    acc[p] = __builtin_fmaf((float)dot, t, acc[p]);
                }
            }
        }
    }
}

// Q6_K rows (210-byte superblocks, 2-byte aligned): the extension mapping — unsigned 6-bit q,
// dd = f16(d*sc), mm = f16(-32*dd), one block per scale (16 values).
template <int P>
__device__ __forceinline__ void down_row_chain_q6k(const uint8_t* __restrict__ rowp, uint32_t nsb,
                                                  const int8_t* __restrict__ aq, uint32_t F,
                                                  const float* __restrict__ as, const float* __restrict__ au,
                                                  uint32_t nbf, float* acc) {
    for (uint32_t sb = 0; sb < nsb; sb++) {
        const uint16_t* s2 = reinterpret_cast<const uint16_t*>(rowp + sb * 210);
        uint16_t w16[105];
#pragma unroll
        for (int i = 0; i < 105; i++) w16[i] = s2[i];
        auto dw = [&](int o) -> uint32_t { return (uint32_t)w16[o >> 1] | ((uint32_t)w16[(o >> 1) + 1] << 16); };
        const float d = h2f(w16[104]);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int8_t sc = (int8_t)((w16[(192 + j) >> 1] >> (((192 + j) & 1) * 8)) & 0xff);
            const float ddv = f16_round(d * (float)sc);
            const float mmv = f16_round(-32.0f * ddv);
            const int nn = j / 8, g = (j % 8) / 2, l0 = 16 * (j % 2);
            const uint32_t b = sb * 16 + j;
#pragma unroll
            for (int p = 0; p < P; p++) {
                const int4 xv = *reinterpret_cast<const int4*>(aq + p * F + b * 16);
                const int xa[4] = {xv.x, xv.y, xv.z, xv.w};
                int dot = 0;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    uint32_t lo = dw(64 * nn + 32 * (g & 1) + l0 + 4 * t);
                    lo = (g >> 1) ? ((lo >> 4) & 0x0f0f0f0fu) : (lo & 0x0f0f0f0fu);
                    const uint32_t hi = (dw(128 + 32 * nn + l0 + 4 * t) >> (2 * g)) & 0x03030303u;
                    dot = sdot4((int)(lo | (hi << 4)), xa[t], dot);
                }
                const float sx = as[p * nbf + b];
                const float t = ddv * sx;
                acc[p] = __builtin_fmaf(mmv, au[p * nbf + b], acc[p]);
                acc[p] = __builtin_fmaf((float)dot, t, acc[p]);
            }
        }
    }
}

template <int P, int NSB>
__global__ __launch_bounds__(256) void decode_down_kernel(Mat down, Mat shd, Workspace ws, float* __restrict__ out,
                                                         int residual) {
    constexpr uint32_t F = NSB * 256, nsb = NSB, nbf = NSB * 16;
    const uint32_t tid = threadIdx.x, row0 = blockIdx.x * DN_R;
    const uint32_t n = ws.n_sel[0], slots = n + 1;

    extern __shared__ __align__(16) uint8_t smem[];
    int8_t* aq = (int8_t*)smem;                               // [slots][P][F]
    float* as = (float*)(smem + (size_t)slots * P * F);       // [slots][P][nbf] folded scale
    float* au = as + slots * P * nbf;                         // [slots][P][nbf] scale * sum
    float* vres = au + slots * P * nbf;                       // [slots][R]

    // stage the slots' activation rows: flat index over (slot, 16-byte piece) with the loads of
    // four pieces in flight per thread
    {
        constexpr uint32_t QP = P * F / 16, SP = P * nbf;  // int4 pieces and scales per slot
        const uint32_t nq = slots * QP, ns = slots * SP;
#pragma unroll 4
        for (uint32_t i = tid; i < nq; i += 256) {
            const uint32_t s = i / QP, o = i % QP;
            const uint32_t a = s < n ? s : (uint32_t)SH_SLOT;
            reinterpret_cast<int4*>(aq)[i] = reinterpret_cast<const int4*>(ws.actq + (size_t)a * P * F)[o];
        }
#pragma unroll 4
        for (uint32_t i = tid; i < ns; i += 256) {
            const uint32_t s = i / SP, o = i % SP;
            const uint32_t a = s < n ? s : (uint32_t)SH_SLOT;
            const float sc = ws.acts[(size_t)a * SP + o];
            as[i] = sc;
            au[i] = sc * (float)ws.actsum[(size_t)a * SP + o];
        }
    }
    __syncthreads();
    for (uint32_t it = tid; it < slots * DN_R; it += blockDim.x) {
        const uint32_t s = it / DN_R, r = it % DN_R;
        const Mat& D = s < n ? down : shd;
        const uint32_t e = s < n ? ws.ids[s] : 0u;
        const uint8_t* rowp = D.ptr + (size_t)e * D.stride + (size_t)(row0 + r) * D.row_bytes;
        float acc[P];
#pragma unroll
        for (int p = 0; p < P; p++) acc[p] = 0.0f;
        const int8_t* a = aq + (size_t)s * P * F;
        if (D.fmt == TRK_FMT_Q4_K)
            down_row_chain_q4k<P, NSB>(rowp, a, F, as + s * P * nbf, au + s * P * nbf, nbf, acc);
        else
            down_row_chain_q6k<P>(rowp, nsb, a, F, as + s * P * nbf, au + s * P * nbf, nbf, acc);
        vres[s * DN_R + r] = P == 2 ? acc[0] + acc[1] : acc[0];  // gemv.rs:154
    }
    __syncthreads();
    if (tid < DN_R) {
        // slot 0 stores, later slots accumulate (gemv.rs:150-160 with accumulate = slot > 0)
        float y = vres[tid];
        for (uint32_t s = 1; s < slots; s++) y = y + vres[s * DN_R + tid];
        float* o = out + row0 + tid;
        *o = residual ? *o + y : y;
    }
}

hipError_t launch_decode_down(const Mat& down, const Mat& sh_down, const Workspace& ws, int pair, uint32_t kcap,
                              float* out, int residual, hipStream_t st) {
    const uint32_t H = down.rows, F = down.k, nbf = F / 16;
    const int P = pair ? 2 : 1;
    const size_t slots = kcap + 1;
    const size_t lds = slots * P * F + slots * P * nbf * 8 + slots * DN_R * 4 + 64;
    switch (F / 256 * 2 + (pair ? 1 : 0)) {
#define DN_CASE(ns) \
    case ns * 2: decode_down_kernel<1, ns><<<H / DN_R, 256, lds, st>>>(down, sh_down, ws, out, residual); break; \
    case ns * 2 + 1: decode_down_kernel<2, ns><<<H / DN_R, 256, lds, st>>>(down, sh_down, ws, out, residual); break;
        DN_CASE(1) DN_CASE(2) DN_CASE(3) DN_CASE(4) DN_CASE(5) DN_CASE(6) DN_CASE(7) DN_CASE(8)
#undef DN_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace trk
