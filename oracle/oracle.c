/*
 * CPU oracle for the tr-infer MoE block — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Compiled with -O2 -ffp-contract=off: every fused multiply-add below is an explicit fmaf()
 * standing for an FMA in the reference; every other product and sum rounds on its own, as the
 * reference's AVX-512 code does.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ========================================================================================== */
/* half precision                                                                             */
/* ========================================================================================== */

/* f16 -> f32, exact (the reference uses half 2.7.1 / F16C: codec.rs:48-51, gemv.rs:104-105). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                sh++;
            }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(113 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0u); /* nan comes back quiet */
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* f32 -> f16, IEEE round-to-nearest-even (numpy astype(float16) in blocks.py:35-36). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan (quiet the nan, keep top payload bits) */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) { /* normal half */
        uint32_t mant = ax & 0x7fffffu;
        uint32_t r = ((((ax >> 23) - 127u + 15u)) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    if (ax < 0x33000000u) /* below 2^-25: rounds to zero */
        return (uint16_t)sign;
    /* subnormal half: value / 2^-24, rounded to nearest even */
    uint32_t M = 0x800000u | (ax & 0x7fffffu);
    int E = (int)(ax >> 23) - 127;
    int shift = -(E + 1);
    uint32_t r = M >> shift;
    uint32_t rem = M & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

__attribute__((target("f16c"))) static uint16_t hw_f32_to_f16(float f) {
    return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
}
__attribute__((target("f16c"))) static float hw_f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }

int orc_have_f16c(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("f16c") ? 1 : 0;
}

uint64_t orc_selftest_f16(uint32_t stride) {
    if (!orc_have_f16c()) return ~0ull;
    uint64_t bad = 0;
    for (uint32_t h = 0; h < 65536u; h++) {
        float a = orc_f16_to_f32((uint16_t)h), b = hw_f16_to_f32((uint16_t)h);
        uint32_t ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        if (ua != ub) bad++;
    }
    if (stride == 0) stride = 1;
    uint64_t x = 0;
    while (x <= 0xffffffffull) {
        uint32_t u = (uint32_t)x;
        float f;
        memcpy(&f, &u, 4);
        uint16_t a = orc_f32_to_f16(f), b = hw_f32_to_f16(f);
        /* nan payloads may differ: compare nan-ness only */
        int na = ((a & 0x7c00u) == 0x7c00u) && (a & 0x3ffu), nb = ((b & 0x7c00u) == 0x7c00u) && (b & 0x3ffu);
        if (na || nb) {
            if (na != nb) bad++;
        } else if (a != b) {
            bad++;
        }
        x += stride;
    }
    return bad;
}

/* ========================================================================================== */
/* TQ codec                                                                                   */
/* ========================================================================================== */

/* codec.rs:22-29 */
size_t orc_tq_block_bytes(int bits, int kb) {
    switch (bits) {
    case 8: return ORC_HDR_BYTES + ORC_STRIP * (size_t)kb;
    case 4: return ORC_HDR_BYTES + ORC_STRIP * (size_t)kb / 2;
    case 5: return ORC_HDR_BYTES + ORC_STRIP * (size_t)kb / 2 + 2 * (size_t)kb;
    default: return 0;
    }
}

static int pad_rows(int rows) { return (rows + ORC_STRIP - 1) / ORC_STRIP * ORC_STRIP; }

/* codec.rs:36-41 */
size_t orc_tq_matrix_bytes(int rows, int k, int bits, int kb) {
    return (size_t)(pad_rows(rows) / ORC_STRIP) * (size_t)(k / kb) * orc_tq_block_bytes(bits, kb);
}

/* codec.rs:80-100 */
uint32_t orc_tq_block_q(const uint8_t *blk, int bits, int kb, int r, int kk) {
    const uint8_t *qb = blk + ORC_HDR_BYTES;
    if (bits == 8) return qb[(kk / 4) * 64 + r * 4 + kk % 4];
    int half = kb / 2;
    int h = kk < half ? 0 : 1, kh = kk < half ? kk : kk - half;
    int j = kh / 4, i = kh % 4;
    uint8_t byte = qb[j * 64 + r * 4 + i];
    uint32_t q = h == 0 ? (byte & 0x0fu) : (uint32_t)(byte >> 4);
    if (bits == 5) {
        const uint8_t *plane = qb + kb / 8 * 64;
        int bit = r * 4 + i;
        uint8_t pb = plane[j * 16 + h * 8 + bit / 8];
        q |= (uint32_t)((pb >> (bit % 8)) & 1u) << 4;
    }
    return q;
}

/* codec.rs:143-169 */
static void set_block_q(uint8_t *blk, int bits, int kb, int r, int kk, uint32_t q) {
    uint8_t *qb = blk + ORC_HDR_BYTES;
    if (bits == 8) {
        qb[(kk / 4) * 64 + r * 4 + kk % 4] = (uint8_t)q;
        return;
    }
    int half = kb / 2;
    int h = kk < half ? 0 : 1, kh = kk < half ? kk : kk - half;
    int j = kh / 4, i = kh % 4;
    int idx = j * 64 + r * 4 + i;
    uint8_t nib = (uint8_t)(q & 0xfu);
    if (h == 0)
        qb[idx] = (uint8_t)((qb[idx] & 0xf0u) | nib);
    else
        qb[idx] = (uint8_t)((qb[idx] & 0x0fu) | (nib << 4));
    if (bits == 5) {
        int bit = r * 4 + i;
        int pidx = kb / 8 * 64 + j * 16 + h * 8 + bit / 8;
        if ((q >> 4) & 1u)
            qb[pidx] |= (uint8_t)(1u << (bit % 8));
        else
            qb[pidx] &= (uint8_t)~(1u << (bit % 8));
    }
}

/* codec.rs:118-141 (python/trpack/codec.py:41-71 writes the same bytes) */
void orc_pack_tq(int rows, int k, int bits, int kb, const uint8_t *q, const uint16_t *d,
                 const uint16_t *m, uint8_t *out) {
    int rp = pad_rows(rows), nb = k / kb;
    size_t bb = orc_tq_block_bytes(bits, kb);
    memset(out, 0, orc_tq_matrix_bytes(rows, k, bits, kb));
    for (int s = 0; s < rp / ORC_STRIP; s++)
        for (int b = 0; b < nb; b++) {
            uint8_t *blk = out + ((size_t)s * nb + b) * bb;
            for (int r = 0; r < ORC_STRIP; r++) {
                int row = s * ORC_STRIP + r;
                if (row >= rows) continue;
                uint16_t dv = d[(size_t)row * nb + b], mv = m[(size_t)row * nb + b];
                blk[2 * r] = (uint8_t)(dv & 0xff);
                blk[2 * r + 1] = (uint8_t)(dv >> 8);
                blk[32 + 2 * r] = (uint8_t)(mv & 0xff);
                blk[32 + 2 * r + 1] = (uint8_t)(mv >> 8);
                for (int kk = 0; kk < kb; kk++)
                    set_block_q(blk, bits, kb, r, kk, q[(size_t)row * k + (size_t)b * kb + kk]);
            }
        }
}

/* codec.rs:54-77: w = d*q + m (product and sum rounded separately) */
void orc_dequant_tq(const uint8_t *buf, int rows, int k, int bits, int kb, float *out) {
    int rp = pad_rows(rows), nb = k / kb;
    size_t bb = orc_tq_block_bytes(bits, kb);
    for (int s = 0; s < rp / ORC_STRIP; s++)
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = buf + ((size_t)s * nb + b) * bb;
            for (int r = 0; r < ORC_STRIP; r++) {
                int row = s * ORC_STRIP + r;
                if (row >= rows) continue;
                float d = orc_f16_to_f32((uint16_t)(blk[2 * r] | (blk[2 * r + 1] << 8)));
                float m = orc_f16_to_f32((uint16_t)(blk[32 + 2 * r] | (blk[32 + 2 * r + 1] << 8)));
                for (int kk = 0; kk < kb; kk++) {
                    float qv = (float)orc_tq_block_q(blk, bits, kb, r, kk);
                    float p = d * qv;
                    out[(size_t)row * k + (size_t)b * kb + kk] = p + m;
                }
            }
        }
}

/* ========================================================================================== */
/* GGUF block quants                                                                          */
/* ========================================================================================== */

size_t orc_gguf_row_bytes(int fmt, int K) {
    if (fmt == ORC_FMT_Q4_K) return (size_t)(K / 256) * 144;
    if (fmt == ORC_FMT_Q6_K) return (size_t)(K / 256) * 210;
    if (fmt == ORC_FMT_Q8_0) return (size_t)(K / 32) * 34;
    if (fmt == ORC_FMT_Q5_1) return (size_t)(K / 32) * 24;
    return 0;
}

/* blocks.py:16-22 (_scale_min_k): 12 bytes -> sc[8], mn[8], 6 bits each */
static void scale_min_k(const uint8_t *s, uint8_t *sc, uint8_t *mn) {
    for (int j = 0; j < 4; j++) {
        uint8_t d = s[j], m = s[4 + j], md = s[8 + j];
        sc[j] = d & 0x3f;
        sc[4 + j] = (uint8_t)((md & 0x0f) | ((d >> 2) & 0x30));
        mn[j] = m & 0x3f;
        mn[4 + j] = (uint8_t)((md >> 4) | ((m >> 2) & 0x30));
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* blocks.py:25-37 (q4k_rows): sub-block j = 2c + h holds nibble h of qs[32c + i];
 * dd = f16(d * sc), mm = f16(-(dmin * mn)) with d, dmin widened to f32 first. */
void orc_q4k_rows(const uint8_t *raw, int rows, int K, uint8_t *q, uint16_t *dd, uint16_t *mm) {
    int nsb = K / 256;
    for (int r = 0; r < rows; r++)
        for (int sb = 0; sb < nsb; sb++) {
            const uint8_t *b = raw + ((size_t)r * nsb + sb) * 144;
            float d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
            uint8_t sc[8], mn[8];
            scale_min_k(b + 4, sc, mn);
            const uint8_t *qs = b + 16;
            for (int c = 0; c < 4; c++)
                for (int h = 0; h < 2; h++)
                    for (int i = 0; i < 32; i++) {
                        uint8_t byte = qs[c * 32 + i];
                        q[(size_t)r * K + (size_t)sb * 256 + (2 * c + h) * 32 + i] =
                            h == 0 ? (byte & 0x0f) : (byte >> 4);
                    }
            for (int j = 0; j < 8; j++) {
                size_t o = (size_t)r * (K / 32) + (size_t)sb * 8 + j;
                dd[o] = orc_f32_to_f16(d * (float)sc[j]);
                mm[o] = orc_f32_to_f16(-(dmin * (float)mn[j]));
            }
        }
}

/* blocks.py:71-78 (q8_0_rows): the signed int8 offset by 128 into an unsigned q, the offset folded
 * into m = f16(-128 * d) (computed in f32, then rounded), d as stored */
void orc_q80_rows(const uint8_t *raw, int rows, int K, uint8_t *q, uint16_t *d, uint16_t *m) {
    int nb = K / 32;
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = raw + ((size_t)r * nb + b) * 34;
            uint16_t dh = rd16(blk);
            size_t o = (size_t)r * nb + b;
            d[o] = dh;
            m[o] = orc_f32_to_f16(-128.0f * orc_f16_to_f32(dh));
            for (int i = 0; i < 32; i++) q[(size_t)r * K + (size_t)b * 32 + i] = (uint8_t)((int)(int8_t)blk[2 + i] + 128);
        }
}

/* blocks.py:57-68 (q5_1_rows): element i of a block is the low (i < 16) or high (i >= 16) nibble
 * of qs[i % 16] with bit i of qh as its fifth bit; d and m as stored */
void orc_q51_rows(const uint8_t *raw, int rows, int K, uint8_t *q, uint16_t *d, uint16_t *m) {
    int nb = K / 32;
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = raw + ((size_t)r * nb + b) * 24;
            size_t o = (size_t)r * nb + b;
            d[o] = rd16(blk);
            m[o] = rd16(blk + 2);
            uint32_t qh = (uint32_t)blk[4] | ((uint32_t)blk[5] << 8) | ((uint32_t)blk[6] << 16) | ((uint32_t)blk[7] << 24);
            for (int i = 0; i < 32; i++) {
                uint8_t nib = i < 16 ? (blk[8 + i] & 0x0f) : (blk[8 + i - 16] >> 4);
                q[(size_t)r * K + (size_t)b * 32 + i] = (uint8_t)(nib | (((qh >> i) & 1u) << 4));
            }
        }
}

/* Q6_K (ggml block_q6_K: ql[128] qh[64] scales[16] int8, d f16) -> 6-bit unsigned q with
 * per-16 (dd, mm) = (f16(d*sc), -32*dd).  Extension: follows the offset-folding of q8_0_rows
 * (blocks.py:71-78); the reference itself has no Q6_K converter. */
void orc_q6k_rows(const uint8_t *raw, int rows, int K, uint8_t *q, uint16_t *dd, uint16_t *mm) {
    int nsb = K / 256;
    for (int r = 0; r < rows; r++)
        for (int sb = 0; sb < nsb; sb++) {
            const uint8_t *b = raw + ((size_t)r * nsb + sb) * 210;
            const uint8_t *ql = b, *qh = b + 128;
            const int8_t *sc = (const int8_t *)(b + 192);
            float d = orc_f16_to_f32(rd16(b + 208));
            uint8_t *qo = q + (size_t)r * K + (size_t)sb * 256;
            for (int n = 0; n < 2; n++)
                for (int l = 0; l < 32; l++) {
                    uint8_t h = qh[32 * n + l];
                    qo[128 * n + l] = (uint8_t)((ql[64 * n + l] & 0x0f) | ((h & 3) << 4));
                    qo[128 * n + l + 32] = (uint8_t)((ql[64 * n + l + 32] & 0x0f) | (((h >> 2) & 3) << 4));
                    qo[128 * n + l + 64] = (uint8_t)((ql[64 * n + l] >> 4) | (((h >> 4) & 3) << 4));
                    qo[128 * n + l + 96] = (uint8_t)((ql[64 * n + l + 32] >> 4) | (((h >> 6) & 3) << 4));
                }
            for (int j = 0; j < 16; j++) {
                size_t o = (size_t)r * (K / 16) + (size_t)sb * 16 + j;
                uint16_t dh = orc_f32_to_f16(d * (float)sc[j]);
                dd[o] = dh;
                mm[o] = orc_f32_to_f16(-32.0f * orc_f16_to_f32(dh));
            }
        }
}

int orc_gguf_to_tq(int fmt, const uint8_t *raw, int rows, int K, int kb, uint8_t *out) {
    uint8_t *q = (uint8_t *)malloc((size_t)rows * K);
    int bits = -1;
    if (fmt == ORC_FMT_Q4_K && (kb == 32 || kb == 16)) {
        int n32 = K / 32;
        uint16_t *d = (uint16_t *)malloc((size_t)rows * n32 * 2), *m = (uint16_t *)malloc((size_t)rows * n32 * 2);
        orc_q4k_rows(raw, rows, K, q, d, m);
        if (kb == 32) {
            orc_pack_tq(rows, K, 4, 32, q, d, m, out);
        } else { /* rows_to_groups (blocks.py:107-113): repeat each per-32 (d, m) twice */
            uint16_t *d16 = (uint16_t *)malloc((size_t)rows * n32 * 4), *m16 = (uint16_t *)malloc((size_t)rows * n32 * 4);
            for (size_t i = 0; i < (size_t)rows * n32; i++) {
                d16[2 * i] = d16[2 * i + 1] = d[i];
                m16[2 * i] = m16[2 * i + 1] = m[i];
            }
            orc_pack_tq(rows, K, 4, 16, q, d16, m16, out);
            free(d16);
            free(m16);
        }
        free(d);
        free(m);
        bits = 4;
    } else if ((fmt == ORC_FMT_Q8_0 || fmt == ORC_FMT_Q5_1) && (kb == 32 || kb == 16)) {
        int n32 = K / 32, nbits = fmt == ORC_FMT_Q8_0 ? 8 : 5;
        uint16_t *d = (uint16_t *)malloc((size_t)rows * n32 * 2), *m = (uint16_t *)malloc((size_t)rows * n32 * 2);
        if (fmt == ORC_FMT_Q8_0)
            orc_q80_rows(raw, rows, K, q, d, m);
        else
            orc_q51_rows(raw, rows, K, q, d, m);
        if (kb == 32) {
            orc_pack_tq(rows, K, nbits, 32, q, d, m, out);
        } else { /* rows_to_groups (blocks.py:107-113) */
            uint16_t *d16 = (uint16_t *)malloc((size_t)rows * n32 * 4), *m16 = (uint16_t *)malloc((size_t)rows * n32 * 4);
            for (size_t i = 0; i < (size_t)rows * n32; i++) {
                d16[2 * i] = d16[2 * i + 1] = d[i];
                m16[2 * i] = m16[2 * i + 1] = m[i];
            }
            orc_pack_tq(rows, K, nbits, 16, q, d16, m16, out);
            free(d16);
            free(m16);
        }
        free(d);
        free(m);
        bits = nbits;
    } else if (fmt == ORC_FMT_Q6_K && kb == 16) {
        int n16 = K / 16;
        uint16_t *d = (uint16_t *)malloc((size_t)rows * n16 * 2), *m = (uint16_t *)malloc((size_t)rows * n16 * 2);
        orc_q6k_rows(raw, rows, K, q, d, m);
        orc_pack_tq(rows, K, 8, 16, q, d, m, out);
        free(d);
        free(m);
        bits = 8;
    }
    free(q);
    return bits;
}

void orc_gguf_dequant(int fmt, const uint8_t *raw, int rows, int K, float *out) {
    int kb = fmt == ORC_FMT_Q4_K ? 32 : 16;
    size_t tb = orc_tq_matrix_bytes(rows, K, 8, kb);
    uint8_t *tq = (uint8_t *)malloc(tb);
    int bits = orc_gguf_to_tq(fmt, raw, rows, K, kb, tq);
    if (bits > 0) orc_dequant_tq(tq, rows, K, bits, kb, out);
    free(tq);
}

/* ========================================================================================== */
/* activation quantisation                                                                    */
/* ========================================================================================== */

/* x86 maxps semantics: a > b ? a : b */
static inline float mx_ps(float a, float b) { return a > b ? a : b; }
static inline float mn_ps(float a, float b) { return a < b ? a : b; }

/* _mm512_cvtps_epi32 under the default MXCSR: round to nearest even */
static inline int32_t cvt_rne(float v) { return (int32_t)nearbyintf(v); }
static inline int8_t sat_i8(int32_t v) { return (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v)); }

/* quant.rs:141-166 */
void orc_quant_block(const float *src, int n, int8_t *dst, float *scale, int32_t *sum) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) amax = mx_ps(amax, fabsf(src[i]));
    float s = amax / 127.0f;
    float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    int32_t su = 0;
    for (int i = 0; i < n; i++) {
        int32_t qi = cvt_rne(src[i] * inv);
        su += qi;
        dst[i] = sat_i8(qi);
    }
    *scale = s;
    *sum = su;
}

/* quant.rs:112-137: also r = fnmadd(q, scale, x) = x - q*scale, one rounding */
void orc_quant_block_resid(const float *src, int n, int8_t *dst, float *resid, float *scale,
                           int32_t *sum) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) amax = mx_ps(amax, fabsf(src[i]));
    float s = amax / 127.0f;
    float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    int32_t su = 0;
    for (int i = 0; i < n; i++) {
        int32_t qi = cvt_rne(src[i] * inv);
        su += qi;
        dst[i] = sat_i8(qi);
        resid[i] = fmaf(-(float)qi, s, src[i]);
    }
    *scale = s;
    *sum = su;
}

/* exec_batch.rs:228-237 (quant_rows), quant.rs:36-48 (quantize_into) */
void orc_quant_rows(const float *x, int m, int k, int kb, int8_t *q, float *s, int32_t *su) {
    int nb = k / kb;
    for (int r = 0; r < m; r++)
        for (int b = 0; b < nb; b++)
            orc_quant_block(x + (size_t)r * k + (size_t)b * kb, kb, q + (size_t)r * k + (size_t)b * kb,
                            s + (size_t)r * nb + b, su + (size_t)r * nb + b);
}

/* quant.rs:96-108 (quantize_pair_blocks over all blocks) */
void orc_quant_pair(const float *x, int k, int kb, int8_t *q, float *s, int32_t *su) {
    int nb = k / kb;
    float resid[32];
    for (int b = 0; b < nb; b++) {
        orc_quant_block_resid(x + (size_t)b * kb, kb, q + (size_t)b * kb, resid, s + b, su + b);
        orc_quant_block(resid, kb, q + k + (size_t)b * kb, s + nb + b, su + nb + b);
    }
}

/* ========================================================================================== */
/* TQ x int8 GEMV (gemv.rs:81-172)                                                            */
/* ========================================================================================== */

static void gemv_impl(const uint8_t *w, int k, int bits, int kb, int s0, int s1, const orc_qact *xq,
                      float *y, size_t ldy, const uint32_t *rows, int accumulate) {
    int m = xq->m;
    size_t bb = orc_tq_block_bytes(bits, kb);
    int nb = k / kb;
    const uint8_t *wp = w;
    for (int s = s0; s < s1; s++) {
        float accf[ORC_MAX_M][ORC_STRIP];
        memset(accf, 0, sizeof accf);
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = wp;
            wp += bb;
            float d[ORC_STRIP], mnv[ORC_STRIP];
            for (int r = 0; r < ORC_STRIP; r++) {
                d[r] = orc_f16_to_f32(rd16(blk + 2 * r));
                mnv[r] = orc_f16_to_f32(rd16(blk + 32 + 2 * r));
            }
            int32_t acc32[ORC_MAX_M][ORC_STRIP];
            for (int mi = 0; mi < m; mi++)
                for (int r = 0; r < ORC_STRIP; r++) {
                    int32_t a = 0;
                    const int8_t *xp = xq->q + (size_t)mi * k + (size_t)b * kb;
                    for (int kk = 0; kk < kb; kk++) a += (int32_t)orc_tq_block_q(blk, bits, kb, r, kk) * xp[kk];
                    acc32[mi][r] = a;
                }
            /* gemv.rs:141-148: acc = fma(m, sx*sum, acc); acc = fma(float(dot), d*sx, acc) */
            for (int mi = 0; mi < m; mi++) {
                float sx = xq->scale[(size_t)mi * nb + b];
                float u = sx * (float)xq->sum[(size_t)mi * nb + b];
                for (int r = 0; r < ORC_STRIP; r++) {
                    float t = d[r] * sx;
                    accf[mi][r] = fmaf(mnv[r], u, accf[mi][r]);
                    accf[mi][r] = fmaf((float)acc32[mi][r], t, accf[mi][r]);
                }
            }
        }
        if (xq->pair) { /* gemv.rs:150-160 */
            for (int mi = 0; mi < m / 2; mi++) {
                size_t yr = rows ? rows[mi] : (size_t)mi;
                float *yp = y + yr * ldy + (size_t)s * ORC_STRIP;
                for (int r = 0; r < ORC_STRIP; r++) {
                    float v = accf[2 * mi][r] + accf[2 * mi + 1][r];
                    yp[r] = accumulate ? yp[r] + v : v;
                }
            }
        } else { /* gemv.rs:161-169 */
            for (int mi = 0; mi < m; mi++) {
                size_t yr = rows ? rows[mi] : (size_t)mi;
                float *yp = y + yr * ldy + (size_t)s * ORC_STRIP;
                for (int r = 0; r < ORC_STRIP; r++) yp[r] = accumulate ? yp[r] + accf[mi][r] : accf[mi][r];
            }
        }
    }
}

/* gemv.rs:25-37 */
void orc_gemv_tq_rows(const uint8_t *w, int k, int bits, int kb, int s0, int s1,
                      const orc_qact *xq, float *y, size_t ldy, const uint32_t *rows,
                      int accumulate) {
    gemv_impl(w, k, bits, kb, s0, s1, xq, y, ldy, rows, accumulate);
}

/* gemv.rs:55-78: chunk the logical rows into MAX_M physical rows per pass */
void orc_gemm_tq_rows(const uint8_t *w, int k, int bits, int kb, int s0, int s1,
                      const orc_qact *xq, float *y, size_t ldy, const uint32_t *rows,
                      int accumulate) {
    int per = xq->pair ? 2 : 1;
    int nb = k / xq->kb;
    int logical = xq->m / per;
    int group = ORC_MAX_M / per;
    for (int r0 = 0; r0 < logical; r0 += group) {
        int r1 = r0 + group < logical ? r0 + group : logical;
        orc_qact sub = {(r1 - r0) * per, k, xq->kb, xq->q + (size_t)r0 * per * k,
                        xq->scale + (size_t)r0 * per * nb, xq->sum + (size_t)r0 * per * nb, xq->pair};
        if (rows)
            gemv_impl(w, k, bits, kb, s0, s1, &sub, y, ldy, rows + r0, accumulate);
        else
            gemv_impl(w, k, bits, kb, s0, s1, &sub, y + (size_t)r0 * ldy, ldy, NULL, accumulate);
    }
}

/* ========================================================================================== */
/* f32 reductions and elementwise                                                             */
/* ========================================================================================== */

/* _mm512_reduce_add_ps: halving tree (lanes i + i+8, then i + i+4, i + i+2, 0 + 1) */
static float reduce16(const float *v) {
    float a[8], b[4], c[2];
    for (int i = 0; i < 8; i++) a[i] = v[i] + v[i + 8];
    for (int i = 0; i < 4; i++) b[i] = a[i] + a[i + 4];
    for (int i = 0; i < 2; i++) c[i] = b[i] + b[i + 2];
    return c[0] + c[1];
}

/* attn.rs:329-357: four 16-lane FMA chains over 64-wide steps, then a 16-wide tail into chain 0,
 * lanewise (c0+c1)+(c2+c3), tree reduce, scalar tail. */
float orc_dot(const float *a, const float *b, int n) {
    float acc[4][16];
    memset(acc, 0, sizeof acc);
    int i = 0;
    for (; i + 64 <= n; i += 64)
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 16; l++) acc[c][l] = fmaf(a[i + 16 * c + l], b[i + 16 * c + l], acc[c][l]);
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; l++) acc[0][l] = fmaf(a[i + l], b[i + l], acc[0][l]);
    float v[16];
    for (int l = 0; l < 16; l++) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    float s = reduce16(v);
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* smallgemm.rs:8-59: y[i][j] = reduce16(lanes l: fma chain over kk of x[i][kk+l] * w[j][kk+l]) */
void orc_gemm_f32_nt(const float *x, int ldx, int mr, const float *w, int ldw, int n, int k,
                     float *y, int ldy) {
    for (int i = 0; i < mr; i++)
        for (int j = 0; j < n; j++) {
            float acc[16] = {0};
            for (int kk = 0; kk < k; kk += 16)
                for (int l = 0; l < 16; l++)
                    acc[l] = fmaf(x[(size_t)i * ldx + kk + l], w[(size_t)j * ldw + kk + l], acc[l]);
            y[(size_t)i * ldy + j] = reduce16(acc);
        }
}

/* elem.rs:224-252 */
float orc_sumsq(const float *x, int n) { return orc_dot(x, x, n); }

/* elem.rs:255-262: r = 1/sqrt(sumsq/n + eps); y = (x*r)*w */
void orc_rmsnorm(const float *x, const float *w, float eps, float *y, int n) {
    float r = 1.0f / sqrtf(orc_sumsq(x, n) / (float)n + eps);
    for (int i = 0; i < n; i++) y[i] = w ? (x[i] * r) * w[i] : x[i] * r;
}

/* elem.rs:7-25 (tr-infer's own clamped degree-6 exp) */
float orc_exp512(float x) {
    x = mn_ps(mx_ps(x, -87.3f), 88.3f);
    float fx = nearbyintf(x * 1.442695041f);
    float r = fmaf(-fx, 0.693145752f, x);
    r = fmaf(-fx, 1.42860677e-6f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    float r2 = r * r;
    p = fmaf(p, r2, r);
    p = p + 1.0f;
    return scalbnf(p, (int)fx);
}

float orc_sigmoid512(float x) { return 1.0f / (1.0f + orc_exp512(0.0f - x)); }
float orc_silu512(float x) { return x * orc_sigmoid512(x); }
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
static float silu_scalar(float x) { return x * orc_sigmoid(x); }

/* elem.rs:173-175 via zip16 (elem.rs:209-221): 16-wide body uses silu512, tail uses scalar silu */
void orc_swiglu(const float *g, const float *u, float *y, int n) {
    int body = n / 16 * 16;
    for (int i = 0; i < body; i++) y[i] = orc_silu512(g[i]) * u[i];
    for (int i = body; i < n; i++) y[i] = silu_scalar(g[i]) * u[i];
}

void orc_add_inplace(float *y, const float *a, int n) {
    for (int i = 0; i < n; i++) y[i] = y[i] + a[i];
}

/* ========================================================================================== */
/* router (router.rs)                                                                         */
/* ========================================================================================== */

/* router.rs:32-44 */
int orc_policy_validate(const orc_policy *p, int n_expert, char *err, int errlen) {
    if (p->min < 1 || p->min > p->max) {
        if (err) snprintf(err, errlen, "moe policy: need 1 <= min (%u) <= max (%u)", p->min, p->max);
        return -1;
    }
    if (p->max > ORC_MOE_K_MAX || (int)p->max > n_expert) {
        if (err)
            snprintf(err, errlen, "moe policy: max (%u) above the limit (%d)", p->max,
                     ORC_MOE_K_MAX < n_expert ? ORC_MOE_K_MAX : n_expert);
        return -1;
    }
    if (!(p->mass > 0.0f) || isnan(p->mass)) {
        if (err) snprintf(err, errlen, "moe policy: target mass (%g) must be positive", (double)p->mass);
        return -1;
    }
    return 0;
}

/* router.rs:70-89: insertion top-k; ties keep the lowest index; nan never enters */
static void topk_sorted(const float *logits, int n, int k, float *top_v, uint32_t *top_i) {
    for (int j = 0; j < ORC_MOE_K_MAX; j++) {
        top_v[j] = -INFINITY;
        top_i[j] = 0xffffffffu;
    }
    for (int i = 0; i < n; i++) {
        float v = logits[i];
        if (!(v > top_v[k - 1])) continue;
        int p = k - 1;
        while (p > 0 && top_v[p - 1] < v) {
            top_v[p] = top_v[p - 1];
            top_i[p] = top_i[p - 1];
            p--;
        }
        top_v[p] = v;
        top_i[p] = (uint32_t)i;
    }
}

/* router.rs:93-104 */
static void renorm(const float *top_v, int k, float *w) {
    float mx = top_v[0], sum = 0.0f;
    for (int j = 0; j < k; j++) {
        w[j] = expf(top_v[j] - mx);
        sum += w[j];
    }
    for (int j = 0; j < k; j++) w[j] /= sum;
}

/* router.rs:106-113 */
void orc_route_topk(const float *logits, int n, int k, uint32_t *ids, float *w) {
    float tv[ORC_MOE_K_MAX];
    uint32_t ti[ORC_MOE_K_MAX];
    topk_sorted(logits, n, k, tv, ti);
    memcpy(ids, ti, sizeof(uint32_t) * k);
    renorm(tv, k, w);
}

/* router.rs:118-148 */
int orc_route_mass(const float *logits, int n, const orc_policy *p, uint32_t *ids, float *w) {
    float tv[ORC_MOE_K_MAX];
    uint32_t ti[ORC_MOE_K_MAX];
    int kmax = (int)p->max;
    topk_sorted(logits, n, kmax, tv, ti);
    float mx = tv[0], denom = 0.0f;
    if (p->basis == ORC_BASIS_ALL) {
        for (int i = 0; i < n; i++) denom += expf(logits[i] - mx);
    } else {
        for (int j = 0; j < kmax; j++) denom += expf(tv[j] - mx);
    }
    int count = 0;
    float mass = 0.0f;
    while (count < kmax) {
        mass += expf(tv[count] - mx) / denom;
        count++;
        if (count >= (int)p->min && mass >= p->mass) break;
    }
    memcpy(ids, ti, sizeof(uint32_t) * count);
    renorm(tv, count, w);
    return count;
}

/* router.rs:152-166 */
void orc_mass_profile(const float *logits, int n, float *cum) {
    float tv[ORC_MOE_K_MAX];
    uint32_t ti[ORC_MOE_K_MAX];
    int k = n < ORC_MOE_K_MAX ? n : ORC_MOE_K_MAX;
    topk_sorted(logits, n, k, tv, ti);
    float mx = tv[0], denom = 0.0f, mass = 0.0f;
    for (int i = 0; i < n; i++) denom += expf(logits[i] - mx);
    for (int j = 0; j < ORC_MOE_K_MAX; j++) {
        if (j < k) mass += expf(tv[j] - mx) / denom;
        cum[j] = mass;
    }
}

/* exec_batch.rs:214-225 (fold_ids): subset packs map the routed ids onto the packed experts,
 * keeping them distinct within the token */
int orc_fold_ids(uint32_t *ids, int n, uint32_t packed) {
    if (n > (int)packed) return -1; /* exec_batch.rs:217: more routed experts than packed experts */
    for (int i = 0; i < n; i++) {
        uint32_t id = ids[i] % packed;
        for (;;) {
            int taken = 0;
            for (int j = 0; j < i; j++) taken |= ids[j] == id;
            if (!taken) break;
            id = (id + 1) % packed;
        }
        ids[i] = id;
    }
    return 0;
}

/* exec.rs:630-639 (Model::route), then the subset-pack fold of exec.rs:1545-1549 /
 * exec_batch.rs:1418-1420 */
static int route_w(const orc_moe_w *W, const float *logits, int k, const orc_policy *p, uint32_t *ids, float *w) {
    int n = W->E, used;
    if (p)
        used = orc_route_mass(logits, n, p, ids, w);
    else {
        orc_route_topk(logits, n, k, ids, w);
        used = k;
    }
    if (W->packed > 0 && W->packed < W->E && orc_fold_ids(ids, used, (uint32_t)W->packed) != 0) return -1;
    return used;
}

static int tiles_of(const orc_moe_w *W) { return W->tiles > 1 ? W->tiles : 1; }

/* bytes of one tile's gate/up [F/T][H] and down [H][F/T] matrices */
static size_t gu_tile_bytes(const orc_moe_w *W, int bits) {
    return orc_tq_matrix_bytes(W->F / tiles_of(W), W->H, bits, 32);
}
static size_t dn_tile_bytes(const orc_moe_w *W, int bits) {
    return orc_tq_matrix_bytes(W->H, W->F / tiles_of(W), bits, 16);
}

/* ========================================================================================== */
/* MoE block                                                                                  */
/* ========================================================================================== */

/* Router logits of one row in dot order (exec.rs:1003-1011): with T tiles, tile t's partial is
 * dot(router_t[e], x[H/T t ..]) over its H/T columns, and the partials are summed in tile order
 * (Mailboxes::reduce, exchange.rs:122-136: the first copied, the others added). */
static void router_logits_dot(const orc_moe_w *W, const float *x, float *rlog) {
    const int T = tiles_of(W), hl = W->H / T;
    for (int e = 0; e < W->E; e++) {
        float v = 0.0f;
        for (int t = 0; t < T; t++) {
            const float p = orc_dot(W->router + ((size_t)t * W->E + e) * hl, x + (size_t)t * hl, hl);
            v = t == 0 ? p : v + p;
        }
        rlog[e] = W->router_bias ? v + W->router_bias[e] : v;
    }
}

/* The batch router (exec_batch.rs:1008-1016): per tile gemm_f32_nt over the tile's H/T columns,
 * the partials summed in tile order.  (The reference's batch all-reduce starts each row's sum at a
 * tile that depends on which core handles the row, exec_batch.rs:741-747; tile order 0..T-1 is its
 * sum where that is core 0 of a single-socket pack.) */
static void router_logits_gemm(const orc_moe_w *W, const float *x, int M, float *lg) {
    const int T = tiles_of(W), hl = W->H / T, E = W->E;
    if (T == 1) {
        orc_gemm_f32_nt(x, W->H, M, W->router, W->H, E, W->H, lg, E);
    } else {
        float *p = (float *)malloc(sizeof(float) * (size_t)M * E);
        for (int t = 0; t < T; t++) {
            orc_gemm_f32_nt(x + (size_t)t * hl, W->H, M, W->router + (size_t)t * E * hl, hl, E, hl,
                            t == 0 ? lg : p, E);
            if (t > 0)
                for (size_t i = 0; i < (size_t)M * E; i++) lg[i] = lg[i] + p[i];
        }
        free(p);
    }
    if (W->router_bias)
        for (int mi = 0; mi < M; mi++)
            for (int e = 0; e < E; e++) lg[(size_t)mi * E + e] = lg[(size_t)mi * E + e] + W->router_bias[e];
}

/* Router logits of M rows as the decode path (dot_rows: per-row dot) or the batch gemm computes
 * them, tiles and bias included. */
void orc_moe_logits(const orc_moe_w *W, const float *x, int M, int dot_rows, float *out) {
    if (dot_rows)
        for (int mi = 0; mi < M; mi++) router_logits_dot(W, x + (size_t)mi * W->H, out + (size_t)mi * W->E);
    else
        router_logits_gemm(W, x, M, out);
}

/* Tile t's slice [F/T t, F/T (t+1)) of `rows` activation rows of length F (with their per-16
 * scales and sums), copied out contiguously. */
static void act_slice(const int8_t *q, const float *s, const int32_t *su, int rows, int F, int T, int t, int8_t *tq,
                      float *ts, int32_t *tsu) {
    const int per = F / T, nbf = F / 16, nbt = per / 16;
    for (int r = 0; r < rows; r++) {
        memcpy(tq + (size_t)r * per, q + (size_t)r * F + (size_t)per * t, per);
        memcpy(ts + (size_t)r * nbt, s + (size_t)r * nbf + (size_t)nbt * t, sizeof(float) * nbt);
        memcpy(tsu + (size_t)r * nbt, su + (size_t)r * nbf + (size_t)nbt * t, sizeof(int32_t) * nbt);
    }
}

/* exec.rs:1540-1623 (moe_block), one tile (T = 1): route, shared gate, (pair-)quantise x per 32,
 * gate/up per slot (shared expert last), SwiGLU + quantise per down.kb with the routing weight
 * folded into the scales, then down with slot 0 overwriting and later slots accumulating. */
int orc_moe_block(const orc_moe_w *W, const float *x, const float *rlog, int k,
                  const orc_policy *policy, int hiprec, float *out, float *rlog_out,
                  uint32_t *ids, float *w, orc_moe_stats *stats) {
    int H = W->H, F = W->F, E = W->E;
    float *lg = (float *)malloc(sizeof(float) * E);
    if (rlog)
        memcpy(lg, rlog, sizeof(float) * E);
    else
        router_logits_dot(W, x, lg);
    if (rlog_out) memcpy(rlog_out, lg, sizeof(float) * E);
    int k_used = route_w(W, lg, k, policy, ids, w);
    if (k_used < 0) {
        free(lg);
        return -1;
    }
    int slots = k_used + 1;
    for (int s = 0; s < k_used; s++)
        if (!W->gate[ids[s]] || !W->up[ids[s]] || !W->down[ids[s]]) {
            free(lg);
            return -1;
        }
    if (stats) {
        stats->rows += 1;
        stats->experts += (uint64_t)k_used;
    }
    float sh_gate = orc_sigmoid(orc_dot(W->shexp_gate, x, H));
    /* CoreScratch::qz (exec.rs:284-290) */
    int mrows = hiprec ? 2 : 1;
    int8_t *xq = (int8_t *)malloc((size_t)2 * H);
    float *xs = (float *)malloc(sizeof(float) * 2 * (H / 32));
    int32_t *xsu = (int32_t *)malloc(sizeof(int32_t) * 2 * (H / 32));
    if (hiprec)
        orc_quant_pair(x, H, 32, xq, xs, xsu);
    else
        orc_quant_rows(x, 1, H, 32, xq, xs, xsu);
    orc_qact qa = {mrows, H, 32, xq, xs, xsu, hiprec};
    float *hg = (float *)malloc(sizeof(float) * (size_t)slots * F);
    float *hu = (float *)malloc(sizeof(float) * (size_t)slots * F);
    /* tasks A (exec.rs:1563-1577); tile t computes rows [F/T t, F/T (t+1)) */
    const int T = tiles_of(W), per = F / T;
    for (int slot = 0; slot < slots; slot++) {
        const uint8_t *g = slot < k_used ? W->gate[ids[slot]] : W->sh_gate;
        const uint8_t *u = slot < k_used ? W->up[ids[slot]] : W->sh_up;
        int gb = slot < k_used ? W->gate_bits : W->sh_gate_bits;
        const size_t tb = gu_tile_bytes(W, gb);
        for (int t = 0; t < T; t++) {
            orc_gemv_tq_rows(g + t * tb, H, gb, 32, 0, per / ORC_STRIP, &qa, hg + (size_t)slot * F + (size_t)per * t, 0,
                             NULL, 0);
            orc_gemv_tq_rows(u + t * tb, H, gb, 32, 0, per / ORC_STRIP, &qa, hu + (size_t)slot * F + (size_t)per * t, 0,
                             NULL, 0);
        }
    }
    /* tasks B (exec.rs:1584-1606): kb = down.kb = 16 */
    int kb = 16, nb = F / kb;
    int8_t *aq = (int8_t *)malloc((size_t)2 * slots * F);
    float *as = (float *)malloc(sizeof(float) * 2 * slots * nb);
    int32_t *asu = (int32_t *)malloc(sizeof(int32_t) * 2 * slots * nb);
    float *act = (float *)malloc(sizeof(float) * F);
    for (int slot = 0; slot < slots; slot++) {
        orc_swiglu(hg + (size_t)slot * F, hu + (size_t)slot * F, act, F);
        float wgt = slot < k_used ? w[slot] : sh_gate;
        int8_t *q = aq + (size_t)2 * slot * F;
        float *sc = as + (size_t)2 * slot * nb;
        int32_t *su = asu + (size_t)2 * slot * nb;
        if (hiprec)
            orc_quant_pair(act, F, kb, q, sc, su);
        else
            orc_quant_rows(act, 1, F, kb, q, sc, su);
        for (int i = 0; i < mrows * nb; i++) sc[i] *= wgt;
    }
    /* tasks C (exec.rs:1610-1621): each tile's partial over its columns of F, slot 0 stored and
     * later slots added, the shared expert last; then the tiles' partials in tile order
     * (exec.rs:1035-1038, Mailboxes::reduce) */
    int8_t *tq = (int8_t *)malloc((size_t)2 * per);
    float *ts = (float *)malloc(sizeof(float) * 2 * (per / kb));
    int32_t *tsu = (int32_t *)malloc(sizeof(int32_t) * 2 * (per / kb));
    float *part = T > 1 ? (float *)malloc(sizeof(float) * H) : out;
    for (int t = 0; t < T; t++) {
        for (int slot = 0; slot < slots; slot++) {
            const uint8_t *dm = slot < k_used ? W->down[ids[slot]] : W->sh_down;
            int db = slot < k_used ? W->down_bits : W->sh_down_bits;
            act_slice(aq + (size_t)2 * slot * F, as + (size_t)2 * slot * nb, asu + (size_t)2 * slot * nb, mrows, F, T, t,
                      tq, ts, tsu);
            orc_qact da = {mrows, per, kb, tq, ts, tsu, hiprec};
            orc_gemv_tq_rows(dm + t * dn_tile_bytes(W, db), per, db, kb, 0, H / ORC_STRIP, &da, part, 0, NULL, slot > 0);
        }
        if (T > 1)
            for (int h = 0; h < H; h++) out[h] = t == 0 ? part[h] : out[h] + part[h];
    }
    if (T > 1) free(part);
    free(tq);
    free(ts);
    free(tsu);
    free(lg);
    free(xq);
    free(xs);
    free(xsu);
    free(hg);
    free(hu);
    free(aq);
    free(as);
    free(asu);
    free(act);
    return k_used;
}

/* Hyper-connection mix, part B, on one tile (T = 1): the MoE input `mixed` of every row from the
 * normed streams xn [m][hc][hh] and the low-rank projection lo [m][lr] (summed over tiles).
 * up: the TQ matrix [hc * hh][lr] with (bits, 32).
 *   decode (exec.rs:1196-1234, hc_mix_b): lo <- silu(lo / hc) with the scalar silu; quantised in
 *     pairs when hiprec (CoreScratch::qz, exec.rs:284-290); gate = sigmoid(up . q) with the scalar
 *     sigmoid; mixed[c] = (sum_s xn[s][c] * gate[s][c], accumulated from 0 with separate multiply
 *     and add) * (1 / hc).
 *   batch (exec_batch.rs:929-968, hc_b_batch): lo <- lo * (1 / hc), then silu_inplace (silu512 on
 *     16-blocks, scalar tail); quant_rows per 32; gate = sigmoid_inplace(up . q) (sigmoid512 on
 *     16-blocks); mixed = xn_0 * gate_0, then fma_inplace for s >= 1 (fused on 16-blocks, multiply
 *     and add on the tail), then scale_inplace(1 / hc). */
void orc_hc_mix(const uint8_t *up, int bits, int hc, int hh, int lr, const float *xn, const float *lo, int m,
                int decode, int hiprec, float *mixed) {
    const int nb = lr / 32, rows = hc * hh, mrows = decode && hiprec ? 2 : 1;
    const float inv = 1.0f / (float)hc;
    float *l2 = (float *)malloc(sizeof(float) * lr);
    int8_t *q = (int8_t *)malloc((size_t)2 * lr);
    float *qs = (float *)malloc(sizeof(float) * 2 * nb);
    int32_t *qsu = (int32_t *)malloc(sizeof(int32_t) * 2 * nb);
    float *gate = (float *)malloc(sizeof(float) * rows);
    for (int mi = 0; mi < m; mi++) {
        const float *lr_in = lo + (size_t)mi * lr;
        if (decode) {
            for (int j = 0; j < lr; j++) l2[j] = silu_scalar(lr_in[j] / (float)hc);
            if (hiprec)
                orc_quant_pair(l2, lr, 32, q, qs, qsu);
            else
                orc_quant_rows(l2, 1, lr, 32, q, qs, qsu);
        } else {
            const int body = lr / 16 * 16;
            for (int j = 0; j < lr; j++) l2[j] = lr_in[j] * inv;
            for (int j = 0; j < lr; j++) l2[j] = j < body ? orc_silu512(l2[j]) : silu_scalar(l2[j]);
            orc_quant_rows(l2, 1, lr, 32, q, qs, qsu);
        }
        orc_qact qa = {mrows, lr, 32, q, qs, qsu, mrows == 2};
        orc_gemv_tq_rows(up, lr, bits, 32, 0, rows / ORC_STRIP, &qa, gate, 0, NULL, 0);
        const int gbody = rows / 16 * 16;
        for (int i = 0; i < rows; i++)
            gate[i] = decode ? orc_sigmoid(gate[i]) : (i < gbody ? orc_sigmoid512(gate[i]) : orc_sigmoid(gate[i]));
        const float *x = xn + (size_t)mi * rows;
        float *out = mixed + (size_t)mi * hh;
        if (decode) {
            for (int c = 0; c < hh; c++) {
                float acc = 0.0f;
                for (int sI = 0; sI < hc; sI++) acc += x[sI * hh + c] * gate[sI * hh + c];
                out[c] = acc * inv;
            }
        } else {
            const int body = hh / 16 * 16;
            for (int c = 0; c < hh; c++) out[c] = x[c] * gate[c];
            for (int sI = 1; sI < hc; sI++)
                for (int c = 0; c < hh; c++)
                    out[c] = c < body ? fmaf(x[sI * hh + c], gate[sI * hh + c], out[c])
                                      : out[c] + x[sI * hh + c] * gate[sI * hh + c];
            for (int c = 0; c < hh; c++) out[c] = out[c] * inv;
        }
    }
    free(l2);
    free(q);
    free(qs);
    free(qsu);
    free(gate);
}

/* exec_batch.rs:1404-1580 (moe_batch) with the router of exec_batch.rs:989-1019 */
int orc_moe_batch(const orc_moe_w *W, const float *x, const float *rlog, int M, int k,
                  const orc_policy *policy, int router_dot_max_m, float *out, float *rlog_out,
                  uint32_t *ids, float *w, uint32_t *n_sel, uint32_t *ent_tok, float *ent_w,
                  uint32_t *ent_expert, uint32_t *grp_start, uint32_t *grp_expert,
                  uint32_t *grp_order, uint32_t *n_groups, orc_moe_stats *stats) {
    int H = W->H, F = W->F, E = W->E, ka = ORC_MOE_K_MAX;
    float *lg = (float *)malloc(sizeof(float) * (size_t)M * E);
    if (rlog) {
        memcpy(lg, rlog, sizeof(float) * (size_t)M * E);
    } else if (M < router_dot_max_m) {
        for (int mi = 0; mi < M; mi++) router_logits_dot(W, x + (size_t)mi * H, lg + (size_t)mi * E);
    } else {
        router_logits_gemm(W, x, M, lg);
    }
    if (rlog_out) memcpy(rlog_out, lg, sizeof(float) * (size_t)M * E);
    /* routing + quant_rows per token (exec_batch.rs:1415-1425) */
    int nbx = H / 32;
    int8_t *xq = (int8_t *)malloc((size_t)M * H);
    float *xs = (float *)malloc(sizeof(float) * (size_t)M * nbx);
    int32_t *xsu = (int32_t *)malloc(sizeof(int32_t) * (size_t)M * nbx);
    for (int mi = 0; mi < M; mi++) {
        const int used = route_w(W, lg + (size_t)mi * E, k, policy, ids + (size_t)mi * ka, w + (size_t)mi * ka);
        if (used < 0) {
            free(lg); free(xq); free(xs); free(xsu);
            return -1;
        }
        n_sel[mi] = (uint32_t)used;
    }
    orc_quant_rows(x, M, H, 32, xq, xs, xsu);
    /* grouping (exec_batch.rs:1428-1462): stable sort of token-major (token, slot) by expert */
    int n_ent = 0;
    for (int mi = 0; mi < M; mi++) n_ent += (int)n_sel[mi];
    uint32_t *cnt = (uint32_t *)calloc((size_t)E + 1, sizeof(uint32_t));
    for (int mi = 0; mi < M; mi++)
        for (uint32_t s = 0; s < n_sel[mi]; s++) cnt[ids[(size_t)mi * ka + s] + 1]++;
    for (int e = 0; e < E; e++) cnt[e + 1] += cnt[e];
    for (int mi = 0; mi < M; mi++) /* counting sort = stable sort by key */
        for (uint32_t s = 0; s < n_sel[mi]; s++) {
            uint32_t e = ids[(size_t)mi * ka + s];
            uint32_t j = cnt[e]++;
            ent_tok[j] = (uint32_t)mi;
            ent_w[j] = w[(size_t)mi * ka + s];
            ent_expert[j] = e;
        }
    int ng = 0;
    uint32_t last = 0xffffffffu;
    for (int j = 0; j < n_ent; j++)
        if (ent_expert[j] != last) {
            grp_start[ng] = (uint32_t)j;
            grp_expert[ng] = ent_expert[j];
            ng++;
            last = ent_expert[j];
        }
    grp_start[ng] = (uint32_t)n_ent;
    n_groups[0] = (uint32_t)ng;
    n_groups[1] = (uint32_t)n_ent;
    if (stats) {
        stats->rows += (uint64_t)M;
        stats->experts += (uint64_t)n_ent;
    }
    /* grp_order: groups by size descending, stable (exec_batch.rs:1459-1461) */
    for (int g = 0; g < ng; g++) grp_order[g] = (uint32_t)g;
    for (int a = 1; a < ng; a++) { /* insertion sort, stable */
        uint32_t v = grp_order[a];
        uint32_t sv = grp_start[v + 1] - grp_start[v];
        int b = a - 1;
        while (b >= 0 && (grp_start[grp_order[b] + 1] - grp_start[grp_order[b]]) < sv) {
            grp_order[b + 1] = grp_order[b];
            b--;
        }
        grp_order[b + 1] = v;
    }
    for (int g = 0; g < ng; g++) {
        uint32_t e = grp_expert[g];
        if (!W->gate[e] || !W->up[e] || !W->down[e]) {
            free(lg); free(xq); free(xs); free(xsu); free(cnt);
            return -1;
        }
    }
    /* tasks A (exec_batch.rs:1481-1509): gate/up per group on the gathered rows, shared on all;
     * tile t computes rows [F/T t, F/T (t+1)) */
    const int T = tiles_of(W), per = F / T;
    int rows_all = n_ent + M;
    float *hg = (float *)malloc(sizeof(float) * (size_t)rows_all * F);
    float *hu = (float *)malloc(sizeof(float) * (size_t)rows_all * F);
    int8_t *gq = (int8_t *)malloc((size_t)M * H);
    float *gs = (float *)malloc(sizeof(float) * (size_t)M * nbx);
    int32_t *gsu = (int32_t *)malloc(sizeof(int32_t) * (size_t)M * nbx);
    for (int g = 0; g < ng; g++) {
        int r0 = (int)grp_start[g], r1 = (int)grp_start[g + 1];
        uint32_t e = grp_expert[g];
        for (int r = r0; r < r1; r++) {
            int tok = (int)ent_tok[r], i = r - r0;
            memcpy(gq + (size_t)i * H, xq + (size_t)tok * H, H);
            memcpy(gs + (size_t)i * nbx, xs + (size_t)tok * nbx, sizeof(float) * nbx);
            memcpy(gsu + (size_t)i * nbx, xsu + (size_t)tok * nbx, sizeof(int32_t) * nbx);
        }
        orc_qact ga = {r1 - r0, H, 32, gq, gs, gsu, 0};
        const size_t tb = gu_tile_bytes(W, W->gate_bits);
        for (int t = 0; t < T; t++) {
            orc_gemm_tq_rows(W->gate[e] + t * tb, H, W->gate_bits, 32, 0, per / ORC_STRIP, &ga,
                             hg + (size_t)r0 * F + (size_t)per * t, F, NULL, 0);
            orc_gemm_tq_rows(W->up[e] + t * tb, H, W->gate_bits, 32, 0, per / ORC_STRIP, &ga,
                             hu + (size_t)r0 * F + (size_t)per * t, F, NULL, 0);
        }
    }
    orc_qact all = {M, H, 32, xq, xs, xsu, 0};
    {
        const size_t tb = gu_tile_bytes(W, W->sh_gate_bits);
        for (int t = 0; t < T; t++) {
            orc_gemm_tq_rows(W->sh_gate + t * tb, H, W->sh_gate_bits, 32, 0, per / ORC_STRIP, &all,
                             hg + (size_t)n_ent * F + (size_t)per * t, F, NULL, 0);
            orc_gemm_tq_rows(W->sh_up + t * tb, H, W->sh_gate_bits, 32, 0, per / ORC_STRIP, &all,
                             hu + (size_t)n_ent * F + (size_t)per * t, F, NULL, 0);
        }
    }
    /* tasks B (exec_batch.rs:1513-1536) */
    int kb = 16, nbd = F / kb;
    int8_t *aq = (int8_t *)malloc((size_t)rows_all * F);
    float *as = (float *)malloc(sizeof(float) * (size_t)rows_all * nbd);
    int32_t *asu = (int32_t *)malloc(sizeof(int32_t) * (size_t)rows_all * nbd);
    float *act = (float *)malloc(sizeof(float) * F);
    for (int r = 0; r < rows_all; r++) {
        orc_swiglu(hg + (size_t)r * F, hu + (size_t)r * F, act, F);
        float wgt = r < n_ent ? ent_w[r] : orc_sigmoid(orc_dot(W->shexp_gate, x + (size_t)(r - n_ent) * H, H));
        orc_quant_rows(act, 1, F, kb, aq + (size_t)r * F, as + (size_t)r * nbd, asu + (size_t)r * nbd);
        for (int i = 0; i < nbd; i++) as[(size_t)r * nbd + i] *= wgt;
    }
    /* tasks C (exec_batch.rs:1539-1561), per tile over its columns of F: shared first
     * (overwrite), then groups ascending by expert, each group's rows accumulated into their
     * tokens' rows; then the tiles' partials in tile order (exec_batch.rs:821-849) */
    int8_t *tq = (int8_t *)malloc((size_t)rows_all * per);
    float *ts = (float *)malloc(sizeof(float) * (size_t)rows_all * (per / kb));
    int32_t *tsu = (int32_t *)malloc(sizeof(int32_t) * (size_t)rows_all * (per / kb));
    float *part = T > 1 ? (float *)malloc(sizeof(float) * (size_t)M * H) : out;
    const int nbt = per / kb;
    for (int t = 0; t < T; t++) {
        act_slice(aq, as, asu, rows_all, F, T, t, tq, ts, tsu);
        orc_qact sa = {M, per, kb, tq + (size_t)n_ent * per, ts + (size_t)n_ent * nbt, tsu + (size_t)n_ent * nbt, 0};
        orc_gemm_tq_rows(W->sh_down + t * dn_tile_bytes(W, W->sh_down_bits), per, W->sh_down_bits, kb, 0, H / ORC_STRIP,
                         &sa, part, H, NULL, 0);
        for (int g = 0; g < ng; g++) {
            int r0 = (int)grp_start[g], r1 = (int)grp_start[g + 1];
            uint32_t e = grp_expert[g];
            orc_qact da = {r1 - r0, per, kb, tq + (size_t)r0 * per, ts + (size_t)r0 * nbt, tsu + (size_t)r0 * nbt, 0};
            orc_gemm_tq_rows(W->down[e] + t * dn_tile_bytes(W, W->down_bits), per, W->down_bits, kb, 0, H / ORC_STRIP, &da,
                             part, H, ent_tok + r0, 1);
        }
        if (T > 1)
            for (size_t i = 0; i < (size_t)M * H; i++) out[i] = t == 0 ? part[i] : out[i] + part[i];
    }
    if (T > 1) free(part);
    free(tq); free(ts); free(tsu);
    free(lg); free(xq); free(xs); free(xsu); free(cnt);
    free(hg); free(hu); free(gq); free(gs); free(gsu);
    free(aq); free(as); free(asu); free(act);
    return n_ent;
}

/* ========================================================================================== */
/* deterministic synthetic data                                                               */
/* ========================================================================================== */

static inline uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* counter-based: one 64-bit draw per (seed, stream, idx) */
uint64_t orc_rng_u64(uint64_t seed, uint64_t stream, uint64_t idx) {
    uint64_t key = mix64(seed ^ mix64(stream));
    return mix64(key + idx * 0xd1b54a32d192ed03ull);
}

/* U(lo, hi) from 24 random bits, rounded in f32 as lo + u*(hi-lo) (mul then add) */
static float unif24(uint64_t r, float lo, float hi) {
    float u = (float)(r & 0xffffffu) * (1.0f / 16777216.0f);
    float span = hi - lo;
    float p = u * span;
    return lo + p;
}

void orc_gen_gguf(int fmt, uint64_t seed, uint64_t stream, int rows, int K, float dlo, float dhi,
                  uint8_t *out) {
    size_t sbb = fmt == ORC_FMT_Q6_K ? 210 : 144;
    size_t nsb = (size_t)rows * (K / 256);
    if (fmt == ORC_FMT_Q5_1) { /* units of 8 blocks (192 bytes): 24 random words, then each d, m */
        for (size_t sb = 0; sb < nsb; sb++) {
            uint8_t *b = out + sb * 192;
            for (size_t wi = 0; wi < 24; wi++) {
                uint64_t r = orc_rng_u64(seed, stream, sb * 64 + wi);
                for (int j = 0; j < 8; j++) b[wi * 8 + j] = (uint8_t)(r >> (8 * j));
            }
            for (int c = 0; c < 8; c++) {
                uint64_t rd = orc_rng_u64(seed, stream, sb * 64 + 48 + c);
                uint16_t d = orc_f32_to_f16(unif24(rd, dlo, dhi));
                uint16_t m = orc_f32_to_f16(-16.0f * unif24(rd >> 24, dlo, dhi));
                b[24 * c] = (uint8_t)(d & 0xff);
                b[24 * c + 1] = (uint8_t)(d >> 8);
                b[24 * c + 2] = (uint8_t)(m & 0xff);
                b[24 * c + 3] = (uint8_t)(m >> 8);
            }
        }
        return;
    }
    if (fmt == ORC_FMT_Q8_0) { /* units of 8 blocks (272 bytes): 34 random words, then each d */
        for (size_t sb = 0; sb < nsb; sb++) {
            uint8_t *b = out + sb * 272;
            for (size_t wi = 0; wi < 34; wi++) {
                uint64_t r = orc_rng_u64(seed, stream, sb * 64 + wi);
                for (int j = 0; j < 8; j++) b[wi * 8 + j] = (uint8_t)(r >> (8 * j));
            }
            for (int c = 0; c < 8; c++) {
                uint16_t d = orc_f32_to_f16(unif24(orc_rng_u64(seed, stream, sb * 64 + 48 + c), dlo, dhi));
                b[34 * c] = (uint8_t)(d & 0xff);
                b[34 * c + 1] = (uint8_t)(d >> 8);
            }
        }
        return;
    }
    for (size_t sb = 0; sb < nsb; sb++) {
        uint8_t *b = out + sb * sbb;
        size_t nw = (sbb + 7) / 8; /* 18 or 27 draws of 8 random bytes */
        for (size_t wi = 0; wi < nw; wi++) {
            uint64_t r = orc_rng_u64(seed, stream, sb * 32 + wi);
            for (int j = 0; j < 8 && wi * 8 + j < sbb; j++) b[wi * 8 + j] = (uint8_t)(r >> (8 * j));
        }
        uint64_t rd = orc_rng_u64(seed, stream, sb * 32 + 31);
        uint16_t d = orc_f32_to_f16(unif24(rd, dlo, dhi));
        if (fmt == ORC_FMT_Q6_K) {
            b[208] = (uint8_t)(d & 0xff);
            b[209] = (uint8_t)(d >> 8);
        } else {
            uint16_t dm = orc_f32_to_f16(unif24(rd >> 24, dlo, dhi));
            b[0] = (uint8_t)(d & 0xff);
            b[1] = (uint8_t)(d >> 8);
            b[2] = (uint8_t)(dm & 0xff);
            b[3] = (uint8_t)(dm >> 8);
        }
    }
}

void orc_gen_normal(uint64_t seed, uint64_t stream, size_t n, double sigma, float *out) {
    for (size_t i = 0; i < n; i++) {
        uint64_t a = orc_rng_u64(seed, stream, 2 * i), b = orc_rng_u64(seed, stream, 2 * i + 1);
        double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = (float)(z * sigma);
    }
}

void orc_gen_uniform(uint64_t seed, uint64_t stream, size_t n, float lo, float hi, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = unif24(orc_rng_u64(seed, stream, i), lo, hi);
}
