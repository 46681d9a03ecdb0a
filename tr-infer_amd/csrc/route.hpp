// Routing of one token on one wave: route_topk / route_mass (crates/tr-kernels/src/router.rs:70-148).
//
// Selection.  Each lane holds NJ logits (index lane + 64 j) as order-preserving u32 keys.  The
// winners come out in exactly the order of the reference's insertion sort: value descending, the
// lower index first among equal values (a later index only displaces strictly smaller values).
// NaN and -inf map to key 0 and are never selected, as `v > top_v[k-1]` never holds for them.
//
// Weights.  exp of (v - max) in f32 through a double exp (Rust's f32::exp, see expf_libm), the
// mass loop of route_mass, then the renormalisation of renorm() with its sequential f32 sum.
#pragma once

#include "common.hpp"

namespace trk {

// order-preserving key of a logit (-0 and +0 share one key, as they compare equal); 0 for values
// that never enter the top-k (nan, -inf: router.rs:75-76)
__device__ __forceinline__ uint32_t fkey(float v) {
    const uint32_t u = __float_as_uint(v + 0.0f);
    const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return v > -__builtin_inff() ? k : 0u;  // selects, no branch
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ float rdl(float v, uint32_t l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)l));
}

// Fallback selection (more than 64 candidates, i.e. many equal logits): each lane sorts its keys
// (key desc, j asc), then kk rounds of a wave arg-max over the lane heads.  Lane rd < ksel gets
// the key and index of the rd-th winner; returns ksel.
template <int NJ, bool COH>
__device__ __forceinline__ uint32_t route_select_rounds(const float* __restrict__ lg, uint32_t E, uint32_t kk,
                                                        uint32_t lane, uint32_t& my_key, uint32_t& my_idx) {
    uint32_t key[NJ], jj[NJ];
    float v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t i = lane + 64u * j, ic = i < E ? i : E - 1;
        v[j] = COH ? ld_devf(lg + ic) : lg[ic];
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        key[j] = lane + 64u * j < E ? fkey(v[j]) : 0u;
        jj[j] = (uint32_t)j;
    }
    // odd-even transposition sort, descending key; equal keys keep ascending j (stable)
#pragma unroll
    for (int pass = 0; pass < NJ; pass++)
#pragma unroll
        for (int j = pass & 1; j + 1 < NJ; j += 2)
            if (key[j + 1] > key[j]) {
                const uint32_t tk = key[j], tj = jj[j];
                key[j] = key[j + 1];
                jj[j] = jj[j + 1];
                key[j + 1] = tk;
                jj[j + 1] = tj;
            }
    uint32_t ksel = 0;
    for (uint32_t rd = 0; rd < kk; rd++) {
        const uint32_t wmax = wave_max_u32(key[0]);
        if (wmax == 0u) break;  // no selectable logit left
        const uint32_t widx = wave_min_u32(key[0] == wmax ? lane + 64u * jj[0] : 0xffffffffu);
        if (lane == widx % 64u) {  // pop this lane's head
#pragma unroll
            for (int j = 0; j + 1 < NJ; j++) {
                key[j] = key[j + 1];
                jj[j] = jj[j + 1];
            }
            key[NJ - 1] = 0u;
        }
        if (lane == rd) {
            my_key = wmax;
            my_idx = widx;
        }
        ksel = rd + 1;
    }
    return ksel;
}

constexpr uint32_t ROUTE_CAND_DUMMY = 95;  // the candidate slot lanes without a candidate write

// One token on one whole wave.  Lanes < count write ids_out[lane] / w_out[lane]; returns count.
// `cand` is 96 entries of LDS for this wave; `ex` (E floats of LDS) is used only for
// MassBasis::All.
//
// Selection: T = the kk-th largest of the 64 lane maxima, truncated to its top 16 bits (a radix
// select over ballots), is a lower bound on the kk-th largest key, since the kk lanes with the
// largest maxima hold kk keys >= T.  The keys >= T (usually a few more than kk) are compacted
// into LDS in ascending index order; each candidate's rank is the number of candidates with a
// larger key plus the earlier ones with an equal key, and the candidates of rank < kk are written
// to their rank's slot.
// COH: the logits were written earlier in the same launch by other workgroups (device-coherent
// loads).
// Selection: lane j < ksel gets the key and index of the j-th winner (my_key, my_idx); returns ksel.
template <int NJ, bool COH = false>
__device__ uint32_t route_select(const float* __restrict__ lg, uint32_t E, uint32_t k, const Policy& pol,
                                 uint32_t lane, uint2* cand, uint32_t& my_key, uint32_t& my_idx) {
    // all NJ loads go out together: clamped indices, no per-load branch
    float v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t i = lane + 64u * j, ic = i < E ? i : E - 1;
        v[j] = COH ? ld_devf(lg + ic) : lg[ic];
    }
    uint32_t key[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t kf = fkey(v[j]);
        key[j] = lane + 64u * j < E ? kf : 0u;
    }
    const uint32_t kk = pol.enabled ? pol.max : k;
    uint32_t lmax = key[0];
#pragma unroll
    for (int j = 1; j < NJ; j++) lmax = lmax > key[j] ? lmax : key[j];
    // two bits per step over the top 16 bits of the keys: T is the kk-th largest lane maximum
    // with its low 16 bits cleared, still a lower bound (candidates sharing its top 16 bits join
    // the ranking); the three candidate prefixes of a step are counted independently
    uint32_t T = 0;
#pragma unroll
    for (int b = 30; b >= 16; b -= 2) {
        const uint32_t t1 = T | (1u << b), t2 = T | (2u << b), t3 = T | (3u << b);
        const uint32_t c1 = (uint32_t)__popcll(__ballot(lmax >= t1));
        const uint32_t c2 = (uint32_t)__popcll(__ballot(lmax >= t2));
        const uint32_t c3 = (uint32_t)__popcll(__ballot(lmax >= t3));
        T = c3 >= kk ? t3 : (c2 >= kk ? t2 : (c1 >= kk ? t1 : T));
    }
    const uint32_t L = T > 1u ? T : 1u;  // key 0 (nan, -inf) is never selectable
    // every lane writes (those without a candidate to slot 95, which the ranking below rewrites
    // before it is read): no branch per j
    uint32_t C = 0;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const bool c = key[j] >= L;
        const uint64_t m = __ballot(c);
        const uint32_t pos =
                C + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        cand[c && pos < 64u ? pos : ROUTE_CAND_DUMMY] = make_uint2(key[j], lane + 64u * j);
        C += (uint32_t)__popcll(m);
    }
    my_key = 0;
    my_idx = 0xffffffffu;
    uint32_t ksel;
    if (C <= 64u) {
        wave_sync();
        const uint2 me = lane < C ? cand[lane] : make_uint2(0u, 0u);
        uint32_t rank = 0;
        if (C <= 16u) {  // the usual case: 16 independent lane reads, no loop
            // lanes >= C hold key 0, below every candidate's key (>= 1), so they add nothing
#pragma unroll
            for (uint32_t t = 0; t < 16u; t++) {
                const uint32_t kt = (uint32_t)__builtin_amdgcn_readlane((int)me.x, (int)t);
                rank += (kt > me.x || (kt == me.x && t < lane)) ? 1u : 0u;
            }
        } else {
            for (uint32_t t = 0; t < C; t++) {  // candidate t's key from lane t's register
                const uint32_t kt = (uint32_t)__builtin_amdgcn_readlane((int)me.x, (int)t);
                rank += (kt > me.x || (kt == me.x && t < lane)) ? 1u : 0u;
            }
        }
        if (lane < C && rank < kk) cand[64 + rank] = me;
        wave_sync();
        ksel = C < kk ? C : kk;
        if (lane < ksel) {
            const uint2 w = cand[64 + lane];
            my_key = w.x;
            my_idx = w.y;
        }
    } else {
        ksel = route_select_rounds<NJ, COH>(lg, E, kk, lane, my_key, my_idx);
    }
    return ksel;
}

// fold_ids (exec_batch.rs:214-225) on one wave: lane i < n holds id i; in order, id i becomes the
// first of id % packed, +1, +2, ... (mod packed) not taken by a lane below it.  The loops are
// wave-uniform (id and the ballot are the same on every lane).
__device__ __forceinline__ uint32_t fold_ids_wave(uint32_t id, uint32_t n, uint32_t packed, uint32_t lane) {
    uint32_t f = 0;
    for (uint32_t i = 0; i < n; i++) {
        uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)id, (int)i) % packed;
        while (__ballot(lane < i && f == v)) v = v + 1 == packed ? 0u : v + 1;
        if (lane == i) f = v;
    }
    return lane < n ? f : id;
}

// Weights of a selection (route_select's per-lane winners): exp of (v - max), the mass loop of
// route_mass, the renormalisation.  Lanes < count write ids_out / w_out; returns count.
template <bool COH = false>
__device__ uint32_t route_weights(const float* __restrict__ lg, uint32_t E, uint32_t k, const Policy& pol,
                                  uint32_t lane, float* ex, uint32_t ksel, uint32_t my_key, uint32_t my_idx,
                                  uint32_t* __restrict__ ids_out, float* __restrict__ w_out) {
    const uint32_t kk = pol.enabled ? pol.max : k;
    if (ksel == 0) return 0;  // nothing selectable (the reference would index u32::MAX)
    const float my_tv = lane < ksel ? fkey_inv(my_key) : -__builtin_inff();
    const float mx = rdl(my_tv, 0);
    const float e = lane < kk ? expf_libm(my_tv - mx) : 0.0f;  // slots past ksel: exp(-inf) = 0
    uint32_t count = kk;
    if (pol.enabled) {  // route_mass (router.rs:118-148)
        float denom = 0.0f;
        if (pol.basis == TRK_BASIS_ALL) {
            for (uint32_t i = lane; i < E; i += 64u) ex[i] = expf_libm((COH ? ld_devf(lg + i) : lg[i]) - mx);
            wave_sync();
            if (lane == 0)
                for (uint32_t i = 0; i < E; i++) denom += ex[i];
            denom = rdl(denom, 0);
        } else {
            for (uint32_t j = 0; j < kk; j++) denom += rdl(e, j);
        }
        float mass = 0.0f;
        count = 0;
        while (count < kk) {
            mass += rdl(e, count) / denom;
            count++;
            if (count >= pol.min && mass >= pol.mass) break;
        }
    }
    if (count > ksel) count = ksel;
    // a subset pack: the ids folded onto its experts (fold_ids, exec_batch.rs:214-225); the weights
    // stay those of the routing
    if (pol.packed) my_idx = fold_ids_wave(my_idx, count, pol.packed, lane);
    float sum = 0.0f;  // renorm (router.rs:93-104): the sequential f32 sum, four lane reads at a time
    for (uint32_t j0 = 0; j0 < count; j0 += 4) {
        float ev[4];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) ev[i] = rdl(e, j0 + i < 64u ? j0 + i : 63u);
#pragma unroll
        for (uint32_t i = 0; i < 4; i++)
            if (j0 + i < count) sum += ev[i];
    }
    if (lane < count) {
        ids_out[lane] = my_idx;
        w_out[lane] = e / sum;
    }
    return count;
}

// One token on one whole wave: selection, then weights.
template <int NJ, bool COH = false>
__device__ uint32_t route_row(const float* __restrict__ lg, uint32_t E, uint32_t k, const Policy& pol, uint32_t lane,
                              uint2* cand, float* ex, uint32_t* __restrict__ ids_out, float* __restrict__ w_out) {
    uint32_t my_key, my_idx;
    const uint32_t ksel = route_select<NJ, COH>(lg, E, k, pol, lane, cand, my_key, my_idx);
    return route_weights<COH>(lg, E, k, pol, lane, ex, ksel, my_key, my_idx, ids_out, w_out);
}

constexpr uint32_t ROUTE_CAND = 96;  // LDS entries (uint2) of route_row's candidate lists per wave

// Logits per lane for E experts: 8 up to 512 experts, 16 up to 1024.
constexpr uint32_t route_nj(uint32_t E) { return E <= 512 ? 8u : 16u; }

}  // namespace trk
