/*
 * The timed CPU baseline: the reference's CPU MoE path restated with AVX-512 / VNNI intrinsics and
 * run on a pinned thread pool the way the reference's tile does (one thread per core, at most 16
 * per tile, crates/tr-sys/src/pool.rs:16,167).  TEST AND MEASUREMENT INFRASTRUCTURE ONLY: bench.py's
 * cpu_baseline leg and tests/ load it; the GPU library never does.
 *
 * What it restates (tokenring-ai/tr-infer):
 *   gemv_impl<BITS, KB>          crates/tr-kernels/src/gemv.rs:81-172 (VNNI dpbusd block dots, the
 *                                per-block f32 epilogue, pair rows summed at the end)
 *   quant_block[_resid]          crates/tr-kernels/src/quant.rs:112-166
 *   dot                          crates/tr-kernels/src/attn.rs:329-357
 *   gemm_f32_nt                  crates/tr-kernels/src/smallgemm.rs:8-59
 *   moe_block tasks A / B / C    crates/tr-model/src/exec.rs:1540-1623 (router S5: 1003-1011)
 *   moe_batch tasks A / B / C    crates/tr-model/src/exec_batch.rs:1404-1580 (router 989-1019)
 * with one tile (T = 1): every core of the tile takes the reference's share of each task list, and
 * the per-output arithmetic order is that of one core, so results are bit-identical to the scalar
 * oracle (oracle.c), which tests/test_cpu_baseline.py checks.  Routing, the grouping sort and
 * SwiGLU are the oracle's own functions (not the hot loops).
 *
 * AMX is probed as crates/tr-kernels/src/amx.rs:18-30 does (arch_prctl ARCH_REQ_XCOMP_PERM); the
 * routed experts never use AMX in the reference, and the shared expert's AMX-BF16 path
 * (exec_batch.rs:294-296) is not reproduced: this is the VNNI path (TR_AMX=0 semantics).
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <sys/syscall.h>
#include <unistd.h>

#include "oracle.h"

/* ---- thread pool with a sense-reversing spin barrier (pool.rs:57-98) ---------------------- */

typedef struct cpu_pool cpu_pool;
typedef void (*cpu_task_fn)(cpu_pool *p, void *arg, int tid);

struct cpu_pool {
    int n;
    pthread_t *th;
    int *cpu;  /* the CPU each thread is pinned to */
    _Atomic int bar_count;
    _Atomic int bar_sense;
    _Atomic unsigned gen; /* job generation: workers start a job when it moves */
    _Atomic int quit;
    cpu_task_fn fn;
    void *arg;
};

typedef struct {
    cpu_pool *p;
    int tid;
} worker_arg;

static __thread int t_sense;

/* spin with pause, yielding the CPU now and then: the threads are pinned one per core, as in the
 * reference, but a host that gives the process fewer cores than threads must not livelock */
static inline void spin_pause(unsigned *n) {
    if (++*n % 4096 == 0)
        sched_yield();
    else
        _mm_pause();
}

void cpu_pool_barrier(cpu_pool *p) {
    t_sense = !t_sense;
    if (atomic_fetch_add(&p->bar_count, 1) == p->n - 1) {
        atomic_store(&p->bar_count, 0);
        atomic_store(&p->bar_sense, t_sense);
    } else {
        unsigned n = 0;
        while (atomic_load(&p->bar_sense) != t_sense) spin_pause(&n);
    }
}

static void pin(int cpu) {
    if (cpu < 0) return;
    cpu_set_t s;
    CPU_ZERO(&s);
    CPU_SET(cpu, &s);
    (void)pthread_setaffinity_np(pthread_self(), sizeof s, &s);
}

static void *worker(void *a) {
    worker_arg wa = *(worker_arg *)a;
    free(a);
    cpu_pool *p = wa.p;
    pin(p->cpu[wa.tid]);
    unsigned seen = 0;
    for (;;) {
        unsigned g, n = 0;
        while ((g = atomic_load(&p->gen)) == seen && !atomic_load(&p->quit)) spin_pause(&n);
        if (atomic_load(&p->quit)) break;
        seen = g;
        p->fn(p, p->arg, wa.tid);
        cpu_pool_barrier(p);
    }
    return NULL;
}

/* A pool of n threads (0: one per CPU this process may run on, at most 16: one tile), pinned to
 * the CPUs of the process's affinity mask in order.  The caller is thread 0. */
cpu_pool *cpu_pool_create(int n) {
    cpu_set_t s;
    int cpus[1024], nc = 0;
    if (sched_getaffinity(0, sizeof s, &s) == 0)
        for (int c = 0; c < CPU_SETSIZE && nc < 1024; c++)
            if (CPU_ISSET(c, &s)) cpus[nc++] = c;
    if (nc == 0) cpus[nc++] = -1;
    if (n <= 0) n = nc < 16 ? nc : 16;
    cpu_pool *p = (cpu_pool *)calloc(1, sizeof *p);
    p->n = n;
    p->th = (pthread_t *)calloc((size_t)n, sizeof(pthread_t));
    p->cpu = (int *)calloc((size_t)n, sizeof(int));
    for (int i = 0; i < n; i++) p->cpu[i] = i < nc ? cpus[i] : -1;
    t_sense = 0;
    for (int i = 1; i < n; i++) {
        worker_arg *wa = (worker_arg *)malloc(sizeof *wa);
        wa->p = p;
        wa->tid = i;
        pthread_create(&p->th[i], NULL, worker, wa);
    }
    pin(p->cpu[0]);
    return p;
}

int cpu_pool_size(const cpu_pool *p) { return p->n; }
int cpu_pool_cpu(const cpu_pool *p, int i) { return i < p->n ? p->cpu[i] : -1; }

void cpu_pool_destroy(cpu_pool *p) {
    if (!p) return;
    atomic_store(&p->quit, 1);
    for (int i = 1; i < p->n; i++) pthread_join(p->th[i], NULL);
    free(p->th);
    free(p->cpu);
    free(p);
}

/* run fn on every thread (the caller is thread 0) and wait for all */
static void pool_run(cpu_pool *p, cpu_task_fn fn, void *arg) {
    p->fn = fn;
    p->arg = arg;
    atomic_fetch_add(&p->gen, 1);
    fn(p, arg, 0);
    cpu_pool_barrier(p);
}

/* pool.rs:110-116 split: the i-th of k near-equal ranges of n */
static void split(int n, int i, int k, int *lo, int *hi) {
    int base = n / k, rem = n % k;
    *lo = i * base + (i < rem ? i : rem);
    *hi = *lo + base + (i < rem ? 1 : 0);
}

/* ---- feature probes -------------------------------------------------------------------- */

int cpu_have_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni");
}

/* amx.rs:18-30: request XTILEDATA permission; 0 when AMX is unavailable */
int cpu_amx_available(void) {
    return syscall(SYS_arch_prctl, 0x1023 /* ARCH_REQ_XCOMP_PERM */, 18 /* XFEATURE_XTILEDATA */) == 0;
}

/* ---- kernels ----------------------------------------------------------------------------- */

/* _mm512_reduce_add_ps as a halving tree: lanes i + i+8, i + i+4, i + i+2, 0 + 1 */
static inline float reduce16_ps(__m512 v) {
    __m256 a = _mm256_add_ps(_mm512_castps512_ps256(v), _mm512_extractf32x8_ps(v, 1));
    __m128 b = _mm_add_ps(_mm256_castps256_ps128(a), _mm256_extractf128_ps(a, 1));
    __m128 c = _mm_add_ps(b, _mm_movehl_ps(b, b));
    return _mm_cvtss_f32(c) + _mm_cvtss_f32(_mm_shuffle_ps(c, c, 1));
}

/* attn.rs:329-357 */
static float dot_avx(const float *a, const float *b, int n) {
    __m512 c0 = _mm512_setzero_ps(), c1 = c0, c2 = c0, c3 = c0;
    int i = 0;
    for (; i + 64 <= n; i += 64) {
        c0 = _mm512_fmadd_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i), c0);
        c1 = _mm512_fmadd_ps(_mm512_loadu_ps(a + i + 16), _mm512_loadu_ps(b + i + 16), c1);
        c2 = _mm512_fmadd_ps(_mm512_loadu_ps(a + i + 32), _mm512_loadu_ps(b + i + 32), c2);
        c3 = _mm512_fmadd_ps(_mm512_loadu_ps(a + i + 48), _mm512_loadu_ps(b + i + 48), c3);
    }
    for (; i + 16 <= n; i += 16) c0 = _mm512_fmadd_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i), c0);
    float s = reduce16_ps(_mm512_add_ps(_mm512_add_ps(c0, c1), _mm512_add_ps(c2, c3)));
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* smallgemm.rs:8-59 for rows [i0, i1) x cols [j0, j1): 16 lane chains per output, then the tree */
static void gemm_nt_avx(const float *x, int ldx, const float *w, int ldw, int k, float *y, int ldy, int i0, int i1,
                        int j0, int j1) {
    for (int i = i0; i < i1; i += 4)
        for (int j = j0; j < j1; j += 4) {
            __m512 acc[4][4];
            int ni = i1 - i < 4 ? i1 - i : 4, nj = j1 - j < 4 ? j1 - j : 4;
            for (int a = 0; a < 4; a++)
                for (int b = 0; b < 4; b++) acc[a][b] = _mm512_setzero_ps();
            for (int kk = 0; kk < k; kk += 16) {
                __m512 xv[4], wv[4];
                for (int a = 0; a < ni; a++) xv[a] = _mm512_loadu_ps(x + (size_t)(i + a) * ldx + kk);
                for (int b = 0; b < nj; b++) wv[b] = _mm512_loadu_ps(w + (size_t)(j + b) * ldw + kk);
                for (int a = 0; a < ni; a++)
                    for (int b = 0; b < nj; b++) acc[a][b] = _mm512_fmadd_ps(xv[a], wv[b], acc[a][b]);
            }
            for (int a = 0; a < ni; a++)
                for (int b = 0; b < nj; b++) y[(size_t)(i + a) * ldy + j + b] = reduce16_ps(acc[a][b]);
        }
}

/* quant.rs:141-166 (resid == NULL) and quant.rs:112-138: one block of kb (16 or 32) values */
static void quant_block_avx(const float *src, int kb, int8_t *dst, float *resid, float *scale, int32_t *sum) {
    const __m512 absmask = _mm512_castsi512_ps(_mm512_set1_epi32(0x7fffffff));
    __m512 amaxv = _mm512_setzero_ps();
    for (int i = 0; i < kb; i += 16) amaxv = _mm512_max_ps(amaxv, _mm512_and_ps(_mm512_loadu_ps(src + i), absmask));
    const float amax = _mm512_reduce_max_ps(amaxv);
    const float s = amax / 127.0f;
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    const __m512 vinv = _mm512_set1_ps(inv), vs = _mm512_set1_ps(s);
    int32_t su = 0;
    for (int i = 0; i < kb; i += 16) {
        const __m512 v = _mm512_loadu_ps(src + i);
        const __m512i q = _mm512_cvtps_epi32(_mm512_mul_ps(v, vinv)); /* round to nearest even */
        su += _mm512_reduce_add_epi32(q);
        _mm_storeu_si128((__m128i *)(dst + i), _mm512_cvtsepi32_epi8(q));
        if (resid) _mm512_storeu_ps(resid + i, _mm512_fnmadd_ps(_mm512_cvtepi32_ps(q), vs, v));
    }
    *scale = s;
    *sum = su;
}

/* QActRef::quantize_into (quant.rs:36-48) / quantize_pair_into (quant.rs:50-53, 96-108) */
static void quant_rows_avx(const float *x, int m, int k, int kb, int8_t *q, float *s, int32_t *su) {
    const int nb = k / kb;
    for (int r = 0; r < m; r++)
        for (int b = 0; b < nb; b++)
            quant_block_avx(x + (size_t)r * k + (size_t)b * kb, kb, q + (size_t)r * k + (size_t)b * kb, NULL,
                            s + (size_t)r * nb + b, su + (size_t)r * nb + b);
}
static void quant_pair_avx(const float *x, int k, int kb, int8_t *q, float *s, int32_t *su) {
    const int nb = k / kb;
    float resid[32];
    for (int b = 0; b < nb; b++) {
        quant_block_avx(x + (size_t)b * kb, kb, q + (size_t)b * kb, resid, s + b, su + b);
        quant_block_avx(resid, kb, q + k + (size_t)b * kb, NULL, s + nb + b, su + nb + b);
    }
}

/* gemv.rs:81-172: strips [s0, s1) of a TQ matrix (w at strip s0) against m <= 8 physical rows */
static void gemv_vnni(const uint8_t *w, int k, int bits, int kb, int s0, int s1, const orc_qact *xq, float *y,
                      size_t ldy, const uint32_t *rows, int accumulate) {
    const int m = xq->m, nb = k / kb;
    const size_t bb = orc_tq_block_bytes(bits, kb);
    const __m512i lo_mask = _mm512_set1_epi8(0x0F);
    const uint8_t *wp = w;
    for (int s = s0; s < s1; s++) {
        __m512 accf[ORC_MAX_M];
        for (int mi = 0; mi < m; mi++) accf[mi] = _mm512_setzero_ps();
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = wp;
            wp += bb;
            _mm_prefetch((const char *)(wp + 3 * bb), _MM_HINT_T0);
            _mm_prefetch((const char *)(wp + 3 * bb + 64), _MM_HINT_T0);
            if (bb > 128) {
                _mm_prefetch((const char *)(wp + 3 * bb + 128), _MM_HINT_T0);
                _mm_prefetch((const char *)(wp + 3 * bb + 192), _MM_HINT_T0);
            }
            const __m512 d = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)blk));
            const __m512 mn = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)(blk + 32)));
            const uint8_t *qb = blk + ORC_HDR_BYTES;
            __m512i acc32[ORC_MAX_M];
            for (int mi = 0; mi < m; mi++) acc32[mi] = _mm512_setzero_si512();
            if (bits == 8) {
                for (int j = 0; j < kb / 4; j++) {
                    const __m512i wq = _mm512_loadu_si512((const void *)(qb + j * 64));
                    for (int mi = 0; mi < m; mi++) {
                        int32_t xa;
                        memcpy(&xa, xq->q + (size_t)mi * k + (size_t)b * kb + 4 * j, 4);
                        acc32[mi] = _mm512_dpbusd_epi32(acc32[mi], wq, _mm512_set1_epi32(xa));
                    }
                }
            } else {
                const uint8_t *plane = qb + kb / 8 * 64;
                for (int j = 0; j < kb / 8; j++) {
                    const __m512i raw = _mm512_loadu_si512((const void *)(qb + j * 64));
                    __m512i lo = _mm512_and_si512(raw, lo_mask);
                    __m512i hi = _mm512_and_si512(_mm512_srli_epi16(raw, 4), lo_mask);
                    if (bits == 5) {
                        uint64_t mlo, mhi;
                        memcpy(&mlo, plane + j * 16, 8);
                        memcpy(&mhi, plane + j * 16 + 8, 8);
                        lo = _mm512_or_si512(lo, _mm512_maskz_set1_epi8(mlo, 0x10));
                        hi = _mm512_or_si512(hi, _mm512_maskz_set1_epi8(mhi, 0x10));
                    }
                    for (int mi = 0; mi < m; mi++) {
                        const int8_t *xp = xq->q + (size_t)mi * k + (size_t)b * kb;
                        int32_t xa, xb;
                        memcpy(&xa, xp + 4 * j, 4);
                        memcpy(&xb, xp + kb / 2 + 4 * j, 4);
                        acc32[mi] = _mm512_dpbusd_epi32(acc32[mi], lo, _mm512_set1_epi32(xa));
                        acc32[mi] = _mm512_dpbusd_epi32(acc32[mi], hi, _mm512_set1_epi32(xb));
                    }
                }
            }
            for (int mi = 0; mi < m; mi++) { /* acc += (d * sx) * acc32 + m * (sx * xsum) */
                const float sx = xq->scale[(size_t)mi * nb + b];
                const float u = sx * (float)xq->sum[(size_t)mi * nb + b];
                const __m512 t = _mm512_mul_ps(d, _mm512_set1_ps(sx));
                accf[mi] = _mm512_fmadd_ps(mn, _mm512_set1_ps(u), accf[mi]);
                accf[mi] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(acc32[mi]), t, accf[mi]);
            }
        }
        if (xq->pair) {
            for (int mi = 0; mi < m / 2; mi++) {
                float *yp = y + (rows ? rows[mi] : (size_t)mi) * ldy + (size_t)s * ORC_STRIP;
                const __m512 v = _mm512_add_ps(accf[2 * mi], accf[2 * mi + 1]);
                _mm512_storeu_ps(yp, accumulate ? _mm512_add_ps(_mm512_loadu_ps(yp), v) : v);
            }
        } else {
            for (int mi = 0; mi < m; mi++) {
                float *yp = y + (rows ? rows[mi] : (size_t)mi) * ldy + (size_t)s * ORC_STRIP;
                _mm512_storeu_ps(yp, accumulate ? _mm512_add_ps(_mm512_loadu_ps(yp), accf[mi]) : accf[mi]);
            }
        }
    }
}

/* gemv.rs:55-78: rows in passes of MAX_M physical rows */
static void gemm_vnni(const uint8_t *w, int k, int bits, int kb, int s0, int s1, const orc_qact *xq, float *y,
                      size_t ldy, const uint32_t *rows, int accumulate) {
    const int per = xq->pair ? 2 : 1, nb = k / xq->kb, logical = xq->m / per, group = ORC_MAX_M / per;
    for (int r0 = 0; r0 < logical; r0 += group) {
        const int r1 = r0 + group < logical ? r0 + group : logical;
        const orc_qact sub = {(r1 - r0) * per, k, xq->kb, xq->q + (size_t)r0 * per * k, xq->scale + (size_t)r0 * per * nb,
                              xq->sum + (size_t)r0 * per * nb, xq->pair};
        if (rows)
            gemv_vnni(w, k, bits, kb, s0, s1, &sub, y, ldy, rows + r0, accumulate);
        else
            gemv_vnni(w, k, bits, kb, s0, s1, &sub, y + (size_t)r0 * ldy, ldy, NULL, accumulate);
    }
}

/* TqMat::item / strip_bytes (weights.rs:14-35): strip s of a [rows][k] TQ matrix */
static const uint8_t *strip_ptr(const uint8_t *mat, int k, int bits, int kb, int s) {
    return mat + (size_t)s * (k / kb) * orc_tq_block_bytes(bits, kb);
}

/* ---- the decode layer (exec.rs:1540-1623) ---------------------------------------------- */

typedef struct {
    const orc_moe_w *W;
    const float *x;
    int k, hiprec;
    const orc_policy *pol;
    float *out;
    /* tile-shared */
    float *rlog, *hg, *hu;
    int8_t *aq;
    float *as;
    int32_t *asu;
    uint32_t *ids;
    float *w;
    int k_used;
} block_job;

static void block_task(cpu_pool *p, void *arg, int tid) {
    block_job *j = (block_job *)arg;
    const orc_moe_w *W = j->W;
    const int H = W->H, F = W->F, E = W->E, nc = p->n;
    int lo, hi;
    /* S5: this core's router rows (exec.rs:1003-1011) */
    split(E, tid, nc, &lo, &hi);
    for (int e = lo; e < hi; e++) {
        float v = dot_avx(W->router + (size_t)e * H, j->x, H);
        j->rlog[e] = W->router_bias ? v + W->router_bias[e] : v;
    }
    cpu_pool_barrier(p);
    /* every core routes (Model::route, exec.rs:630-639) and quantises x into its own scratch */
    uint32_t ids[ORC_MOE_K_MAX];
    float wts[ORC_MOE_K_MAX];
    const int k_used = j->pol ? orc_route_mass(j->rlog, E, j->pol, ids, wts)
                              : (orc_route_topk(j->rlog, E, j->k, ids, wts), j->k);
    if (tid == 0) {
        j->k_used = k_used;
        memcpy(j->ids, ids, sizeof ids);
        memcpy(j->w, wts, sizeof wts);
    }
    const int slots = k_used + 1, mrows = j->hiprec ? 2 : 1;
    const float sh_gate = orc_sigmoid(dot_avx(W->shexp_gate, j->x, H));
    int8_t xq[2 * 8192];
    float xs[2 * 256];
    int32_t xsu[2 * 256];
    if (j->hiprec)
        quant_pair_avx(j->x, H, 32, xq, xs, xsu);
    else
        quant_rows_avx(j->x, 1, H, 32, xq, xs, xsu);
    const orc_qact qa = {mrows, H, 32, xq, xs, xsu, j->hiprec};
    /* tasks A: (slot, gate|up, strip) round robin */
    const int ns = F / ORC_STRIP, ntask = slots * 2 * ns;
    for (int t = tid; t < ntask; t += nc) {
        const int slot = t / (2 * ns), which = (t / ns) % 2, s = t % ns;
        const int routed = slot < k_used;
        const uint8_t *mat = which == 0 ? (routed ? W->gate[ids[slot]] : W->sh_gate)
                                        : (routed ? W->up[ids[slot]] : W->sh_up);
        const int bits = routed ? W->gate_bits : W->sh_gate_bits;
        float *dst = (which == 0 ? j->hg : j->hu) + (size_t)slot * F;
        gemv_vnni(strip_ptr(mat, H, bits, 32, s), H, bits, 32, s, s + 1, &qa, dst, 0, NULL, 0);
    }
    cpu_pool_barrier(p);
    /* tasks B: SwiGLU, quantisation per down.kb = 16, the weight folded into the scales */
    const int kb = 16, nb = F / kb;
    float act[8192];
    for (int slot = tid; slot < slots; slot += nc) {
        orc_swiglu(j->hg + (size_t)slot * F, j->hu + (size_t)slot * F, act, F);
        const float wgt = slot < k_used ? wts[slot] : sh_gate;
        int8_t *q = j->aq + (size_t)2 * slot * F;
        float *sc = j->as + (size_t)2 * slot * nb;
        int32_t *su = j->asu + (size_t)2 * slot * nb;
        if (j->hiprec)
            quant_pair_avx(act, F, kb, q, sc, su);
        else
            quant_rows_avx(act, 1, F, kb, q, sc, su);
        for (int i = 0; i < mrows * nb; i++) sc[i] *= wgt;
    }
    cpu_pool_barrier(p);
    /* tasks C: this core's down strips over every slot (slot 0 stores, later slots add) */
    split(H / ORC_STRIP, tid, nc, &lo, &hi);
    if (hi > lo)
        for (int slot = 0; slot < slots; slot++) {
            const int routed = slot < k_used;
            const uint8_t *mat = routed ? W->down[ids[slot]] : W->sh_down;
            const int bits = routed ? W->down_bits : W->sh_down_bits;
            const orc_qact da = {mrows, F, kb, j->aq + (size_t)2 * slot * F, j->as + (size_t)2 * slot * nb,
                                 j->asu + (size_t)2 * slot * nb, j->hiprec};
            gemv_vnni(strip_ptr(mat, F, bits, kb, lo), F, bits, kb, lo, hi, &da, j->out, 0, NULL, slot > 0);
        }
}

/* One decode token through the pool; returns k_used (ids / w [32] may be NULL), -1 on a shape the
 * scratch does not hold (H, F <= 8192). */
int cpu_moe_block(cpu_pool *p, const orc_moe_w *W, const float *x, int k, const orc_policy *pol, int hiprec,
                  float *out, uint32_t *ids, float *w) {
    if (W->H > 8192 || W->F > 8192) return -1;
    const int E = W->E, F = W->F, slots = ORC_MOE_K_MAX + 1, nb = F / 16;
    block_job j = {W, x, k, hiprec, pol, out, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 0};
    uint32_t ids_l[ORC_MOE_K_MAX];
    float w_l[ORC_MOE_K_MAX];
    j.rlog = (float *)malloc(sizeof(float) * E);
    j.hg = (float *)malloc(sizeof(float) * (size_t)slots * F);
    j.hu = (float *)malloc(sizeof(float) * (size_t)slots * F);
    j.aq = (int8_t *)malloc((size_t)2 * slots * F);
    j.as = (float *)malloc(sizeof(float) * 2 * slots * nb);
    j.asu = (int32_t *)malloc(sizeof(int32_t) * 2 * slots * nb);
    j.ids = ids ? ids : ids_l;
    j.w = w ? w : w_l;
    pool_run(p, block_task, &j);
    free(j.rlog);
    free(j.hg);
    free(j.hu);
    free(j.aq);
    free(j.as);
    free(j.asu);
    return j.k_used;
}

/* ---- the batch layer (exec_batch.rs:1404-1580) ------------------------------------------ */

typedef struct {
    const orc_moe_w *W;
    const float *x;
    int M, k, router_dot_max_m;
    const orc_policy *pol;
    float *out;
    float *lg;
    int8_t *xq;
    float *xs;
    int32_t *xsu;
    uint32_t *ids;
    float *w;
    uint32_t *n_sel;
    uint32_t *ent_tok, *ent_expert, *grp_start, *grp_expert, *grp_order;
    float *ent_w;
    int n_ent, ng;
    float *hg, *hu;
    int8_t *aq;
    float *as;
    int32_t *asu;
    int8_t *gq; /* per-core gather buffers [nc][M][H] */
    float *gs;
    int32_t *gsu;
} batch_job;

static void batch_task(cpu_pool *p, void *arg, int tid) {
    batch_job *j = (batch_job *)arg;
    const orc_moe_w *W = j->W;
    const int H = W->H, F = W->F, E = W->E, M = j->M, nc = p->n, ka = ORC_MOE_K_MAX, nbx = H / 32;
    int lo, hi;
    /* router (exec_batch.rs:989-1019): per-row dot below the tile's core count, else the gemm */
    if (M < j->router_dot_max_m) {
        split(E, tid, nc, &lo, &hi);
        for (int mi = 0; mi < M; mi++)
            for (int e = lo; e < hi; e++) j->lg[(size_t)mi * E + e] = dot_avx(W->router + (size_t)e * H, j->x + (size_t)mi * H, H);
    } else {
        split((M + 3) / 4, tid, nc, &lo, &hi);
        gemm_nt_avx(j->x, H, W->router, H, H, j->lg, E, 4 * lo, 4 * hi < M ? 4 * hi : M, 0, E);
    }
    if (W->router_bias) {
        split(M, tid, nc, &lo, &hi);
        for (int mi = lo; mi < hi; mi++)
            for (int e = 0; e < E; e++) j->lg[(size_t)mi * E + e] = j->lg[(size_t)mi * E + e] + W->router_bias[e];
    }
    cpu_pool_barrier(p);
    /* route + quant_rows per token (exec_batch.rs:1415-1425) */
    split(M, tid, nc, &lo, &hi);
    for (int mi = lo; mi < hi; mi++) {
        const float *lgr = j->lg + (size_t)mi * E;
        j->n_sel[mi] = (uint32_t)(j->pol ? orc_route_mass(lgr, E, j->pol, j->ids + (size_t)mi * ka, j->w + (size_t)mi * ka)
                                         : (orc_route_topk(lgr, E, j->k, j->ids + (size_t)mi * ka, j->w + (size_t)mi * ka), j->k));
        quant_rows_avx(j->x + (size_t)mi * H, 1, H, 32, j->xq + (size_t)mi * H, j->xs + (size_t)mi * nbx,
                       j->xsu + (size_t)mi * nbx);
    }
    cpu_pool_barrier(p);
    /* grouping on core 0 (exec_batch.rs:1428-1462): stable counting sort by expert, LPT order */
    if (tid == 0) {
        int n_ent = 0;
        for (int mi = 0; mi < M; mi++) n_ent += (int)j->n_sel[mi];
        uint32_t *cnt = (uint32_t *)calloc((size_t)E + 1, sizeof(uint32_t));
        for (int mi = 0; mi < M; mi++)
            for (uint32_t s = 0; s < j->n_sel[mi]; s++) cnt[j->ids[(size_t)mi * ka + s] + 1]++;
        for (int e = 0; e < E; e++) cnt[e + 1] += cnt[e];
        for (int mi = 0; mi < M; mi++)
            for (uint32_t s = 0; s < j->n_sel[mi]; s++) {
                const uint32_t e = j->ids[(size_t)mi * ka + s], at = cnt[e]++;
                j->ent_tok[at] = (uint32_t)mi;
                j->ent_w[at] = j->w[(size_t)mi * ka + s];
                j->ent_expert[at] = e;
            }
        free(cnt);
        int ng = 0;
        uint32_t last = 0xffffffffu;
        for (int r = 0; r < n_ent; r++)
            if (j->ent_expert[r] != last) {
                j->grp_start[ng] = (uint32_t)r;
                j->grp_expert[ng++] = j->ent_expert[r];
                last = j->ent_expert[r];
            }
        j->grp_start[ng] = (uint32_t)n_ent;
        for (int g = 0; g < ng; g++) j->grp_order[g] = (uint32_t)g;
        for (int a = 1; a < ng; a++) { /* stable insertion sort by group size, descending */
            const uint32_t v = j->grp_order[a], sv = j->grp_start[v + 1] - j->grp_start[v];
            int b = a - 1;
            while (b >= 0 && j->grp_start[j->grp_order[b] + 1] - j->grp_start[j->grp_order[b]] < sv) {
                j->grp_order[b + 1] = j->grp_order[b];
                b--;
            }
            j->grp_order[b + 1] = v;
        }
        j->n_ent = n_ent;
        j->ng = ng;
    }
    cpu_pool_barrier(p);
    const int ng = j->ng, n_ent = j->n_ent;
    /* tasks A: (group, gate|up) in LPT order over all strips on the gathered rows, then the
     * shared expert's gate and up over all M rows */
    const int ns = F / ORC_STRIP, ntask = ng * 2 + 2;
    int8_t *gq = j->gq + (size_t)tid * M * H;
    float *gs = j->gs + (size_t)tid * M * nbx;
    int32_t *gsu = j->gsu + (size_t)tid * M * nbx;
    int gathered = -1;
    for (int t = tid; t < ntask; t += nc) {
        if (t < ng * 2) {
            const int grp = (int)j->grp_order[t / 2], which = t % 2;
            const int r0 = (int)j->grp_start[grp], r1 = (int)j->grp_start[grp + 1];
            const uint32_t e = j->grp_expert[grp];
            if (gathered != grp) {
                for (int r = r0; r < r1; r++) {
                    const int tok = (int)j->ent_tok[r], i = r - r0;
                    memcpy(gq + (size_t)i * H, j->xq + (size_t)tok * H, (size_t)H);
                    memcpy(gs + (size_t)i * nbx, j->xs + (size_t)tok * nbx, sizeof(float) * nbx);
                    memcpy(gsu + (size_t)i * nbx, j->xsu + (size_t)tok * nbx, sizeof(int32_t) * nbx);
                }
                gathered = grp;
            }
            const orc_qact ga = {r1 - r0, H, 32, gq, gs, gsu, 0};
            gemm_vnni(which == 0 ? W->gate[e] : W->up[e], H, W->gate_bits, 32, 0, ns, &ga,
                      (which == 0 ? j->hg : j->hu) + (size_t)r0 * F, F, NULL, 0);
        } else {
            const orc_qact all = {M, H, 32, j->xq, j->xs, j->xsu, 0};
            gemm_vnni(t == ng * 2 ? W->sh_gate : W->sh_up, H, W->sh_gate_bits, 32, 0, ns, &all,
                      (t == ng * 2 ? j->hg : j->hu) + (size_t)n_ent * F, F, NULL, 0);
        }
    }
    cpu_pool_barrier(p);
    /* tasks B: per entry row (and the shared rows), SwiGLU, quantise per 16, fold the weight */
    const int kb = 16, nbd = F / kb, total = n_ent + M;
    float act[8192];
    split(total, tid, nc, &lo, &hi);
    for (int r = lo; r < hi; r++) {
        orc_swiglu(j->hg + (size_t)r * F, j->hu + (size_t)r * F, act, F);
        const float wgt = r < n_ent ? j->ent_w[r] : orc_sigmoid(dot_avx(W->shexp_gate, j->x + (size_t)(r - n_ent) * H, H));
        quant_rows_avx(act, 1, F, kb, j->aq + (size_t)r * F, j->as + (size_t)r * nbd, j->asu + (size_t)r * nbd);
        for (int i = 0; i < nbd; i++) j->as[(size_t)r * nbd + i] *= wgt;
    }
    cpu_pool_barrier(p);
    /* tasks C: this core's down strips: the shared expert over all rows first (overwrite), then every
     * group ascending by expert, accumulated into its tokens' rows */
    split(H / ORC_STRIP, tid, nc, &lo, &hi);
    if (hi > lo) {
        const orc_qact sa = {M, F, kb, j->aq + (size_t)n_ent * F, j->as + (size_t)n_ent * nbd, j->asu + (size_t)n_ent * nbd, 0};
        gemm_vnni(strip_ptr(W->sh_down, F, W->sh_down_bits, kb, lo), F, W->sh_down_bits, kb, lo, hi, &sa, j->out, H, NULL, 0);
        for (int g = 0; g < ng; g++) {
            const int r0 = (int)j->grp_start[g], r1 = (int)j->grp_start[g + 1];
            const uint32_t e = j->grp_expert[g];
            const orc_qact da = {r1 - r0, F, kb, j->aq + (size_t)r0 * F, j->as + (size_t)r0 * nbd, j->asu + (size_t)r0 * nbd, 0};
            gemm_vnni(strip_ptr(W->down[e], F, W->down_bits, kb, lo), F, W->down_bits, kb, lo, hi, &da, j->out, H,
                      j->ent_tok + r0, 1);
        }
    }
}

/* M tokens through the pool (x [M][H] -> out [M][H]); returns the number of entries. */
int cpu_moe_batch(cpu_pool *p, const orc_moe_w *W, const float *x, int M, int k, const orc_policy *pol,
                  int router_dot_max_m, float *out) {
    if (W->H > 8192 || W->F > 8192 || M <= 0) return -1;
    const int H = W->H, F = W->F, E = W->E, ka = ORC_MOE_K_MAX, nbx = H / 32, nc = p->n;
    const size_t ent_cap = (size_t)M * ka, rows = ent_cap + M;
    batch_job j;
    memset(&j, 0, sizeof j);
    j.W = W;
    j.x = x;
    j.M = M;
    j.k = k;
    j.router_dot_max_m = router_dot_max_m;
    j.pol = pol;
    j.out = out;
    j.lg = (float *)malloc(sizeof(float) * (size_t)M * E);
    j.xq = (int8_t *)malloc((size_t)M * H);
    j.xs = (float *)malloc(sizeof(float) * (size_t)M * nbx);
    j.xsu = (int32_t *)malloc(sizeof(int32_t) * (size_t)M * nbx);
    j.ids = (uint32_t *)malloc(sizeof(uint32_t) * ent_cap);
    j.w = (float *)malloc(sizeof(float) * ent_cap);
    j.n_sel = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)M);
    j.ent_tok = (uint32_t *)malloc(sizeof(uint32_t) * ent_cap);
    j.ent_expert = (uint32_t *)malloc(sizeof(uint32_t) * ent_cap);
    j.ent_w = (float *)malloc(sizeof(float) * ent_cap);
    j.grp_start = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)E + 2));
    j.grp_expert = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)E + 1));
    j.grp_order = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)E + 1));
    j.hg = (float *)malloc(sizeof(float) * rows * F);
    j.hu = (float *)malloc(sizeof(float) * rows * F);
    j.aq = (int8_t *)malloc(rows * F);
    j.as = (float *)malloc(sizeof(float) * rows * (F / 16));
    j.asu = (int32_t *)malloc(sizeof(int32_t) * rows * (F / 16));
    j.gq = (int8_t *)malloc((size_t)nc * M * H);
    j.gs = (float *)malloc(sizeof(float) * (size_t)nc * M * nbx);
    j.gsu = (int32_t *)malloc(sizeof(int32_t) * (size_t)nc * M * nbx);
    pool_run(p, batch_task, &j);
    const int n_ent = j.n_ent;
    free(j.lg); free(j.xq); free(j.xs); free(j.xsu); free(j.ids); free(j.w); free(j.n_sel);
    free(j.ent_tok); free(j.ent_expert); free(j.ent_w); free(j.grp_start); free(j.grp_expert);
    free(j.grp_order); free(j.hg); free(j.hu); free(j.aq); free(j.as); free(j.asu); free(j.gq);
    free(j.gs); free(j.gsu);
    return n_ent;
}
