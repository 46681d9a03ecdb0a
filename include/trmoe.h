/*
 * trmoe — MI355X (gfx950) HIP implementation of tr-infer's MoE block behind a C ABI.
 *
 * Drop-in for the CPU MoE path of tokenring-ai/tr-infer: the router, top-k / cumulative-mass
 * routing, the token-to-expert dispatch, the Q4_K/Q6_K SwiGLU experts against int8-quantised
 * activations, the shared expert with its sigmoid gate, and the combine.  Results follow the
 * reference's CPU arithmetic (per-block f32 epilogue, FMA chains, accumulation order).
 *
 * Conventions (mirroring the kernel contracts of crates/tr-kernels/src in the reference):
 *   - every pointer argument is a DEVICE pointer unless stated otherwise; the caller owns all
 *     buffers (the reference preallocates workspaces at load, exec.rs:733-779);
 *   - `stream` is a hipStream_t (0 = the null stream); all work is stream-ordered and
 *     asynchronous unless a function says it synchronises;
 *   - functions return a trk_status; the reference's asserts/panics (gemv.rs:35, quant.rs:68-71,
 *     router.rs:75) become TRK_E_INVALID and MoePolicy::validate errors (router.rs:32-44) become
 *     TRK_E_POLICY, with the message in trk_last_error();
 *   - nothing here allocates device memory except trk_create.
 */
#ifndef TRMOE_H
#define TRMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRK_ABI_VERSION 3
#define TRK_MOE_K_MAX 32 /* router.rs:6 MOE_K_MAX */

typedef enum {
    TRK_OK = 0,
    TRK_E_INVALID = -1,  /* bad shape / pointer / codec: the reference asserts */
    TRK_E_POLICY = -2,   /* MoePolicy::validate (router.rs:32-44) */
    TRK_E_CAPACITY = -3, /* more rows than the context was created for */
    TRK_E_HIP = -4,      /* a HIP runtime call failed */
    TRK_E_NOMEM = -5,
    TRK_E_TIMEOUT = -6   /* a device-side wait of the one-launch decode layer gave up (bounded spin):
                            the outputs of the calls since the last trk_get_stats are invalid */
} trk_status;

enum { TRK_FMT_Q5_1 = 7, TRK_FMT_Q8_0 = 8, TRK_FMT_Q4_K = 12, TRK_FMT_Q6_K = 14 }; /* GGML type ids (python/trpack/blocks.py:11) */
/* The reference's packed TQ codecs (crates/tr-format/src/codec.rs:1-46, Codec {bits, kb}):
 * fmt = bits << 8 | kb.  A TQ matrix is ceil(rows / 16) strips of k / kb blocks, each block
 * d[16] f16 | m[16] f16 | q | (5-bit) high-bit plane, exactly as trpack writes it. */
enum {
    TRK_FMT_TQ4_16 = 0x410, TRK_FMT_TQ4_32 = 0x420, TRK_FMT_TQ5_16 = 0x510,
    TRK_FMT_TQ5_32 = 0x520, TRK_FMT_TQ8_16 = 0x810, TRK_FMT_TQ8_32 = 0x820
};
enum { TRK_BASIS_ALL = 0, TRK_BASIS_TOP = 1 }; /* MassBasis (router.rs:9-16) */

/* A stack of `count` weight matrices [rows][k], `stride` bytes apart.  Replaces
 * tr_model::weights::TqMat {ptr, rows, k, codec, count, stride} (crates/tr-model/src/weights.rs:
 * 14-35); `fmt` says how the bytes are laid out:
 *   - a TQ codec (TRK_FMT_TQ*): the reference's packed strips exactly as trpack writes them, a
 *     pack's TensorKind::Tq entry uploaded unchanged.  register() (weights.rs:207-210) fills
 *     rows, k, codec, count and stride from the manifest entry (manifest.rs:65-94): pass the same
 *     values, with fmt = bits << 8 | kb.  Gate/up take a kb-32 codec, downs a kb-16 codec (the
 *     activations' block sizes).  16-byte aligned (every TQ block is a multiple of 16 bytes).
 *   - a GGUF block format read in place on the GPU (the CPU path reads its TQ re-layout):
 *     gate/up Q4_K; down (routed and shared alike) Q4_K, Q6_K, Q8_0 or Q5_1 (blocks.py:57-78);
 *     row-major rows of superblocks.  Q4_K, Q8_0 and Q5_1 stacks are 16-byte aligned, Q6_K 2-byte.
 * tile_stride: bytes from one tile's tensor to the next in a layer packed for n_tiles > 1 tiles
 * (trk_cfg): tile t's tensor (the pack's entry for tile t) starts at ptr + t * tile_stride, and
 * rows / k give ONE tile's shape (gate/up [n_ff / T][H], down [H][n_ff / T], python/trpack/
 * plan.py:106-118).  Ignored with one tile. */
typedef struct {
    const void *ptr;
    uint32_t rows, k;
    uint32_t fmt;
    uint32_t count;
    uint64_t stride;
    uint64_t tile_stride;
} trk_mat;

/* One layer's MoE weights. Replaces tr_model::exec::MoeW (crates/tr-model/src/exec.rs:86-96). */
typedef struct {
    const float *router;      /* [E][H] f32 (ffn_gate_inp); packed for T > 1 tiles: the tiles'
                                 K-split slices back to back, [T][E][H / T] (plan.py:174-181) */
    const float *router_bias; /* [E] f32 or NULL: additive logit bias for synthetic load skew;
                                 the reference has no bias (pass NULL for its semantics) */
    const float *shexp_gate;  /* [H] f32 (ffn_gate_inp_shexp) */
    trk_mat gate, up, down;   /* routed experts: gate/up [F][H] (Q4_K), down [H][F] (Q4_K|Q6_K) */
    trk_mat sh_gate, sh_up, sh_down; /* shared expert, count 1 */
} trk_moe_w;

/* Cumulative-mass routing. Replaces tr_kernels::router::MoePolicy (router.rs:18-30). */
typedef struct {
    uint32_t min, max;
    float mass;
    uint32_t basis;
} trk_moe_policy;

/* Layer shape and workspace sizing (ModelConfig, crates/tr-model/src/config.rs:5-99). */
typedef struct {
    uint32_t hidden;           /* H (multiple of 256) */
    uint32_t n_expert;         /* E (<= 1024) */
    uint32_t n_ff;             /* F, per routed and shared expert (a multiple of 256 for GGUF
                                  experts, of 16 per tile for TQ experts) */
    uint32_t n_expert_used;    /* k of the fixed top-k routing (<= 32) */
    uint32_t m_max;            /* most rows one call may carry (the reference's batch_max) */
    uint32_t k_cap;            /* most experts one token may select, sizes the entry buffers
                                  (0 = n_expert_used; a policy's max must not exceed it) */
    uint32_t router_dot_max_m; /* batch logits use the per-row dot order when M < this, else the
                                  gemm_f32_nt order (exec_batch.rs:989-1019: the reference
                                  switches at its tile's core count); 0 = 16 */
    int32_t hiprec;            /* M == 1: two-level activations (TR_HIPREC, exec.rs:782) */
    uint32_t n_tiles;          /* T, the tiles the pack was written for (ModelConfig::n_tiles,
                                  plan.py:88): 0 or 1 = one.  With T > 1 (TQ experts only) the
                                  router is K-split and every expert is split by n_ff into T
                                  tiles, as trpack shards them; the layer then sums the tiles'
                                  router partials and down partials in tile order (exchange.rs:
                                  122-136), as the reference's tiles do */
    uint32_t n_expert_packed;  /* experts in the pack (ModelConfig::n_expert_packed, a subset
                                  pack of the first experts, exec.rs:1545-1549): routed ids are
                                  folded onto them (fold_ids, exec_batch.rs:214-225); 0 = n_expert */
} trk_cfg;

/* Replaces tr_model::exec::MoeStats counters rows/experts (exec.rs:558-605). */
typedef struct {
    uint64_t rows, experts;
} trk_moe_stats;

typedef struct trk_ctx trk_ctx;

/* ---- layer-level entry points ---------------------------------------------------------- */

/* Allocate the device workspaces for cfg (Model::load_with sizing, exec.rs:733-779) on the
 * current HIP device. */
int trk_create(const trk_cfg *cfg, trk_ctx **out);
int trk_destroy(trk_ctx *ctx);

/* Switch the routing policy; NULL = the fixed top-n_expert_used.
 * Replaces Model::set_moe (exec.rs:619-625). */
int trk_set_moe(trk_ctx *ctx, const trk_moe_policy *policy);

/* out[M][H] = MoE(x[M][H]).  M == 1 follows Model::moe_block (exec.rs:1540-1623, with the S5
 * router dot of exec.rs:1003-1011); M >= 2 follows Model::moe_batch (exec_batch.rs:1404-1580,
 * with the router of exec_batch.rs:989-1019).  rlog: [M][E] precomputed logits or NULL to
 * compute them from w->router.  Replaces both call sites' worker-side bodies (one call per layer
 * from one host thread instead of an SPMD pool run). */
int trk_moe_forward(trk_ctx *ctx, const trk_moe_w *w, const float *x, const float *rlog, uint32_t m,
                    float *out, void *stream);

/* The device workspace, in bytes, that the layer needs for m rows of this configuration: what
 * trk_create allocates for m_max = m, and what trk_moe_forward_noalloc needs of its static scratch.
 * Host-only (no GPU call); errors as for trk_create.  Sizing helper for callers that preallocate,
 * as Model::load_with sizes its arenas (exec.rs:733-779, exec_batch.rs:127-211). */
int trk_workspace_bytes(const trk_cfg *cfg, uint32_t m, size_t *bytes);

/* Config-5 layer: h[M][H] += MoE(rmsnorm(h; rms_w, eps)).  Composes elem::rmsnorm
 * (elem.rs:255-262), the MoE block and elem::add_inplace (elem.rs:104-118).  Below the router
 * GEMM threshold (and with the one-launch decode layer off) the logits launch normalises h as it
 * reads it, with the same bits as a separate rmsnorm; otherwise rmsnorm runs as its own launch. */
int trk_moe_residual(trk_ctx *ctx, const trk_moe_w *w, const float *rms_w, float eps, float *h,
                     uint32_t m, void *stream);

/* trk_moe_forward without a context and without allocating anything: no counterpart in the
 * reference.  For callers that cannot allocate (code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc).  cfg gives the layer shape as for trk_create (m_max is
 * ignored: the workspace is laid out for this call's m), policy the routing (NULL = top
 * n_expert_used).  The workspace lives in a static device array of TRK_NOALLOC_SCRATCH_BYTES per
 * GPU, held until the process ends; a call whose workspace does not fit returns TRK_E_CAPACITY (at
 * H = 2048, E = 512, F = 512, k = 10 that is M above 100; trk_workspace_bytes gives the need of any
 * shape).  Every call on one GPU shares that array:
 * calls that overlap on one GPU (several host threads or streams) race.  MoeStats are not counted
 * and the one-launch decode layer is not used.  Results are those of trk_moe_forward. */
#define TRK_NOALLOC_SCRATCH_BYTES (16u << 20)
int trk_moe_forward_noalloc(const trk_cfg *cfg, const trk_moe_policy *policy, const trk_moe_w *w, const float *x,
                            const float *rlog, uint32_t m, float *out, void *stream);

/* Read (and optionally reset) the routing counters, ordered after the work queued on `stream`
 * (synchronises that stream only).  Returns TRK_E_TIMEOUT, with the counters filled, when a
 * device-side wait of the one-launch decode layer timed out since the last call (and clears that
 * flag): the outputs of those calls are invalid.  Replaces MoeStats::snapshot (exec.rs:593-595). */
int trk_get_stats(trk_ctx *ctx, trk_moe_stats *out, int reset, void *stream);

/* Router-mass profiling: MoeStats::profile_start (exec.rs:567-573) zeroes the profile and turns it
 * on; every later forward then adds each row's router::mass_profile (router.rs:152-166: the
 * cumulative softmax mass of its best 1..32 experts, fixed point 1e-6) to it, as
 * MoeStats::profile_row (exec.rs:582-592) does.  trk_profile_report (exec.rs:575-581) writes the
 * mean cumulative mass of the best k experts, k = 1..32, to cum[32] (host memory) and the number of
 * profiled rows to *rows, ordered after `stream` (synchronises it); on = 0 in trk_profile_start
 * turns profiling off. */
int trk_profile_start(trk_ctx *ctx, int on, void *stream);
int trk_profile_report(trk_ctx *ctx, double *cum, uint64_t *rows, void *stream);

/* Message of the last error on this thread (static storage). */
const char *trk_last_error(void);

/* ---- kernel-level entry points (mirrors of tr-kernels, on caller buffers) --------------- */

/* Router logits rlog[m][E] = router . x[m] (+ bias): gemm_order 0 = attn::dot per row
 * (attn.rs:329-357), 1 = smallgemm::gemm_f32_nt (smallgemm.rs:8-59).  Also the shared-gate
 * logit sh[m] = dot(shexp_gate, x[m]) when shexp_gate is not NULL. */
int trk_router_logits(const float *router, const float *bias, const float *shexp_gate, const float *x,
                      uint32_t m, uint32_t n_expert, uint32_t hidden, int gemm_order, float *rlog,
                      float *sh, void *stream);

/* The hyper-connection mix of the FFN input, part B (tr_model::exec::HcW {up}, exec.rs:49-55):
 * up = the low-rank up projection [hc * hidden][lr] in a kb-32 TQ codec, hc streams (1..8), low
 * rank lr (a multiple of 32, at most 1024).  A batch call keeps the quantised lo rows (1.375 lr
 * bytes per row, rows rounded up to 16) in the context's per-entry output rows, which hold at least
 * 4 (k + 1) m_max hidden bytes; a call beyond them returns TRK_E_CAPACITY. */
typedef struct {
    trk_mat up;
    uint32_t hc, lr;
} trk_hc_w;

/* out[M][H] = MoE(mixed) where mixed is the MoE input the hyper-connection mix produces from the
 * normed streams xn[M][hc][H] (hc_mix_a's output) and the low-rank projection lo[M][lr] summed
 * over tiles: Model::hc_mix_b (exec.rs:1196-1234) + the S5 router + moe_block at M = 1 (two-level
 * lo with hiprec), hc_b_batch (exec_batch.rs:929-1019) + moe_batch at M >= 2, on one tile.  The
 * mix runs as the layer's input stage (one launch at M = 1; at M >= 2 a quantisation of lo, then
 * the mix); the router then reads the mixed rows. */
int trk_moe_forward_hc(trk_ctx *ctx, const trk_moe_w *w, const trk_hc_w *hc, const float *xn, const float *lo,
                       uint32_t m, float *out, void *stream);

/* Per-row routing: route_topk (router.rs:106-113) or, with a policy, route_mass
 * (router.rs:118-148).  ids/w: [m][32], n_sel: [m]. */
int trk_route(const float *logits, uint32_t m, uint32_t n_expert, uint32_t k, const trk_moe_policy *policy,
              uint32_t *ids, float *w, uint32_t *n_sel, void *stream);

/* int8 activation quantisation per kb-block (kb 16 or 32): QActRef::quantize_into
 * (quant.rs:36-48); pair != 0 quantises ONE row into (coarse, residual) rows, quantize_pair_into
 * (quant.rs:50-53).  q [m or 2][k], scale/sum [m or 2][k/kb]. */
int trk_quantize(const float *x, uint32_t m, uint32_t k, uint32_t kb, int pair, int8_t *q, float *scale,
                 int32_t *sum, void *stream);

/* y[rows[i] * ldy + r] (+)= W_item[r] . x_i for the rows r of 16-row strips [s0, s1) and int8
 * activation rows x: gemv_tq_rows / gemm_tq_rows (gemv.rs:16-78) with w = the strip-s0 pointer of
 * matrix `item`.  Any number of activation rows (gemm_tq_rows' chunking is internal); logical
 * rows are written in order, so a row map with repeats accumulates as the reference's does.
 *   w->fmt  a TQ codec (kb must equal the codec's, gemv.rs:27; k a multiple of kb), or a GGUF
 *           block format (k a multiple of 256) read as its TQ conversion: Q4_K with kb 32 or 16,
 *           Q6_K with kb 16, Q8_0 / Q5_1 with kb 32 or 16 (blocks.py:57-113);
 *   s1      at most ceil(rows / 16).  TQ writes every row of each strip (zero padding rows
 *           included, as the reference's 16-wide stores do); GGUF writes rows < w->rows;
 *   pair    rows come in (coarse, residual) pairs, m counts physical rows;
 *   rows    NULL = identity (logical row i to y row i).
 * q: 16-byte aligned, [m][k]; scale / sum: [m][k / kb]. */
int trk_gemv(const trk_mat *w, uint32_t item, uint32_t s0, uint32_t s1, uint32_t kb, const int8_t *q,
             const float *scale, const int32_t *sum, uint32_t m, int pair, float *y, uint32_t ldy,
             const uint32_t *rows, int accumulate, void *stream);

/* y = silu(g) * u (elem::swiglu_vec, elem.rs:173-175) over n floats. */
int trk_swiglu(const float *g, const float *u, float *y, size_t n, void *stream);

/* y[m][n] = rmsnorm(x[m][n]; w, eps) (elem.rs:255-262). */
int trk_rmsnorm(const float *x, const float *w, float eps, uint32_t m, uint32_t n, float *y, void *stream);

/* y[i] += a[i] (elem.rs:104-118). */
int trk_add_inplace(float *y, const float *a, size_t n, void *stream);

/* ---- synthetic data (bit-identical to the test oracle's generator) ---------------------- */
/* GGUF superblocks of a [rows][k] matrix: d (and dmin) ~ U(dlo, dhi) as f16, all other bytes
 * uniform; fmt Q4_K, Q6_K, Q8_0 or Q5_1 (Q8_0 / Q5_1: every block's d, Q5_1 m = -16 U). */
int trk_gen_gguf(uint32_t fmt, uint64_t seed, uint64_t stream_id, uint32_t rows, uint32_t k, float dlo,
                 float dhi, void *out, void *stream);
/* The same for a stack of `count` matrices `stride` bytes apart, matrix e drawing from stream
 * stream0 + e * stream_step (one launch; what trk_gen_gguf gives per matrix). */
int trk_gen_gguf_stack(uint32_t fmt, uint64_t seed, uint64_t stream0, uint64_t stream_step, uint32_t count,
                       uint32_t rows, uint32_t k, float dlo, float dhi, void *out, uint64_t stride, void *stream);
/* n normals N(0, sigma) (Box-Muller in double, rounded to f32). */
int trk_gen_normal(uint64_t seed, uint64_t stream_id, size_t n, double sigma, float *out, void *stream);

/* ---- measurement and introspection ------------------------------------------------------ */
/* M == 1: run the whole layer as one launch when the layer's shape has a fused kernel and the GPU
 * can hold its grid at once (on), or as the three launches router / gate-up / down (off, the
 * default).  Both follow exec.rs:1540-1623 with identical results; no counterpart in the
 * reference, whose decode layer is one pool run. */
int trk_set_fusion(trk_ctx *ctx, int on);

/* M >= 2: grouped work items (one expert's entry rows, at most 16) of at most `rows` rows run on
 * the streaming GEMV kernels, larger ones on the int8 MFMA tiles.  rows = -1 (the default) picks
 * 16 for M <= 16 (every item streams), 4 while M * k_cap <= 2 * n_expert, else 0 (every item on
 * the tiles).  Every choice gives the same bits (moe_batch, exec_batch.rs:1404-1580); no
 * counterpart in the reference, which runs one grouped kernel per expert matrix. */
int trk_set_stream_rows(trk_ctx *ctx, int rows);

/* 2 <= M <= rows (default 8, 0..16): every token runs as a decode (its routing inside its gate/up
 * workgroups, its rows added by the down launch in the batch combine's order: shared expert
 * first, then ascending expert), three launches with no dispatch, grouped items or combine.  GGUF
 * layers with one tile; TQ layers where the decode kernels take the shape (the real one: kb-32
 * gate/up, kb-16 down, one tile, k_cap <= 15).  The same bits as the grouped path
 * (exec_batch.rs:1404-1580); the dispatch arrays (TRK_WS_ENT_*, items) are then not written.
 * No counterpart in the reference. */
int trk_set_decode_rows(trk_ctx *ctx, int rows);

/* Layers on TQ experts: the int8 MFMA kernels (on, the default, where H / 32 units of staged
 * activations fit a workgroup's LDS) or the generic grouped TQ GEMV (off).  Both give the same
 * bits; no counterpart in the reference. */
int trk_set_tq_mfma(trk_ctx *ctx, int on);

/* Per-kernel timing (the HIP counterpart of the reference's TR_PROFILE laps, exec.rs:344-430):
 * when on, every kernel a forward launches is bracketed by HIP events on the call's stream. */
int trk_set_timing(trk_ctx *ctx, int on);
/* Sum of the recorded durations per kernel since the last call, then forget them (synchronises).
 * Fills up to cap entries (kernel name, total ms, launches); returns the number of kernels. */
int trk_get_timing(trk_ctx *ctx, const char **names, double *ms, uint64_t *launches, int cap);

/* Launch only the kernel `name` (a name trk_get_timing reports) of the forward sequence for
 * (w, x, rlog, m, out), on the workspace as the previous calls left it.  For timing one kernel in
 * isolation (bench.py; the reference's kbench, crates/tr-kernels/benches): the results are only
 * meaningful when the calls before it prepared the workspace for the same inputs. */
int trk_launch_kernel(trk_ctx *ctx, const trk_moe_w *w, const float *x, const float *rlog, uint32_t m,
                      float *out, const char *name, void *stream);

/* Copy an internal workspace buffer of the last forward to host memory. */
enum {
    TRK_WS_RLOG = 1,     /* [M][E] f32 */
    TRK_WS_IDS = 2,      /* [M][32] u32 */
    TRK_WS_W = 3,        /* [M][32] f32 */
    TRK_WS_NSEL = 4,     /* [M] u32 */
    TRK_WS_ENT_TOK = 5,  /* [n_ent] u32 */
    TRK_WS_ENT_W = 6,    /* [n_ent] f32 */
    TRK_WS_ENT_EXP = 7,  /* [n_ent] u32 */
    TRK_WS_GRP_START = 8,/* [n_groups+1] u32 */
    TRK_WS_GRP_EXP = 9,  /* [n_groups] u32 */
    TRK_WS_NGROUPS = 10, /* [2] u32: n_groups, n_ent */
    TRK_WS_XQ = 11,      /* [rows][H] i8 (pair: 2 rows) */
    TRK_WS_XS = 12,      /* [rows][H/32] f32 */
    TRK_WS_ACTQ = 13,    /* activation rows of the down input, i8 */
    TRK_WS_ACTS = 14,    /* their folded scales, f32 */
    TRK_WS_SHLOGIT = 15, /* [M] f32: dot(shexp_gate, x) */
    TRK_WS_BARRIER_ERR = 16, /* u32: nonzero if a one-launch decode layer ever timed out at a grid barrier */
    TRK_WS_MIXED = 17    /* [M][H] f32: the MoE input trk_moe_forward_hc mixed */
};
/* Ordered after the work queued on `stream` (synchronises that stream only). */
int trk_debug_read(trk_ctx *ctx, int which, void *host_dst, size_t bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif
