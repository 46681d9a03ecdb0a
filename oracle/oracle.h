/*
 * CPU oracle for the tr-infer MoE block — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU MoE path (tokenring-ai/tr-infer, Rust), used
 * as the parity checker for the HIP library and as the timed CPU baseline ("port").  Nothing in
 * the product path may link or call it: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.
 *
 * Every function cites the reference file:line it follows.  The arithmetic order follows the
 * reference exactly (explicit fmaf where the reference uses FMA, no contraction elsewhere; the
 * library is compiled with -ffp-contract=off), so results are bit-identical to the reference
 * wherever the reference's own arithmetic is fixed by its source.  Two pieces are fixed only by
 * assumption and are therefore "pinned to tolerance":
 *   - the lane order of _mm512_reduce_add_ps (taken as the halving tree 16->8->4->2->1, the
 *     order Intel documents and stdarch implements) inside dot / gemm_f32_nt / sumsq;
 *   - Rust's f32::exp, taken as glibc expf (what rustc links on x86_64 Linux).
 * One piece has no reference at all and is "parity unpinned":
 *   - Q6_K (orc_q6k_rows and its uses): the reference has no Q6_K converter or kernel; this
 *     restatement's mapping (unsigned 6-bit q, dd = f16(d*sc), mm = f16(-32*dd), one block per
 *     scale) is checked only against a brute-force f64 dequantisation of the same bytes.
 */
#ifndef TR_ORACLE_H
#define TR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_STRIP 16      /* crates/tr-format/src/codec.rs:9  */
#define ORC_HDR_BYTES 64  /* crates/tr-format/src/codec.rs:10 */
#define ORC_MAX_M 8       /* crates/tr-kernels/src/gemv.rs:9  */
#define ORC_MOE_K_MAX 32  /* crates/tr-kernels/src/router.rs:6 */

/* GGML type ids used by the weight converters (python/trpack/blocks.py:11). Q6_K (14) is an
 * extension: the reference has no Q6_K converter. */
#define ORC_FMT_Q4_K 12
#define ORC_FMT_Q6_K 14
#define ORC_FMT_Q8_0 8
#define ORC_FMT_Q5_1 7

/* ---- half precision (IEEE binary16, round-to-nearest-even) ------------------------------ */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
/* Compare the software conversions with the F16C instructions over a strided sweep of all
 * 2^32 f32 bit patterns (and all 2^16 halves).  Returns the number of mismatches. */
uint64_t orc_selftest_f16(uint32_t stride);
int orc_have_f16c(void);

/* ---- TQ codec (crates/tr-format/src/codec.rs, python/trpack/codec.py) ------------------- */
size_t orc_tq_block_bytes(int bits, int kb);
size_t orc_tq_matrix_bytes(int rows, int k, int bits, int kb);
/* q [rows][k] unsigned, d/m [rows][k/kb] f16 bits -> packed bytes (codec.rs:118-169). */
void orc_pack_tq(int rows, int k, int bits, int kb, const uint8_t *q, const uint16_t *d,
                 const uint16_t *m, uint8_t *out);
uint32_t orc_tq_block_q(const uint8_t *blk, int bits, int kb, int r, int kk);
void orc_dequant_tq(const uint8_t *buf, int rows, int k, int bits, int kb, float *out);

/* ---- GGUF block quants -> (q, d, m) (python/trpack/blocks.py) ---------------------------- */
/* Q4_K rows: raw [rows][K/256*144] -> q [rows][K], dd/mm [rows][K/32] f16 bits. */
void orc_q4k_rows(const uint8_t *raw, int rows, int K, uint8_t *q, uint16_t *dd, uint16_t *mm);
/* Q6_K rows (extension, no reference math): q in [0,63], dd = f16(d*sc), mm = -32*dd per 16. */
void orc_q6k_rows(const uint8_t *raw, int rows, int K, uint8_t *q, uint16_t *dd, uint16_t *mm);
/* Q8_0 (34-byte blocks: f16 d, 32 int8) -> u8 q = int8 + 128, d, m = f16(-128 d) per 32 (blocks.py:71-78) */
void orc_q80_rows(const uint8_t *raw, int rows, int K, uint8_t *q, uint16_t *d, uint16_t *m);
/* Q5_1 (24-byte blocks: f16 d, f16 m, u32 qh, 16 qs) -> 5-bit q, d, m per 32 (blocks.py:57-68) */
void orc_q51_rows(const uint8_t *raw, int rows, int K, uint8_t *q, uint16_t *d, uint16_t *m);
/* Whole matrix GGUF -> TQ(bits, kb) bytes; returns bits, or -1 on an unsupported (fmt, kb). */
int orc_gguf_to_tq(int fmt, const uint8_t *raw, int rows, int K, int kb, uint8_t *out);
size_t orc_gguf_row_bytes(int fmt, int K);
/* Reference dequant of a raw GGUF matrix to f32 (for f64 brute-force checks). */
void orc_gguf_dequant(int fmt, const uint8_t *raw, int rows, int K, float *out);

/* ---- activation quantisation (crates/tr-kernels/src/quant.rs) ---------------------------- */
void orc_quant_block(const float *src, int n, int8_t *dst, float *scale, int32_t *sum);
void orc_quant_block_resid(const float *src, int n, int8_t *dst, float *resid, float *scale,
                           int32_t *sum);
void orc_quant_rows(const float *x, int m, int k, int kb, int8_t *q, float *s, int32_t *su);
/* Two-level: q [2][k] (coarse | residual), s/su [2][k/kb]. */
void orc_quant_pair(const float *x, int k, int kb, int8_t *q, float *s, int32_t *su);

/* ---- TQ x int8 GEMV (crates/tr-kernels/src/gemv.rs) -------------------------------------- */
typedef struct {
    int m, k, kb;          /* physical rows (pair: 2 per logical row) */
    const int8_t *q;       /* [m][k] */
    const float *scale;    /* [m][k/kb] */
    const int32_t *sum;    /* [m][k/kb] */
    int pair;
} orc_qact;

void orc_gemv_tq_rows(const uint8_t *w, int k, int bits, int kb, int s0, int s1,
                      const orc_qact *xq, float *y, size_t ldy, const uint32_t *rows,
                      int accumulate);
void orc_gemm_tq_rows(const uint8_t *w, int k, int bits, int kb, int s0, int s1,
                      const orc_qact *xq, float *y, size_t ldy, const uint32_t *rows,
                      int accumulate);

/* ---- f32 elementwise / reductions -------------------------------------------------------- */
float orc_dot(const float *a, const float *b, int n);                 /* attn.rs:329-357 */
void orc_gemm_f32_nt(const float *x, int ldx, int mr, const float *w, int ldw, int n, int k,
                     float *y, int ldy);                              /* smallgemm.rs:8-59 */
float orc_sumsq(const float *x, int n);                               /* elem.rs:224-252 */
void orc_rmsnorm(const float *x, const float *w, float eps, float *y, int n); /* elem.rs:255-262 */
float orc_exp512(float x);                                            /* elem.rs:7-25 */
float orc_sigmoid512(float x);                                        /* elem.rs:27-32 */
float orc_silu512(float x);                                           /* elem.rs:34-38 */
float orc_sigmoid(float x);                                           /* elem.rs:57-59 */
void orc_swiglu(const float *g, const float *u, float *y, int n);     /* elem.rs:173-175 */
void orc_add_inplace(float *y, const float *a, int n);                /* elem.rs:104-118 */

/* ---- router (crates/tr-kernels/src/router.rs) -------------------------------------------- */
#define ORC_BASIS_ALL 0
#define ORC_BASIS_TOP 1
typedef struct {
    uint32_t min, max;
    float mass;
    uint32_t basis;
} orc_policy;

int orc_policy_validate(const orc_policy *p, int n_expert, char *err, int errlen);
void orc_route_topk(const float *logits, int n, int k, uint32_t *ids, float *w);
int orc_route_mass(const float *logits, int n, const orc_policy *p, uint32_t *ids, float *w);
void orc_mass_profile(const float *logits, int n, float *cum /* [32] */);

/* ---- the MoE block (crates/tr-model/src/exec.rs, exec_batch.rs) -------------------------- */
typedef struct {
    int H, E, F;                /* hidden, experts, intermediate (per expert and shared) */
    const float *router;        /* [E][H] f32 */
    const float *router_bias;   /* [E] or NULL: synthetic-load bias added to the logits */
    const float *shexp_gate;    /* [H] */
    int gate_bits, down_bits;   /* TQ codecs: gate/up (bits, 32), down (bits, 16) */
    const uint8_t *const *gate; /* [E] TQ matrices [F][H] (NULL for experts never touched) */
    const uint8_t *const *up;   /* [E] [F][H] */
    const uint8_t *const *down; /* [E] [H][F] */
    int sh_gate_bits, sh_down_bits;
    const uint8_t *sh_gate, *sh_up, *sh_down;
    /* T tiles (python/trpack/plan.py:106-118,174-181): 0 or 1 = one tile.  With T > 1 the
     * router is [T][E][H/T] (tile t: columns [H/T t, H/T (t+1)) of every expert's row), each
     * gate/up pointer holds the T tiles' [F/T][H] matrices back to back (tile t: rows
     * [F/T t, F/T (t+1))), each down pointer the T tiles' [H][F/T] matrices (tile t: columns
     * [F/T t, F/T (t+1))), and the shared expert's likewise. */
    int tiles;
    /* n_expert_packed of a subset pack (exec.rs:1545-1549): routed ids are folded onto the first
     * `packed` experts by fold_ids (exec_batch.rs:214-225); 0 = E (no folding). */
    int packed;
} orc_moe_w;

/* fold_ids (exec_batch.rs:214-225): ids[i] <- the first of ids[i] % packed, +1, +2, ... (mod
 * packed) not among ids[0..i).  Returns -1 (the reference asserts) when n > packed. */
int orc_fold_ids(uint32_t *ids, int n, uint32_t packed);

/* Router logits of M rows x [M][H] into out [M][E]: per-row dot order (dot_rows) or the batch gemm
 * order, with the layer's tiles and bias. */
void orc_moe_logits(const orc_moe_w *W, const float *x, int M, int dot_rows, float *out);

typedef struct {
    uint64_t rows, experts; /* MoeStats::add (exec.rs:602-605) */
} orc_moe_stats;

/* Hyper-connection mix part B on one tile: mixed [m][hh] from xn [m][hc][hh] and lo [m][lr]
 * (exec.rs:1196-1234 when decode, exec_batch.rs:929-968 otherwise); up: TQ [hc*hh][lr], kb 32. */
void orc_hc_mix(const uint8_t *up, int bits, int hc, int hh, int lr, const float *xn, const float *lo, int m,
                int decode, int hiprec, float *mixed);

/* Decode path, one token (exec.rs:1540-1623 with the S5 router at exec.rs:1003-1011).
 * rlog: [E] logits or NULL (then computed with dot + optional bias into rlog_out).
 * ids/w: [32]; returns k_used (or -1 on error: untouched expert weights missing). */
int orc_moe_block(const orc_moe_w *W, const float *x, const float *rlog, int k,
                  const orc_policy *policy, int hiprec, float *out, float *rlog_out,
                  uint32_t *ids, float *w, orc_moe_stats *stats);

/* Batch path (exec_batch.rs:1404-1580, router exec_batch.rs:989-1019).  x [M][H] -> out [M][H].
 * router_dot_max_m: rows M < this use per-row dot, else gemm_f32_nt (the reference switches at
 * its tile's core count).  Dispatch outputs (ent_*, grp_*) are returned for bit-exact checks;
 * their capacities: ent_* >= M*32, grp_* >= E+1.  Returns n_ent, or -1 on error. */
int orc_moe_batch(const orc_moe_w *W, const float *x, const float *rlog, int M, int k,
                  const orc_policy *policy, int router_dot_max_m, float *out, float *rlog_out,
                  uint32_t *ids, float *w, uint32_t *n_sel, uint32_t *ent_tok, float *ent_w,
                  uint32_t *ent_expert, uint32_t *grp_start, uint32_t *grp_expert,
                  uint32_t *grp_order, uint32_t *n_groups, orc_moe_stats *stats);

/* ---- deterministic synthetic data (shared bit-for-bit with the GPU generator) ------------ */
uint64_t orc_rng_u64(uint64_t seed, uint64_t stream, uint64_t idx);
/* Q4_K / Q6_K superblocks of a [rows][K] matrix: d, dmin ~ U(dlo, dhi) as f16, other bytes
 * uniform random.  out must hold rows*row_bytes. */
void orc_gen_gguf(int fmt, uint64_t seed, uint64_t stream, int rows, int K, float dlo, float dhi,
                  uint8_t *out);
/* n normals N(0, sigma) (Box-Muller in f64, rounded to f32). */
void orc_gen_normal(uint64_t seed, uint64_t stream, size_t n, double sigma, float *out);
void orc_gen_uniform(uint64_t seed, uint64_t stream, size_t n, float lo, float hi, float *out);

#ifdef __cplusplus
}
#endif
#endif
