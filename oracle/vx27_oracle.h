/*
 * vx27 oracle: a CPU restatement of the reference token-mixer math.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  It is used by tests/ (as the parity checker), by
 * __graft_entry__.smoke() (as the checker of the smoke run) and by bench.py's
 * cpu_baseline leg (as the timed CPU path).  Each function follows the
 * reference operation for operation, including its float/double casts and
 * evaluation order, so that it reproduces the reference bit-for-bit on the
 * same machine; the citation on each declaration names the reference code it
 * restates.  Build with -std=c11 -ffp-contract=off (no FMA contraction),
 * exactly as the reference's own -std=c11 build evaluates.
 *
 * Pinning status (how each function is checked, in tests/test_oracle.py):
 *   orc_gate_params, orc_l2norm, orc_step_exact, orc_conv1d_step,
 *   orc_update_simple / orc_retrieve_simple, orc_rmsnorm_w, orc_attn_1q,
 *   orc_rope_cos_sin, orc_rope_apply                -> golden vectors minted
 *     from the compiled reference (oracle/_ref) + the reference's own
 *     known-answer checks + closed forms.
 *   orc_dn_layer_token, orc_gqa_layer_token (the vx27_qlayer glue)
 *     -> golden vectors minted from the compiled reference vx27_qlayer with
 *        synthetic F32 weights and a zero FFN.
 *   orc_attend (bf16 KV, long context, batches) -> orc_gqa_token (pinned
 *     above) + closed forms (one key -> its value, identical keys -> mean).
 *   orc_dn_run (multi-token, batched; the DeltaNet prefill oracle) and
 *   orc_gqa_prefill (token-ordered GQA prefill) -> bit-exact against chains
 *     of the pinned per-token functions.
 *   orc_update_avx2_pub / orc_retrieve_avx2_pub -> bit-exact against the
 *     compiled reference's AVX2 outputs (simple_update fixture);
 *     orc_dn_run_avx2 (a CPU timing baseline, not a checker) -> equal to a
 *     chain of those two on one head.
 */
#ifndef VX27_ORACLE_H
#define VX27_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 helpers: round-to-nearest-even narrowing, exact widening. */
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float *x, uint16_t *y, size_t n);
void orc_bf16_to_f32_n(const uint16_t *x, float *y, size_t n);

/* --- DeltaNet (src/vx27_deltanet.c) --- */
/* vx27_deltanet_state_per_layer / _total / _mb (vx27_deltanet.c:5-13) */
int orc_state_per_layer(void);
int orc_state_total(void);
double orc_state_mb(int bytes_per_elem);
/* vx27_deltanet_update_ref / retrieve_ref (vx27_deltanet.c:15-25) */
void orc_update_simple(float *S, const float *k, const float *v, float decay, int hd);
void orc_retrieve_simple(const float *S, const float *q, float *o, int hd);
/* vx27_deltanet_l2norm (vx27_deltanet.c:51-56) */
void orc_l2norm(const float *x, float *y, int n);
/* vx27_deltanet_gate_params + softplus (vx27_deltanet.c:58-69) */
void orc_gate_params(double a, double A_log, double b, double dt_bias,
                     double *beta, double *g_log);
/* vx27_deltanet_step_exact (vx27_deltanet.c:71-102) */
void orc_step_exact(float *S, const float *q, const float *k, const float *v,
                    double beta, double g_log, float *o, int hd);
/* vx27_conv1d_step + silu (vx27_deltanet.c:104-122) */
void orc_conv1d_step(float *state, const float *x, const float *w, float *y,
                     int C, int apply_silu);

/* --- GQA / norms (src/vx27_gqa.c, src/vx27_qfwd.c:32-48) --- */
int orc_kv_for_q(int q_head);                                   /* vx27_gqa.c:6-8 */
void orc_rmsnorm_w(const float *x, const float *w, float *y, int n, float eps); /* vx27_gqa.c:10-15 */
void orc_rmsn_1pw(const float *x, const float *w, float *y, int n);  /* rmsn, vx27_qfwd.c:32-39 */
void orc_rmsn_std(const float *x, const float *w, float *y, int n);  /* rmsn_std, vx27_qfwd.c:42-47 */
float orc_silu(float v);                                         /* silu1, vx27_qfwd.c:48 */
/* vx27_attn_1q (vx27_gqa.c:17-45) without the 1024-position cap. */
void orc_attn_1q(const float *q, const float *kcache, const float *vcache,
                 int n_pos, float *out);

/* Generic single-query attention for one sequence, the inline loop of
 * vx27_qlayer (vx27_qfwd.c:186-209): per Q head h (KV head h*n_kv/n_q),
 * scores over keys 0..n_keys-1, two-pass float softmax, float P.V.
 *   dot_double = 1: score = (float)(sum_i (double)q*k * scale)  (vx27_qfwd.c:196-197)
 *   dot_double = 0: score = (float sum_i q*k) * scale           (vx27_gqa.c:30-32)
 * K/V element (pos p, kv head h, dim i) is read at base + p*pos_stride +
 * h*head_stride + i; kv_bf16 selects uint16 bf16 storage instead of float. */
typedef struct {
    int n_q, n_kv, hd, n_keys, dot_double, kv_bf16;
    const float *q;          /* [n_q][hd] */
    const void *k, *v;
    size_t k_pos_stride, k_head_stride, v_pos_stride, v_head_stride;
    float *out;              /* [n_q][hd] */
} orc_attend_args;
void orc_attend(const orc_attend_args *a);
/* One Q head h of orc_attend; sc is scratch of n_keys floats. */
void orc_attend_one(const orc_attend_args *a, int h, float *sc);

/* --- RoPE (src/vx27_rope.c) --- */
void orc_rope_cos_sin(int pos, float *cosv, float *sinv, int rope_dim,
                      float theta, float yarn_factor);           /* vx27_rope.c:5-16 */
void orc_rope_apply(float *v, int n_heads, int head_dim, int rope_dim,
                    const float *cosv, const float *sinv);       /* vx27_rope.c:18-29 */
void orc_mrope_cos_sin_text(int pos, float *cosv, float *sinv);  /* vx27_rope.c:31-33 */

/* --- Projection: the F32 matvec of vx27_pmat (vx27_pmat.c:98-101, 119-125):
 * y[r] = (float) sum_c (double)W[r][c] * (double)x[c], serial in c.
 * w_bf16 = 1 reads W as bf16 widened exactly. --- */
void orc_matvec(const void *W, int w_bf16, const float *x, float *y, int rows, int cols);

/* --- DeltaNet mixer glue for one token of one sequence (vx27_qfwd.c:92-155)
 * flags select which stages run, so the same restatement covers the
 * step_exact-only configs and the full vx27_qlayer branch:
 *   ORC_DN_CONV      causal conv + SiLU over the q|k|v channels (:110-116)
 *   ORC_DN_PRE_RMS   rmsn(1+w) with norm_w before the l2norm (:119-126)
 *   ORC_DN_PRE_L2    l2norm q,k + q *= 1/sqrt(hd) before step_exact (:124-130)
 *   ORC_DN_OUT_GATE  out = rmsn_std(ret, norm_w) * silu(z) (:144-151)
 * Inputs: qkv [2*nqk*hd + nv*hd] (projection output, conv input), a,b [nv],
 * A_log, dt_bias [nv], norm_w [hd], z [nv*hd]; state S [nv][hd][hd],
 * conv_state [C][3], conv_w [C][4] (float).  Output [nv*hd]. */
enum { ORC_DN_CONV = 1, ORC_DN_PRE_RMS = 2, ORC_DN_PRE_L2 = 4, ORC_DN_OUT_GATE = 8 };
typedef struct {
    int nqk, nv, hd, flags;
    const float *A_log, *dt_bias, *norm_w, *conv_w;
} orc_dn_cfg;
void orc_dn_token(const orc_dn_cfg *c, const float *qkv, const float *a, const float *b,
                  const float *z, float *S, float *conv_state, float *out);

/* --- GQA mixer glue for one token of one sequence (vx27_qfwd.c:156-211):
 * qg [n_q][2*hd] interleaved (q | gate) or q/gate separate (gate != NULL);
 * k1, v1 [n_kv][hd] raw projections; rmsn(1+w) on q and k; RoPE with the
 * given table; append k,v at position pos of the caller's cache (layout by
 * strides, float or bf16 storage); attend over 0..pos (double dot);
 * out [n_q][hd] = attention * sigmoid(gate), or attention alone with no_gate
 * (the MTP drafter's use_gate = 0, vx27_mtp.c:258). */
typedef struct {
    int n_q, n_kv, hd, rope_dim, kv_bf16;
    const float *q_norm_w, *k_norm_w;      /* [hd] each, (1+w) form */
    void *k_cache, *v_cache;
    size_t k_pos_stride, k_head_stride, v_pos_stride, v_head_stride;
    int no_gate;
} orc_gqa_cfg;
void orc_gqa_token(const orc_gqa_cfg *c, const float *q_raw, size_t q_head_stride,
                   const float *gate, size_t gate_head_stride,
                   const float *k1, const float *v1, int pos,
                   const float *cosv, const float *sinv, float *out);

/* Whole reference layer minus the FFN, for pinning against vx27_qlayer with a
 * zero FFN: out = x + mixer(rmsn(x, ln_w)).  Weights are float [rows][cols].
 * DeltaNet: nqk=16, nv=48, hd=128 fixed as vx27_qfwd.c:97. */
typedef struct {
    const float *ln_w;                     /* [5120] input_layernorm */
    const float *w_qkv, *w_z, *w_a, *w_b;  /* [10240|6144|48|48][5120] */
    const float *conv_w;                   /* [10240][4] */
    const float *A_log, *dt_bias, *norm_w; /* [48],[48],[128] */
    const float *w_out;                    /* [5120][6144] */
} orc_dn_layer_w;
void orc_dn_layer_token(const orc_dn_layer_w *w, const float *x, float *S, float *conv,
                        float *out);
typedef struct {
    const float *ln_w;                     /* [5120] */
    const float *w_q, *w_k, *w_v;          /* [12288|1024|1024][5120] */
    const float *q_norm_w, *k_norm_w;      /* [256] */
    const float *w_o;                      /* [5120][6144] */
} orc_gqa_layer_w;
/* kcache/vcache float [T][4*256] (one slot of vx27_qfwd's cache). */
void orc_gqa_layer_token(const orc_gqa_layer_w *w, const float *x, int n_pos,
                         float *kcache, float *vcache, float *out);

/* --- CPU baseline drivers (POSIX thread pool, parallel over independent
 * (sequence, head) units).  Return wall seconds. --- */
/* B sequences x nv heads x steps of step_exact on per-step q,k,v,a,b
 * (layouts [steps][B][nqk|nv][hd], [steps][B][nv]); with conv when
 * conv_w != NULL (x [steps][B][C]).  Mirrors the decode descriptor. */
typedef struct {
    int B, nqk, nv, hd, steps, flags, threads;
    float *S;               /* [B][nv][hd][hd] */
    float *conv_state;      /* [B][C][3] or NULL */
    const float *conv_w;    /* [C][4] or NULL */
    const float *x;         /* conv input [steps][B][C] (flags & ORC_DN_CONV) */
    const float *q, *k, *v; /* direct inputs when no conv */
    const float *a, *b, *A_log, *dt_bias, *norm_w, *z;
    float *out;             /* [steps][B][nv][hd] */
} orc_dn_run_args;
double orc_dn_run(const orc_dn_run_args *r);

/* The reference AVX2 primitives vx27_deltanet_update_avx2 /
 * retrieve_avx2 (vx27_deltanet_avx2.c:6-45), restated: row r of S becomes
 * fma(S, decay, k[r]*v); o accumulates fma(S_row, q[r], o) over rows. */
void orc_update_avx2_pub(float *S, const float *k, const float *v, float decay, int hd);
void orc_retrieve_avx2_pub(const float *S, const float *q, float *o, int hd);
typedef void (*orc_update_fn)(float *S, const float *k, const float *v, float decay, int hd);
typedef void (*orc_retrieve_fn)(const float *S, const float *q, float *o, int hd);

/* The AVX2 primitives composed into the gated delta rule
 * (decay*retrieve(S,k) -> d=beta(v-kv) -> update(S,k,d,decay) -> retrieve(S,q)),
 * q/k/v already normalised.  Float arithmetic, FMA, as vx27_deltanet_avx2.c.
 * upd/ret: the primitives to call -- the compiled reference's own
 * vx27_deltanet_update_avx2 / retrieve_avx2 when given, else the
 * restatement above. */
double orc_dn_run_avx2(int B, int nv, int hd, int steps, int threads, float *S,
                       const float *qn, const float *kn, const float *v,
                       const double *beta, const double *decay, float *out,
                       orc_update_fn upd, orc_retrieve_fn ret);

/* GQA decode for B sequences over caches with per-sequence key counts. */
typedef struct {
    int B, n_q, n_kv, hd, threads, kv_bf16, dot_double;
    const int *n_keys;      /* [B] */
    const float *q;         /* [B][n_q][hd], already normed + roped */
    const void *k, *v;      /* per sequence: base + b*seq_stride */
    size_t seq_stride, k_pos_stride, k_head_stride, v_pos_stride, v_head_stride;
    float *out;             /* [B][n_q][hd] */
} orc_attend_batch_args;
double orc_attend_batch(const orc_attend_batch_args *a);

/* GQA prefill of T tokens per sequence in the order of vx27_qlayer_batch
 * (vx27_qfwd.c:314-376): for each token, rmsn(1+w) on q and k, RoPE at
 * pos0+t (orc_rope_cos_sin), k,v appended to a float cache
 * [B][L][n_kv][hd] (rows < pos0 supplied by the caller), then the token's
 * attention over positions 0..pos0+t (double dot, float softmax) times
 * sigmoid(gate) (or not, with no_gate).  The attention units (b, t, h) run
 * in parallel. */
typedef struct {
    int B, T, n_q, n_kv, hd, rope_dim, pos0, L, threads;
    float rope_theta, rope_yarn;
    const float *q, *gate;          /* [B][T][n_q][hd] */
    const float *k, *v;             /* [B][T][n_kv][hd] raw */
    const float *q_norm_w, *k_norm_w;
    float *k_cache, *v_cache;       /* [B][L][n_kv][hd] */
    float *out;                     /* [B][T][n_q][hd] */
    int no_gate;
} orc_gqa_prefill_args;
double orc_gqa_prefill(const orc_gqa_prefill_args *a);

/* Row-parallel matvec for B vectors (W bf16 widened), double serial sums. */
double orc_matvec_batch(const void *W, int w_bf16, const float *x, float *y,
                        int rows, int cols, int B, int threads);

#ifdef __cplusplus
}
#endif
#endif
