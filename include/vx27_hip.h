/*
 * vx27_hip.h -- C ABI of the MI355X (gfx950) token-mixer library.
 *
 * The reference (DavidPandleton/vx27) runs its mixers on the host, inline in
 * vx27_qlayer (src/vx27_qfwd.c:92-215), through the void functions of
 * vx27_deltanet.h / vx27_gqa.h / vx27_rope.h.  This header is the thin C ABI
 * those callers use to run the same mixers on device-resident data:
 *   - a context (device + HIP stream) and device memory helpers,
 *   - DeltaNet recurrent decode (gate mapping, causal conv, delta rule,
 *     gated output norm), one or many tokens per call,
 *   - gated GQA decode over a bf16 KV cache (split-K flash decode),
 *   - RoPE tables and KV-cache format helpers.
 * The reference's own void API (include/vx27_deltanet.h etc.) is exported by
 * the same library and routes through these entry points.
 *
 * Conventions: every entry point returns 0 on success and -1 on failure;
 * the reason is in vx27_hip_last_error() (thread-local).  All pointers in
 * descriptors are device pointers unless stated.  Calls on one context are
 * serialised on its stream and are not thread-safe; distinct contexts are
 * independent.  Kernels are enqueued asynchronously: call vx27_hip_sync()
 * (or synchronise the stream) before reading results on the host.
 */
#ifndef VX27_HIP_H
#define VX27_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct vx27_hip_ctx vx27_hip_ctx;

/* ------------------------------------------------------------- context */
/* Open a context on `device` with its own stream.  Mirrors the reference's
 * init convention (int status + caller message buffer, vx27_gpu_reg.h:9). */
int vx27_hip_open(vx27_hip_ctx **ctx, int device, char *err, size_t errlen);
void vx27_hip_close(vx27_hip_ctx *ctx);
/* Waits for the context stream.  Also returns -1 if a call since the last
 * sync was given a device-side index outside its range: a GQA decode
 * position outside its KV cache (pos < 0 or pos >= L: the kernels clamp it
 * so no access leaves the cache) or a vx27_hip_dn_commit index past its
 * checkpoints (nothing is copied for it).  That call's outputs are
 * undefined. */
int vx27_hip_sync(vx27_hip_ctx *ctx);
/* Use a caller stream (hipStream_t) for subsequent calls; NULL restores the
 * context's own stream. */
int vx27_hip_set_stream(vx27_hip_ctx *ctx, void *hip_stream);
void *vx27_hip_get_stream(vx27_hip_ctx *ctx);
const char *vx27_hip_last_error(void);
int vx27_hip_device_count(void);
/* Library version string and the gfx target it was built for. */
const char *vx27_hip_version(void);

/* Kernel profiler: while enabled, the library records HIP events around
 * each of its kernel launches on the context stream; prof_read synchronises
 * and returns how many launches of `kernel` were recorded and their summed
 * duration; a template kernel's instances (name<...>) count under its
 * name.  Enabling (or disabling) clears the records. */
int vx27_hip_prof_enable(vx27_hip_ctx *ctx, int on);
int vx27_hip_prof_read(vx27_hip_ctx *ctx, const char *kernel, int *count, double *total_ms);

/* The context used by the reference-API drop-ins (opened on first use on
 * device VX27_HIP_DEVICE from the environment, default 0). */
vx27_hip_ctx *vx27_hip_default_ctx(void);

/* Route switch for callers that keep their own CPU path, mirroring
 * vx27_gpu_reg_on/off (vx27_gpu_reg.h:10-11): enable turns the route on only
 * if the default context opens (returns 0, else -1 with last_error set);
 * vx27_hip_enabled() is what the caller tests before taking the device path.
 * Off by default.  The library's own functions do not consult it. */
int vx27_hip_enable(void);
void vx27_hip_disable(void);
int vx27_hip_enabled(void);

/* Error behaviour of the void drop-ins, which cannot return a status:
 * VX27_HIP_ERR_ABORT (default) prints the error and aborts the process;
 * VX27_HIP_ERR_POISON fills the outputs with NaN, records the error and
 * returns.  There is no host fallback in either mode. */
#define VX27_HIP_ERR_ABORT 0
#define VX27_HIP_ERR_POISON 1
void vx27_hip_set_error_mode(int mode);

/* -------------------------------------------------------------- memory */
int vx27_hip_alloc(vx27_hip_ctx *ctx, void **dptr, size_t bytes);
int vx27_hip_free(vx27_hip_ctx *ctx, void *dptr);
int vx27_hip_h2d(vx27_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
int vx27_hip_d2h(vx27_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
int vx27_hip_d2d(vx27_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Fills `bytes` bytes at dst with `byte`, by a kernel on the context stream
 * (never hipMemsetAsync), so it may be captured into a graph. */
int vx27_hip_memset(vx27_hip_ctx *ctx, void *dst, int byte, size_t bytes);
/* Diagnostics with no counterpart in the reference: the context's scratch
 * size, how many device buffers it keeps retired for live graphs, how many
 * prefill attention schedules it caches and how many graphs captured on it
 * are alive.  Any output pointer may be NULL. */
int vx27_hip_mem_info(vx27_hip_ctx *ctx, size_t *scratch_bytes, int *retired_buffers, int *cached_schedules,
                      int *live_graphs);
/* HBM bandwidth probe, a measurement utility with no counterpart in the
 * reference: allocates `bytes` of device memory (at least 1 MiB; use far
 * more than the 256 MiB Infinity Cache), then `iters` times (after one
 * warm-up) streams it with a plain read kernel and copies its first half
 * into its second with a plain copy kernel, timed with events on the
 * context stream, and frees it.  Returns the best rates in GB/s, counting
 * `bytes` moved per kernel (the copy: bytes/2 read + bytes/2 written).  Not
 * allowed inside a graph capture. */
int vx27_hip_bw_probe(vx27_hip_ctx *ctx, size_t bytes, int iters, double *read_GBs, double *copy_GBs);

/* dtype codes */
#define VX27_F32 0
#define VX27_BF16 1

/* ------------------------------------------------------ DeltaNet decode */
/* Stages of the reference DeltaNet branch (vx27_qfwd.c:92-155) applied
 * around the exact gated delta rule (vx27_deltanet_step_exact,
 * vx27_deltanet.c:71-102, which always l2-normalises q,k and scales q):
 *   VX27_DN_CONV     causal conv width 4 + SiLU on the q|k|v channels, with
 *                    the conv state carried in place (vx27_deltanet.c:106-122)
 *   VX27_DN_PRE_RMS  rmsn(x)*(1+norm_w) on each q,k head (vx27_qfwd.c:123)
 *   VX27_DN_PRE_L2   l2norm q,k and q *= 1/sqrt(hd) (vx27_qfwd.c:124-130)
 *   VX27_DN_OUT_GATE out = rmsn_std(o)*norm_w * silu(z) (vx27_qfwd.c:147-151)
 * No flags = step_exact on the given q,k,v (the recurrence alone). */
#define VX27_DN_CONV 1u
#define VX27_DN_PRE_RMS 2u
#define VX27_DN_PRE_L2 4u
#define VX27_DN_OUT_GATE 8u

typedef struct {
    int B;          /* independent sequences */
    int nqk, nv;    /* QK heads and value heads; value head vh uses QK head vh*nqk/nv
                       (vx27_qfwd.c:137); nv must be a multiple of nqk */
    int hd;         /* head dim: 128 */
    int steps;      /* tokens per sequence in this call (>= 1), run in order */
    unsigned flags; /* VX27_DN_* */
    float *S;       /* [B][nv][hd][hd] fp32 state, row = key dim, column = value dim; in/out */
    float *conv_state;  /* [B][C][3] fp32, oldest first (VX27_DN_CONV); in/out */
    const void *conv_w; /* [C][4] weights, tap 3 = newest, 16-byte aligned (VX27_DN_CONV) */
    int conv_w_dtype;   /* VX27_F32 or VX27_BF16 */
    /* Per-token inputs, fp32, token t of sequence b at [t][b]:
     *   VX27_DN_CONV:  x [steps][B][C], C = 2*nqk*hd + nv*hd, channels q|k|v
     *   otherwise:     q,k [steps][B][nqk][hd], v [steps][B][nv][hd] */
    const float *x, *q, *k, *v;
    const float *a, *b;          /* [steps][B][nv] gate projections */
    const float *A_log, *dt_bias;/* [nv] */
    const float *norm_w;         /* [hd] (PRE_RMS uses 1+w, OUT_GATE uses w) */
    const float *z;              /* [steps][B][nv][hd] (OUT_GATE) */
    float *out;                  /* [steps][B][nv][hd] */
} vx27_dn_desc;

/* Run `steps` tokens of the DeltaNet mixer core for B sequences.  The state
 * stays in registers across the steps of one call, so multi-step calls read
 * and write S once per call. */
int vx27_hip_dn_decode(vx27_hip_ctx *ctx, const vx27_dn_desc *d);

/* DeltaNet prefill: T tokens of each of B sequences, in order, as
 * vx27_qlayer_batch runs the DeltaNet branch token by token
 * (vx27_qfwd.c:276-308): optional conv with carried state, optional
 * rmsn(1+w) + l2norm pre-norm, step_exact (vx27_deltanet.c:71-102, which
 * l2-normalises q,k and scales q again), optional gated output norm, and
 * optional per-token state checkpoints (Sckpt/Cckpt, vx27_qfwd.c:306-307).
 * The flags are the decode's (VX27_DN_CONV, _PRE_RMS, _PRE_L2, _OUT_GATE).
 *
 * Two algorithms:
 *   chunked (default): the chunked WY form over chunks of 64 tokens, the
 *     fp32 state carried between chunks, the chunk products on bf16 MFMA
 *     with every operand split into a bf16 pair hi + lo (hi*hi + lo*hi +
 *     hi*lo: ~16 significand bits per operand, results within ~1e-5
 *     relative of the fp32 recurrence); the glue stages run in fp32 and
 *     hand q, k, v over as such pairs.  VX27_DN_BF16 uses single bf16
 *     operands instead (about 2x faster, bf16 accuracy).
 *   exact (VX27_DN_EXACT, or whenever a checkpoint is asked for): the
 *     decode kernels' fp32 recurrence token by token, the reference's own
 *     arithmetic (bit-identical to vx27_hip_dn_decode called token by
 *     token when checkpoints are written).  Meant for short windows such as
 *     an MTP verify batch (the reference's batch is at most 8 tokens).
 * Inputs are [B][T][...] (token t of sequence b at row b*T + t). */
#define VX27_DN_EXACT 16u
#define VX27_DN_BF16 32u

typedef struct {
    int B, T;
    int nqk, nv;    /* value head vh uses QK head vh*nqk/nv; nv a multiple of nqk */
    int hd;         /* 128 */
    unsigned flags; /* VX27_DN_CONV | _PRE_RMS | _PRE_L2 | _OUT_GATE | _EXACT | _BF16 */
    float *S;       /* [B][nv][hd][hd] fp32: initial state in, final state out */
    /* without VX27_DN_CONV: bf16 q,k [B][T][nqk][hd], v [B][T][nv][hd] */
    const uint16_t *q, *k;
    const uint16_t *v;
    const float *a, *b;          /* [B][T][nv] gate projections */
    const float *A_log, *dt_bias;/* [nv] */
    float *out;                  /* [B][T][nv][hd] */
    /* VX27_DN_CONV: fp32 projection output x [B][T][C], C = 2*nqk*hd + nv*hd,
     * channels q|k|v; the conv state [B][C][3] (oldest first) is read and
     * left as after token T-1; conv_w [C][4] as in vx27_dn_desc */
    const float *x;
    float *conv_state;
    const void *conv_w;
    int conv_w_dtype;
    const float *norm_w;         /* [hd] (PRE_RMS uses 1+w, OUT_GATE uses w) */
    const float *z;              /* [B][T][nv][hd] (OUT_GATE; then z, norm_w and out 16-byte aligned) */
    /* optional checkpoints (either selects the exact algorithm):
     * S_ckpt [B][T][nv][hd][hd] the state after each token,
     * conv_ckpt [B][T][C][3] the conv state after each token (VX27_DN_CONV) */
    float *S_ckpt;
    float *conv_ckpt;
} vx27_dn_prefill_desc;
int vx27_hip_dn_prefill(vx27_hip_ctx *ctx, const vx27_dn_prefill_desc *d);

/* Make checkpoint m[b] of sequence b its live state (the device form of
 * vx27_engine_commit_ckpt, vx27_run.c:250-255: a partial commit after a
 * verify batch, the drafts past m rejected).  S [B][nv][hd][hd] and
 * conv_state [B][C][3] take S_ckpt[b][m[b]] and conv_ckpt[b][m[b]] (layouts
 * of vx27_dn_prefill_desc, T checkpoints per sequence); m is a device int
 * array [B]; m[b] < 0 leaves sequence b unchanged, m[b] >= T is an error
 * flagged like a position outside the cache (reported by vx27_hip_sync).
 * Either checkpoint array may be NULL (its state is then not touched). */
int vx27_hip_dn_commit(vx27_hip_ctx *ctx, int B, int T, int nv, int hd, int C, const int *m,
                       const float *S_ckpt, const float *conv_ckpt, float *S, float *conv_state);

/* ---------------------------------------------------------- GQA decode */
/* KV cache format (bf16), for B sequences x n_kv heads x L positions, hd 256:
 *   K: [B][n_kv][L][hd]            one row per position
 *   V: [B][n_kv][L/32][hd][32]     32-position blocks stored dim-major
 * L (the capacity) must be a multiple of 64.  Use vx27_hip_kv_write /
 * vx27_hip_kv_read to move rows in or out of this layout. */
#define VX27_GQA_NORM_W 1u  /* q/k norm as x*s*w (vx27_gqa.c:10-15) instead of x*s*(1+w) */
#define VX27_GQA_NO_GATE 2u /* no output gate: out = attention (the MTP drafter's use_gate = 0,
                               vx27_mtp.c:258); gate may be NULL */

typedef struct {
    int B;
    int n_q, n_kv, hd;       /* 24, 4, 256 (hd must be 256, n_q/n_kv <= 16) */
    int rope_dim;            /* rotated leading dims per head (NeoX half split), 64 */
    float rope_theta;        /* 1e7 */
    float rope_yarn;         /* linear position scale, >= 1 */
    int L;                   /* cache capacity (positions), multiple of 64 */
    unsigned flags;          /* VX27_GQA_* */
    const int *pos;          /* [B] device: position of the new token; keys 0..pos attended */
    /* raw q (before norm/rope), element (b, h, i) at q[b*q_seq_stride + h*q_head_stride + i];
     * the interleaved q_proj output of vx27_qfwd.c:160-167 is q_head_stride = 2*hd and
     * gate = q + hd with the same strides. */
    const float *q;
    size_t q_seq_stride, q_head_stride;
    const float *gate;       /* gate logits, same addressing with its own strides */
    size_t gate_seq_stride, gate_head_stride;
    const float *k_new, *v_new;  /* [B][n_kv][hd] raw k (before norm/rope) and v
                                    (sequence stride kv_seq_stride) */
    const float *q_norm_w, *k_norm_w;  /* [hd] */
    uint16_t *k_cache, *v_cache;       /* bf16, format above; row pos is written */
    float *out;              /* [B][n_q][hd]: attention * sigmoid(gate) (attention alone with VX27_GQA_NO_GATE) */
    int n_split;             /* key splits per (sequence, KV head); 0 = automatic */
    size_t kv_seq_stride;    /* per-sequence stride of k_new / v_new in floats; 0 = n_kv*hd */
} vx27_gqa_desc;

/* One decode step of the gated GQA mixer core (vx27_qfwd.c:172-211):
 * rmsn q,k -> RoPE at pos -> append k,v (bf16) at pos -> softmax attention
 * over positions 0..pos -> * sigmoid(gate). */
int vx27_hip_gqa_decode(vx27_hip_ctx *ctx, const vx27_gqa_desc *d);

/* The same decode step without any allocation in the call.  No counterpart
 * in the reference: it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Its
 * scratch (normed q and the split-K partials) is a static 16 MiB device
 * array, one per GPU, set up by vx27_hip_open and held until the process
 * ends; a call needing more (B * n_kv * n_split * (n_q/n_kv) partials of
 * 258 floats plus B * n_q * 256 floats) returns -1 with the size.  Every
 * call on one GPU shares that array and leaves its contents there: calls
 * that overlap on one GPU (two streams or two contexts) race.  Results are
 * bit-identical to vx27_hip_gqa_decode's.  The profiler does not record it. */
int vx27_hip_gqa_decode_noalloc(vx27_hip_ctx *ctx, const vx27_gqa_desc *d);

/* GQA prefill: T new tokens of each of B sequences at positions pos0..pos0+T-1
 * (token by token as vx27_qlayer_batch runs the decode glue,
 * vx27_qfwd.c:314-376): rmsn q,k -> RoPE -> k,v written to the cache (bf16,
 * format above) -> causal attention of each token over positions 0..its own
 * (earlier cache rows included) -> * sigmoid(gate).  bf16 MFMA products,
 * fp32 softmax.
 * Requirements (checked; -1 with a message otherwise): hd == 256; rope_dim a
 * multiple of 64, at most 128; q 16-byte aligned with q strides multiples of
 * 8 elements; gate 8-byte aligned with gate strides multiples of 4 elements;
 * k_new 8-byte aligned; v_new, q_norm_w, out, k_cache and v_cache 16-byte
 * aligned.  Buffers from hipMalloc and the
 * interleaved q_proj layout (gate = q + 256) meet all of them. */
typedef struct {
    int B, T;
    int n_q, n_kv, hd;       /* 24, 4, 256 */
    int rope_dim;            /* 64 (0 = no rotation) */
    float rope_theta, rope_yarn;
    int L;                   /* cache capacity, multiple of 64; pos0 + T <= L */
    int pos0;                /* position of token 0 (same for every sequence) */
    unsigned flags;          /* VX27_GQA_NORM_W, VX27_GQA_NO_GATE */
    /* bf16 raw q and gate logits: element (b, t, h, i) at
     * q[(b*T + t)*q_tok_stride + h*q_head_stride + i]; 0 strides = dense
     * [B][T][n_q][hd].  Interleaved q_proj output: head stride 2*hd, gate = q + hd. */
    const uint16_t *q;
    size_t q_tok_stride, q_head_stride;
    const uint16_t *gate;
    size_t gate_tok_stride, gate_head_stride;
    const uint16_t *k_new, *v_new;   /* bf16 [B][T][n_kv][hd] raw k and v */
    const float *q_norm_w, *k_norm_w;/* [hd] */
    uint16_t *k_cache, *v_cache;
    float *out;                      /* [B][T][n_q][hd] */
} vx27_gqa_prefill_desc;
int vx27_hip_gqa_prefill(vx27_hip_ctx *ctx, const vx27_gqa_prefill_desc *d);

/* Copy n rows of fp32 [n][n_kv][hd] K and V (positions p0..p0+n-1 of
 * sequence b) into / out of the cache format, rounding to bf16 on write. */
int vx27_hip_kv_write(vx27_hip_ctx *ctx, uint16_t *k_cache, uint16_t *v_cache, int B_total,
                      int n_kv, int hd, int L, int b, int p0, int n,
                      const float *k_rows, const float *v_rows);
int vx27_hip_kv_read(vx27_hip_ctx *ctx, const uint16_t *k_cache, const uint16_t *v_cache,
                     int B_total, int n_kv, int hd, int L, int b, int p0, int n,
                     float *k_rows, float *v_rows);

/* RoPE cos/sin tables on the device for n positions (device int array):
 * cos/sin [n][rope_dim/2].  The frequency table powf(theta, -2i/rope_dim) is
 * evaluated on the host exactly as vx27_rope.c:11; the angle is the same
 * float product; cos/sin are the device's float functions. */
int vx27_hip_rope_table(vx27_hip_ctx *ctx, const int *pos, int n, int rope_dim,
                        float theta, float yarn, float *cosv, float *sinv);

/* ------------------------------------------------ projections and layers */
/* y[b*y_stride + n] = sum_k W[n][k] * x[b*x_stride + k] for B >= 1 vectors:
 * W bf16 row-major [N][K] (N % 16 == 0, K % 32 == 0), x and y fp32.  The
 * F32 matvec of the reference (vx27_pmat.c:98-101, 119-125) on bf16 weights;
 * x enters the MFMA exactly (split into three bf16 parts), fp32 accumulation.
 * W is read once per 65 vectors. */
int vx27_hip_gemv_bf16(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x,
                       size_t x_stride, int B, float *y, size_t y_stride);

/* The same product for many tokens at once (a prompt's projections): y[r*y_stride + n] =
 * sum_k W[n][k] * x[r*x_stride + k] for R >= 1 rows, W tiled (vx27_hip_pack_weights_bf16,
 * N % 16 == 0, K % 64 == 0), x and y fp32 with 16-byte aligned rows (strides % 4 == 0).
 * A bf16 MFMA GEMM (tiles of 256 tokens x 256 rows, W read once per 256 tokens); each x
 * enters as two bf16 parts hi + lo (16 significand bits: relative error about 2^-17 per
 * product), fp32 accumulation.  Context scratch holds x packed for the MFMAs (R*K*4 bytes,
 * R rounded up to 256).  No counterpart in the reference, whose batched matvec
 * (vx27_pmat.c:212-227) serves at most 8 tokens; the layer prefill entry points use it from
 * 256 tokens on. */
int vx27_hip_gemm_bf16(vx27_hip_ctx *ctx, const uint16_t *W_tiled, int N, int K, const float *x,
                       size_t x_stride, int R, float *y, size_t y_stride);

/* Weight tiling for the layer entry points: row-major bf16 W [N][K] into the
 * MFMA tile layout [K/32][N/16][64 lanes][8]: lane (g,m) of tile (k-step s,
 * row block rb) holds W[16rb + m][32s + 8g .. 8g+7].  Each wave loads 1 KiB
 * of contiguous weights per tile and the row blocks of one k-step are
 * adjacent, so a launch streams long contiguous runs.  (A build option,
 * VX_GEMV_KG = 2 or 4, groups that many k-steps of a row block together.)
 * Done once per weight, like the reference's offline forge of its packed
 * weight format (src/vx_forge.c). */
int vx27_hip_pack_weights_bf16(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, uint16_t *W_tiled);

/* The mixer of one Gated DeltaNet layer for one decode token of B
 * sequences (any B; the projections stream their weights once per 65
 * sequences), from the layer input xn to the out_proj output (the DeltaNet
 * branch of vx27_qlayer, vx27_qfwd.c:102-153):
 *   [qkv | z | a | b] = W_in xn      (in_proj_qkv, in_proj_z, in_proj_a, in_proj_b
 *                                      stacked row-wise: C + nv*hd + 2*nv rows)
 *   causal conv + SiLU on qkv (state in place), gates from a, b,
 *   rmsn(1+w) + l2norm on q,k, exact delta rule per value head,
 *   rmsn_std(o)*w * silu(z), out = W_out o.
 * hd = 128, C = 2*nqk*hd + nv*hd. */
typedef struct {
    int B, nqk, nv, hd, hidden;
    const float *x;             /* [B][hidden] layer input (after input_layernorm) */
    const uint16_t *x_packed;   /* optional: x already packed by vx27_hip_pack_x (or NULL) */
    const uint16_t *w_in;       /* bf16 [C + nv*hd + 2*nv][hidden], tiled (vx27_hip_pack_weights_bf16) */
    const uint16_t *w_out;      /* bf16 [hidden][nv*hd], tiled */
    const void *conv_w;         /* [C][4], 16-byte aligned */
    int conv_w_dtype;           /* VX27_F32 or VX27_BF16 */
    const float *A_log, *dt_bias, *norm_w;  /* [nv], [nv], [hd] */
    float *S;                   /* [B][nv][hd][hd] in/out */
    float *conv_state;          /* [B][C][3] in/out */
    float *out;                 /* [B][hidden] */
} vx27_dn_layer_desc;
int vx27_hip_dn_layer_decode(vx27_hip_ctx *ctx, const vx27_dn_layer_desc *d);

/* The mixer of one gated GQA layer for one decode token of B sequences
 * (any B; weights streamed once per 65 sequences)
 * (the attention branch of vx27_qlayer, vx27_qfwd.c:162-213):
 *   [q|gate interleaved per head | k | v] = W_qkv xn  (q_proj, k_proj, v_proj
 *                                      stacked: n_q*2*hd + 2*n_kv*hd rows),
 *   vx27_hip_gqa_decode on them, out = W_o att. */
typedef struct {
    int B, n_q, n_kv, hd, hidden, rope_dim;
    float rope_theta, rope_yarn;
    int L;                      /* KV cache capacity */
    const float *x;             /* [B][hidden] */
    const uint16_t *x_packed;   /* optional pre-packed x (or NULL) */
    const uint16_t *w_qkv;      /* bf16 [n_q*2*hd + 2*n_kv*hd][hidden], tiled */
    const uint16_t *w_o;        /* bf16 [hidden][n_q*hd], tiled */
    const float *q_norm_w, *k_norm_w;
    const int *pos;             /* [B] device */
    uint16_t *k_cache, *v_cache;
    float *out;                 /* [B][hidden] */
    int n_split;                /* 0 = automatic */
} vx27_gqa_layer_desc;
int vx27_hip_gqa_layer_decode(vx27_hip_ctx *ctx, const vx27_gqa_layer_desc *d);

/* The DeltaNet layer for T tokens of each of B sequences, in order: the
 * device form of vx27_qlayer_batch's DeltaNet branch (vx27_qfwd.c:249-313)
 * as vx27_engine_batch_step runs it per layer (vx27_run.c:187-238):
 * [qkv|z|a|b] = W_in x for every token, then vx27_hip_dn_prefill with every
 * glue stage (and the checkpoints, when given), then out = W_out o.  The
 * projections stream their weights once per 65 tokens, so this is for short
 * windows such as an MTP verify batch (the reference's batch is at most 8
 * tokens); a long prompt's projections belong in a GEMM.  x and out are
 * [B][T][hidden]; the other fields as vx27_dn_layer_desc; flags
 * VX27_DN_EXACT / VX27_DN_BF16 choose the prefill algorithm (checkpoints
 * imply the exact one, bit-identical to T vx27_hip_dn_layer_decode calls). */
typedef struct {
    int B, T, nqk, nv, hd, hidden;
    unsigned flags;
    const float *x;
    const uint16_t *w_in, *w_out;   /* tiled */
    const void *conv_w;             /* 16-byte aligned */
    int conv_w_dtype;
    const float *A_log, *dt_bias, *norm_w;  /* norm_w 16-byte aligned */
    float *S, *conv_state;
    float *out;
    float *S_ckpt, *conv_ckpt;      /* optional: [B][T][nv][hd][hd], [B][T][C][3] */
} vx27_dn_layer_prefill_desc;
int vx27_hip_dn_layer_prefill(vx27_hip_ctx *ctx, const vx27_dn_layer_prefill_desc *d);

/* The gated GQA layer for T tokens of each of B sequences at positions
 * pos0 .. pos0+T-1 (vx27_qlayer_batch's attention branch,
 * vx27_qfwd.c:314-376): [q|gate|k|v] = W_qkv x for every token, rounded to
 * bf16, vx27_hip_gqa_prefill (cache rows written, causal attention, gate),
 * out = W_o att.  Same window note as vx27_hip_dn_layer_prefill; flags as
 * vx27_gqa_prefill_desc. */
typedef struct {
    int B, T, n_q, n_kv, hd, hidden, rope_dim;
    float rope_theta, rope_yarn;
    int L, pos0;
    unsigned flags;
    const float *x;                 /* [B][T][hidden] */
    const uint16_t *w_qkv, *w_o;    /* tiled */
    const float *q_norm_w, *k_norm_w;
    uint16_t *k_cache, *v_cache;
    float *out;                     /* [B][T][hidden] */
} vx27_gqa_layer_prefill_desc;
int vx27_hip_gqa_layer_prefill(vx27_hip_ctx *ctx, const vx27_gqa_layer_prefill_desc *d);

/* Pack x [B][K] once for several layers that read the same input
 * (x_packed of the layer descriptors); packed holds vx27_hip_pack_bytes(K, B). */
size_t vx27_hip_pack_bytes(int K, int B);
int vx27_hip_pack_x(vx27_hip_ctx *ctx, const float *x, int B, int K, uint16_t *packed);

/* pos[b] += 1 for b < B (advances decode positions inside a captured graph) */
int vx27_hip_advance_pos(vx27_hip_ctx *ctx, int *pos, int B);

/* --------------------------------------------------------- HIP graphs
 * Capture the calls made on ctx between graph_begin and graph_end into an
 * executable graph; graph_launch replays it on the context stream.
 *   - A call that needs more context scratch than the context holds fails
 *     inside a capture (-1): run the same call once before capturing.
 *   - A captured graph keeps the addresses of the scratch buffer and the
 *     prefill schedules it was captured with.  While any graph captured on
 *     a context is alive, the context frees none of them: a later call that
 *     grows the scratch, or a prefill of a new shape, leaves the graph's
 *     memory in place until graph_destroy of the last live graph (or
 *     vx27_hip_close).  So eager calls of any size may run between replays.
 *   - The graph and the eager calls share that scratch: replays and eager
 *     calls must be ordered on one stream (the context's), never overlapped. */
int vx27_hip_graph_begin(vx27_hip_ctx *ctx);
int vx27_hip_graph_end(vx27_hip_ctx *ctx, void **graph_exec);
int vx27_hip_graph_launch(vx27_hip_ctx *ctx, void *graph_exec);
int vx27_hip_graph_destroy(void *graph_exec);

/* ---------------------------------------------- synthetic data on device
 * Deterministic N(mean, std^2) values from a counter-based generator
 * (splitmix64 of (seed, index), Box-Muller) -- for benchmarks and tests. */
int vx27_hip_fill_normal_f32(vx27_hip_ctx *ctx, float *p, size_t n, uint64_t seed, float mean,
                             float std);
int vx27_hip_fill_normal_bf16(vx27_hip_ctx *ctx, uint16_t *p, size_t n, uint64_t seed, float mean,
                              float std);

/* ------------------------------------ device forms of the reference API
 * Same arguments, sizes and arithmetic as the reference function named, on
 * device pointers.  The host-pointer drop-ins of vx27_deltanet.h, vx27_gqa.h
 * and vx27_rope.h stage their buffers and call these. */
/* vx27_deltanet_step_exact (vx27_deltanet.c:71-102) with decay = exp(g_log)
 * given (the drop-in evaluates it with the host's exp); hd in [1, 256]. */
int vx27_hip_step_exact(vx27_hip_ctx *ctx, float *S, const float *q, const float *k,
                        const float *v, double beta, double decay, float *o, int hd);
/* vx27_deltanet_update_{ref,tiled} (variant 0) / _avx2 (variant 1, fused
 * multiply-add) -- vx27_deltanet.c:15-19, vx27_deltanet_avx2.c:6-24 */
int vx27_hip_update_simple(vx27_hip_ctx *ctx, float *S, const float *k, const float *v,
                           float decay, int hd, int variant);
/* vx27_deltanet_retrieve_ref (0) / _avx2 (1) / _tiled (2) -- vx27_deltanet.c:20-49,
 * vx27_deltanet_avx2.c:28-45 */
int vx27_hip_retrieve_simple(vx27_hip_ctx *ctx, const float *S, const float *q, float *o,
                             int hd, int variant);
int vx27_hip_l2norm(vx27_hip_ctx *ctx, const float *x, float *y, int n);  /* vx27_deltanet.c:51-56 */
int vx27_hip_rmsnorm(vx27_hip_ctx *ctx, const float *x, const float *w, float *y, int n,
                     float eps);                                         /* vx27_gqa.c:10-15 */
int vx27_hip_conv1d_step(vx27_hip_ctx *ctx, float *state, const float *x, const float *w,
                         float *y, int C, int apply_silu);               /* vx27_deltanet.c:106-122 */
int vx27_hip_rope_apply(vx27_hip_ctx *ctx, float *v, int n_heads, int head_dim, int rope_dim,
                        const float *cosv, const float *sinv);           /* vx27_rope.c:18-29 */
/* vx27_attn_1q (vx27_gqa.c:17-45) without its 1024-position cap; its scratch
 * is the context's, so concurrent calls need distinct contexts. */
int vx27_hip_attn_1q(vx27_hip_ctx *ctx, const float *q, const float *kcache,
                     const float *vcache, int n_pos, float *out);
/* Context-owned device staging buffer of at least `bytes` for host-pointer
 * callers (valid until the next vx27_hip_staging call on ctx). */
int vx27_hip_staging(vx27_hip_ctx *ctx, size_t bytes, void **dptr);
int vx27_hip_get_error_mode(void);

#ifdef __cplusplus
}
#endif
#endif
