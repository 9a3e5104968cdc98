/*
 * Host-pointer drop-ins for the reference's mixer API (vx27_deltanet.h,
 * vx27_gqa.h, vx27_rope.h), in C, on top of the vx27_hip.h C ABI.
 *
 * Each compute function stages its host buffers into the default context's
 * device staging area, runs the device form of the same function and copies
 * the results back; the call is synchronous, like the reference's.  There is
 * no host fallback: on failure the process aborts with the library's error
 * message, or (error mode VX27_HIP_ERR_POISON) the outputs are set to NaN.
 * Scalar helpers (state sizing, the KV-head map, gate parameters and the
 * per-position RoPE table) are host functions in the reference's own
 * arithmetic, as the reference evaluates them once per token on the host.
 *
 * The drop-ins may be called from several threads: the default context is
 * opened once (vx27_hip_default_ctx), and each call holds one process-wide
 * lock from staging its inputs to reading back its outputs, because all of
 * them share the default context's stream and staging buffer.  Concurrent
 * calls are therefore serialised, not run side by side.
 */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vx27_deltanet.h"
#include "vx27_gqa.h"
#include "vx27_hip.h"
#include "vx27_rope.h"

/* ---------------------------------------------------------------- helpers */
static void poison(float *p, size_t n) {
    if (!p) return;
    for (size_t i = 0; i < n; i++) p[i] = NAN;
}

static void dropin_fail(const char *fn, float *o1, size_t n1, float *o2, size_t n2) {
    if (vx27_hip_get_error_mode() == VX27_HIP_ERR_POISON) {
        poison(o1, n1);
        poison(o2, n2);
        return;
    }
    fprintf(stderr, "vx27_hip: %s failed: %s\n", fn, vx27_hip_last_error());
    fflush(stderr);
    abort();
}

/* A staging area carved into up to 8 float arrays, 256-byte aligned. */
typedef struct {
    vx27_hip_ctx *ctx;
    char *base;
    size_t off[8];
    size_t len[8];
    int n;
    int locked;
} stage_t;

static pthread_mutex_t g_dropin_mu = PTHREAD_MUTEX_INITIALIZER;

/* Ends a call that opened a stage: releases the drop-in lock. */
static void stage_close(stage_t *s) {
    if (s->locked) pthread_mutex_unlock(&g_dropin_mu);
    s->locked = 0;
}

static size_t align256(size_t x) { return (x + 255u) & ~(size_t)255u; }

static int stage_open(stage_t *s, const size_t *counts, int n) {
    memset(s, 0, sizeof *s);
    s->ctx = vx27_hip_default_ctx();
    if (!s->ctx) return -1;
    pthread_mutex_lock(&g_dropin_mu);
    s->locked = 1;
    size_t total = 0;
    for (int i = 0; i < n; i++) {
        s->off[i] = total;
        s->len[i] = counts[i] * sizeof(float);
        total += align256(s->len[i] ? s->len[i] : 1);
    }
    s->n = n;
    void *p = NULL;
    if (vx27_hip_staging(s->ctx, total, &p)) return -1;
    s->base = (char *)p;
    return 0;
}
static float *dptr(stage_t *s, int i) { return (float *)(s->base + s->off[i]); }
static int up(stage_t *s, int i, const float *h) {
    return s->len[i] ? vx27_hip_h2d(s->ctx, dptr(s, i), h, s->len[i]) : 0;
}
static int down(stage_t *s, int i, float *h) {
    return s->len[i] ? vx27_hip_d2h(s->ctx, h, dptr(s, i), s->len[i]) : 0;
}

/* --------------------------------------------------------------- DeltaNet */
/* vx27_deltanet.c:5-13 with the model constants of vx27_config.h:14-16. */
int vx27_deltanet_state_per_layer(void) { return 16 * 128 * 128; }
int vx27_deltanet_state_total(void) { return vx27_deltanet_state_per_layer() * 48; }
double vx27_deltanet_state_mb(int bytes_per_elem) {
    return (double)vx27_deltanet_state_total() * bytes_per_elem / 1e6;
}

static void simple_update(const char *fn, float *S, const float *k, const float *v, float decay,
                          int hd, int variant) {
    stage_t s = {0};
    size_t c[3] = {(size_t)hd * hd, (size_t)hd, (size_t)hd};
    if (hd < 1 || stage_open(&s, c, 3) || up(&s, 0, S) || up(&s, 1, k) || up(&s, 2, v) ||
        vx27_hip_update_simple(s.ctx, dptr(&s, 0), dptr(&s, 1), dptr(&s, 2), decay, hd, variant) ||
        down(&s, 0, S))
        dropin_fail(fn, S, hd > 0 ? (size_t)hd * hd : 0, NULL, 0);
    stage_close(&s);
}
static void simple_retrieve(const char *fn, const float *S, const float *q, float *o, int hd,
                            int variant) {
    stage_t s = {0};
    size_t c[3] = {(size_t)hd * hd, (size_t)hd, (size_t)hd};
    if (hd < 1 || stage_open(&s, c, 3) || up(&s, 0, S) || up(&s, 1, q) ||
        vx27_hip_retrieve_simple(s.ctx, dptr(&s, 0), dptr(&s, 1), dptr(&s, 2), hd, variant) ||
        down(&s, 2, o))
        dropin_fail(fn, o, hd > 0 ? (size_t)hd : 0, NULL, 0);
    stage_close(&s);
}

void vx27_deltanet_update_ref(float *S, const float *k, const float *v, float decay, int hd) {
    simple_update("vx27_deltanet_update_ref", S, k, v, decay, hd, 0);
}
void vx27_deltanet_update_tiled(float *S, const float *k, const float *v, float decay, int hd) {
    simple_update("vx27_deltanet_update_tiled", S, k, v, decay, hd, 0);
}
void vx27_deltanet_update_avx2(float *S, const float *k, const float *v, float decay, int hd) {
    simple_update("vx27_deltanet_update_avx2", S, k, v, decay, hd, 1);
}
void vx27_deltanet_retrieve_ref(const float *S, const float *q, float *o, int hd) {
    simple_retrieve("vx27_deltanet_retrieve_ref", S, q, o, hd, 0);
}
void vx27_deltanet_retrieve_tiled(const float *S, const float *q, float *o, int hd) {
    simple_retrieve("vx27_deltanet_retrieve_tiled", S, q, o, hd, 2);
}
void vx27_deltanet_retrieve_avx2(const float *S, const float *q, float *o, int hd) {
    simple_retrieve("vx27_deltanet_retrieve_avx2", S, q, o, hd, 1);
}

void vx27_deltanet_l2norm(const float *x, float *y, int n) {
    stage_t s = {0};
    size_t c[2] = {(size_t)(n > 0 ? n : 0), (size_t)(n > 0 ? n : 0)};
    if (n <= 0) return;
    if (stage_open(&s, c, 2) || up(&s, 0, x) || vx27_hip_l2norm(s.ctx, dptr(&s, 0), dptr(&s, 1), n) ||
        down(&s, 1, y))
        dropin_fail("vx27_deltanet_l2norm", y, (size_t)n, NULL, 0);
    stage_close(&s);
}

/* Scalar: vx27_deltanet.c:58-69. */
static double softplus_ref(double x) {
    if (x > 20.0) return x;
    if (x < -20.0) return exp(x);
    return log(1.0 + exp(x));
}
void vx27_deltanet_gate_params(double a, double A_log, double b, double dt_bias, double *beta,
                               double *g_log) {
    if (beta) *beta = 1.0 / (1.0 + exp(-b));
    if (g_log) *g_log = -exp(A_log) * softplus_ref(a + dt_bias);
}

void vx27_deltanet_step_exact(float *S, const float *q, const float *k, const float *v, double beta,
                              double g_log, float *o, int hd) {
    stage_t s = {0};
    size_t c[5] = {(size_t)hd * hd, (size_t)hd, (size_t)hd, (size_t)hd, (size_t)hd};
    if (hd < 1 || hd > 256 || stage_open(&s, c, 5) || up(&s, 0, S) || up(&s, 1, q) || up(&s, 2, k) ||
        up(&s, 3, v) ||
        vx27_hip_step_exact(s.ctx, dptr(&s, 0), dptr(&s, 1), dptr(&s, 2), dptr(&s, 3), beta, exp(g_log),
                            dptr(&s, 4), hd) ||
        down(&s, 0, S) || down(&s, 4, o))
        dropin_fail("vx27_deltanet_step_exact", o, hd > 0 ? (size_t)hd : 0, S,
                    hd > 0 ? (size_t)hd * hd : 0);
    stage_close(&s);
}

void vx27_conv1d_step(float *state, const float *x, const float *w, float *y, int C, int apply_silu) {
    stage_t s = {0};
    if (C <= 0) return;
    size_t c[4] = {(size_t)C * 3, (size_t)C, (size_t)C * 4, (size_t)C};
    if (stage_open(&s, c, 4) || up(&s, 0, state) || up(&s, 1, x) || up(&s, 2, w) ||
        vx27_hip_conv1d_step(s.ctx, dptr(&s, 0), dptr(&s, 1), dptr(&s, 2), dptr(&s, 3), C, apply_silu) ||
        down(&s, 0, state) || down(&s, 3, y))
        dropin_fail("vx27_conv1d_step", y, (size_t)C, state, (size_t)C * 3);
    stage_close(&s);
}

/* -------------------------------------------------------------------- GQA */
int vx27_gqa_kv_for_q(int q_head) { return q_head * 4 / 24; }   /* vx27_gqa.c:6-8 */

void vx27_rmsnorm(const float *x, const float *w, float *y, int n, float eps) {
    stage_t s = {0};
    if (n <= 0) return;
    size_t c[3] = {(size_t)n, (size_t)n, (size_t)n};
    if (stage_open(&s, c, 3) || up(&s, 0, x) || up(&s, 1, w) ||
        vx27_hip_rmsnorm(s.ctx, dptr(&s, 0), dptr(&s, 1), dptr(&s, 2), n, eps) || down(&s, 2, y))
        dropin_fail("vx27_rmsnorm", y, (size_t)n, NULL, 0);
    stage_close(&s);
}

void vx27_attn_1q(const float *q, const float *kcache, const float *vcache, int n_pos, float *out) {
    stage_t s = {0};
    const size_t nq = 24 * 256, nkv = (size_t)(n_pos > 0 ? n_pos : 0) * 4 * 256;
    size_t c[4] = {nq, nkv, nkv, nq};
    if (n_pos < 1 || stage_open(&s, c, 4) || up(&s, 0, q) || up(&s, 1, kcache) || up(&s, 2, vcache) ||
        vx27_hip_attn_1q(s.ctx, dptr(&s, 0), dptr(&s, 1), dptr(&s, 2), n_pos, dptr(&s, 3)) ||
        down(&s, 3, out))
        dropin_fail("vx27_attn_1q", out, nq, NULL, 0);
    stage_close(&s);
}

/* ------------------------------------------------------------------- RoPE */
/* Per-position table, the reference's float formula (vx27_rope.c:5-16). */
void vx27_rope_cos_sin(int pos, float *cosv, float *sinv, int rope_dim, float theta,
                       float yarn_factor) {
    if (yarn_factor < 1.0f) yarn_factor = 1.0f;
    const float ps = (float)pos / yarn_factor;
    for (int i = 0; i < rope_dim / 2; i++) {
        const float expo = (-2.0f * (float)i) / (float)rope_dim;
        const float ang = ps * powf(theta, expo);
        cosv[i] = cosf(ang);
        sinv[i] = sinf(ang);
    }
}
void vx27_mrope_cos_sin_text(int pos, float *cosv, float *sinv) {
    vx27_rope_cos_sin(pos, cosv, sinv, 64, 10000000.0f, 1.0f);   /* vx27_rope.c:31-33 */
}

void vx27_rope_apply(float *v, int n_heads, int head_dim, int rope_dim, const float *cosv,
                     const float *sinv) {
    stage_t s = {0};
    if (n_heads <= 0 || rope_dim < 2) return;
    const size_t nv = (size_t)n_heads * head_dim, half = (size_t)rope_dim / 2;
    size_t c[3] = {nv, half, half};
    if (rope_dim > head_dim || stage_open(&s, c, 3) || up(&s, 0, v) || up(&s, 1, cosv) ||
        up(&s, 2, sinv) ||
        vx27_hip_rope_apply(s.ctx, dptr(&s, 0), n_heads, head_dim, rope_dim, dptr(&s, 1), dptr(&s, 2)) ||
        down(&s, 0, v))
        dropin_fail("vx27_rope_apply", v, nv, NULL, 0);
    stage_close(&s);
}
