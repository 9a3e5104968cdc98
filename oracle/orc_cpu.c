/*
 * CPU baseline drivers for the oracle.  TEST / BENCH INFRASTRUCTURE ONLY.
 *
 * A POSIX fork-join pool with the shape of the reference's threadpool.h API
 * (tp_run(fn(arg, tid, nthreads)), src/threadpool.h:8-13), whose own
 * implementation is Win32-only (src/threadpool.c:4).  Work is split over
 * independent (sequence, head) units, each unit running all of its steps,
 * so one fork-join covers a whole run.  Wall time is CLOCK_MONOTONIC.
 */
#define _POSIX_C_SOURCE 200809L
#include "vx27_oracle.h"
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

typedef void (*orc_task_fn)(void *arg, int tid, int nthreads);
typedef struct { orc_task_fn fn; void *arg; int tid, n; } orc_task;

static void *orc_task_main(void *p) {
    orc_task *t = (orc_task *)p;
    t->fn(t->arg, t->tid, t->n);
    return NULL;
}

/* Run fn on `threads` workers (the caller is worker 0) and join. */
static void orc_tp_run(int threads, orc_task_fn fn, void *arg) {
    if (threads < 1) threads = 1;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
    orc_task *ts = (orc_task *)malloc(sizeof(orc_task) * (size_t)threads);
    for (int i = 0; i < threads; i++) {
        ts[i].fn = fn; ts[i].arg = arg; ts[i].tid = i; ts[i].n = threads;
    }
    for (int i = 1; i < threads; i++) pthread_create(&th[i], NULL, orc_task_main, &ts[i]);
    fn(arg, 0, threads);
    for (int i = 1; i < threads; i++) pthread_join(th[i], NULL);
    free(th);
    free(ts);
}

static double orc_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* ---------------------------------------------------- DeltaNet decode run */
/* One unit = (sequence b, QK head g): owns the conv channels of q_g, k_g and
 * of the value heads mapped to g, so units never share state. */
static void orc_dn_unit(const orc_dn_run_args *r, int b, int g) {
    const int hd = r->hd, nqk = r->nqk, nv = r->nv;
    const int qd = nqk * hd, vd = nv * hd, C = 2 * qd + vd;
    const int vh0 = (g * nv + nqk - 1) / nqk;          /* first vh with vh*nqk/nv == g */
    int vh1 = vh0;
    while (vh1 < nv && vh1 * nqk / nv == g) vh1++;
    float qa[256], ka[256], tq[256], tk[256], ret[256], tn[256];
    float *cst = r->conv_state;
    for (int t = 0; t < r->steps; t++) {
        const size_t sb = (size_t)t * r->B + b;
        /* gather this unit's q,k (and per value head v) activations */
        if (r->flags & ORC_DN_CONV) {
            const float *x = r->x + sb * C;
            float *cs = cst + (size_t)b * C * 3;
            orc_conv1d_step(cs + (size_t)(g * hd) * 3, x + g * hd, r->conv_w + (size_t)(g * hd) * 4,
                            qa, hd, 1);
            orc_conv1d_step(cs + (size_t)(qd + g * hd) * 3, x + qd + g * hd,
                            r->conv_w + (size_t)(qd + g * hd) * 4, ka, hd, 1);
        } else {
            memcpy(qa, r->q + sb * qd + (size_t)g * hd, sizeof(float) * hd);
            memcpy(ka, r->k + sb * qd + (size_t)g * hd, sizeof(float) * hd);
        }
        if (r->flags & (ORC_DN_PRE_RMS | ORC_DN_PRE_L2)) {
            if (r->flags & ORC_DN_PRE_RMS) {
                orc_rmsn_1pw(qa, r->norm_w, tq, hd);
                orc_rmsn_1pw(ka, r->norm_w, tk, hd);
            } else {
                memcpy(tq, qa, sizeof(float) * hd);
                memcpy(tk, ka, sizeof(float) * hd);
            }
            if (r->flags & ORC_DN_PRE_L2) {
                orc_l2norm(tq, qa, hd);
                orc_l2norm(tk, ka, hd);
                const float qs = 1.0f / sqrtf((float)hd);
                for (int i = 0; i < hd; i++) qa[i] = qa[i] * qs;
            } else {
                memcpy(qa, tq, sizeof(float) * hd);
                memcpy(ka, tk, sizeof(float) * hd);
            }
        }
        for (int vh = vh0; vh < vh1; vh++) {
            float va[256];
            if (r->flags & ORC_DN_CONV) {
                const float *x = r->x + sb * C;
                float *cs = cst + (size_t)b * C * 3;
                orc_conv1d_step(cs + (size_t)(2 * qd + vh * hd) * 3, x + 2 * qd + vh * hd,
                                r->conv_w + (size_t)(2 * qd + vh * hd) * 4, va, hd, 1);
            } else {
                memcpy(va, r->v + sb * vd + (size_t)vh * hd, sizeof(float) * hd);
            }
            double beta, glog;
            orc_gate_params((double)r->a[sb * nv + vh], (double)r->A_log[vh],
                            (double)r->b[sb * nv + vh], (double)r->dt_bias[vh], &beta, &glog);
            float *S = r->S + ((size_t)b * nv + vh) * hd * hd;
            orc_step_exact(S, qa, ka, va, beta, glog, ret, hd);
            float *o = r->out + sb * vd + (size_t)vh * hd;
            if (r->flags & ORC_DN_OUT_GATE) {
                orc_rmsn_std(ret, r->norm_w, tn, hd);
                const float *z = r->z + sb * vd + (size_t)vh * hd;
                for (int i = 0; i < hd; i++) o[i] = tn[i] * orc_silu(z[i]);
            } else {
                memcpy(o, ret, sizeof(float) * hd);
            }
        }
    }
}

static void orc_dn_worker(void *arg, int tid, int n) {
    const orc_dn_run_args *r = (const orc_dn_run_args *)arg;
    const int units = r->B * r->nqk;
    for (int u = tid; u < units; u += n) orc_dn_unit(r, u / r->nqk, u % r->nqk);
}

double orc_dn_run(const orc_dn_run_args *r) {
    const double t0 = orc_now();
    orc_tp_run(r->threads, orc_dn_worker, (void *)r);
    return orc_now() - t0;
}

/* -------------------------------- the reference AVX2 primitives, composed */
/* Restates vx27_deltanet_update_avx2 (vx27_deltanet_avx2.c:6-24): row r of S
 * becomes fma(S, decay, k[r]*v), and vx27_deltanet_retrieve_avx2 (:28-45):
 * o accumulates fma(S_row, q[r], o) over rows. */
__attribute__((target("avx2,fma")))
static void orc_update_avx2(float *S, const float *k, const float *v, float decay, int hd) {
    const __m256 dv = _mm256_set1_ps(decay);
    for (int r = 0; r < hd; r++) {
        const __m256 kr = _mm256_set1_ps(k[r]);
        float *row = S + (size_t)r * hd;
        for (int c = 0; c < hd; c += 8) {
            __m256 prod = _mm256_mul_ps(kr, _mm256_loadu_ps(v + c));
            _mm256_storeu_ps(row + c, _mm256_fmadd_ps(_mm256_loadu_ps(row + c), dv, prod));
        }
    }
}
__attribute__((target("avx2,fma")))
static void orc_retrieve_avx2(const float *S, const float *q, float *o, int hd) {
    __m256 acc[32];
    for (int c = 0; c < hd / 8; c++) acc[c] = _mm256_setzero_ps();
    for (int r = 0; r < hd; r++) {
        const __m256 qr = _mm256_set1_ps(q[r]);
        const float *row = S + (size_t)r * hd;
        for (int c = 0; c < hd / 8; c++)
            acc[c] = _mm256_fmadd_ps(_mm256_loadu_ps(row + 8 * c), qr, acc[c]);
    }
    for (int c = 0; c < hd / 8; c++) _mm256_storeu_ps(o + 8 * c, acc[c]);
}

void orc_update_avx2_pub(float *S, const float *k, const float *v, float decay, int hd) {
    orc_update_avx2(S, k, v, decay, hd);
}
void orc_retrieve_avx2_pub(const float *S, const float *q, float *o, int hd) {
    orc_retrieve_avx2(S, q, o, hd);
}

typedef struct {
    int B, nv, hd, steps;
    float *S;
    const float *qn, *kn, *v;
    const double *beta, *decay;
    float *out;
    orc_update_fn upd;
    orc_retrieve_fn ret;
} orc_avx2_args;

static void orc_avx2_worker(void *arg, int tid, int n) {
    const orc_avx2_args *a = (const orc_avx2_args *)arg;
    const int hd = a->hd, units = a->B * a->nv;
    float kv[256], d[256];
    for (int u = tid; u < units; u += n) {
        float *S = a->S + (size_t)u * hd * hd;
        for (int t = 0; t < a->steps; t++) {
            const size_t e = (size_t)t * units + u;
            const float *q = a->qn + e * hd, *k = a->kn + e * hd, *v = a->v + e * hd;
            const float dec = (float)a->decay[e], bt = (float)a->beta[e];
            a->ret(S, k, kv, hd);
            for (int c = 0; c < hd; c++) d[c] = bt * (v[c] - dec * kv[c]);
            a->upd(S, k, d, dec, hd);
            a->ret(S, q, a->out + e * hd, hd);
        }
    }
}

double orc_dn_run_avx2(int B, int nv, int hd, int steps, int threads, float *S,
                       const float *qn, const float *kn, const float *v,
                       const double *beta, const double *decay, float *out,
                       orc_update_fn upd, orc_retrieve_fn ret) {
    orc_avx2_args a = {B, nv, hd, steps, S, qn, kn, v, beta, decay, out,
                       upd ? upd : orc_update_avx2, ret ? ret : orc_retrieve_avx2};
    const double t0 = orc_now();
    orc_tp_run(threads, orc_avx2_worker, &a);
    return orc_now() - t0;
}

/* ------------------------------------------------------- attention runs */
static void orc_attend_worker(void *arg, int tid, int n) {
    const orc_attend_batch_args *a = (const orc_attend_batch_args *)arg;
    const int units = a->B * a->n_q;
    int maxk = 1;
    for (int b = 0; b < a->B; b++) if (a->n_keys[b] > maxk) maxk = a->n_keys[b];
    float *sc = (float *)malloc(sizeof(float) * (size_t)maxk);
    float *one = (float *)malloc(sizeof(float) * (size_t)a->n_q * a->hd);
    const size_t esz = a->kv_bf16 ? 2 : 4;
    for (int u = tid; u < units; u += n) {
        const int b = u / a->n_q, h = u % a->n_q;
        orc_attend_args s = {a->n_q, a->n_kv, a->hd, a->n_keys[b], a->dot_double, a->kv_bf16,
                             a->q + (size_t)b * a->n_q * a->hd,
                             (const char *)a->k + (size_t)b * a->seq_stride * esz,
                             (const char *)a->v + (size_t)b * a->seq_stride * esz,
                             a->k_pos_stride, a->k_head_stride, a->v_pos_stride,
                             a->v_head_stride, one};
        orc_attend_one(&s, h, sc);
        memcpy(a->out + ((size_t)b * a->n_q + h) * a->hd, one + (size_t)h * a->hd,
               sizeof(float) * (size_t)a->hd);
    }
    free(sc);
    free(one);
}

double orc_attend_batch(const orc_attend_batch_args *a) {
    const double t0 = orc_now();
    orc_tp_run(a->threads, orc_attend_worker, (void *)a);
    return orc_now() - t0;
}

/* -------------------------------------------------------- GQA prefill */
typedef struct {
    const orc_gqa_prefill_args *a;
    const float *q_rot;     /* [B][T][n_q][hd] normed + roped */
} orc_gp_ctx;

static void orc_gp_worker(void *arg, int tid, int n) {
    const orc_gp_ctx *c = (const orc_gp_ctx *)arg;
    const orc_gqa_prefill_args *a = c->a;
    const int hd = a->hd;
    const long long units = (long long)a->B * a->T * a->n_q;
    float *sc = (float *)malloc(sizeof(float) * (size_t)a->L);
    float *one = (float *)malloc(sizeof(float) * (size_t)a->n_q * hd);
    for (long long u = tid; u < units; u += n) {
        const int h = (int)(u % a->n_q);
        const long long bt = u / a->n_q;
        const int t = (int)(bt % a->T), b = (int)(bt / a->T);
        const size_t kvs = (size_t)a->n_kv * hd;
        orc_attend_args s = {a->n_q, a->n_kv, hd, a->pos0 + t + 1, 1, 0,
                             c->q_rot + (size_t)bt * a->n_q * hd,
                             a->k_cache + (size_t)b * a->L * kvs, a->v_cache + (size_t)b * a->L * kvs,
                             kvs, (size_t)hd, kvs, (size_t)hd, one};
        orc_attend_one(&s, h, sc);
        const size_t o = ((size_t)bt * a->n_q + h) * hd;
        for (int i = 0; i < hd; i++)
            a->out[o + i] = a->no_gate ? one[(size_t)h * hd + i]
                                       : one[(size_t)h * hd + i] * (1.0f / (1.0f + expf(-a->gate[o + i])));
    }
    free(sc);
    free(one);
}

double orc_gqa_prefill(const orc_gqa_prefill_args *a) {
    const double t0 = orc_now();
    const int hd = a->hd, half = a->rope_dim / 2;
    float *q_rot = (float *)malloc(sizeof(float) * (size_t)a->B * a->T * a->n_q * hd);
    float cosv[128], sinv[128];
    for (int b = 0; b < a->B; b++)
        for (int t = 0; t < a->T; t++) {
            const size_t bt = (size_t)b * a->T + t;
            const int pos = a->pos0 + t;
            if (half > 0) orc_rope_cos_sin(pos, cosv, sinv, a->rope_dim, a->rope_theta, a->rope_yarn);
            float *qr = q_rot + bt * a->n_q * hd;
            for (int h = 0; h < a->n_q; h++)
                orc_rmsn_1pw(a->q + (bt * a->n_q + h) * hd, a->q_norm_w, qr + (size_t)h * hd, hd);
            float *kc = a->k_cache + ((size_t)b * a->L + pos) * a->n_kv * hd;
            float *vc = a->v_cache + ((size_t)b * a->L + pos) * a->n_kv * hd;
            for (int h = 0; h < a->n_kv; h++)
                orc_rmsn_1pw(a->k + (bt * a->n_kv + h) * hd, a->k_norm_w, kc + (size_t)h * hd, hd);
            if (half > 0) {
                orc_rope_apply(qr, a->n_q, hd, a->rope_dim, cosv, sinv);
                orc_rope_apply(kc, a->n_kv, hd, a->rope_dim, cosv, sinv);
            }
            memcpy(vc, a->v + bt * a->n_kv * hd, sizeof(float) * (size_t)a->n_kv * hd);
        }
    orc_gp_ctx c = {a, q_rot};
    orc_tp_run(a->threads, orc_gp_worker, &c);
    free(q_rot);
    return orc_now() - t0;
}

/* --------------------------------------------------------- matvec runs */
typedef struct { const void *W; int w_bf16; const float *x; float *y; int rows, cols, B; } orc_mv_args;

static void orc_mv_worker(void *arg, int tid, int n) {
    const orc_mv_args *m = (const orc_mv_args *)arg;
    const int r0 = (int)((long long)m->rows * tid / n), r1 = (int)((long long)m->rows * (tid + 1) / n);
    for (int b = 0; b < m->B; b++) {
        const size_t off = (size_t)r0 * m->cols;
        const void *Wr = m->w_bf16 ? (const void *)((const uint16_t *)m->W + off)
                                   : (const void *)((const float *)m->W + off);
        orc_matvec(Wr, m->w_bf16, m->x + (size_t)b * m->cols, m->y + (size_t)b * m->rows + r0,
                   r1 - r0, m->cols);
    }
}

double orc_matvec_batch(const void *W, int w_bf16, const float *x, float *y,
                        int rows, int cols, int B, int threads) {
    orc_mv_args m = {W, w_bf16, x, y, rows, cols, B};
    const double t0 = orc_now();
    orc_tp_run(threads, orc_mv_worker, &m);
    return orc_now() - t0;
}
