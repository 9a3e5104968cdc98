/*
 * vx27 oracle: CPU restatement of the reference token-mixer math.
 * TEST INFRASTRUCTURE ONLY (see vx27_oracle.h for the contract and the
 * pinning status of every function).  Compiled with -std=c11
 * -ffp-contract=off so that every float/double operation below is evaluated
 * as written, one rounding per operation, like the reference's own build.
 */
#define _POSIX_C_SOURCE 200809L
#include "vx27_oracle.h"
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------ bf16 */
uint16_t orc_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
void orc_f32_to_bf16_n(const float *x, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_f32_to_bf16(x[i]);
}
void orc_bf16_to_f32_n(const uint16_t *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------- DeltaNet */
/* Model constants of vx27_config.h:14-16 (16 QK heads, head dim 128, 48 layers). */
int orc_state_per_layer(void) { return 16 * 128 * 128; }
int orc_state_total(void) { return orc_state_per_layer() * 48; }
double orc_state_mb(int bytes_per_elem) {
    return (double)orc_state_total() * bytes_per_elem / 1e6;
}

/* vx27_deltanet.c:15-19: S <- decay*S + k v^T, float, no fused multiply-add. */
void orc_update_simple(float *S, const float *k, const float *v, float decay, int hd) {
    for (int r = 0; r < hd; r++) {
        float *row = S + (size_t)r * hd;
        const float kr = k[r];
        for (int c = 0; c < hd; c++) {
            float dec = decay * row[c];
            float add = kr * v[c];
            row[c] = dec + add;
        }
    }
}
/* vx27_deltanet.c:20-25: o[c] = float running sum over rows of S[r][c]*q[r]. */
void orc_retrieve_simple(const float *S, const float *q, float *o, int hd) {
    for (int c = 0; c < hd; c++) {
        float acc = 0.0f;
        for (int r = 0; r < hd; r++) acc = acc + S[(size_t)r * hd + c] * q[r];
        o[c] = acc;
    }
}

/* vx27_deltanet.c:51-56: double sum of squares, eps 1e-6 inside the sqrt, no /n. */
void orc_l2norm(const float *x, float *y, int n) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) {
        double xi = (double)x[i];
        ss = ss + xi * xi;
    }
    float inv = 1.0f / sqrtf((float)ss + 1e-6f);
    for (int i = 0; i < n; i++) y[i] = x[i] * inv;
}

/* vx27_deltanet.c:58-63: softplus with linear / exponential tails at |x|>20. */
static double orc_softplus(double x) {
    if (x > 20.0) return x;
    if (x < -20.0) return exp(x);
    return log(1.0 + exp(x));
}
/* vx27_deltanet.c:65-69: beta = sigmoid(b) (no dt_bias); g = -exp(A_log)*softplus(a+dt_bias). */
void orc_gate_params(double a, double A_log, double b, double dt_bias,
                     double *beta, double *g_log) {
    if (beta) *beta = 1.0 / (1.0 + exp(-b));
    if (g_log) *g_log = -exp(A_log) * orc_softplus(a + dt_bias);
}

/* vx27_deltanet.c:71-102, one token of one value head:
 *   qn = l2norm(q) * (1/sqrtf(hd)), kn = l2norm(k)        (float)
 *   S  = (float)((double)S * exp(g))
 *   kv = S^T kn                                              (double, rows in order)
 *   S  = (float)((double)S + (double)kn[r] * ((v - kv)*beta))
 *   o  = (float)(S^T qn)                                     (double, rows in order) */
void orc_step_exact(float *S, const float *q, const float *k, const float *v,
                    double beta, double g_log, float *o, int hd) {
    float qn[256], kn[256];
    double kv[256];
    orc_l2norm(q, qn, hd);
    orc_l2norm(k, kn, hd);
    const float qscale = 1.0f / sqrtf((float)hd);
    for (int r = 0; r < hd; r++) qn[r] = qn[r] * qscale;
    const double decay = exp(g_log);
    const size_t n = (size_t)hd * hd;
    for (size_t e = 0; e < n; e++) S[e] = (float)((double)S[e] * decay);
    for (int c = 0; c < hd; c++) {
        double acc = 0.0;
        for (int r = 0; r < hd; r++) acc = acc + (double)S[(size_t)r * hd + c] * (double)kn[r];
        kv[c] = acc;
    }
    for (int r = 0; r < hd; r++) {
        const double kr = (double)kn[r];
        float *row = S + (size_t)r * hd;
        for (int c = 0; c < hd; c++) {
            const double delta = ((double)v[c] - kv[c]) * beta;
            row[c] = (float)((double)row[c] + kr * delta);
        }
    }
    for (int c = 0; c < hd; c++) {
        double acc = 0.0;
        for (int r = 0; r < hd; r++) acc = acc + (double)S[(size_t)r * hd + c] * (double)qn[r];
        o[c] = (float)acc;
    }
}

/* vx27_qfwd.c:48 / vx27_deltanet.c:104. */
float orc_silu(float v) { return v / (1.0f + expf(-v)); }

/* vx27_deltanet.c:106-122: window = (state[0] oldest, state[1], state[2], x);
 * acc = w0*s0 + w1*s1 + w2*s2 + w3*x evaluated left to right; state shifts. */
void orc_conv1d_step(float *state, const float *x, const float *w, float *y,
                     int C, int apply_silu) {
    for (int c = 0; c < C; c++) {
        float *st = state + (size_t)c * 3;
        const float *wc = w + (size_t)c * 4;
        float acc = wc[0] * st[0];
        acc = acc + wc[1] * st[1];
        acc = acc + wc[2] * st[2];
        acc = acc + wc[3] * x[c];
        y[c] = apply_silu ? orc_silu(acc) : acc;
        st[0] = st[1];
        st[1] = st[2];
        st[2] = x[c];
    }
}

/* ----------------------------------------------------------- GQA, norms */
/* vx27_gqa.c:6-8 with 24 Q / 4 KV heads (vx27_config.h:19-20). */
int orc_kv_for_q(int q_head) { return q_head * 4 / 24; }

static float orc_rms_inv(const float *x, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) {
        double xi = (double)x[i];
        ss = ss + xi * xi;
    }
    return 1.0f / sqrtf((float)(ss / n) + eps);
}
/* vx27_gqa.c:10-15: y = x*s*w. */
void orc_rmsnorm_w(const float *x, const float *w, float *y, int n, float eps) {
    const float s = orc_rms_inv(x, n, eps);
    for (int i = 0; i < n; i++) y[i] = (x[i] * s) * w[i];
}
/* vx27_qfwd.c:32-39: y = x*s*(1+w) (zero-centred weight), eps 1e-6; w NULL -> x*s. */
void orc_rmsn_1pw(const float *x, const float *w, float *y, int n) {
    const float s = orc_rms_inv(x, n, 1e-6f);
    for (int i = 0; i < n; i++) y[i] = w ? (x[i] * s) * (w[i] + 1.0f) : x[i] * s;
}
/* vx27_qfwd.c:42-47: y = x*s*w; w NULL -> x*s. */
void orc_rmsn_std(const float *x, const float *w, float *y, int n) {
    const float s = orc_rms_inv(x, n, 1e-6f);
    for (int i = 0; i < n; i++) y[i] = w ? (x[i] * s) * w[i] : x[i] * s;
}

static inline float orc_kv_load(const void *base, int bf16, size_t idx) {
    return bf16 ? orc_bf16_to_f32(((const uint16_t *)base)[idx]) : ((const float *)base)[idx];
}

/* Two-pass softmax attention of one query head over n_keys keys; scores in
 * a caller scratch of n_keys floats.  Follows vx27_qfwd.c:190-207 (double
 * dot) or vx27_gqa.c:37-58 (float dot). */
void orc_attend_one(const orc_attend_args *a, int h, float *sc) {
    const int hd = a->hd;
    const int kvh = h * a->n_kv / a->n_q;
    const float *qh = a->q + (size_t)h * hd;
    const float scale = 1.0f / sqrtf((float)hd);
    float smax = -1e30f, ssum = 0.0f;
    for (int p = 0; p < a->n_keys; p++) {
        const size_t kb = (size_t)p * a->k_pos_stride + (size_t)kvh * a->k_head_stride;
        float s;
        if (a->dot_double) {
            double acc = 0.0;
            for (int i = 0; i < hd; i++)
                acc = acc + (double)qh[i] * (double)orc_kv_load(a->k, a->kv_bf16, kb + i);
            s = (float)(acc * (double)scale);
        } else {
            float acc = 0.0f;
            for (int i = 0; i < hd; i++) acc = acc + qh[i] * orc_kv_load(a->k, a->kv_bf16, kb + i);
            s = acc * scale;
        }
        sc[p] = s;
        if (s > smax) smax = s;
    }
    for (int p = 0; p < a->n_keys; p++) {
        sc[p] = expf(sc[p] - smax);
        ssum = ssum + sc[p];
    }
    float *oh = a->out + (size_t)h * hd;
    for (int i = 0; i < hd; i++) oh[i] = 0.0f;
    for (int p = 0; p < a->n_keys; p++) {
        const float wgt = sc[p] / ssum;
        const size_t vb = (size_t)p * a->v_pos_stride + (size_t)kvh * a->v_head_stride;
        for (int i = 0; i < hd; i++) oh[i] = oh[i] + wgt * orc_kv_load(a->v, a->kv_bf16, vb + i);
    }
}

void orc_attend(const orc_attend_args *a) {
    float *sc = (float *)malloc(sizeof(float) * (size_t)(a->n_keys > 0 ? a->n_keys : 1));
    for (int h = 0; h < a->n_q; h++) orc_attend_one(a, h, sc);
    free(sc);
}

/* vx27_gqa.c:17-45: float dot, caches [pos][4][256] float. */
void orc_attn_1q(const float *q, const float *kcache, const float *vcache,
                 int n_pos, float *out) {
    orc_attend_args a = {24, 4, 256, n_pos, 0, 0, q, kcache, vcache,
                         4 * 256, 256, 4 * 256, 256, out};
    orc_attend(&a);
}

/* ----------------------------------------------------------------- RoPE */
/* vx27_rope.c:5-16: float position / yarn, freq = powf(theta, -2i/rd), float angle. */
void orc_rope_cos_sin(int pos, float *cosv, float *sinv, int rope_dim,
                      float theta, float yarn_factor) {
    if (yarn_factor < 1.0f) yarn_factor = 1.0f;
    const float ps = (float)pos / yarn_factor;
    const int half = rope_dim / 2;
    for (int i = 0; i < half; i++) {
        const float expo = (-2.0f * (float)i) / (float)rope_dim;
        const float freq = powf(theta, expo);
        const float ang = ps * freq;
        cosv[i] = cosf(ang);
        sinv[i] = sinf(ang);
    }
}
/* vx27_rope.c:18-29: NeoX half-split rotation of the first rope_dim dims. */
void orc_rope_apply(float *v, int n_heads, int head_dim, int rope_dim,
                    const float *cosv, const float *sinv) {
    const int half = rope_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        float *p = v + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            const float a = p[i], b = p[i + half];
            p[i] = a * cosv[i] - b * sinv[i];
            p[i + half] = a * sinv[i] + b * cosv[i];
        }
    }
}
/* vx27_rope.c:31-33: text M-RoPE == standard RoPE, rope_dim 64, theta 1e7. */
void orc_mrope_cos_sin_text(int pos, float *cosv, float *sinv) {
    orc_rope_cos_sin(pos, cosv, sinv, 64, 10000000.0f, 1.0f);
}

/* ----------------------------------------------------------- projection */
void orc_matvec(const void *W, int w_bf16, const float *x, float *y, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        const size_t base = (size_t)r * cols;
        double acc = 0.0;
        for (int c = 0; c < cols; c++)
            acc = acc + (double)orc_kv_load(W, w_bf16, base + c) * (double)x[c];
        y[r] = (float)acc;
    }
}

/* ------------------------------------------------------ DeltaNet glue */
void orc_dn_token(const orc_dn_cfg *c, const float *qkv, const float *a, const float *b,
                  const float *z, float *S, float *conv_state, float *out) {
    const int hd = c->hd, nqk = c->nqk, nv = c->nv;
    const int qd = nqk * hd, vd = nv * hd, C = 2 * qd + vd;
    float *act = (float *)malloc(sizeof(float) * (size_t)C);
    float *ret = (float *)malloc(sizeof(float) * (size_t)vd);
    if (c->flags & ORC_DN_CONV)
        orc_conv1d_step(conv_state, qkv, c->conv_w, act, C, 1);
    else
        memcpy(act, qkv, sizeof(float) * (size_t)C);
    float *q = act, *k = act + qd, *v = act + 2 * qd;
    if (c->flags & (ORC_DN_PRE_RMS | ORC_DN_PRE_L2)) {
        float tq[256], tk[256];
        for (int h = 0; h < nqk; h++) {
            float *qh = q + (size_t)h * hd, *kh = k + (size_t)h * hd;
            if (c->flags & ORC_DN_PRE_RMS) {
                orc_rmsn_1pw(qh, c->norm_w, tq, hd);
                orc_rmsn_1pw(kh, c->norm_w, tk, hd);
            } else {
                memcpy(tq, qh, sizeof(float) * (size_t)hd);
                memcpy(tk, kh, sizeof(float) * (size_t)hd);
            }
            if (c->flags & ORC_DN_PRE_L2) {
                orc_l2norm(tq, qh, hd);
                orc_l2norm(tk, kh, hd);
            } else {
                memcpy(qh, tq, sizeof(float) * (size_t)hd);
                memcpy(kh, tk, sizeof(float) * (size_t)hd);
            }
        }
        if (c->flags & ORC_DN_PRE_L2) {
            const float qs = 1.0f / sqrtf((float)hd);
            for (int i = 0; i < qd; i++) q[i] = q[i] * qs;
        }
    }
    for (int vh = 0; vh < nv; vh++) {
        const int g = vh * nqk / nv;
        double beta, glog;
        orc_gate_params((double)a[vh], (double)c->A_log[vh], (double)b[vh],
                        (double)c->dt_bias[vh], &beta, &glog);
        orc_step_exact(S + (size_t)vh * hd * hd, q + (size_t)g * hd, k + (size_t)g * hd,
                       v + (size_t)vh * hd, beta, glog, ret + (size_t)vh * hd, hd);
    }
    if (c->flags & ORC_DN_OUT_GATE) {
        float tn[256];
        for (int vh = 0; vh < nv; vh++) {
            orc_rmsn_std(ret + (size_t)vh * hd, c->norm_w, tn, hd);
            for (int i = 0; i < hd; i++)
                out[(size_t)vh * hd + i] = tn[i] * orc_silu(z[(size_t)vh * hd + i]);
        }
    } else {
        memcpy(out, ret, sizeof(float) * (size_t)vd);
    }
    free(act);
    free(ret);
}

/* ----------------------------------------------------------- GQA glue */
static void orc_kv_store(void *base, int bf16, size_t idx, float x) {
    if (bf16) ((uint16_t *)base)[idx] = orc_f32_to_bf16(x);
    else ((float *)base)[idx] = x;
}

void orc_gqa_token(const orc_gqa_cfg *c, const float *q_raw, size_t q_head_stride,
                   const float *gate, size_t gate_head_stride,
                   const float *k1, const float *v1, int pos,
                   const float *cosv, const float *sinv, float *out) {
    const int nq = c->n_q, nkv = c->n_kv, hd = c->hd;
    float *q = (float *)malloc(sizeof(float) * (size_t)nq * hd);
    float *k = (float *)malloc(sizeof(float) * (size_t)nkv * hd);
    float *att = (float *)malloc(sizeof(float) * (size_t)nq * hd);
    for (int h = 0; h < nq; h++)
        orc_rmsn_1pw(q_raw + (size_t)h * q_head_stride, c->q_norm_w, q + (size_t)h * hd, hd);
    for (int h = 0; h < nkv; h++)
        orc_rmsn_1pw(k1 + (size_t)h * hd, c->k_norm_w, k + (size_t)h * hd, hd);
    orc_rope_apply(q, nq, hd, c->rope_dim, cosv, sinv);
    orc_rope_apply(k, nkv, hd, c->rope_dim, cosv, sinv);
    for (int h = 0; h < nkv; h++)
        for (int i = 0; i < hd; i++) {
            orc_kv_store(c->k_cache, c->kv_bf16,
                         (size_t)pos * c->k_pos_stride + (size_t)h * c->k_head_stride + i,
                         k[(size_t)h * hd + i]);
            orc_kv_store(c->v_cache, c->kv_bf16,
                         (size_t)pos * c->v_pos_stride + (size_t)h * c->v_head_stride + i,
                         v1[(size_t)h * hd + i]);
        }
    orc_attend_args a = {nq, nkv, hd, pos + 1, 1, c->kv_bf16, q, c->k_cache, c->v_cache,
                         c->k_pos_stride, c->k_head_stride, c->v_pos_stride,
                         c->v_head_stride, att};
    orc_attend(&a);
    for (int h = 0; h < nq; h++)
        for (int i = 0; i < hd; i++) {
            if (c->no_gate) {   /* vx27_mtp.c:258 with use_gate = 0 */
                out[(size_t)h * hd + i] = att[(size_t)h * hd + i];
                continue;
            }
            const float gl = gate[(size_t)h * gate_head_stride + i];
            out[(size_t)h * hd + i] = att[(size_t)h * hd + i] * (1.0f / (1.0f + expf(-gl)));
        }
    free(q);
    free(k);
    free(att);
}

/* ------------------------------------------------ whole layers (no FFN) */
void orc_dn_layer_token(const orc_dn_layer_w *w, const float *x, float *S, float *conv,
                        float *out) {
    const int H = 5120, nqk = 16, nv = 48, hd = 128;
    const int qkvd = 2 * nqk * hd + nv * hd, vd = nv * hd;
    float *xn = (float *)malloc(sizeof(float) * H);
    float *qkv = (float *)malloc(sizeof(float) * (size_t)qkvd);
    float *z = (float *)malloc(sizeof(float) * (size_t)vd);
    float *o = (float *)malloc(sizeof(float) * (size_t)vd);
    float *ao = (float *)malloc(sizeof(float) * H);
    float av[48], bv[48];
    orc_rmsn_1pw(x, w->ln_w, xn, H);
    orc_matvec(w->w_qkv, 0, xn, qkv, qkvd, H);
    orc_matvec(w->w_z, 0, xn, z, vd, H);
    orc_matvec(w->w_a, 0, xn, av, nv, H);
    orc_matvec(w->w_b, 0, xn, bv, nv, H);
    orc_dn_cfg cfg = {nqk, nv, hd, ORC_DN_CONV | ORC_DN_PRE_RMS | ORC_DN_PRE_L2 | ORC_DN_OUT_GATE,
                      w->A_log, w->dt_bias, w->norm_w, w->conv_w};
    orc_dn_token(&cfg, qkv, av, bv, z, S, conv, o);
    orc_matvec(w->w_out, 0, o, ao, H, vd);
    for (int i = 0; i < H; i++) out[i] = x[i] + ao[i];
    free(xn); free(qkv); free(z); free(o); free(ao);
}

void orc_gqa_layer_token(const orc_gqa_layer_w *w, const float *x, int n_pos,
                         float *kcache, float *vcache, float *out) {
    const int H = 5120, nq = 24, nkv = 4, hd = 256;
    float *xn = (float *)malloc(sizeof(float) * H);
    float *qg = (float *)malloc(sizeof(float) * (size_t)nq * hd * 2);
    float *k1 = (float *)malloc(sizeof(float) * (size_t)nkv * hd);
    float *v1 = (float *)malloc(sizeof(float) * (size_t)nkv * hd);
    float *att = (float *)malloc(sizeof(float) * (size_t)nq * hd);
    float *ao = (float *)malloc(sizeof(float) * H);
    float cs[32], sn[32];
    orc_rmsn_1pw(x, w->ln_w, xn, H);
    orc_matvec(w->w_q, 0, xn, qg, nq * hd * 2, H);
    orc_matvec(w->w_k, 0, xn, k1, nkv * hd, H);
    orc_matvec(w->w_v, 0, xn, v1, nkv * hd, H);
    orc_rope_cos_sin(n_pos, cs, sn, 64, 10000000.0f, 1.0f);
    orc_gqa_cfg cfg = {nq, nkv, hd, 64, 0, w->q_norm_w, w->k_norm_w, kcache, vcache,
                       (size_t)nkv * hd, hd, (size_t)nkv * hd, hd};
    orc_gqa_token(&cfg, qg, 2 * hd, qg + hd, 2 * hd, k1, v1, n_pos, cs, sn, att);
    orc_matvec(w->w_o, 0, att, ao, H, nq * hd);
    for (int i = 0; i < H; i++) out[i] = x[i] + ao[i];
    free(xn); free(qg); free(k1); free(v1); free(att); free(ao);
}
