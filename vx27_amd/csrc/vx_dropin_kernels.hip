// Device forms of the reference's own mixer API (vx27_deltanet.h,
// vx27_gqa.h, vx27_rope.h): same arguments and sizes the reference accepts,
// on device pointers.  They serve the host-pointer drop-ins in vx27_dropin.c
// and any caller that keeps the reference's per-head calling pattern; the
// batched decode/prefill kernels are the fast path.
//
// Each lane owns one output element and walks the reduction in the
// reference's order, so the float/double roundings match the reference's
// (sums of squares are done serially by one lane for the same reason).
#include "vx_common.h"

namespace {

constexpr int MAXHD = 256;

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

// serial double sum of squares of x[0..n) (reference order), done by lane 0
__device__ double serial_ssq(const float *x, int n, double *slot) {
    if (threadIdx.x == 0) {
        double ss = 0.0;
        for (int i = 0; i < n; i++) ss = ss + (double)x[i] * (double)x[i];
        *slot = ss;
    }
    __syncthreads();
    return *slot;
}

// vx27_deltanet_step_exact (vx27_deltanet.c:71-102); block of hd threads
__global__ void step_exact_kernel(float *S, const float *q, const float *k, const float *v,
                                  double beta, double decay, float *o, int hd) {
    __shared__ float qn[MAXHD], kn[MAXHD];
    __shared__ double ss[2];
    const int j = threadIdx.x;
    const double sq = serial_ssq(q, hd, &ss[0]);
    const double sk = serial_ssq(k, hd, &ss[1]);
    const float iq = 1.0f / sqrtf((float)sq + 1e-6f), ik = 1.0f / sqrtf((float)sk + 1e-6f);
    const float qs = 1.0f / sqrtf((float)hd);
    qn[j] = (q[j] * iq) * qs;
    kn[j] = k[j] * ik;
    __syncthreads();
    double kv = 0.0;
    for (int i = 0; i < hd; i++) {
        const float sd = (float)((double)S[(size_t)i * hd + j] * decay);
        S[(size_t)i * hd + j] = sd;
        kv = kv + (double)sd * (double)kn[i];
    }
    const double dl = ((double)v[j] - kv) * beta;
    double acc = 0.0;
    for (int i = 0; i < hd; i++) {
        const float su = (float)((double)S[(size_t)i * hd + j] + (double)kn[i] * dl);
        S[(size_t)i * hd + j] = su;
        acc = acc + (double)su * (double)qn[i];
    }
    o[j] = (float)acc;
}

// vx27_deltanet_update_{ref,tiled} (variant 0: decay*S + k*v) and
// vx27_deltanet_update_avx2 (variant 1: fma(S, decay, k*v)); grid hd rows
__global__ void update_simple_kernel(float *S, const float *k, const float *v, float decay, int hd,
                                     int variant) {
    const int r = blockIdx.x;
    for (int c = threadIdx.x; c < hd; c += blockDim.x) {
        float *p = S + (size_t)r * hd + c;
        const float kv = k[r] * v[c];
        if (variant == 1) {
            *p = __builtin_fmaf(*p, decay, kv);
        } else {
            const float dec = decay * *p;
            *p = dec + kv;
        }
    }
}

// vx27_deltanet_retrieve_ref (0: serial float sum), _avx2 (1: serial fma),
// _tiled (2: 16-row partial sums added in row-block order)
__global__ void retrieve_simple_kernel(const float *S, const float *q, float *o, int hd, int variant) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= hd) return;
    float acc = 0.0f;
    if (variant == 2) {
        for (int r0 = 0; r0 < hd; r0 += 16) {
            float part = 0.0f;
            const int r1 = r0 + 16 < hd ? r0 + 16 : hd;
            for (int r = r0; r < r1; r++) part = part + S[(size_t)r * hd + c] * q[r];
            acc = acc + part;
        }
    } else if (variant == 1) {
        for (int r = 0; r < hd; r++) acc = __builtin_fmaf(S[(size_t)r * hd + c], q[r], acc);
    } else {
        for (int r = 0; r < hd; r++) acc = acc + S[(size_t)r * hd + c] * q[r];
    }
    o[c] = acc;
}

// vx27_deltanet_l2norm (vx27_deltanet.c:51-56)
__global__ void l2norm_kernel(const float *x, float *y, int n) {
    __shared__ double ss;
    const double s2 = serial_ssq(x, n, &ss);
    const float inv = 1.0f / sqrtf((float)s2 + 1e-6f);
    for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = x[i] * inv;
}

// vx27_rmsnorm (vx27_gqa.c:10-15)
__global__ void rmsnorm_kernel(const float *x, const float *w, float *y, int n, float eps) {
    __shared__ double ss;
    const double s2 = serial_ssq(x, n, &ss);
    const float s = 1.0f / sqrtf((float)(s2 / n) + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = (x[i] * s) * w[i];
}

// vx27_conv1d_step (vx27_deltanet.c:106-122), one thread per channel
__global__ void conv1d_kernel(float *state, const float *x, const float *w, float *y, int C, int silu) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    float *st = state + (size_t)c * 3;
    const float *wc = w + (size_t)c * 4;
    float acc = wc[0] * st[0];
    acc = acc + wc[1] * st[1];
    acc = acc + wc[2] * st[2];
    acc = acc + wc[3] * x[c];
    y[c] = silu ? silu_f(acc) : acc;
    st[0] = st[1];
    st[1] = st[2];
    st[2] = x[c];
}

// vx27_rope_apply (vx27_rope.c:18-29), one block per head
__global__ void rope_apply_kernel(float *v, int head_dim, int half, const float *cosv, const float *sinv) {
    float *p = v + (size_t)blockIdx.x * head_dim;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float a = p[i], b = p[i + half];
        p[i] = a * cosv[i] - b * sinv[i];
        p[i + half] = a * sinv[i] + b * cosv[i];
    }
}

// vx27_attn_1q (vx27_gqa.c:17-45): 24 Q / 4 KV heads, hd 256, fp32 caches
// [pos][4][256]; float dot in dim order, float softmax, float P.V in position
// order.  One block per Q head; sc is [24][n_pos] device scratch.
__global__ __launch_bounds__(256) void attn_1q_kernel(const float *q, const float *kc, const float *vc,
                                                      int n_pos, float *sc, float *out) {
    const int h = blockIdx.x, kvh = h * 4 / 24, hd = 256;
    const float *qh = q + (size_t)h * hd;
    const float scale = 1.0f / sqrtf((float)hd);
    float *s = sc + (size_t)h * n_pos;
    __shared__ float red[256];
    __shared__ float bc[2];
    float lmax = -1e30f;
    for (int p = threadIdx.x; p < n_pos; p += blockDim.x) {
        const float *kh = kc + ((size_t)p * 4 + kvh) * hd;
        float acc = 0.0f;
        for (int i = 0; i < hd; i++) acc = acc + qh[i] * kh[i];
        acc = acc * scale;
        s[p] = acc;
        lmax = acc > lmax ? acc : lmax;
    }
    red[threadIdx.x] = lmax;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = -1e30f;
        for (int t = 0; t < (int)blockDim.x; t++) m = red[t] > m ? red[t] : m;
        bc[0] = m;
    }
    __syncthreads();
    const float smax = bc[0];
    for (int p = threadIdx.x; p < n_pos; p += blockDim.x) s[p] = expf(s[p] - smax);
    __syncthreads();
    if (threadIdx.x == 0) {   // serial float sum, reference order
        float sum = 0.0f;
        for (int p = 0; p < n_pos; p++) sum = sum + s[p];
        bc[1] = sum;
    }
    __syncthreads();
    const float ssum = bc[1];
    const int i = threadIdx.x;
    float o = 0.0f;
    for (int p = 0; p < n_pos; p++) {
        const float wgt = s[p] / ssum;
        o = o + wgt * vc[((size_t)p * 4 + kvh) * hd + i];
    }
    out[(size_t)h * hd + i] = o;
}

}  // namespace

extern "C" int vx27_hip_step_exact(vx27_hip_ctx *ctx, float *S, const float *q, const float *k,
                                   const float *v, double beta, double decay, float *o, int hd) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(hd >= 1 && hd <= MAXHD, "vx27_hip_step_exact: hd must be in [1, 256] (got %d)", hd);
    VX_LAUNCH(ctx, step_exact_kernel, dim3(1), dim3(hd), S, q, k, v, beta, decay, o, hd);
    return 0;
}

extern "C" int vx27_hip_update_simple(vx27_hip_ctx *ctx, float *S, const float *k, const float *v,
                                      float decay, int hd, int variant) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(hd >= 1, "vx27_hip_update_simple: hd must be >= 1");
    VX_REQUIRE(variant == 0 || variant == 1, "vx27_hip_update_simple: variant 0 (ref) or 1 (fma)");
    VX_LAUNCH(ctx, update_simple_kernel, dim3(hd), dim3(128), S, k, v, decay, hd, variant);
    return 0;
}

extern "C" int vx27_hip_retrieve_simple(vx27_hip_ctx *ctx, const float *S, const float *q, float *o,
                                        int hd, int variant) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(hd >= 1, "vx27_hip_retrieve_simple: hd must be >= 1");
    VX_REQUIRE(variant >= 0 && variant <= 2, "vx27_hip_retrieve_simple: variant 0 (ref), 1 (fma), 2 (tiled)");
    VX_LAUNCH(ctx, retrieve_simple_kernel, dim3((hd + 127) / 128), dim3(128), S, q, o, hd,
                       variant);
    return 0;
}

extern "C" int vx27_hip_l2norm(vx27_hip_ctx *ctx, const float *x, float *y, int n) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(n >= 0, "vx27_hip_l2norm: n must be >= 0");
    if (n == 0) return 0;
    VX_LAUNCH(ctx, l2norm_kernel, dim3(1), dim3(256), x, y, n);
    return 0;
}

extern "C" int vx27_hip_rmsnorm(vx27_hip_ctx *ctx, const float *x, const float *w, float *y, int n, float eps) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(n >= 1, "vx27_hip_rmsnorm: n must be >= 1");
    VX_LAUNCH(ctx, rmsnorm_kernel, dim3(1), dim3(256), x, w, y, n, eps);
    return 0;
}

extern "C" int vx27_hip_conv1d_step(vx27_hip_ctx *ctx, float *state, const float *x, const float *w,
                                    float *y, int C, int apply_silu) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(C >= 0, "vx27_hip_conv1d_step: C must be >= 0");
    if (C == 0) return 0;
    VX_LAUNCH(ctx, conv1d_kernel, dim3((C + 255) / 256), dim3(256), state, x, w, y, C,
                       apply_silu ? 1 : 0);
    return 0;
}

extern "C" int vx27_hip_rope_apply(vx27_hip_ctx *ctx, float *v, int n_heads, int head_dim, int rope_dim,
                                   const float *cosv, const float *sinv) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(n_heads >= 0 && rope_dim >= 0 && rope_dim <= head_dim,
               "vx27_hip_rope_apply: need 0 <= rope_dim <= head_dim");
    if (n_heads == 0 || rope_dim < 2) return 0;
    VX_LAUNCH(ctx, rope_apply_kernel, dim3(n_heads), dim3(64), v, head_dim, rope_dim / 2,
                       cosv, sinv);
    return 0;
}

extern "C" int vx27_hip_attn_1q(vx27_hip_ctx *ctx, const float *q, const float *kcache, const float *vcache,
                                int n_pos, float *out) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(n_pos >= 1, "vx27_hip_attn_1q: n_pos must be >= 1");
    void *scr;
    if (vx_ctx_scratch(ctx, (size_t)24 * n_pos * sizeof(float), &scr)) return -1;
    VX_LAUNCH(ctx, attn_1q_kernel, dim3(24), dim3(256), q, kcache, vcache, n_pos,
                       (float *)scr, out);
    return 0;
}

extern "C" int vx27_hip_staging(vx27_hip_ctx *ctx, size_t bytes, void **dptr) {
    if (vx_ctx_enter(ctx)) return -1;
    return vx_ctx_stage(ctx, bytes, dptr);
}
