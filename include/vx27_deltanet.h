/*
 * vx27_deltanet.h -- the reference's Gated DeltaNet API, served by the GPU.
 *
 * Same declarations as the reference's src/vx27_deltanet.h:10-59; each is
 * exported by libvx27_hip and replaces the reference function of the same
 * name (cited per declaration).  Buffers are caller-owned host memory, as in
 * the reference: the library stages them to the device, runs the kernel and
 * copies results back before returning.  On a device error the call aborts
 * with a message (or, with vx27_hip_set_error_mode(VX27_HIP_ERR_POISON),
 * fills its outputs with NaN); there is no host fallback.
 * Batched, device-resident calls are in vx27_hip.h (vx27_hip_dn_decode).
 */
#ifndef VX27_DELTANET_H
#define VX27_DELTANET_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* State sizing of the model: 16 QK heads x 128 x 128 per layer, 48 linear
 * layers (vx27_deltanet.c:5-13). */
int vx27_deltanet_state_per_layer(void);
int vx27_deltanet_state_total(void);
double vx27_deltanet_state_mb(int bytes_per_elem);

/* Simplified decayed outer product S = decay*S + k v^T and o = S^T q on one
 * row-major hd x hd state (vx27_deltanet.c:15-49, vx27_deltanet_avx2.c:6-45).
 * _ref/_tiled: separate multiply and add; _avx2: fused multiply-add. */
void vx27_deltanet_update_ref(float *S, const float *k, const float *v, float decay, int hd);
void vx27_deltanet_retrieve_ref(const float *S, const float *q, float *o, int hd);
void vx27_deltanet_update_tiled(float *S, const float *k, const float *v, float decay, int hd);
void vx27_deltanet_retrieve_tiled(const float *S, const float *q, float *o, int hd);
void vx27_deltanet_update_avx2(float *S, const float *k, const float *v, float decay, int hd);
void vx27_deltanet_retrieve_avx2(const float *S, const float *q, float *o, int hd);

/* y = x / sqrtf(sum x^2 + 1e-6), sum in double (vx27_deltanet.c:51-56). */
void vx27_deltanet_l2norm(const float *x, float *y, int n);

/* One exact gated delta-rule step of one value head (vx27_deltanet.c:71-102):
 * q,k l2-normalised, q scaled by 1/sqrt(hd); S *= exp(g_log);
 * kv = S^T k; S += k (x) (v - kv)*beta; o = S^T q.  S row-major [hd][hd],
 * updated in place; hd <= 256. */
void vx27_deltanet_step_exact(float *S, const float *q, const float *k, const float *v,
                              double beta, double g_log, float *o, int hd);

/* beta = sigmoid(b); g_log = -exp(A_log) * softplus(a + dt_bias)
 * (vx27_deltanet.c:58-69).  Scalar; evaluated on the host. */
void vx27_deltanet_gate_params(double a, double A_log, double b, double dt_bias,
                               double *beta, double *g_log);

/* Depthwise causal conv, width 4, over C channels, state [C][3] oldest first,
 * weights [C][4] with tap 3 the newest, optional SiLU (vx27_deltanet.c:106-122). */
void vx27_conv1d_step(float *state, const float *x, const float *w, float *y,
                      int C, int apply_silu);

#ifdef __cplusplus
}
#endif
#endif
