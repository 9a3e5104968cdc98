/*
 * vx27_gqa.h -- the reference's gated-GQA helpers, served by the GPU.
 *
 * Same declarations as the reference's src/vx27_gqa.h:8-13, exported by
 * libvx27_hip (host buffers staged to the device; no host fallback).  The
 * reference's real attention is inline in vx27_qlayer (vx27_qfwd.c:186-211);
 * its GPU form, batched over sequences with a bf16 KV cache, is
 * vx27_hip_gqa_decode in vx27_hip.h.
 */
#ifndef VX27_GQA_H
#define VX27_GQA_H

#ifdef __cplusplus
extern "C" {
#endif

/* KV head of query head h for 24 Q / 4 KV heads: h*4/24 (vx27_gqa.c:6-8). */
int vx27_gqa_kv_for_q(int q_head);

/* y = x / sqrtf(mean(x^2) + eps) * w, sum in double (vx27_gqa.c:10-15). */
void vx27_rmsnorm(const float *x, const float *w, float *y, int n, float eps);

/* Single-query attention of one layer (vx27_gqa.c:17-45): q [24*256],
 * caches [n_pos][4][256] fp32, out [24*256], scale 1/16, float dot products.
 * The reference's 1024-position cap and static scratch are lifted here: any
 * n_pos >= 1, and the function is thread-safe (the library serialises
 * concurrent drop-in calls on its default context). */
void vx27_attn_1q(const float *q, const float *kcache, const float *vcache, int n_pos,
                  float *out);

#ifdef __cplusplus
}
#endif
#endif
