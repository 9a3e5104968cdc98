/*
 * vx27_rope.h -- the reference's partial RoPE API (src/vx27_rope.h:11-17).
 *
 * head_dim 256, rope_dim 64 (NeoX half split), theta 1e7; YaRN as a linear
 * position scale.  The cos/sin table functions are scalar per position and
 * are evaluated on the host with the reference's float formula (the batched
 * decode path evaluates its own table on the device from positions, see
 * vx27_hip_rope_table); vx27_rope_apply runs on the GPU.
 */
#ifndef VX27_ROPE_H
#define VX27_ROPE_H

#ifdef __cplusplus
extern "C" {
#endif

/* cos/sin of pos/yarn * theta^(-2i/rope_dim), i < rope_dim/2 (vx27_rope.c:5-16). */
void vx27_rope_cos_sin(int pos, float *cosv, float *sinv, int rope_dim,
                       float theta, float yarn_factor);
/* Rotate pairs (i, i+rope_dim/2) of each head's first rope_dim dims
 * (vx27_rope.c:18-29). */
void vx27_rope_apply(float *v, int n_heads, int head_dim, int rope_dim,
                     const float *cosv, const float *sinv);
/* Text-only M-RoPE == standard RoPE with rope_dim 64, theta 1e7 (vx27_rope.c:31-33). */
void vx27_mrope_cos_sin_text(int pos, float *cosv, float *sinv);

#ifdef __cplusplus
}
#endif
#endif
