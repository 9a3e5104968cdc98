// Internal interface of the skinny bf16 GEMM (vx_gemv.hip), shared with the
// layer kernels that fuse their own reduction epilogues.
#pragma once
#include "vx_common.h"

// Split-K plan for an N x K GEMV: n_seg K segments of ks_per 32-wide k-steps.
int vx_gemv_plan(int N, int K, int *n_seg, int *ks_per);
size_t vx_gemv_part_bytes(int N, int n_seg);
size_t vx_pack_bytes(int K);
// x [B][K] (row stride x_stride) -> packed MFMA B operand with P bf16 parts.
int vx_pack(vx27_hip_ctx *ctx, const float *x, size_t x_stride, int B, int P, int K, uint16_t *packed);
// partial sums [n_seg][N][16] of W [N][K] bf16 times the packed operand
int vx_gemv_part(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const uint16_t *packed, int n_seg,
                 int ks_per, float *part);
// y[b*y_stride + n] = sum of partials (P parts of vector b)
int vx_gemv_reduce_store(vx27_hip_ctx *ctx, const float *part, int N, int B, int P, int n_seg, float *y,
                         size_t y_stride);

// Sum of the partials of output (n, b): segments in order, parts in order
// within a segment.
__device__ __forceinline__ float vx_gemv_sum(const float *part, int N, int B, int P, int n_seg, int n, int b) {
    float acc = 0.0f;
    for (int s = 0; s < n_seg; s++) {
        const float *p = part + ((size_t)s * N + n) * 16 + b;
        float v = p[0];
        for (int q = 1; q < P; q++) v += p[q * B];
        acc += v;
    }
    return acc;
}
