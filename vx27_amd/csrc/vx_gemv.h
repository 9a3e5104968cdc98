// Internal interface of the skinny bf16 GEMM (vx_gemv.hip), shared with the
// kernels that produce its packed operand or fuse its reduction epilogue.
#pragma once
#include "vx_common.h"

// Split-K plan of the row-major path for an N x K GEMV: n_seg K segments of
// ks_per 32-wide k-steps; segments are combined four at a time inside a
// workgroup, so vx_gemv_pseg(n_seg) partial sets [N][16] fp32 are written.
int vx_gemv_plan(int N, int K, int *n_seg, int *ks_per);
int vx_gemv_pseg(int n_seg);
size_t vx_gemv_part_bytes(int N, int n_seg);
// Packed activations: vectors go in groups of VX_PACK_GV, each group one
// 16-column MFMA B operand (the three parts of its <= 5 vectors): layout
// [K/32 k-steps][groups][64 lanes][8] bf16.
constexpr int VX_PACK_GV = 5;
__host__ __device__ __forceinline__ int vx_pack_groups(int B) { return (B + VX_PACK_GV - 1) / VX_PACK_GV; }
size_t vx_pack_bytes(int K, int B);
// x [B][K] (row stride x_stride) -> packed MFMA B operand (three bf16 parts).
int vx_pack(vx27_hip_ctx *ctx, const float *x, size_t x_stride, int B, int K, uint16_t *packed);
// y[b*y_stride + n] = sum over k of W[n][k] x_b[k] for tiled W and a packed x
// of B vectors (any B: passes of up to three groups, 15 vectors, each
// streaming W once)
int vx_gemv_store(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const uint16_t *packed, int B, float *y,
                  size_t y_stride);

// Part p (0 = hi, 1 = mid, 2 = lo) of the exact three-way bf16 split of x:
// hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid); each difference
// is exact in fp32.
__device__ __forceinline__ uint16_t vx_bf16_part(float x, int p) {
    uint16_t h = vx_f32_to_bf16(x);
    for (int q = 0; q < p; q++) {
        x = x - vx_bf16_to_f32(h);
        h = vx_f32_to_bf16(x);
    }
    return h;
}

// Element k of vector b (of B) as the three parts of the packed operand:
// group j = b / 5 holds its Bj <= 5 vectors' part p of vector b' at column
// p*Bj + b'.
__device__ __forceinline__ void vx_pack_store(uint16_t *packed, int B, int b, int k, float x) {
    const int G = vx_pack_groups(B), j = b / VX_PACK_GV, bl = b - VX_PACK_GV * j;
    const int Bj = min(VX_PACK_GV, B - VX_PACK_GV * j);
    const size_t base = (((size_t)(k >> 5) * G + j) * 64 + ((k >> 3) & 3) * 16) * 8 + (k & 7);
    uint16_t h = vx_f32_to_bf16(x);
    packed[base + (size_t)bl * 8] = h;
    x = x - vx_bf16_to_f32(h);
    h = vx_f32_to_bf16(x);
    packed[base + (size_t)(Bj + bl) * 8] = h;
    x = x - vx_bf16_to_f32(h);
    packed[base + (size_t)(2 * Bj + bl) * 8] = vx_f32_to_bf16(x);
}

// Sums of the partials of row n for each vector b < B (three parts):
// partial sets in order, parts hi + mid + lo within a set.
template <int B>
__device__ __forceinline__ void vx_gemv_sum_row_t(const float *part, int N, int n_pseg, int n, float *acc) {
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = 0.0f;
    for (int s = 0; s < n_pseg; s++) {
        const float4 *p4 = (const float4 *)(part + ((size_t)s * N + n) * 16);
        const float4 c0 = p4[0], c1 = p4[1], c2 = p4[2], c3 = p4[3];
        const float c[16] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w,
                             c2.x, c2.y, c2.z, c2.w, c3.x, c3.y, c3.z, c3.w};
#pragma unroll
        for (int b = 0; b < B; b++) acc[b] += (c[b] + c[B + b]) + c[2 * B + b];
    }
}
__device__ __forceinline__ void vx_gemv_sum_row(const float *part, int N, int B, int n_pseg, int n,
                                                float *acc) {
    switch (B) {
        case 1: vx_gemv_sum_row_t<1>(part, N, n_pseg, n, acc); break;
        case 2: vx_gemv_sum_row_t<2>(part, N, n_pseg, n, acc); break;
        case 3: vx_gemv_sum_row_t<3>(part, N, n_pseg, n, acc); break;
        case 4: vx_gemv_sum_row_t<4>(part, N, n_pseg, n, acc); break;
        default: vx_gemv_sum_row_t<5>(part, N, n_pseg, n, acc); break;
    }
}
