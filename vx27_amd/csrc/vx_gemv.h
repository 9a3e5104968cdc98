// Internal interface of the skinny bf16 GEMM (vx_gemv.hip), shared with the
// kernels that produce its packed operand or fuse its reduction epilogue.
#pragma once
#include "vx_common.h"

// Packed activations: vectors go in groups of VX_PACK_GV, each group one
// 16-column MFMA B operand (the three parts of its <= 5 vectors): layout
// [K/32 k-steps][groups][64 lanes][8] bf16.
// Above three groups the count is rounded up to 4, 7, 10 or 13 (one GEMV
// pass covers up to 65 vectors; larger batches take whole multiples of 13):
// the padding groups are never written and feed output columns nobody reads.
constexpr int VX_PACK_GV = 5;
constexpr int VX_PASS_G = 13;   // most groups per pass over the weights
// groups of a pass holding the g <= VX_PASS_G groups that have vectors
__host__ __device__ __forceinline__ int vx_round_groups(int g) {
    return g <= 3 ? g : g <= 4 ? 4 : g <= 7 ? 7 : g <= 10 ? 10 : 13;
}

__host__ __device__ __forceinline__ int vx_pack_groups(int B) {
    const int g = (B + VX_PACK_GV - 1) / VX_PACK_GV;
    return g <= VX_PASS_G ? vx_round_groups(g) : (g + VX_PASS_G - 1) / VX_PASS_G * VX_PASS_G;
}
// groups of the pass that starts at vector b0 of B (its last group may be
// followed by padding groups of the layout that the pass skips)
__host__ __device__ __forceinline__ int vx_pass_groups(int B, int b0) {
    const int g = (B - b0 + VX_PACK_GV - 1) / VX_PACK_GV;
    return vx_round_groups(g < VX_PASS_G ? g : VX_PASS_G);
}
size_t vx_pack_bytes(int K, int B);
// x [B][K] (row stride x_stride) -> packed MFMA B operand (three bf16 parts).
int vx_pack(vx27_hip_ctx *ctx, const float *x, size_t x_stride, int B, int K, uint16_t *packed);
// y[b*y_stride + n] = sum over k of W[n][k] x_b[k] for tiled W and a packed x
// of B vectors (one pass over W for up to 65 vectors; passes of 13 groups
// beyond).  Each row's sum order is the same for any B.  y_zeroed: y holds
// zeros (written by an earlier kernel on the stream), so the rows may be
// added in two halves.
int vx_gemv_store(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const uint16_t *packed, int B, float *y,
                  size_t y_stride, bool y_zeroed = false);

// The projection of R tokens at once (vx_gemm.hip): y[r][n] = sum over k of
// W[n][k] x_r[k] for tiled W, fp32 x rows (x as two bf16 parts; K % 64 == 0,
// 16-byte aligned rows).
// ws: vx_gemm_ws_bytes of device scratch (the tokens packed for the MFMAs,
// and the partial sums of a last round of tiles split along k)
int vx_gemm_store(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x, size_t x_stride, int R,
                  float *y, size_t y_stride, void *ws);
size_t vx_gemm_ws_bytes(int N, int K, int R, int n_cu);
// whether vx_gemm_store takes this shape (else the GEMV passes)
bool vx_gemm_fits(int N, int K, int R, const float *x, size_t x_stride, const float *y, size_t y_stride);
// Output in segments: rows n >= 16 rb0 of segment s (up to the next
// segment's) go to p[r * stride + n - 16 rb0], as fp32 or as bf16 (round to
// nearest even, vx_f32_to_bf16).  Segment 0 starts at rb0 = 0.
struct GemmSeg {
    int rb0, bf16;
    size_t stride;
    void *p;
};
constexpr int VX_GEMM_SEGS = 4;
struct GemmOut {
    int n;
    GemmSeg s[VX_GEMM_SEGS];
};
int vx_gemm_store_seg(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x, size_t x_stride, int R,
                      const GemmOut &out, void *ws);
bool vx_gemm_fits_seg(int N, int K, int R, const float *x, size_t x_stride, const GemmOut &out);
constexpr int VX_GEMM_MIN_ROWS = 256;   // layer prefills use the GEMM from this many tokens (one token tile)
// The GEMM's packed tokens: one 32 KiB image per (256-token tile, 32-wide
// k-step), [token tiles][K/32][32 KiB].  In an image, part p (0: hi =
// bf16(x), 1: lo = bf16(x - hi)) of token t's elements 8g .. 8g+7 sit in
// 1 KiB block ((t % 256) / 16) * 2 + p, 16-byte unit g * 16 + ((t % 16) ^ 2g)
// (the XOR spreads a token column over the LDS banks).  Byte offset of the
// hi unit holding element k of token t (its lo unit: + 1024):
__host__ __device__ __forceinline__ size_t vx_gemm_pack_unit(int t, int k, int K) {
    const int tb = (t >> 4) & 15, n = t & 15, g = (k >> 3) & 3;
    return ((size_t)(t >> 8) * (K >> 5) + (k >> 5)) * 32768 + (size_t)tb * 2048 + (size_t)(g * 16 + (n ^ (g << 1))) * 16;
}
size_t vx_gemm_pack_bytes(int K, int R);
// vx_gemm_store_seg on tokens already packed (xp: vx_gemm_pack_bytes, rows
// past R may hold anything: they feed only outputs that are not stored);
// ws: vx_gemm_ws_bytes.
int vx_gemm_store_packed(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const char *xp, int R,
                         const GemmOut &out, void *ws);

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
