// Skinny bf16 GEMM (the mixer projections) on gfx950 MFMA.
//
// y[b][n] = sum_k W[n][k] * x[b][k] for B activation vectors (decode: one
// token per sequence), W bf16 [N][K] (the reference's weight tensors,
// vx27_pmat.h:6-8), x and y fp32.
//
// The fp32 activations enter the MFMA exactly: each x is split into three
// bf16 parts hi + mid + lo (8 mantissa bits each, 24 in all), and the parts
// of up to 5 vectors are the columns of one MFMA B operand (3*5 <= 15 of the
// 16 columns): one v_mfma_f32_16x16x32_bf16 multiplies 16 weight rows by
// every part of 5 vectors; the products are exact in fp32 and the only
// rounding is the fp32 accumulation, as in a plain fp32 dot product.  More
// vectors go in more such groups: a weight tile loaded once feeds one MFMA
// per group, up to 13 groups (65 vectors) per pass over the weights.
// Output column n of an MFMA depends only on operand column n, so operand
// columns >= 3*B may hold anything: they feed output columns nobody reads.
//
// Layouts:
//   packed activations  [K/32 k-steps][groups][64 lanes][8] bf16: lane (g,n)
//                       of group j (its Bj <= 5 vectors 5j..) at k-step s
//                       holds part n/Bj of vector 5j + n%Bj at k = 32s + 8g + 0..7
//   tiled weights       [K/(32 KG) k-groups][N/16 row blocks][KG][64 lanes][8]
//                       bf16 (KG = 1 by default): lane (g,m) of tile (s, rb)
//                       holds W[16*rb + m][32s + 8g + 0..7].  A wave's A
//                       operand is 1 KiB contiguous and the row blocks of a
//                       k-step are adjacent (a 1 MiB slab for N = 16K rows)
//                       (vx27_hip_pack_weights_bf16 converts row-major W)
//
// Both layouts go through gemv_wk_store (vx_gemv_body.h): whole-K
// workgroups with the wave partials reduced in LDS, reading the weights once
// for up to 65 vectors.  Row-major weights (the plain vx27_hip_gemv_bf16
// call) are read as 16 rows x 64 bytes per tile.
#include <algorithm>

#include "vx_gemv_body.h"

namespace {


// pack activations: grid (K/32, groups), block 64; lane (g,n) of group j
// writes its 8 elements
__global__ __launch_bounds__(64) void pack_x(const float *x, size_t x_stride, int B, uint16_t *out) {
    const int s = blockIdx.x, j = blockIdx.y, lane = threadIdx.x, g = lane >> 4, n = lane & 15;
    const int Bj = min(VX_PACK_GV, B - VX_PACK_GV * j);
    if (n >= 3 * Bj) return;   // padding columns feed unread output columns
    const int p = n / Bj, b = VX_PACK_GV * j + n % Bj;
    const float *xr = x + (size_t)b * x_stride + 32 * s + 8 * g;
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = vx_bf16_part(xr[e], p);

    uint4 w;
    w.x = v[0] | ((uint32_t)v[1] << 16);
    w.y = v[2] | ((uint32_t)v[3] << 16);
    w.z = v[4] | ((uint32_t)v[5] << 16);
    w.w = v[6] | ((uint32_t)v[7] << 16);
    *(uint4 *)(out + (((size_t)s * gridDim.y + j) * 64 + lane) * 8) = w;
}

// row-major W [N][K] -> tiled; grid (N/16, K/32), block 64
__global__ __launch_bounds__(64) void pack_w(const uint16_t *W, int K, uint16_t *Wt) {
    const int rb = blockIdx.x, s = blockIdx.y, lane = threadIdx.x, g = lane >> 4, m = lane & 15;
    const uint4 v = *(const uint4 *)(W + (size_t)(16 * rb + m) * K + 32 * s + 8 * g);
    *(uint4 *)(Wt + vx_tile_off(s, rb, gridDim.x, vx_gemv_kg(K)) + lane * 8) = v;
}

template <int RB, int G>
__global__ __launch_bounds__(VX_WK_NW * 64) void gemv_wk_store(WkWeights wt, int N, int K, const uint16_t *xp,
                                                              int Gt, int g0, int B, int halves, WkStore epi) {
    vx_gemv_wk_body<RB, G>(wt, N, K, xp, Gt, g0, B, halves, epi);
}

}  // namespace

WkPlan vx_gemv_wk_plan(int N, int K, int n_cu, int G, bool allow_halves) {
    (void)K;
    const int nb = N / 16;
    WkPlan best = {0, G, 0, 1};
    double best_t = 0.0;
    for (int single = 1; single >= 0 && best.rb == 0; single--)
        for (int halves = 1; halves <= (allow_halves ? 2 : 1); halves++)
            for (int rb = 1; rb <= vx_wk_max_rb(G); rb++) {
                const int wgs = halves * ((nb + rb - 1) / rb);
                if (single && wgs > n_cu) continue;
                // CU time ~ rounds x (rb weight tiles + G operand tiles per
                // k-step, an operand tile from L2 costing about a quarter of
                // a weight tile from HBM) x the share of the k-steps; ties
                // keep whole workgroups, then the smaller rb
                const double t = (double)((wgs + n_cu - 1) / n_cu) * (rb + 0.25 * G) / halves;
                if (best.rb == 0 || t < best_t - 1e-9) {
                    best_t = t;
                    best = {rb, G, wgs, halves};
                }
            }
    return best;
}

int vx_gemv_store(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const uint16_t *packed, int B, float *y,
                  size_t y_stride, bool y_zeroed) {
    VX_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0 && B >= 1,
               "gemv: N must be a multiple of 16, K of 32, B >= 1 (N=%d K=%d B=%d)", N, K, B);
    const int Gt = vx_pack_groups(B);
    for (int g0 = 0; g0 < Gt; g0 += VX_PASS_G) {   // one pass up to 13 groups (65 vectors)
        const int b0 = g0 * VX_PACK_GV, G = vx_pass_groups(B, b0);
        const int Bp = std::min(B - b0, G * VX_PACK_GV);
        const WkPlan p = vx_gemv_wk_plan(N, K, ctx->n_cu, G, y_zeroed);
        VX_WK_DISPATCH(ctx, gemv_wk_store, p, (WkWeights{W, 0}), N, K, packed, Gt, g0, Bp, p.halves,
                       (WkStore{y, y_stride, b0}));
    }
    return 0;
}

size_t vx_pack_bytes(int K, int B) {
    return (size_t)(K / 32) * vx_pack_groups(B) * 64 * 8 * sizeof(uint16_t);
}

int vx_pack(vx27_hip_ctx *ctx, const float *x, size_t x_stride, int B, int K, uint16_t *packed) {
    VX_REQUIRE(B >= 1 && K % 32 == 0, "pack: need B >= 1, K %% 32 == 0");
    VX_LAUNCH(ctx, pack_x, dim3(K / 32, vx_pack_groups(B)), dim3(64), x, x_stride, B, packed);
    return 0;
}

extern "C" int vx27_hip_pack_weights_bf16(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, uint16_t *Wt) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(W && Wt && W != Wt, "vx27_hip_pack_weights_bf16: need distinct source and destination");
    VX_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0,
               "vx27_hip_pack_weights_bf16: N must be a multiple of 16 and K of 32");
    VX_LAUNCH(ctx, pack_w, dim3(N / 16, K / 32), dim3(64), W, K, Wt);
    return 0;
}

extern "C" int vx27_hip_gemv_bf16(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x,
                                  size_t x_stride, int B, float *y, size_t y_stride) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(W && x && y, "vx27_hip_gemv_bf16: null pointer");
    VX_REQUIRE(B >= 1, "vx27_hip_gemv_bf16: B must be >= 1 (got %d)", B);
    VX_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0,
               "vx27_hip_gemv_bf16: N must be a multiple of 16 and K of 32 (N=%d K=%d)", N, K);
    // one pass over W per 13 groups (65 vectors), each packing its vectors
    const int Bp0 = std::min(B, VX_PASS_G * VX_PACK_GV);
    void *scr;
    if (vx_ctx_scratch(ctx, vx_pack_bytes(K, Bp0), &scr)) return -1;
    uint16_t *packed = (uint16_t *)scr;
    for (int b0 = 0; b0 < B; b0 += VX_PASS_G * VX_PACK_GV) {
        const int Bp = std::min(B - b0, VX_PASS_G * VX_PACK_GV), G = vx_pack_groups(Bp);
        if (vx_pack(ctx, x + (size_t)b0 * x_stride, x_stride, Bp, K, packed)) return -1;
        const WkPlan p = vx_gemv_wk_plan(N, K, ctx->n_cu, G);
        VX_WK_DISPATCH(ctx, gemv_wk_store, p, (WkWeights{W, 1}), N, K, packed, G, 0, Bp, p.halves,
                       (WkStore{y, y_stride, b0}));
    }
    return 0;
}
