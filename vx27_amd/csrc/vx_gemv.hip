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
// per group, up to 3 groups (15 vectors) per pass over the weights.
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
// Tiled weights (the layer entry points): gemv_wk_store, whole-K workgroups
// with the reduction in LDS (vx_gemv_body.h).  Row-major weights (the plain
// vx27_hip_gemv_bf16 call): gemv_part_rm, 4-wave workgroups of 64 rows over
// K segments, partial sums [pseg][N][16] reduced by gemv_reduce_store in a
// fixed order.
#include <algorithm>

#include "vx_gemv_body.h"

namespace {

constexpr int RB = 4;   // row blocks per workgroup of the row-major path
#ifndef VX_GEMV_WAVES
#define VX_GEMV_WAVES 2048   // target waves per launch (row-major path)
#endif
#ifndef VX_GEMV_MINKS
#define VX_GEMV_MINKS 8      // at least this many 32-wide k-steps per wave
#endif

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

template <int RBW, bool NT, int G>
__global__ __launch_bounds__(1024) void gemv_wk_store(const uint16_t *W, int N, int K, const uint16_t *xp, int Gt,
                                                      int g0, int B, WkStore epi) {
    vx_gemv_wk_body<RBW, NT, G>(W, N, K, xp, Gt, g0, B, epi);
}

// Row-major W: grid (ceil(N/64), ceil(n_seg/4)), block 256; wave w takes K
// segment 4*blockIdx.y + w of its workgroup's 64 rows; the four segments are
// summed in LDS and one partial set [64][16] is written per workgroup.
__global__ __launch_bounds__(256) void gemv_part_rm(const uint16_t *W, int N, int K, const uint16_t *xp,
                                                    int ks_per, int n_seg, float *part) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, m = lane & 15;
    const int seg = blockIdx.y * 4 + wave;
    const int rb0 = blockIdx.x * RB;
    const int nks = K / 32;
    const int s0 = seg * ks_per, s1 = seg < n_seg ? min(nks, s0 + ks_per) : s0;
    __shared__ vx_floatx4_t red[4][RB][64];
    vx_floatx4_t acc[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) acc[r] = (vx_floatx4_t){0.f, 0.f, 0.f, 0.f};
    bool live[RB];
    const uint16_t *wp[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) {
        live[r] = (rb0 + r) * 16 < N;          // whole 16-row block in or out (N % 16 == 0)
        wp[r] = W + (size_t)(16 * (live[r] ? rb0 + r : 0) + m) * K + 8 * g;
    }
    const vx_bf16x8_t *xb = (const vx_bf16x8_t *)xp + lane;
    for (int s = s0; s < s1; s++) {
        const vx_bf16x8_t bop = xb[(size_t)s * 64];
        vx_bf16x8_t aop[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) aop[r] = *(const vx_bf16x8_t *)(wp[r] + (size_t)s * 32);
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[r], bop, acc[r], 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < RB; r++) red[wave][r][lane] = acc[r];
    __syncthreads();
    // wave w sums the four segments of row block w in segment order
    const int r = wave;
    if (!live[r]) return;
    vx_floatx4_t v = red[0][r][lane];
    v += red[1][r][lane];
    v += red[2][r][lane];
    v += red[3][r][lane];
    // lane (g,m) holds C[4g+i][m]: row 16*(rb0+r) + 4g + i, column m
#pragma unroll
    for (int i = 0; i < 4; i++) part[((size_t)blockIdx.y * N + 16 * (rb0 + r) + 4 * g + i) * 16 + m] = v[i];
}

// plain reduction, one thread per row: y[b*y_stride + n] for b < B
__global__ __launch_bounds__(256) void gemv_reduce_store(const float *part, int N, int B, int n_pseg,
                                                         float *y, size_t y_stride) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    float acc[5];
    vx_gemv_sum_row(part, N, B, n_pseg, n, acc);
    for (int b = 0; b < B; b++) y[(size_t)b * y_stride + n] = acc[b];
}

}  // namespace

#ifndef VX_GEMV_NT_MIB
#define VX_GEMV_NT_MIB 32   // matrices of at least this many MiB are read with streaming loads
#endif
WkPlan vx_gemv_wk_plan(int N, int K, int n_cu, int G) {
    const int nb = N / 16;
    const int max_rb = VX_WK_MAX_RB / G;   // RB x G accumulator tiles (LDS reduction space)
    WkPlan p;
    p.g = G;
    p.rb = max_rb;
    for (int rb = 1; rb <= max_rb; rb++)
        if ((nb + rb - 1) / rb <= n_cu) {
            p.rb = rb;
            break;
        }
    p.grid = (nb + p.rb - 1) / p.rb;
    // streaming loads pay off on matrices read once between other traffic
    // (every projection of a decode step); small ones may stay cached
    p.nt = (size_t)N * K * 2 >= ((size_t)VX_GEMV_NT_MIB << 20);
    return p;
}

int vx_gemv_store(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const uint16_t *packed, int B, float *y,
                  size_t y_stride) {
    VX_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0 && B >= 1,
               "gemv: N must be a multiple of 16, K of 32, B >= 1 (N=%d K=%d B=%d)", N, K, B);
    const int Gt = vx_pack_groups(B);
    for (int g0 = 0; g0 < Gt; g0 += 3) {   // passes of up to three groups (15 vectors)
        const int G = std::min(3, Gt - g0), b0 = g0 * VX_PACK_GV;
        const int Bp = std::min(B - b0, G * VX_PACK_GV);
        const WkPlan p = vx_gemv_wk_plan(N, K, ctx->n_cu, G);
        VX_WK_DISPATCH(ctx, gemv_wk_store, p, W, N, K, packed, Gt, g0, Bp, (WkStore{y, y_stride, b0}));
    }
    return 0;
}

int vx_gemv_plan(int N, int K, int *n_seg, int *ks_per) {
    VX_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0,
               "gemv: N must be a multiple of 16 and K of 32 (N=%d K=%d)", N, K);
    const int groups = (N + 16 * RB - 1) / (16 * RB);
    const int nks = K / 32;
    // about VX_GEMV_WAVES waves in all, at least VX_GEMV_MINKS k-steps per wave
    int seg = (VX_GEMV_WAVES + groups - 1) / groups;
    if (seg > nks / VX_GEMV_MINKS) seg = nks / VX_GEMV_MINKS;
    if (seg < 1) seg = 1;
    const int per = (nks + seg - 1) / seg;
    *n_seg = (nks + per - 1) / per;
    *ks_per = per;
    return 0;
}

int vx_gemv_pseg(int n_seg) { return (n_seg + 3) / 4; }
size_t vx_gemv_part_bytes(int N, int n_seg) { return (size_t)vx_gemv_pseg(n_seg) * N * 16 * sizeof(float); }
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
    int n_seg, ks_per;
    if (vx_gemv_plan(N, K, &n_seg, &ks_per)) return -1;
    const size_t pk = (vx_pack_bytes(K, VX_PACK_GV) + 255) & ~(size_t)255;
    void *scr;
    if (vx_ctx_scratch(ctx, pk + vx_gemv_part_bytes(N, n_seg), &scr)) return -1;
    uint16_t *packed = (uint16_t *)scr;
    float *part = (float *)((char *)scr + pk);
    // passes of up to 5 vectors (one packed group each)
    for (int b0 = 0; b0 < B; b0 += VX_PACK_GV) {
        const int Bp = std::min(VX_PACK_GV, B - b0);
        if (vx_pack(ctx, x + (size_t)b0 * x_stride, x_stride, Bp, K, packed)) return -1;
        const dim3 grid((N + 16 * RB - 1) / (16 * RB), vx_gemv_pseg(n_seg));
        VX_LAUNCH(ctx, gemv_part_rm, grid, dim3(256), W, N, K, packed, ks_per, n_seg, part);
        VX_LAUNCH(ctx, gemv_reduce_store, dim3((N + 255) / 256), dim3(256), part, N, Bp, vx_gemv_pseg(n_seg),
                  y + (size_t)b0 * y_stride, y_stride);
    }
    return 0;
}
