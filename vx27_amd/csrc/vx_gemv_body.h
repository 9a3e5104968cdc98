// Whole-K workgroup GEMV for the tiled weight layout (vx_gemv.hip), shared
// with the kernels that put their own epilogue after it (vx_layer.hip).
//
// A workgroup of 16 waves owns RB row blocks (16 RB rows) over all of K:
// wave w takes the k-steps w, w + 16, ... (so the waves of a workgroup read
// neighbouring 1 MiB k-step slabs of the tiled weights at any moment), the
// 16 wave partials are summed in LDS in wave order, then the three bf16
// parts of each vector (hi + mid + lo), and the epilogue gets whole rows:
// no split-K partials in memory and no second kernel.  The host picks the
// smallest RB that keeps the launch to one workgroup per CU (a launch with
// some CUs running two workgroups takes about as long as two launches).
#pragma once
#include "vx_gemv.h"

typedef __bf16 vx_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float vx_floatx4_t __attribute__((ext_vector_type(4)));

constexpr int VX_WK_WAVES = 16;   // waves per workgroup (K split)
constexpr int VX_WK_MAX_RB = 8;
#ifndef VX_GEMV_KG
#define VX_GEMV_KG 1              // k-steps per group of the tiled layout (1, 2 or 4)
#endif

// k-steps per group of the tiled weight layout
__host__ __device__ __forceinline__ int vx_gemv_kg(int K) {
    const int nks = K / 32;
    return nks % VX_GEMV_KG == 0 ? VX_GEMV_KG : 1;
}
// element offset of tile (k-step s, row block rb) in the tiled layout
__device__ __forceinline__ size_t vx_tile_off(int s, int rb, int nb, int kg) {
    return ((size_t)(s / kg) * nb + rb) * kg * 512 + (size_t)(s % kg) * 512;
}

// Summed rows handed to an epilogue: y(r, b) for local row r < rows and
// vector b < B of the pass (its groups g0 .. g0+G-1 of the packed operand).
template <int RB, int G>
struct WkRows {
    const float (*c)[16 * G + 1];   // [16 RB][16 G + 1]: the MFMA output columns of the G groups
    int B;                          // vectors in this pass (<= 5 G)
    __device__ __forceinline__ float y(int r, int b) const {
        const int j = b / VX_PACK_GV, bl = b - VX_PACK_GV * j, Bj = min(VX_PACK_GV, B - VX_PACK_GV * j);
        const float *cr = c[r] + 16 * j;
        return (cr[bl] + cr[Bj + bl]) + cr[2 * Bj + bl];
    }
};

// Epilogue interface, both called by all 1024 threads (rows = valid rows
// from row0, <= 16 RB):
//   Pre prefetch(int row0, int rows, int tid) const      before the K loop:
//       issues the loads the epilogue needs besides the sums (their latency
//       then hides under the loop instead of trailing it)
//   void operator()(int row0, int rows, const WkRows<RB, G> &, int tid, const Pre &) const
// One pass covers the B vectors of groups g0 .. g0+G-1 of a packed operand
// with Gt groups in all.
template <int RB, bool NT, int G, class Epi>
__device__ __forceinline__ void vx_gemv_wk_body(const uint16_t *W, int N, int K, const uint16_t *xp, int Gt, int g0,
                                                int B, const Epi &epi) {
    constexpr int NW = VX_WK_WAVES;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb0 = blockIdx.x * RB, nb = N / 16;
    const int nks = K / 32, kg = vx_gemv_kg(K);
    const int row0 = rb0 * 16;
    const int rows = min(16 * RB, N - row0);
    const auto pre = epi.prefetch(row0, rows, tid);
    vx_floatx4_t acc[RB][G];
#pragma unroll
    for (int r = 0; r < RB; r++)
#pragma unroll
        for (int j = 0; j < G; j++) acc[r][j] = (vx_floatx4_t){0.f, 0.f, 0.f, 0.f};
    const uint16_t *wp[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) {
        const int rb = rb0 + r < nb ? rb0 + r : 0;   // dead blocks re-read block 0, never stored
        wp[r] = W + vx_tile_off(0, rb, nb, kg) + lane * 8;
    }
    const vx_bf16x8_t *xb = (const vx_bf16x8_t *)xp + (size_t)g0 * 64 + lane;
    const size_t gstride = (size_t)nb * kg * 512;
    for (int s = wave; s < nks; s += NW) {
        vx_bf16x8_t bop[G];
#pragma unroll
        for (int j = 0; j < G; j++) bop[j] = xb[((size_t)s * Gt + j) * 64];
        const size_t off = (size_t)(s / kg) * gstride + (size_t)(s % kg) * 512;
        vx_bf16x8_t aop[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const vx_bf16x8_t *a = (const vx_bf16x8_t *)(wp[r] + off);
            aop[r] = NT ? __builtin_nontemporal_load(a) : *a;
        }
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int j = 0; j < G; j++)
                acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[r], bop[j], acc[r][j], 0, 0, 0);
    }
    __shared__ vx_floatx4_t red[NW][RB * G][64];
    __shared__ float ct[16 * RB][16 * G + 1];
#pragma unroll
    for (int r = 0; r < RB; r++)
#pragma unroll
        for (int j = 0; j < G; j++) red[wave][r * G + j][lane] = acc[r][j];
    __syncthreads();
    for (int t = tid; t < RB * G * 64; t += NW * 64) {   // (row block r, group j, lane l): wave partials in order
        const int rj = t >> 6, l = t & 63, g = l >> 4, m = l & 15;
        const int r = rj / G, j = rj % G;
        vx_floatx4_t v = red[0][rj][l];
#pragma unroll
        for (int w = 1; w < NW; w++) v += red[w][rj][l];
        // lane (g,m) holds C[4g+i][m]: row 16r + 4g + i, column 16j + m
#pragma unroll
        for (int i = 0; i < 4; i++) ct[16 * r + 4 * g + i][16 * j + m] = v[i];
    }
    __syncthreads();
    epi(row0, rows, WkRows<RB, G>{ct, B}, tid, pre);
}

// Epilogue: y[(b0 + b)*y_stride + n] for every row n of the workgroup.
struct WkStore {
    float *y;
    size_t y_stride;
    int b0;
    struct Pre {};
    __device__ __forceinline__ Pre prefetch(int, int, int) const { return {}; }
    template <int RB, int G>
    __device__ __forceinline__ void operator()(int row0, int rows, const WkRows<RB, G> &c, int tid, const Pre &) const {
        for (int t = tid; t < rows * c.B; t += blockDim.x) {
            const int r = t % rows, b = t / rows;
            y[(size_t)(b0 + b) * y_stride + row0 + r] = c.y(r, b);
        }
    }
};

// Launch plan: row blocks per workgroup (1..VX_WK_MAX_RB / G) and whether
// the weight loads are streaming (nontemporal, for large matrices).
struct WkPlan {
    int rb, nt, grid, g;
};
WkPlan vx_gemv_wk_plan(int N, int K, int n_cu, int G);

// Launch KERNEL<rb, nt, g>(args...) for a plan (grid plan.grid, block 1024).
#define VX_WK_CASE(ctx, KERNEL, p, R, GG, ...)                                                                  \
    if (p.rb == R && p.g == GG) {                                                                              \
        if (p.nt)                                                                                              \
            VX_LAUNCH_NAMED(ctx, #KERNEL, (KERNEL<R, true, GG>), dim3((unsigned)p.grid), dim3(1024), __VA_ARGS__); \
        else                                                                                                   \
            VX_LAUNCH_NAMED(ctx, #KERNEL, (KERNEL<R, false, GG>), dim3((unsigned)p.grid), dim3(1024), __VA_ARGS__); \
        break;                                                                                                 \
    }
#define VX_WK_DISPATCH(ctx, KERNEL, p, ...)                   \
    do {                                                      \
        VX_WK_CASE(ctx, KERNEL, p, 1, 1, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 2, 1, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 3, 1, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 4, 1, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 5, 1, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 6, 1, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 7, 1, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 8, 1, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 1, 2, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 2, 2, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 3, 2, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 4, 2, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 1, 3, __VA_ARGS__)         \
        VX_WK_CASE(ctx, KERNEL, p, 2, 3, __VA_ARGS__)         \
        VX_REQUIRE(false, "internal: no GEMV instance for rb=%d g=%d", p.rb, p.g); \
    } while (0)
