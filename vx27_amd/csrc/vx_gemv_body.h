// Whole-K workgroup GEMV body for the skinny projections (vx_gemv.hip),
// shared with the kernels that put their own epilogue after it
// (vx_layer.hip).
//
// A workgroup of 8 waves owns RB row blocks (16 RB rows) over all of K:
// wave w takes the k-steps w, w + 8, ... (so the waves of a workgroup read
// neighbouring k-step slabs of the tiled weights at any moment) and
// multiplies each weight tile it loads by all G operand groups of the pass
// (one pass over the weights for up to 65 vectors).  Each wave keeps a ring
// of D operand sets: the loads of its next D - 1 k-steps are in flight
// while the MFMAs of the current one run, so that a workgroup keeps about
// 8 D (RB + G) KiB of loads outstanding.  A row's value is fixed as
//   y = y0 + y1,   yh = (hi_h + mid_h) + lo_h,
// where hi_h, mid_h, lo_h are the column sums of waves 4h .. 4h+3 in wave
// order: the 8 partials are summed in LDS as two halves.  A plain-store
// epilogue may instead run the two halves as two workgroups of 4 waves
// that add y0 and y1 into a zeroed output with fp32 atomics: two addends
// commute, so the bits are the same, and the finer grid fills the CUs
// where whole rows would leave some idle.  The sum order is the same
// whatever RB, D, the halves or the number of vectors in the pass.
// (A split of K over workgroups, whose last arrival sums the slices, was
// measured slower on every projection shape of the model, with or without
// device-scope fences.)
#pragma once
#include "vx_gemv.h"

typedef __bf16 vx_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float vx_floatx4_t __attribute__((ext_vector_type(4)));

constexpr int VX_WK_NW = 8;   // waves per workgroup
#ifndef VX_WK_DMAX
#define VX_WK_DMAX 4              // most operand sets in a wave's ring
#endif
#ifndef VX_GEMV_KG
#define VX_GEMV_KG 1              // k-steps per group of the tiled layout (1, 2 or 4)
#endif

static __device__ vx_bf16x8_t vx_wk_zero[64];   // zero operand tile (static storage)

// largest RB for G groups: RB x G accumulator tiles and the operand sets
// within the register budget of 8-wave workgroups
__host__ __device__ constexpr int vx_wk_max_rb(int G) {
    return G == 1 ? 20 : G == 2 ? 16 : G == 3 ? 10 : G == 4 ? 8 : G == 7 ? 4 : G == 10 ? 3 : 2;
}
// operand sets in a wave's ring: as many as fit beside the 4 RB G
// accumulator registers in about 200 (an operand set takes 4 (RB + G)),
// 1 .. VX_WK_DMAX
__host__ __device__ constexpr int vx_wk_depth_raw(int RB, int G) { return (200 - 4 * RB * G) / (4 * (RB + G)); }
__host__ __device__ constexpr int vx_wk_depth(int RB, int G) {
    return vx_wk_depth_raw(RB, G) < 1 ? 1 : vx_wk_depth_raw(RB, G) > VX_WK_DMAX ? VX_WK_DMAX : vx_wk_depth_raw(RB, G);
}

// k-steps per group of the tiled weight layout
__host__ __device__ __forceinline__ int vx_gemv_kg(int K) {
    const int nks = K / 32;
    return nks % VX_GEMV_KG == 0 ? VX_GEMV_KG : 1;
}
// element offset of tile (k-step s, row block rb) in the tiled layout
__host__ __device__ __forceinline__ size_t vx_tile_off(int s, int rb, int nb, int kg) {
    return ((size_t)(s / kg) * nb + rb) * kg * 512 + (size_t)(s % kg) * 512;
}

// Weights: tiled (vx27_hip_pack_weights_bf16) or row-major [N][K].
struct WkWeights {
    const uint16_t *W;
    int row_major;
    // this lane's 8 elements of tile (0, rb)
    __device__ __forceinline__ const uint16_t *base(int rb, int nb, int K, int kg, int lane) const {
        return row_major ? W + (size_t)(16 * rb + (lane & 15)) * K + 8 * (lane >> 4)
                         : W + vx_tile_off(0, rb, nb, kg) + lane * 8;
    }
    // offset of k-step s from tile (0, rb)
    __device__ __forceinline__ size_t off(int s, int nb, int kg) const {
        return row_major ? (size_t)s * 32 : (size_t)(s / kg) * nb * kg * 512 + (size_t)(s % kg) * 512;
    }
};

// Summed rows handed to an epilogue: y(r, b) for local row r < rows and
// vector b < B of the pass (its groups g0 .. g0+G-1 of the packed operand):
// the nh halves' values added in order (nh = 1 in a half workgroup).
template <int RB, int G>
struct WkRows {
    const float (*c)[16 * RB][16 * G + 1];   // [2][16 RB][16 G + 1]: each half's MFMA output columns
    int B;                                   // vectors in this pass (<= 5 G)
    int nh;                                  // halves summed here (2, or 1 in a half workgroup)
    __device__ __forceinline__ float y(int r, int b) const {
        const int j = b / VX_PACK_GV, bl = b - VX_PACK_GV * j, Bj = min(VX_PACK_GV, B - VX_PACK_GV * j);
        const float *c0 = c[0][r] + 16 * j;
        const float y0 = (c0[bl] + c0[Bj + bl]) + c0[2 * Bj + bl];
        if (nh == 1) return y0;
        const float *c1 = c[1][r] + 16 * j;
        return y0 + ((c1[bl] + c1[Bj + bl]) + c1[2 * Bj + bl]);
    }
};

// Epilogue interface, both called by all threads of the workgroup (rows =
// valid rows from row0, <= 16 RB):
//   Pre prefetch(int row0, int rows, int tid) const      before the K loop:
//       issues the loads the epilogue needs besides the sums (their latency
//       then hides under the loop instead of trailing it)
//   void operator()(int row0, int rows, const WkRows<RB, G> &, int tid, const Pre &) const
// One pass covers the B vectors of groups g0 .. g0+G-1 of a packed operand
// with Gt groups in all.  halves = 1: grid ceil(N / 16 RB), block 512;
// halves = 2: grid 2 ceil(N / 16 RB), block 256, workgroup 2i + h running
// waves 4h .. 4h+3 of row group i (the epilogue then gets only its half).
template <int RB, int G, class Epi>
__device__ __forceinline__ void vx_gemv_wk_body(const WkWeights &wt, int N, int K, const uint16_t *xp, int Gt,
                                                int g0, int B, int halves, const Epi &epi) {
    constexpr int NW = VX_WK_NW, D = vx_wk_depth(RB, G);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = halves == 2 ? (int)(blockIdx.x & 1) : 0;
    const int nwp = halves == 2 ? NW / 2 : NW;   // waves in this workgroup
    const int vw = h * (NW / 2) + wave;          // the wave's place in the 8-wave split
    const int rb0 = (halves == 2 ? (int)(blockIdx.x >> 1) : (int)blockIdx.x) * RB, nb = N / 16;
    const int nks = K / 32, kg = vx_gemv_kg(K);
    const int k0 = 0, k1 = nks;
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
    for (int r = 0; r < RB; r++)   // dead blocks re-read block 0, never stored
        wp[r] = wt.base(rb0 + r < nb ? rb0 + r : 0, nb, K, kg, lane);
    const vx_bf16x8_t *xb = (const vx_bf16x8_t *)xp + (size_t)g0 * 64 + lane;
    // operands of k-step s; past the end (s >= k1) both operands come from
    // a zero tile, so that every path issues the same loads and MFMAs (the
    // waits before each MFMA then leave the later sets in flight) and the
    // extra products add exact zeros
    const vx_bf16x8_t *zt = vx_wk_zero + lane;
    auto load = [&](int s, vx_bf16x8_t(&ao)[RB], vx_bf16x8_t(&bo)[G]) {
        const bool live = s < k1;
#pragma unroll
        for (int j = 0; j < G; j++) bo[j] = *(live ? xb + ((size_t)s * Gt + j) * 64 : zt);
        const size_t off = wt.off(s, nb, kg);
#pragma unroll
        for (int r = 0; r < RB; r++) ao[r] = *(live ? (const vx_bf16x8_t *)(wp[r] + off) : zt);
    };
    auto mma = [&](const vx_bf16x8_t(&ao)[RB], const vx_bf16x8_t(&bo)[G]) {
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int j = 0; j < G; j++)
                acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ao[r], bo[j], acc[r][j], 0, 0, 0);
    };
    // D operand sets in a ring: the loads of the next D - 1 k-steps of this
    // wave are in flight during the MFMAs of the current one (the branches
    // are uniform: s is a wave constant)
    vx_bf16x8_t a[D][RB], b[D][G];
#pragma unroll
    for (int d = 0; d < D; d++) load(k0 + vw + d * NW, a[d], b[d]);
    for (int s = k0 + vw; s < k1; s += D * NW) {   // whole rounds of D k-steps
#pragma unroll
        for (int d = 0; d < D; d++) {
            mma(a[d], b[d]);
            load(s + (d + D) * NW, a[d], b[d]);
        }
    }
    constexpr int NTL = RB * G;                         // accumulator tiles
    constexpr int RC = NTL < 64 / NW ? NTL : 64 / NW;   // tiles reduced per round (64 KiB of LDS)
    __shared__ vx_floatx4_t red[NW][RC][64];
    __shared__ float ct[2][16 * RB][16 * G + 1];
    const int nh = nwp / 4;   // halves summed in this workgroup
#pragma unroll
    for (int t0 = 0; t0 < NTL; t0 += RC) {
        if (t0) __syncthreads();   // the previous round's partials are read out
#pragma unroll
        for (int q = 0; q < RC; q++)
            if (t0 + q < NTL) red[wave][q][lane] = acc[(t0 + q) / G][(t0 + q) % G];
        __syncthreads();
        for (int t = tid; t < RC * 64; t += nwp * 64) {   // (tile t0 + q, lane l): each half's 4 partials in order
            const int q = t >> 6, l = t & 63, g = l >> 4, m = l & 15;
            const int rj = t0 + q;
            if (rj >= NTL) continue;
            const int r = rj / G, j = rj % G;
            for (int hh = 0; hh < nh; hh++) {
                const vx_floatx4_t v = ((red[4 * hh][q][l] + red[4 * hh + 1][q][l]) + red[4 * hh + 2][q][l]) +
                                       red[4 * hh + 3][q][l];
                // lane (g,m) holds C[4g+i][m]: row 16r + 4g + i, column 16j + m
#pragma unroll
                for (int i = 0; i < 4; i++) ct[hh][16 * r + 4 * g + i][16 * j + m] = v[i];
            }
        }
    }
    __syncthreads();
    epi(row0, rows, WkRows<RB, G>{ct, B, nh}, tid, pre);
}

// Epilogue: y[(b0 + b)*y_stride + n] for every row n of the workgroup
// (added with an atomic in a half workgroup: y must then start at zero).
struct WkStore {
    float *y;
    size_t y_stride;
    int b0;
    struct Pre {};
    __device__ __forceinline__ Pre prefetch(int, int, int) const { return {}; }
    template <int RB, int G>
    __device__ __forceinline__ void operator()(int row0, int rows, const WkRows<RB, G> &c, int tid, const Pre &) const {
        for (int t = tid; t < rows * c.B; t += c.nh * 4 * 64) {
            const int r = t % rows, b = t / rows;
            float *yp = y + (size_t)(b0 + b) * y_stride + row0 + r;
            if (c.nh == 1) atomicAdd(yp, c.y(r, b));
            else *yp = c.y(r, b);
        }
    }
};

// Launch plan for an N x K matrix and a pass of G groups: RB row blocks per
// workgroup, whole (halves = 1, grid ceil(N / 16 RB)) or split in two half
// workgroups (halves = 2, twice the grid, only when allow_halves: an
// epilogue that adds into a zeroed output).  The plan takes the shape that
// best balances the CUs in one round of workgroups (several rounds only
// when no single-round plan exists).
struct WkPlan {
    int rb, g, grid, halves;
};
WkPlan vx_gemv_wk_plan(int N, int K, int n_cu, int G, bool allow_halves = false);

// every (RB, G) instance: RB = 1 .. vx_wk_max_rb(G)
#define VX_WK_RB_G1(X, ...)                                                                                      \
    X(1, 1, __VA_ARGS__) X(2, 1, __VA_ARGS__) X(3, 1, __VA_ARGS__) X(4, 1, __VA_ARGS__) X(5, 1, __VA_ARGS__)    \
    X(6, 1, __VA_ARGS__) X(7, 1, __VA_ARGS__) X(8, 1, __VA_ARGS__) X(9, 1, __VA_ARGS__) X(10, 1, __VA_ARGS__)   \
    X(11, 1, __VA_ARGS__) X(12, 1, __VA_ARGS__) X(13, 1, __VA_ARGS__) X(14, 1, __VA_ARGS__)                     \
    X(15, 1, __VA_ARGS__) X(16, 1, __VA_ARGS__) X(17, 1, __VA_ARGS__) X(18, 1, __VA_ARGS__)                     \
    X(19, 1, __VA_ARGS__) X(20, 1, __VA_ARGS__)
#define VX_WK_RB_G2(X, ...)                                                                                      \
    X(1, 2, __VA_ARGS__) X(2, 2, __VA_ARGS__) X(3, 2, __VA_ARGS__) X(4, 2, __VA_ARGS__) X(5, 2, __VA_ARGS__)    \
    X(6, 2, __VA_ARGS__) X(7, 2, __VA_ARGS__) X(8, 2, __VA_ARGS__) X(9, 2, __VA_ARGS__) X(10, 2, __VA_ARGS__)   \
    X(11, 2, __VA_ARGS__) X(12, 2, __VA_ARGS__) X(13, 2, __VA_ARGS__) X(14, 2, __VA_ARGS__)                     \
    X(15, 2, __VA_ARGS__) X(16, 2, __VA_ARGS__)
#define VX_WK_RB_G3(X, ...)                                                                                      \
    X(1, 3, __VA_ARGS__) X(2, 3, __VA_ARGS__) X(3, 3, __VA_ARGS__) X(4, 3, __VA_ARGS__) X(5, 3, __VA_ARGS__)    \
    X(6, 3, __VA_ARGS__) X(7, 3, __VA_ARGS__) X(8, 3, __VA_ARGS__) X(9, 3, __VA_ARGS__) X(10, 3, __VA_ARGS__)
#define VX_WK_RB_BIG(X, ...)                                                                                     \
    X(1, 4, __VA_ARGS__) X(2, 4, __VA_ARGS__) X(3, 4, __VA_ARGS__) X(4, 4, __VA_ARGS__) X(5, 4, __VA_ARGS__)    \
    X(6, 4, __VA_ARGS__) X(7, 4, __VA_ARGS__) X(8, 4, __VA_ARGS__) X(1, 7, __VA_ARGS__) X(2, 7, __VA_ARGS__)    \
    X(3, 7, __VA_ARGS__) X(4, 7, __VA_ARGS__) X(1, 10, __VA_ARGS__) X(2, 10, __VA_ARGS__) X(3, 10, __VA_ARGS__) \
    X(1, 13, __VA_ARGS__) X(2, 13, __VA_ARGS__)
#define VX_WK_ALL(X, ...)                                                                                        \
    VX_WK_RB_G1(X, __VA_ARGS__) VX_WK_RB_G2(X, __VA_ARGS__) VX_WK_RB_G3(X, __VA_ARGS__) VX_WK_RB_BIG(X, __VA_ARGS__)

// Launch KERNEL<rb, g>(args...) for a plan (grid plan.grid, block 512 or
// 256 for half workgroups).
#define VX_WK_CASE(R, GG, ctx, KERNEL, p, ...)                                                                 \
    case GG * 64 + R:                                                                                          \
        VX_LAUNCH_NAMED(ctx, #KERNEL, (KERNEL<R, GG>), dim3((unsigned)p.grid),                                 \
                        dim3(VX_WK_NW * 64 / p.halves), __VA_ARGS__);                                          \
        break;
#define VX_WK_DISPATCH(ctx, KERNEL, p, ...)                                                   \
    do {                                                                                      \
        switch (p.g * 64 + p.rb) {                                                            \
            VX_WK_ALL(VX_WK_CASE, ctx, KERNEL, p, __VA_ARGS__)                                \
            default: VX_REQUIRE(false, "internal: no GEMV instance for rb=%d g=%d", p.rb, p.g); \
        }                                                                                     \
    } while (0)
