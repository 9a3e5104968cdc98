// Long-prompt projections on gfx950 MFMA: y[r][n] = sum_k W[n][k] x[r][k]
// for R tokens at once (the layer prefills from 256 tokens), the weights read once per
// tile of 256 tokens instead of once per 65 (the skinny GEMV of vx_gemv.hip).
// The reference applies its fp32 matvec (vx27_pmat.c:98-101, 119-125) token
// by token; this is the same product for a whole prompt.
//
// Numerics: W is bf16 (the tiled layout of vx27_hip_pack_weights_bf16); each
// fp32 activation enters the MFMAs as two bf16 parts, hi = bf16(x) and
// lo = bf16(x - hi) (16 significand bits, a relative error of at most
// 2^-16 per product, about 2^-17 typical), both accumulated in fp32 in one
// accumulator per output, k-step by k-step, hi before lo.  (The GEMV splits
// x three ways and is exact; two parts halve the MFMA work of a third.)
//
// Shape: one workgroup of 8 waves (two a SIMD) per output tile of 256 tokens
// x 256 rows (16 row blocks); wave (wm, wn) = (wave & 3, wave >> 2) owns
// tokens 64 wm .. +63 and rows 128 wn .. +127: 8 x 4 accumulator tiles of
// v_mfma_f32_16x16x32_bf16 (128 registers: with 256 in AGPRs the compiler
// copied a loop-carried share of them through VGPRs every k-step; 64 x 128
// rather than 128 x 64 since the token operand comes twice, hi and lo, so
// this shape reads the least from LDS), the W tile as operand A (lane
// (g, m): row m, k 8g..8g+7: exactly the tiled layout) and the token tile
// as operand B (lane (g, n): token n, k 8g..8g+7), so a lane's four outputs
// are four consecutive rows of one token (one 16-byte store).  Per 32-wide
// k-step a stage in LDS holds the 16 W tiles (16 KiB) and the 16 token
// tiles as hi and lo parts (32 KiB), both brought in by direct-to-LDS loads
// of 1 KiB runs; three stages rotate (the loads run two k-steps ahead), one
// barrier per k-step.  The token tiles come as their LDS image, written
// once per call by gemm_pack: the fp32 rows read and split into hi and lo
// once, where splitting them on the way into LDS cost every row tile of a
// token tile the loads, conversions and LDS stores again (9-10% of the
// kernel).  Per k-step and wave: 16 operand reads of 1 KiB from LDS, 64
// MFMAs (two waves a SIMD: about 2048 cycles of the SIMD's matrix core) and
// 6 DMAs of 1 KiB (2 W tiles, 4 KiB of the token image).
//
// Tiles are ordered per XCD (workgroup i runs on XCD i % 8): XCD x takes a
// contiguous range of tile indices, numbered in groups of 4 token tiles x
// all row tiles (token tile fastest), so the tiles an XCD runs together
// share 4 token slabs and about 8 weight slabs in its L2.
#include <algorithm>

#include "vx_gemv.h"
#include "vx_gemv_body.h"
#include "vx_lds.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int GT = 256;                  // tokens per tile
constexpr int GRB = 16;                  // row blocks (16 rows) per tile
constexpr int G_W = 0;                   // stage: W tiles [16][1 KiB]
constexpr int G_X = GRB * 1024;          // stage: token tiles [16 token blocks][hi, lo][1 KiB]
constexpr int G_STAGE = G_X + 32 * 1024; // 48 KiB
constexpr int G_GM = 4;                  // token tiles per group of the tile order
constexpr int G_XIMG = 32 * 1024;        // packed token tile image per k-step
#ifndef GEMM_NST
#define GEMM_NST 3                       // LDS stages (the loads run GEMM_NST - 1 k-steps ahead)
#endif
constexpr int G_NST = GEMM_NST;
constexpr int G_DMA = 6;                 // DMAs per wave and k-step (2 W tiles, 4 KiB of tokens)

// two floats as packed bf16, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = (bf16x2_t){(__bf16)x, (__bf16)y};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
    bf16x8_t r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

struct GemmArgs {
    const uint16_t *W;    // tiled [K/(32 kg)][N/16][kg][64][8]
    int N, K, R, kg;
    const char *xp;       // packed token tiles [n_tm][K/32][32 KiB] (gemm_pack)
    GemmOut out;          // where the rows of the product go (fp32 or bf16 segments)
    int n_tm, n_tn;
    // this launch: tiles tile0 .. tile0 + n_t - 1 of the tile order; P = 1:
    // whole tiles, XCD-grouped (per_xcd a XCD); P > 1: each tile's k-steps in
    // P parts (workgroup w: tile w % n_t, part w / n_t), the partial sums
    // into ws, for gemm_reduce
    int tile0, n_t, per_xcd, P;
    floatx4_t *ws;        // [P][n_t][32 accumulators (j, i)][512 lanes], float4s
};

// (tm, tn) of tile t: groups of G_GM token tiles x all row tiles, token tile fastest
__device__ __forceinline__ void gemm_tile(const GemmArgs &a, int t, int &tm, int &tn) {
    const int gsize = G_GM * a.n_tn, grp = t / gsize, first_m = grp * G_GM;
    const int msz = min(G_GM, a.n_tm - first_m), rr = t - grp * gsize;
    tm = first_m + rr % msz;
    tn = rr / msz;
}

// Accumulator (j, i) of lane (g, n) of wave (wm, wn): token 16 i + n of the
// wave's 64, rows 16 j + 4 g .. +3 of its 128, into the segment that holds
// the row block (wave-uniform).
__device__ __forceinline__ void gemm_store1(const GemmArgs &a, int tm, int tn, int wm, int wn, int g, int n, int j,
                                            int i, floatx4_t v) {
    const int rb = tn * GRB + wn * 8 + j, tk = tm * GT + wm * 64 + 16 * i + n;
    if (rb >= a.N / 16 || tk >= a.R) return;
    int si = 0;
#pragma unroll
    for (int q = 1; q < VX_GEMM_SEGS; q++)
        if (q < a.out.n && rb >= a.out.s[q].rb0) si = q;
    const GemmSeg sg = a.out.s[si];
    const size_t o = (size_t)tk * sg.stride + (size_t)(rb - sg.rb0) * 16 + 4 * g;
    if (sg.bf16)
        *(uint2 *)((uint16_t *)sg.p + o) = make_uint2(vx_f32_to_bf16(v[0]) | ((uint32_t)vx_f32_to_bf16(v[1]) << 16),
                                                      vx_f32_to_bf16(v[2]) | ((uint32_t)vx_f32_to_bf16(v[3]) << 16));
    else
        *(floatx4_t *)((float *)sg.p + o) = v;
}

// Token tile layout in LDS, per k-step: 16 token blocks x (hi, lo) x 1 KiB;
// lane (g, n)'s 16 bytes (token n of the block, k 8g..8g+7 of the step) sit
// at 16-byte unit g * 16 + (n ^ 2g).  The operand reads (8 lanes a cycle,
// one g) stay one aligned 128-byte block each, and the XOR spreads the
// units that one token column touches over the LDS's 32 banks.
// gemm_pack writes this image for every (token tile, k-step) of x (tokens
// past R as zeros; vx_gemm_pack_unit gives the layout), so that gemm_wx
// copies it into LDS verbatim by direct-to-LDS loads.  grid (K/32, token
// tiles), block 256.
__global__ __launch_bounds__(256) void gemm_pack(const float *x, size_t x_stride, int R, char *xp) {
    const int s = blockIdx.x, tm = blockIdx.y, K = 32 * gridDim.x;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int u = threadIdx.x + 256 * q, tb = u >> 6, g = (u >> 4) & 3, n = u & 15;
        const int t = tm * GT + tb * 16 + n;
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (t < R) {
            const float4 *p = (const float4 *)(x + (size_t)t * x_stride + 32 * s + 8 * g);
            const float4 v0 = p[0], v1 = p[1];
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
            v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
        }
        uint32_t h[4], l[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[e] = pack2(v[2 * e], v[2 * e + 1]);   // hi = bf16(x), then lo = bf16(x - hi)
            l[e] = pack2(v[2 * e] - __uint_as_float(h[e] << 16), v[2 * e + 1] - __uint_as_float(h[e] & 0xffff0000u));
        }
        char *dst = xp + vx_gemm_pack_unit(t, 32 * s + 8 * g, K);
        *(uint4 *)dst = make_uint4(h[0], h[1], h[2], h[3]);
        *(uint4 *)(dst + 1024) = make_uint4(l[0], l[1], l[2], l[3]);
    }
}

__global__ __launch_bounds__(512, 1) void gemm_wx(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) char smem[G_NST * G_STAGE];
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave & 3, wn = wave >> 2;

    // tile (and k-steps ks0 .. ks1 - 1) of this workgroup
    int tl, part = 0;
    if (a.P == 1) {
        tl = (blockIdx.x & 7) * a.per_xcd + (int)(blockIdx.x >> 3);
        if (tl >= a.n_t) return;
    } else {
        tl = (int)blockIdx.x % a.n_t;
        part = (int)blockIdx.x / a.n_t;
    }
    int tm, tn;
    gemm_tile(a, a.tile0 + tl, tm, tn);
    const int nb = a.N / 16, KSall = a.K / 32;
    const int ks0 = part * KSall / a.P, KS = (part + 1) * KSall / a.P;   // (KS: the end)
    const int rb0 = tn * GRB, tok0 = tm * GT;

    // this wave's DMA of W tiles 2 wave, 2 wave + 1 (row blocks clamped:
    // those past N are loaded but never stored)
    const char *Wb = (const char *)a.W;
    auto dma_w = [&](int s, int st) {
        const uint32_t base = vx_lds_addr(smem) + st * G_STAGE + G_W;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int jj = wave * 2 + q, rb = min(rb0 + jj, nb - 1);
            vx_dma16(Wb + vx_tile_off(s, rb, nb, a.kg) * 2, (uint32_t)lane * 16, base + jj * 1024);
        }
    };
    // this wave's 4 KiB of the packed token image of k-step s
    const char *xpt = a.xp + (size_t)tm * KSall * G_XIMG + wave * 4096;
    auto dma_x = [&](int s, int st) {
        const uint32_t base = vx_lds_addr(smem) + st * G_STAGE + G_X + wave * 4096;
#pragma unroll
        for (int q = 0; q < 4; q++) vx_dma16(xpt + (size_t)s * G_XIMG + q * 1024, (uint32_t)lane * 16, base + q * 1024);
    };
    const uint32_t xrd = (uint32_t)(g * 16 + (n ^ (g << 1))) * 16;   // this lane's operand unit

    floatx4_t acc[8][4];
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[j][i] = (floatx4_t){0.f, 0.f, 0.f, 0.f};

    // k-step s (in stage s % G_NST): the W tiles and token image of
    // s + G_NST - 1 are requested first into the stage that step s - 1 read
    // (clamped at the end: the extra loads land in a stage nobody reads
    // again), then the MFMAs on stage s.  No branch in the step, so the
    // waits count only what they need.
    auto step = [&](int s, int cur) {
        const int ld = cur == 0 ? G_NST - 1 : cur - 1;
        dma_w(min(s + G_NST - 1, KS - 1), ld);
        dma_x(min(s + G_NST - 1, KS - 1), ld);
        __builtin_amdgcn_sched_barrier(0);
        const char *sb = smem + cur * G_STAGE;
        bf16x8_t aw[8];
#pragma unroll
        for (int j = 0; j < 8; j++) aw[j] = as_bf16x8(*(const uint4 *)(sb + G_W + (wn * 8 + j) * 1024 + lane * 16));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tb = wm * 4 + i;
            const bf16x8_t bh = as_bf16x8(*(const uint4 *)(sb + G_X + (tb * 2 + 0) * 1024 + xrd));
            const bf16x8_t bl = as_bf16x8(*(const uint4 *)(sb + G_X + (tb * 2 + 1) * 1024 + xrd));
#pragma unroll
            for (int j = 0; j < 8; j++) {
                acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aw[j], bh, acc[j][i], 0, 0, 0);
                acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aw[j], bl, acc[j][i], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // this wave's DMAs of step s + 1 have landed (only the ones just
        // issued may be in flight), then every wave's stage is complete
        __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(G_DMA * (G_NST - 2)) : "memory");
        vx_lds_barrier();
    };

#pragma unroll
    for (int q = 0; q < G_NST - 1; q++) {
        dma_w(min(ks0 + q, KS - 1), (ks0 + q) % G_NST);
        dma_x(min(ks0 + q, KS - 1), (ks0 + q) % G_NST);
    }
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(G_DMA * (G_NST - 2)) : "memory");   // (the first stage)
    vx_lds_barrier();
    for (int s = ks0; s < KS; s++) step(s, s % G_NST);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // (the last, unused loads)

    if (a.P == 1) {
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) gemm_store1(a, tm, tn, wm, wn, g, n, j, i, acc[j][i]);
    } else {   // this part's sums for gemm_reduce (1 KiB runs per wave and accumulator)
        floatx4_t *w = a.ws + ((size_t)part * a.n_t + tl) * 32 * 512 + tid;
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) w[(j * 4 + i) * 512] = acc[j][i];
    }
}

// The tiles of a split launch: the P partial sums of each value added in
// part order (the same bits every run), then stored as the whole-tile
// launch stores them.  grid (n_t, 32 accumulators), block 512.
__global__ __launch_bounds__(512) void gemm_reduce(GemmArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave & 3, wn = wave >> 2;
    const int tl = blockIdx.x, q = blockIdx.y;
    int tm, tn;
    gemm_tile(a, a.tile0 + tl, tm, tn);
    const floatx4_t *w = a.ws + ((size_t)tl * 32 + q) * 512 + tid;
    const size_t pstride = (size_t)a.n_t * 32 * 512;   // float4s between parts
    floatx4_t v = w[0];
    for (int p = 1; p < a.P; p++) v += w[p * pstride];
    gemm_store1(a, tm, tn, wm, wn, g, n, q >> 2, q & 3, v);
}

}  // namespace

namespace {
// the shape and the output segments (N % 16 == 0, K % 64 == 0; segments in
// increasing row-block order from row block 0, aligned for their stores)
bool gemm_shape_ok(int N, int K, int R, const GemmOut &out) {
    if (!(N > 0 && N % 16 == 0 && K > 0 && K % 64 == 0 && R >= 1)) return false;
    if (out.n < 1 || out.n > VX_GEMM_SEGS || out.s[0].rb0 != 0) return false;
    for (int q = 0; q < out.n; q++) {
        const GemmSeg &sg = out.s[q];
        if (!sg.p || sg.stride % 4 != 0 || ((uintptr_t)sg.p & (sg.bf16 ? 7 : 15)) != 0) return false;
        if (q > 0 && (sg.rb0 <= out.s[q - 1].rb0 || sg.rb0 >= N / 16)) return false;
    }
    return true;
}
}  // namespace

bool vx_gemm_fits_seg(int N, int K, int R, const float *x, size_t x_stride, const GemmOut &out) {
    return x_stride % 4 == 0 && ((uintptr_t)x & 15) == 0 && gemm_shape_ok(N, K, R, out);
}

size_t vx_gemm_pack_bytes(int K, int R) {
    return (size_t)((R + GT - 1) / GT) * (K / 32) * G_XIMG;
}

bool vx_gemm_fits(int N, int K, int R, const float *x, size_t x_stride, const float *y, size_t y_stride) {
    GemmOut o = {};
    o.n = 1;
    o.s[0] = GemmSeg{0, 0, y_stride, (void *)y};
    return vx_gemm_fits_seg(N, K, R, x, x_stride, o);
}

namespace {
// Whole rounds of tiles (one per CU) as whole tiles; a last partial round of
// rem tiles, when it fills at most half of the CUs, in P parts along k (at
// least 8 k-steps each), so that it takes about one round of parts instead of
// one round of whole tiles.
struct GemmPlan {
    int n_main, rem, P;
    size_t ws_bytes;   // the split's partial sums (a multiple of 256 bytes), then the packed tokens
};
GemmPlan gemm_plan(int N, int K, int R, int n_cu) {
    const int n_tiles = ((R + GT - 1) / GT) * ((N / 16 + GRB - 1) / GRB);
    GemmPlan pl = {n_tiles, 0, 1, 0};
    const int rem = n_tiles % n_cu;
    if (rem > 0 && 2 * rem <= n_cu) {
        const int P = std::min(n_cu / rem, K / 32 / 8);
        if (P >= 2) pl = {n_tiles - rem, rem, P, (size_t)rem * P * 512 * 32 * sizeof(floatx4_t)};
    }
    return pl;
}
}  // namespace

size_t vx_gemm_ws_bytes(int N, int K, int R, int n_cu) {
    return gemm_plan(N, K, R, n_cu).ws_bytes + vx_gemm_pack_bytes(K, R);
}

int vx_gemm_store_packed(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const char *xp, int R,
                         const GemmOut &out, void *ws) {
    VX_REQUIRE(xp && ((uintptr_t)xp & 15) == 0 && gemm_shape_ok(N, K, R, out),
               "gemm: need N %% 16 == 0, K %% 64 == 0, a 16-byte aligned packed input and aligned output "
               "segments (N=%d K=%d R=%d)", N, K, R);
    VX_REQUIRE(ws != nullptr, "gemm: needs its workspace (vx_gemm_ws_bytes)");
    GemmArgs a;
    a.W = W; a.N = N; a.K = K; a.R = R; a.kg = vx_gemv_kg(K);
    a.out = out;
    a.xp = xp;
    a.n_tm = (R + GT - 1) / GT;
    a.n_tn = (N / 16 + GRB - 1) / GRB;
    const GemmPlan pl = gemm_plan(N, K, R, ctx->n_cu);
    if (pl.n_main > 0) {
        a.tile0 = 0; a.n_t = pl.n_main; a.P = 1; a.ws = nullptr;
        a.per_xcd = (pl.n_main + 7) / 8;
        VX_LAUNCH(ctx, gemm_wx, dim3((unsigned)(8 * a.per_xcd)), dim3(512), a);
    }
    if (pl.rem > 0) {
        a.tile0 = pl.n_main; a.n_t = pl.rem; a.P = pl.P; a.ws = (floatx4_t *)ws; a.per_xcd = 0;
        VX_LAUNCH(ctx, gemm_wx, dim3((unsigned)(pl.rem * pl.P)), dim3(512), a);
        VX_LAUNCH(ctx, gemm_reduce, dim3((unsigned)pl.rem, 32), dim3(512), a);
    }
    return 0;
}

int vx_gemm_store_seg(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x, size_t x_stride, int R,
                      const GemmOut &out, void *ws) {
    VX_REQUIRE(vx_gemm_fits_seg(N, K, R, x, x_stride, out),
               "gemm: need N %% 16 == 0, K %% 64 == 0, 16-byte aligned x rows and aligned output segments "
               "(N=%d K=%d R=%d)", N, K, R);
    VX_REQUIRE(ws != nullptr, "gemm: needs its workspace (vx_gemm_ws_bytes)");
    char *xp = (char *)ws + gemm_plan(N, K, R, ctx->n_cu).ws_bytes;
    VX_LAUNCH(ctx, gemm_pack, dim3((unsigned)(K / 32), (unsigned)((R + GT - 1) / GT)), dim3(256), x, x_stride, R,
              xp);
    return vx_gemm_store_packed(ctx, W, N, K, xp, R, out, ws);
}

int vx_gemm_store(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x, size_t x_stride, int R,
                  float *y, size_t y_stride, void *ws) {
    GemmOut o = {};
    o.n = 1;
    o.s[0] = GemmSeg{0, 0, y_stride, (void *)y};
    return vx_gemm_store_seg(ctx, W, N, K, x, x_stride, R, o, ws);
}

extern "C" int vx27_hip_gemm_bf16(vx27_hip_ctx *ctx, const uint16_t *W_tiled, int N, int K, const float *x,
                                  size_t x_stride, int R, float *y, size_t y_stride) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(W_tiled && x && y, "vx27_hip_gemm_bf16: null pointer");
    void *ws = nullptr;
    const size_t wsb = vx_gemm_ws_bytes(N, K, R, ctx->n_cu);
    if (wsb && vx_ctx_scratch(ctx, wsb, &ws)) return -1;
    return vx_gemm_store(ctx, W_tiled, N, K, x, x_stride, R, y, y_stride, ws);
}
