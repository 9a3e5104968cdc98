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
// (g, m): row m,
// k 8g..8g+7: exactly the tiled layout) and the token tile as operand B
// (lane (g, n): token n, k 8g..8g+7), so a lane's four outputs are four
// consecutive rows of one token (one 16-byte store).  Per 32-wide k-step a
// stage in LDS holds the 16 W tiles (16 KiB, direct-to-LDS loads of their
// 1 KiB runs) and the 16 token tiles as hi and lo parts (32 KiB, split from
// the fp32 rows on the way in); two stages alternate, one barrier per
// k-step.  Per k-step and wave: 16 operand reads of 1 KiB from LDS, 64
// MFMAs (two waves a SIMD: about 2048 cycles of the SIMD's matrix core), 4
// row loads of 16 bytes a lane and 2 tile DMAs, all for the next k-step.
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
    const float *x;       // [R] rows of K, row stride x_stride (16-byte aligned rows)
    size_t x_stride;
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

__global__ __launch_bounds__(512, 1) void gemm_wx(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) char smem[2 * G_STAGE];
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
    // token rows: load i of this wave covers tokens 32 wave + 8 i + lane / 8,
    // floats 4 (lane % 8) .. +3 of the k-step, through a buffer resource: the
    // lane's byte offset plus a scalar one per k-step (tokens past R read row
    // R - 1; the host keeps x within 2^31 bytes)
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.x, (short)0, (int)((size_t)a.R * a.x_stride * 4), 0x00020000);
    const int tok_l = tok0 + wave * 32 + (lane >> 3);
    uint32_t xoff[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        xoff[i] = (uint32_t)((size_t)min(tok_l + i * 8, a.R - 1) * a.x_stride * 4) + 16u * (uint32_t)(lane & 7);
    auto load_x = [&](int s, floatx4_t (&xr)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xres, (int)xoff[i], 128 * s, 0));
            xr[i] = (floatx4_t){__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
        }
    };
    // Token tile layout: lane (g, n)'s 16 bytes (token n, k 8g..8g+7) sit at
    // 16-byte unit g * 16 + (n ^ 2g).  The LDS serves 128 bytes (32 banks) a
    // cycle: a store below writes 8 bytes a lane, 16 lanes a cycle (2 columns
    // x 4 values of g x 2 halves), whose units n ^ 2g then cover all 8
    // 16-byte bank groups once (without the XOR all 16 lanes fell on the
    // same 128 bytes: four ways, the LDS's largest cost here); the operand
    // reads (8 lanes a cycle, one g) stay one aligned 128-byte block each.
    // Token t' = 32 wave + 8 i + lane / 8 is column t' % 16 of token block
    // t' / 16; its floats 4c..4c+3 (c = lane % 8) are elements 4 (c % 2) ..
    // of lane (c / 2, t' % 16).
    auto store_x = [&](int st, const floatx4_t (&xr)[4]) {
        char *xb = smem + st * G_STAGE + G_X;
        const int c = lane & 7, gw = c >> 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tt = wave * 32 + i * 8 + (lane >> 3), tb = tt >> 4, col = tt & 15;
            const uint2 h = make_uint2(pack2(xr[i][0], xr[i][1]), pack2(xr[i][2], xr[i][3]));
            const uint2 l = make_uint2(pack2(xr[i][0] - __uint_as_float(h.x << 16), xr[i][1] - __uint_as_float(h.x & 0xffff0000u)),
                                       pack2(xr[i][2] - __uint_as_float(h.y << 16), xr[i][3] - __uint_as_float(h.y & 0xffff0000u)));
            const int off = (gw * 16 + (col ^ (gw << 1))) * 16 + (c & 1) * 8;
            *(uint2 *)(xb + (tb * 2 + 0) * 1024 + off) = h;
            *(uint2 *)(xb + (tb * 2 + 1) * 1024 + off) = l;
        }
    };
    const uint32_t xrd = (uint32_t)(g * 16 + (n ^ (g << 1))) * 16;   // this lane's operand unit

    floatx4_t acc[8][4];
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[j][i] = (floatx4_t){0.f, 0.f, 0.f, 0.f};

    // k-step s: the W tiles and the rows of s + 1 are requested first
    // (clamped at the end: the extra loads land in a stage nobody reads
    // again), then the MFMAs on stage s, then the rows split into the other
    // stage.  No branch in the step, so the waits count only what they need.
    floatx4_t xr[4];
    auto step = [&](int s) {
        const int cur = s & 1;
        dma_w(min(s + 1, KS - 1), cur ^ 1);
        load_x(min(s + 1, KS - 1), xr);
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
        store_x(cur ^ 1, xr);
        // this wave's W DMA has landed, then every wave's stage is complete
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        vx_lds_barrier();
    };

    dma_w(ks0, ks0 & 1);
    load_x(ks0, xr);
    store_x(ks0 & 1, xr);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // (the W DMA of the first stage)
    vx_lds_barrier();
    for (int s = ks0; s < KS; s++) step(s);
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

bool vx_gemm_fits_seg(int N, int K, int R, const float *x, size_t x_stride, const GemmOut &out) {
    if (!(N > 0 && N % 16 == 0 && K > 0 && K % 64 == 0 && R >= 1 && x_stride % 4 == 0 && ((uintptr_t)x & 15) == 0 &&
          (size_t)R * x_stride * 4 < ((size_t)1 << 31)))
        return false;
    if (out.n < 1 || out.n > VX_GEMM_SEGS || out.s[0].rb0 != 0) return false;
    for (int q = 0; q < out.n; q++) {
        const GemmSeg &sg = out.s[q];
        if (!sg.p || sg.stride % 4 != 0 || ((uintptr_t)sg.p & (sg.bf16 ? 7 : 15)) != 0) return false;
        if (q > 0 && (sg.rb0 <= out.s[q - 1].rb0 || sg.rb0 >= N / 16)) return false;
    }
    return true;
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
    size_t ws_bytes;
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
    return gemm_plan(N, K, R, n_cu).ws_bytes;
}

int vx_gemm_store_seg(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x, size_t x_stride, int R,
                      const GemmOut &out, void *ws) {
    VX_REQUIRE(vx_gemm_fits_seg(N, K, R, x, x_stride, out),
               "gemm: need N %% 16 == 0, K %% 64 == 0, 16-byte aligned x rows within 2^31 bytes and aligned "
               "output segments (N=%d K=%d R=%d)", N, K, R);
    GemmArgs a;
    a.W = W; a.N = N; a.K = K; a.R = R; a.kg = vx_gemv_kg(K);
    a.x = x; a.x_stride = x_stride; a.out = out;
    a.n_tm = (R + GT - 1) / GT;
    a.n_tn = (N / 16 + GRB - 1) / GRB;
    GemmPlan pl = gemm_plan(N, K, R, ctx->n_cu);
    if (!ws) pl = {a.n_tm * a.n_tn, 0, 1, 0};
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
