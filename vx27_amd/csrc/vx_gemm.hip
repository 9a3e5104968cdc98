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
    int n_tm, n_tn, per_xcd;
};

__global__ __launch_bounds__(512, 1) void gemm_wx(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) char smem[2 * G_STAGE];
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave & 3, wn = wave >> 2;

    // tile of this workgroup
    const int xcd = blockIdx.x & 7;
    const int t = xcd * a.per_xcd + (int)(blockIdx.x >> 3);
    if (t >= a.n_tm * a.n_tn) return;
    const int gsize = G_GM * a.n_tn, grp = t / gsize, first_m = grp * G_GM;
    const int msz = min(G_GM, a.n_tm - first_m), rr = t - grp * gsize;
    const int tm = first_m + rr % msz, tn = rr / msz;
    const int nb = a.N / 16, KS = a.K / 32;
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
    // 16-byte unit g * 16 + (n ^ 8 (g & 1)): the hi/lo writes below (8 columns
    // x 4 values of g a store) then meet each bank at most twice, and the
    // operand reads (16 lanes of one g) stay a permutation of 16 units.
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
            const int off = (gw * 16 + (col ^ ((gw & 1) << 3))) * 16 + (c & 1) * 8;
            *(uint2 *)(xb + (tb * 2 + 0) * 1024 + off) = h;
            *(uint2 *)(xb + (tb * 2 + 1) * 1024 + off) = l;
        }
    };
    const uint32_t xrd = (uint32_t)(g * 16 + (n ^ ((g & 1) << 3))) * 16;   // this lane's operand unit

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

    dma_w(0, 0);
    load_x(0, xr);
    store_x(0, xr);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // (the W DMA of stage 0)
    vx_lds_barrier();
    for (int s = 0; s < KS; s++) step(s);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // (the last, unused loads)

    // lane (g, n) of accumulator (j, i): token 16 i + n of the wave's 64,
    // rows 16 j + 4 g .. +3 of its 128, into the segment that holds the row
    // block (wave-uniform)
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int rb = rb0 + wn * 8 + j;
        if (rb >= nb) continue;
        int si = 0;
#pragma unroll
        for (int q = 1; q < VX_GEMM_SEGS; q++)
            if (q < a.out.n && rb >= a.out.s[q].rb0) si = q;
        const GemmSeg sg = a.out.s[si];
        const size_t col = (size_t)(rb - sg.rb0) * 16 + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tk = tok0 + wm * 64 + 16 * i + n;
            if (tk >= a.R) continue;
            const size_t o = (size_t)tk * sg.stride + col;
            if (sg.bf16) {
                const floatx4_t v = acc[j][i];
                *(uint2 *)((uint16_t *)sg.p + o) =
                    make_uint2(vx_f32_to_bf16(v[0]) | ((uint32_t)vx_f32_to_bf16(v[1]) << 16),
                               vx_f32_to_bf16(v[2]) | ((uint32_t)vx_f32_to_bf16(v[3]) << 16));
            } else {
                *(floatx4_t *)((float *)sg.p + o) = acc[j][i];
            }
        }
    }
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

int vx_gemm_store_seg(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x, size_t x_stride, int R,
                      const GemmOut &out) {
    VX_REQUIRE(vx_gemm_fits_seg(N, K, R, x, x_stride, out),
               "gemm: need N %% 16 == 0, K %% 64 == 0, 16-byte aligned x rows within 2^31 bytes and aligned "
               "output segments (N=%d K=%d R=%d)", N, K, R);
    GemmArgs a;
    a.W = W; a.N = N; a.K = K; a.R = R; a.kg = vx_gemv_kg(K);
    a.x = x; a.x_stride = x_stride; a.out = out;
    a.n_tm = (R + GT - 1) / GT;
    a.n_tn = (N / 16 + GRB - 1) / GRB;
    const int n_tiles = a.n_tm * a.n_tn;
    a.per_xcd = (n_tiles + 7) / 8;
    VX_LAUNCH(ctx, gemm_wx, dim3((unsigned)(8 * a.per_xcd)), dim3(512), a);
    return 0;
}

int vx_gemm_store(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x, size_t x_stride, int R,
                  float *y, size_t y_stride) {
    GemmOut o = {};
    o.n = 1;
    o.s[0] = GemmSeg{0, 0, y_stride, (void *)y};
    return vx_gemm_store_seg(ctx, W, N, K, x, x_stride, R, o);
}

extern "C" int vx27_hip_gemm_bf16(vx27_hip_ctx *ctx, const uint16_t *W_tiled, int N, int K, const float *x,
                                  size_t x_stride, int R, float *y, size_t y_stride) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(W_tiled && x && y, "vx27_hip_gemm_bf16: null pointer");
    return vx_gemm_store(ctx, W_tiled, N, K, x, x_stride, R, y, y_stride);
}
