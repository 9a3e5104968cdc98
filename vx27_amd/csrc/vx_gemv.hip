// Skinny bf16 GEMM (the mixer projections) on gfx950 MFMA.
//
// y[b][n] = sum_k W[n][k] * x[b][k] for B <= 5 activation vectors (decode:
// one token per sequence), W bf16 row-major [N][K] (the layout of the
// reference's weight tensors, vx27_pmat.h:6-8), x and y fp32.
//
// The fp32 activations enter the MFMA exactly: each x is split into three
// bf16 parts hi + mid + lo (8 mantissa bits each, 24 in all), and the parts
// of the B vectors are the columns of the MFMA's B operand (3*B <= 16 of the
// 16 columns).  One v_mfma_f32_16x16x32_bf16 therefore multiplies 16 weight
// rows by all parts of all vectors; the products are exact in fp32 and the
// only rounding is the fp32 accumulation, as in a plain fp32 dot product.
// The part sums are formed in the reduction.  No cross-lane reduction is
// needed: the MFMA accumulates over k.
//
// Kernels:
//   pack_x     x [B][K] fp32 -> packed B operand [K/32][64 lanes][8] bf16
//              (lane (g,n) of k-step s holds part n/B of vector n%B at
//              k = 32s + 8g + 0..7; columns n >= P*B are zero)
//   gemv_part  one wave per (64-row group, K segment): 4 row blocks x the
//              segment's k-steps, partial sums [split][N][16] fp32
//   reductions sum the partials in a fixed order (deterministic) and apply
//              an epilogue: plain store, or the DeltaNet input projection's
//              (causal conv + SiLU, z, gate mapping), see vx_layer.hip.
#include "vx_gemv.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint16_t bf16_bits(float x) { return vx_f32_to_bf16(x); }

// pack: grid (K/32), block 64; lane (g,n) writes its 8 elements of k-step s
__global__ __launch_bounds__(64) void pack_x(const float *x, size_t x_stride, int B, int P, uint16_t *out) {
    const int s = blockIdx.x, lane = threadIdx.x, g = lane >> 4, n = lane & 15;
    uint16_t v[8];
    if (n < P * B) {
        const int p = n / B, b = n % B;
        const float *xr = x + (size_t)b * x_stride + 32 * s + 8 * g;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float r = xr[e];
            uint16_t h = bf16_bits(r);
            for (int q = 0; q < p; q++) {   // peel the leading parts
                r = r - vx_bf16_to_f32(h);
                h = bf16_bits(r);
            }
            v[e] = h;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = 0;
    }
    uint4 w;
    w.x = v[0] | ((uint32_t)v[1] << 16);
    w.y = v[2] | ((uint32_t)v[3] << 16);
    w.z = v[4] | ((uint32_t)v[5] << 16);
    w.w = v[6] | ((uint32_t)v[7] << 16);
    *(uint4 *)(out + ((size_t)s * 64 + lane) * 8) = w;
}

constexpr int RB = 4;   // 16-row MFMA blocks per wave

// grid (ceil(N/64), ceil(n_seg/4)), block 256: wave w computes row group
// blockIdx.x (64 rows) over K segment blockIdx.y*4 + w.
__global__ __launch_bounds__(256) void gemv_part(const uint16_t *W, int N, int K, const uint16_t *xp,
                                                 int ks_per, int n_seg, float *part) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, m = lane & 15;
    const int seg = blockIdx.y * 4 + wave;
    if (seg >= n_seg) return;
    const int row0 = blockIdx.x * 16 * RB;
    const int nks = K / 32;
    const int s0 = seg * ks_per, s1 = min(nks, s0 + ks_per);
    floatx4_t acc[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) acc[r] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    const uint16_t *wrow[RB];
    bool live[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) {
        const int row = row0 + r * 16 + m;
        live[r] = row0 + r * 16 < N;          // whole block in or out (N % 16 == 0)
        wrow[r] = W + (size_t)(live[r] ? row : 0) * K + 8 * g;
    }
    const bf16x8_t *xb = (const bf16x8_t *)xp + lane;
#pragma unroll 2
    for (int s = s0; s < s1; s++) {
        const bf16x8_t bop = xb[(size_t)s * 64];
        bf16x8_t aop[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) aop[r] = *(const bf16x8_t *)(wrow[r] + 32 * s);
#pragma unroll
        for (int r = 0; r < RB; r++)
            if (live[r]) acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[r], bop, acc[r], 0, 0, 0);
    }
    // lane (g,m) holds C[4g+i][m]: rows row0 + r*16 + 4g + i, column m
#pragma unroll
    for (int r = 0; r < RB; r++) {
        if (!live[r]) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = row0 + r * 16 + 4 * g + i;
            part[((size_t)seg * N + row) * 16 + m] = acc[r][i];
        }
    }
}

// plain reduction: y[b*y_stride + n] = sum over segments and parts
__global__ __launch_bounds__(256) void gemv_reduce_store(const float *part, int N, int B, int P, int n_seg,
                                                         float *y, size_t y_stride) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)N * B) return;
    const int b = (int)(id / N), n = (int)(id % N);
    y[(size_t)b * y_stride + n] = vx_gemv_sum(part, N, B, P, n_seg, n, b);
}

}  // namespace

int vx_gemv_plan(int N, int K, int *n_seg, int *ks_per) {
    VX_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0,
               "gemv: N must be a multiple of 16 and K of 32 (N=%d K=%d)", N, K);
    const int groups = (N + 16 * RB - 1) / (16 * RB);
    const int nks = K / 32;
    // about 2048 waves in all, at least 8 k-steps per wave
    int seg = (2048 + groups - 1) / groups;
    if (seg > nks / 8) seg = nks / 8;
    if (seg < 1) seg = 1;
    int per = (nks + seg - 1) / seg;
    seg = (nks + per - 1) / per;
    *n_seg = seg;
    *ks_per = per;
    return 0;
}

size_t vx_gemv_part_bytes(int N, int n_seg) { return (size_t)n_seg * N * 16 * sizeof(float); }
size_t vx_pack_bytes(int K) { return (size_t)(K / 32) * 64 * 8 * sizeof(uint16_t); }

int vx_pack(vx27_hip_ctx *ctx, const float *x, size_t x_stride, int B, int P, int K, uint16_t *packed) {
    VX_REQUIRE(B >= 1 && P >= 1 && P * B <= 16 && K % 32 == 0, "pack: need P*B <= 16, K %% 32 == 0");
    VX_LAUNCH(ctx, pack_x, dim3(K / 32), dim3(64), x, x_stride, B, P, packed);
    return 0;
}

int vx_gemv_part(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const uint16_t *packed, int n_seg,
                 int ks_per, float *part) {
    const int groups = (N + 16 * RB - 1) / (16 * RB);
    VX_LAUNCH(ctx, gemv_part, dim3(groups, (n_seg + 3) / 4), dim3(256), W, N, K, packed, ks_per, n_seg, part);
    return 0;
}

extern "C" int vx27_hip_gemv_bf16(vx27_hip_ctx *ctx, const uint16_t *W, int N, int K, const float *x,
                                  size_t x_stride, int B, float *y, size_t y_stride) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(W && x && y, "vx27_hip_gemv_bf16: null pointer");
    VX_REQUIRE(B >= 1 && B <= 5, "vx27_hip_gemv_bf16: B must be 1..5 (got %d)", B);
    int n_seg, ks_per;
    if (vx_gemv_plan(N, K, &n_seg, &ks_per)) return -1;
    const size_t pk = (vx_pack_bytes(K) + 255) & ~(size_t)255;
    void *scr;
    if (vx_ctx_scratch(ctx, pk + vx_gemv_part_bytes(N, n_seg), &scr)) return -1;
    uint16_t *packed = (uint16_t *)scr;
    float *part = (float *)((char *)scr + pk);
    if (vx_pack(ctx, x, x_stride, B, 3, K, packed)) return -1;
    if (vx_gemv_part(ctx, W, N, K, packed, n_seg, ks_per, part)) return -1;
    const size_t n = (size_t)N * B;
    VX_LAUNCH(ctx, gemv_reduce_store, dim3((unsigned)((n + 255) / 256)), dim3(256), part, N, B, 3, n_seg, y,
              y_stride);
    return 0;
}

int vx_gemv_reduce_store(vx27_hip_ctx *ctx, const float *part, int N, int B, int P, int n_seg, float *y,
                         size_t y_stride) {
    const size_t n = (size_t)N * B;
    VX_LAUNCH(ctx, gemv_reduce_store, dim3((unsigned)((n + 255) / 256)), dim3(256), part, N, B, P, n_seg, y,
              y_stride);
    return 0;
}
