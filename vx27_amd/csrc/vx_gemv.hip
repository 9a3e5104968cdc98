// Skinny bf16 GEMM (the mixer projections) on gfx950 MFMA.
//
// y[b][n] = sum_k W[n][k] * x[b][k] for B <= 5 activation vectors (decode:
// one token per sequence), W bf16 [N][K] (the reference's weight tensors,
// vx27_pmat.h:6-8), x and y fp32.
//
// The fp32 activations enter the MFMA exactly: each x is split into three
// bf16 parts hi + mid + lo (8 mantissa bits each, 24 in all), and the parts
// of the B vectors are the columns of the MFMA's B operand (3*B <= 15 of the
// 16 columns).  One v_mfma_f32_16x16x32_bf16 therefore multiplies 16 weight
// rows by every part of every vector; the products are exact in fp32 and the
// only rounding is the fp32 accumulation, as in a plain fp32 dot product.
// Output column n of an MFMA depends only on operand column n, so operand
// columns >= 3*B may hold anything: they feed output columns nobody reads.
//
// Layouts:
//   packed activations  [K/32 k-steps][64 lanes][8] bf16: lane (g,n) of k-step
//                       s holds part n/B of vector n%B at k = 32s + 8g + 0..7
//   tiled weights       [K/(32 KG) k-groups][N/16 row blocks][KG][64 lanes][8]
//                       bf16 (KG = 4 k-steps when K/32 allows): lane (g,m) of
//                       tile (s, rb) holds W[16*rb + m][32s + 8g + 0..7].  A
//                       wave's A operand is 1 KiB contiguous, a row block's KG
//                       k-steps are adjacent, and so are the row blocks of a
//                       workgroup: one wave's batch of KG k-steps over its 4
//                       row blocks is one 16 KiB run, and neighbouring
//                       workgroups read neighbouring runs
//                       (vx27_hip_pack_weights_bf16 converts row-major W)
//
// gemv_part: a workgroup of 4 waves owns 64 rows (4 row blocks); its waves
// take 4 consecutive K segments and are combined in LDS, so one partial
// [N][16] fp32 is written per workgroup-segment; the reductions sum them in a
// fixed order (deterministic) and apply an epilogue.
#include "vx_gemv.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int RB = 4;   // 16-row MFMA blocks per workgroup
#ifndef VX_GEMV_WAVES
#define VX_GEMV_WAVES 2048   // target waves per launch
#endif
#ifndef VX_GEMV_MINKS
#define VX_GEMV_MINKS 8      // at least this many 32-wide k-steps per wave
#endif


// pack activations: grid (K/32), block 64; lane (g,n) writes its 8 elements
__global__ __launch_bounds__(64) void pack_x(const float *x, size_t x_stride, int B, uint16_t *out) {
    const int s = blockIdx.x, lane = threadIdx.x, g = lane >> 4, n = lane & 15;
    if (n >= 3 * B) return;   // padding columns feed unread output columns
    const int p = n / B, b = n % B;
    const float *xr = x + (size_t)b * x_stride + 32 * s + 8 * g;
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = vx_bf16_part(xr[e], p);

    uint4 w;
    w.x = v[0] | ((uint32_t)v[1] << 16);
    w.y = v[2] | ((uint32_t)v[3] << 16);
    w.z = v[4] | ((uint32_t)v[5] << 16);
    w.w = v[6] | ((uint32_t)v[7] << 16);
    *(uint4 *)(out + ((size_t)s * 64 + lane) * 8) = w;
}

#ifndef VX_GEMV_KG
#define VX_GEMV_KG 1         // k-steps per group of the tiled layout (1, 2 or 4)
#endif
#ifndef VX_GEMV_U
#define VX_GEMV_U 1          // k-steps per load batch of a wave
#endif
#ifndef VX_GEMV_STRIDED
#define VX_GEMV_STRIDED 0    // K segments interleaved (segment s: k-steps s, s + n_seg, ...)
#endif
// k-steps per group of the tiled weight layout
__host__ __device__ __forceinline__ int gemv_kg(int K) {
    const int nks = K / 32;
    return nks % VX_GEMV_KG == 0 ? VX_GEMV_KG : 1;
}
// element offset of tile (k-step s, row block rb) in the tiled layout
__device__ __forceinline__ size_t tile_off(int s, int rb, int nb, int kg) {
    return ((size_t)(s / kg) * nb + rb) * kg * 512 + (size_t)(s % kg) * 512;
}

// row-major W [N][K] -> tiled; grid (N/16, K/32), block 64
__global__ __launch_bounds__(64) void pack_w(const uint16_t *W, int K, uint16_t *Wt) {
    const int rb = blockIdx.x, s = blockIdx.y, lane = threadIdx.x, g = lane >> 4, m = lane & 15;
    const uint4 v = *(const uint4 *)(W + (size_t)(16 * rb + m) * K + 32 * s + 8 * g);
    *(uint4 *)(Wt + tile_off(s, rb, gridDim.x, gemv_kg(K)) + lane * 8) = v;
}

#ifndef VX_GEMV_NT
#define VX_GEMV_NT 1         // streaming (nontemporal) weight loads
#endif
__device__ __forceinline__ bf16x8_t wload(const bf16x8_t *p) {
    if (VX_GEMV_NT) return __builtin_nontemporal_load(p);
    return *p;
}

// grid (ceil(N/64), ceil(n_seg/4)), block 256; wave w: K segment 4*blockIdx.y + w
template <bool TILED>
__global__ __launch_bounds__(256) void gemv_part_k(const uint16_t *W, int N, int K, const uint16_t *xp,
                                                   int ks_per, int n_seg, float *part) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, m = lane & 15;
    const int seg = blockIdx.y * 4 + wave;
    const int rb0 = blockIdx.x * RB;
    const int nks = K / 32;
    const int s0 = seg * ks_per, s1 = seg < n_seg ? min(nks, s0 + ks_per) : s0;
    __shared__ floatx4_t red[4][RB][64];
    floatx4_t acc[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) acc[r] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    bool live[RB];
    const uint16_t *wp[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) {
        live[r] = (rb0 + r) * 16 < N;          // whole 16-row block in or out (N % 16 == 0)
        const int rb = live[r] ? rb0 + r : 0;
        wp[r] = TILED ? W + tile_off(0, rb, N / 16, gemv_kg(K)) + lane * 8
                      : W + (size_t)(16 * rb + m) * K + 8 * g;
    }
    const bf16x8_t *xb = (const bf16x8_t *)xp + lane;
    // k-steps of this wave: a contiguous segment [s0, s1), or (strided) the
    // k-steps seg, seg + n_seg, ...; loads of U k-steps are issued before the
    // first MFMA of the batch consumes them
    constexpr int U = VX_GEMV_U;
    const int kg = TILED ? gemv_kg(K) : 1;
    const size_t gstride = (size_t)(N / 16) * kg * 512;
    auto woff = [&](int st) -> size_t {
        return TILED ? (size_t)(st / kg) * gstride + (size_t)(st % kg) * 512 : (size_t)st * 32;
    };
    const int sbeg = VX_GEMV_STRIDED ? (seg < n_seg ? seg : nks) : s0;
    const int send = VX_GEMV_STRIDED ? nks : s1;
    const int sinc = VX_GEMV_STRIDED ? n_seg : 1;
    int s = sbeg;
    for (; s + (U - 1) * sinc < send; s += U * sinc) {
        bf16x8_t bop[U], aop[U][RB];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int st = s + u * sinc;
            bop[u] = xb[(size_t)st * 64];
            const size_t off = woff(st);
#pragma unroll
            for (int r = 0; r < RB; r++) aop[u][r] = wload((const bf16x8_t *)(wp[r] + off));
        }
        // dead row blocks (past N in the last workgroup) multiply row block 0
        // and are never stored: no branch in the streaming loop
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int r = 0; r < RB; r++)
                acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[u][r], bop[u], acc[r], 0, 0, 0);
    }
    for (; s < send; s += sinc) {
        const bf16x8_t bop = xb[(size_t)s * 64];
        const size_t off = woff(s);
        bf16x8_t aop[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) aop[r] = wload((const bf16x8_t *)(wp[r] + off));
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[r], bop, acc[r], 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < RB; r++) red[wave][r][lane] = acc[r];
    __syncthreads();
    // wave w sums the four segments of row block w in segment order
    const int r = wave;
    if (!live[r]) return;
    floatx4_t v = red[0][r][lane];
    v += red[1][r][lane];
    v += red[2][r][lane];
    v += red[3][r][lane];
    // lane (g,m) holds C[4g+i][m]: row 16*(rb0+r) + 4g + i, column m
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = 16 * (rb0 + r) + 4 * g + i;
        part[((size_t)blockIdx.y * N + row) * 16 + m] = v[i];
    }
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

int vx_gemv_plan(int N, int K, int *n_seg, int *ks_per) {
    VX_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0,
               "gemv: N must be a multiple of 16 and K of 32 (N=%d K=%d)", N, K);
    const int groups = (N + 16 * RB - 1) / (16 * RB);
    const int nks = K / 32;
    // about VX_GEMV_WAVES waves in all, at least VX_GEMV_MINKS k-steps per wave
    int seg = (VX_GEMV_WAVES + groups - 1) / groups;
    if (seg > nks / VX_GEMV_MINKS) seg = nks / VX_GEMV_MINKS;
    if (seg < 1) seg = 1;
    int per = (nks + seg - 1) / seg;
    const int kg = gemv_kg(K);
    per = (per + kg - 1) / kg * kg;   // segments start at k-group boundaries
    seg = (nks + per - 1) / per;
    *n_seg = seg;
    *ks_per = per;
    return 0;
}

int vx_gemv_pseg(int n_seg) { return (n_seg + 3) / 4; }
size_t vx_gemv_part_bytes(int N, int n_seg) { return (size_t)vx_gemv_pseg(n_seg) * N * 16 * sizeof(float); }
size_t vx_pack_bytes(int K) { return (size_t)(K / 32) * 64 * 8 * sizeof(uint16_t); }

int vx_pack(vx27_hip_ctx *ctx, const float *x, size_t x_stride, int B, int K, uint16_t *packed) {
    VX_REQUIRE(B >= 1 && B <= 5 && K % 32 == 0, "pack: need B <= 5, K %% 32 == 0");
    VX_LAUNCH(ctx, pack_x, dim3(K / 32), dim3(64), x, x_stride, B, packed);
    return 0;
}

int vx_gemv_part(vx27_hip_ctx *ctx, const uint16_t *W, int tiled, int N, int K, const uint16_t *packed,
                 int n_seg, int ks_per, float *part) {
    const dim3 grid((N + 16 * RB - 1) / (16 * RB), vx_gemv_pseg(n_seg));
    if (tiled)
        VX_LAUNCH(ctx, gemv_part_k<true>, grid, dim3(256), W, N, K, packed, ks_per, n_seg, part);
    else
        VX_LAUNCH(ctx, gemv_part_k<false>, grid, dim3(256), W, N, K, packed, ks_per, n_seg, part);
    return 0;
}

int vx_gemv_reduce_store(vx27_hip_ctx *ctx, const float *part, int N, int B, int n_seg, float *y,
                         size_t y_stride) {
    VX_LAUNCH(ctx, gemv_reduce_store, dim3((N + 255) / 256), dim3(256), part, N, B, vx_gemv_pseg(n_seg), y,
              y_stride);
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
    VX_REQUIRE(B >= 1 && B <= 5, "vx27_hip_gemv_bf16: B must be 1..5 (got %d)", B);
    int n_seg, ks_per;
    if (vx_gemv_plan(N, K, &n_seg, &ks_per)) return -1;
    const size_t pk = (vx_pack_bytes(K) + 255) & ~(size_t)255;
    void *scr;
    if (vx_ctx_scratch(ctx, pk + vx_gemv_part_bytes(N, n_seg), &scr)) return -1;
    uint16_t *packed = (uint16_t *)scr;
    float *part = (float *)((char *)scr + pk);
    if (vx_pack(ctx, x, x_stride, B, K, packed)) return -1;
    if (vx_gemv_part(ctx, W, 0, N, K, packed, n_seg, ks_per, part)) return -1;
    return vx_gemv_reduce_store(ctx, part, N, B, n_seg, y, y_stride);
}
