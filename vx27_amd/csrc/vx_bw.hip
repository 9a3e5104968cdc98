// HBM bandwidth probe: a plain streaming read kernel and a plain copy kernel
// over device memory, timed with events on the context stream.  The rates
// they reach on a buffer far larger than the 256 MiB Infinity Cache are the
// practical ceilings the decode kernels are compared with (a measurement
// utility; no counterpart in the reference).
#include <algorithm>

#include "vx_common.h"

namespace {
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Workgroup w streams its own contiguous chunk of the n 16-byte units (the
// last workgroup also takes the remainder), four streaming loads of 256
// threads in flight per step: on gfx950 this reaches about 7.1 TB/s, against
// 5.7-6.8 TB/s for a grid-stride loop over the same buffer.  The XOR of
// everything read is stored only if it equals a constant (never, in
// practice), which keeps every load live.
__device__ __forceinline__ void bw_chunk(size_t n, size_t &lo, size_t &hi) {
    const size_t per = n / gridDim.x;
    lo = per * blockIdx.x;
    hi = blockIdx.x + 1 == gridDim.x ? n : lo + per;
}
__global__ __launch_bounds__(256) void bw_read_kernel(const u32x4_t *p, size_t n, uint32_t *sink) {
    size_t lo, hi;
    bw_chunk(n, lo, hi);
    u32x4_t acc = {0u, 0u, 0u, 0u};
    size_t i = lo + threadIdx.x;
    for (; i + 3 * 256 < hi; i += 4 * 256) {
        const u32x4_t a = __builtin_nontemporal_load(p + i);
        const u32x4_t b = __builtin_nontemporal_load(p + i + 256);
        const u32x4_t c = __builtin_nontemporal_load(p + i + 512);
        const u32x4_t d = __builtin_nontemporal_load(p + i + 768);
        acc ^= (a ^ b) ^ (c ^ d);
    }
    for (; i < hi; i += 256) acc ^= __builtin_nontemporal_load(p + i);
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == 0x9e3779b9u) sink[0] = x;
}

// dst = src over n 16-byte units, the same chunking, streaming loads and stores
__global__ __launch_bounds__(256) void bw_copy_kernel(const u32x4_t *src, u32x4_t *dst, size_t n) {
    size_t lo, hi;
    bw_chunk(n, lo, hi);
    size_t i = lo + threadIdx.x;
    for (; i + 3 * 256 < hi; i += 4 * 256) {
        const u32x4_t a = __builtin_nontemporal_load(src + i);
        const u32x4_t b = __builtin_nontemporal_load(src + i + 256);
        const u32x4_t c = __builtin_nontemporal_load(src + i + 512);
        const u32x4_t d = __builtin_nontemporal_load(src + i + 768);
        __builtin_nontemporal_store(a, dst + i);
        __builtin_nontemporal_store(b, dst + i + 256);
        __builtin_nontemporal_store(c, dst + i + 512);
        __builtin_nontemporal_store(d, dst + i + 768);
    }
    for (; i < hi; i += 256) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}
}  // namespace

extern "C" int vx27_hip_bw_probe(vx27_hip_ctx *ctx, size_t bytes, int iters, double *read_GBs, double *copy_GBs) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(read_GBs && copy_GBs, "vx27_hip_bw_probe: null result pointer");
    VX_REQUIRE(bytes >= ((size_t)1 << 20) && iters >= 1 && iters <= 1000,
               "vx27_hip_bw_probe: bytes must be at least 1 MiB and iters in [1, 1000]");
    VX_REQUIRE(!vx_ctx_capturing(ctx), "vx27_hip_bw_probe: not inside a graph capture");
    const size_t n = (bytes / 2) / 16;   // units per half: the copy reads one half into the other
    void *buf = nullptr;
    uint32_t *sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = -1;
    double best_r = 0.0, best_c = 0.0;
    const dim3 grid((unsigned)(ctx->n_cu * 2)), block(256);
    auto fail = [&](hipError_t e, const char *what) {
        vx_set_error("vx27_hip_bw_probe: %s: %s", what, hipGetErrorString(e));
    };
    hipError_t e;
    if ((e = hipMalloc(&buf, 2 * n * 16)) != hipSuccess) { fail(e, "hipMalloc"); goto done; }
    if ((e = hipMalloc((void **)&sink, 256)) != hipSuccess) { fail(e, "hipMalloc"); goto done; }
    if ((e = hipMemsetAsync(buf, 0x5a, 2 * n * 16, ctx->stream)) != hipSuccess) { fail(e, "hipMemsetAsync"); goto done; }
    if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess) {
        fail(e, "hipEventCreate");
        goto done;
    }
    for (int it = 0; it <= iters; it++) {   // iteration 0 warms up
        float ms_r = 0.f, ms_c = 0.f;
        const u32x4_t *src = (const u32x4_t *)buf;
        u32x4_t *dst = (u32x4_t *)buf + n;
        (void)hipEventRecord(e0, ctx->stream);
        hipLaunchKernelGGL(bw_read_kernel, grid, block, 0, ctx->stream, src, 2 * n, sink);
        (void)hipEventRecord(e1, ctx->stream);
        if ((e = hipEventSynchronize(e1)) != hipSuccess) { fail(e, "read kernel"); goto done; }
        (void)hipEventElapsedTime(&ms_r, e0, e1);
        (void)hipEventRecord(e0, ctx->stream);
        hipLaunchKernelGGL(bw_copy_kernel, grid, block, 0, ctx->stream, src, dst, n);
        (void)hipEventRecord(e1, ctx->stream);
        if ((e = hipEventSynchronize(e1)) != hipSuccess) { fail(e, "copy kernel"); goto done; }
        (void)hipEventElapsedTime(&ms_c, e0, e1);
        if (it > 0 && ms_r > 0.f) best_r = std::max(best_r, (double)(2 * n * 16) / (ms_r * 1e-3) / 1e9);
        if (it > 0 && ms_c > 0.f) best_c = std::max(best_c, (double)(2 * n * 16) / (ms_c * 1e-3) / 1e9);
    }
    *read_GBs = best_r;
    *copy_GBs = best_c;
    rc = 0;
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (sink) (void)hipFree(sink);
    if (buf) (void)hipFree(buf);
    return rc;
}
