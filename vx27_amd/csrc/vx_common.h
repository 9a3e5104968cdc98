// Internal helpers shared by the HIP translation units of libvx27_hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <vector>

#include "vx27_hip.h"

// one profiled launch: events recorded around it on the context stream
struct vx_prof_rec {
    const char *name;
    hipEvent_t e0, e1;
};

struct vx27_hip_ctx {
    int device;
    hipStream_t stream;      // stream used for every enqueue
    hipStream_t own_stream;  // created by vx27_hip_open
    // grow-only device scratch (split-K partials, prefill chunk records),
    // owned by the context
    void *scratch;
    size_t scratch_bytes;
    // small staging for the drop-ins (host-pointer API)
    void *stage;
    size_t stage_bytes;
    int n_cu;                // compute units of the device
    // prefill attention work schedules, one per shape (vx_gqa_prefill.hip)
    std::vector<void *> gqp_scheds;
    // Executable graphs captured on this context that are not yet destroyed.
    // A captured graph keeps the raw addresses of the scratch buffer and of
    // the schedules it was captured with, so while any is alive a buffer
    // that scratch growth replaces is kept here (not freed) until the last
    // graph is destroyed or the context is closed.
    int live_graphs;
    std::vector<void *> retired;
    // device flag set by a decode kernel that saw a position outside its KV
    // cache; read back (into err_host, pinned) and cleared by vx27_hip_sync
    int *err_flag;
    int *err_host;
    // kernel profiler (vx27_hip_prof_*): off unless enabled
    int prof_on;
    vx_prof_rec *prof;
    int prof_n, prof_cap;
};

// thread-local error message
void vx_set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

#define VX_HIP(expr)                                                                   \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess) {                                                        \
            vx_set_error("%s:%d %s: %s", __FILE__, __LINE__, #expr, hipGetErrorString(e_)); \
            return -1;                                                                 \
        }                                                                              \
    } while (0)

#define VX_REQUIRE(cond, ...)          \
    do {                               \
        if (!(cond)) {                 \
            vx_set_error(__VA_ARGS__); \
            return -1;                 \
        }                              \
    } while (0)

#define VX_LAUNCHED(name)                                                                    \
    do {                                                                                     \
        hipError_t e_ = hipGetLastError();                                                   \
        if (e_ != hipSuccess) {                                                              \
            vx_set_error("%s:%d launch of %s failed: %s", __FILE__, __LINE__, name,          \
                         hipGetErrorString(e_));                                             \
            return -1;                                                                       \
        }                                                                                    \
    } while (0)

// Kernel profiler hooks (see vx27_hip_prof_enable).
void vx_prof_begin(vx27_hip_ctx *ctx);
void vx_prof_end(vx27_hip_ctx *ctx, const char *name);

// Launch `kernel` on the context stream (profiled when enabled) and check it.
#define VX_LAUNCH(ctx, kernel, grid, block, ...)                                  \
    do {                                                                          \
        vx_prof_begin(ctx);                                                       \
        hipLaunchKernelGGL(kernel, grid, block, 0, (ctx)->stream, __VA_ARGS__);   \
        vx_prof_end(ctx, #kernel);                                                \
        VX_LAUNCHED(#kernel);                                                     \
    } while (0)

// The same with the profiler name given (for template instances whose
// argument list needs parentheses in the macro call).
#define VX_LAUNCH_NAMED(ctx, name, kernel, grid, block, ...)                       \
    do {                                                                          \
        vx_prof_begin(ctx);                                                       \
        hipLaunchKernelGGL(kernel, grid, block, 0, (ctx)->stream, __VA_ARGS__);   \
        vx_prof_end(ctx, name);                                                   \
        VX_LAUNCHED(name);                                                        \
    } while (0)

// Make the context's device current (contexts may live on different devices).
int vx_ctx_enter(vx27_hip_ctx *ctx);
// Device scratch of at least `bytes`, owned by ctx (synchronises before growing).
int vx_ctx_scratch(vx27_hip_ctx *ctx, size_t bytes, void **out);
// frees the cached prefill attention schedules (vx_gqa_prefill.hip)
void vx_gqp_sched_free(vx27_hip_ctx *ctx);
// Device memory owned by the context: freed now, or (while a captured graph
// that may reference it is alive) kept until the last such graph is gone.
void vx_ctx_release(vx27_hip_ctx *ctx, void *dptr);
// Nonzero while the context stream is capturing a graph.
bool vx_ctx_capturing(vx27_hip_ctx *ctx);
// Host-pointer staging buffer of at least `bytes` (device memory).
int vx_ctx_stage(vx27_hip_ctx *ctx, size_t bytes, void **out);

// ------------------------------------------------------------ device math
__device__ __forceinline__ float vx_bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}
// round-to-nearest-even narrowing (NaN kept quiet)
__device__ __forceinline__ uint16_t vx_f32_to_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Full-wave (64 lanes) sums and maxima through cross-lane shuffles.
__device__ __forceinline__ double vx_wave_sum_f64(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float vx_wave_sum_f32(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
// The same sum on the VALU's DPP paths, without the LDS crossbar that the
// shuffles go through: a butterfly inside each quad, row rotations by 4 and
// 8 (every lane of a 16-lane row then holds the row sum), the row
// broadcasts 15 and 31 (lane 63 then holds the wave sum), and lane 63 read
// back.  A fixed tree, so the result is the same on every call.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double vx_dpp_f64(double x) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
// The value of lane l ^ 32 (gfx950 v_permlane32_swap: a VALU exchange of
// the wave's two 32-lane halves).
__device__ __forceinline__ uint32_t vx_xor32_u32(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
}
__device__ __forceinline__ double vx_xor32_f64(double x) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint64_t lo = vx_xor32_u32((uint32_t)u), hi = vx_xor32_u32((uint32_t)(u >> 32));
    return __builtin_bit_cast(double, (hi << 32) | lo);
}
__device__ __forceinline__ double vx_wave_sum_f64_dpp(double v) {
    v = v + vx_dpp_f64<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = v + vx_dpp_f64<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = v + vx_dpp_f64<0x124, 0xF>(v);   // row_ror:4
    v = v + vx_dpp_f64<0x128, 0xF>(v);   // row_ror:8
    v = v + vx_dpp_f64<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3 (others add +0)
    v = v + vx_dpp_f64<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
