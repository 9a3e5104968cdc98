// Internal interface of the gated-GQA kernels: the bf16 KV-cache format, the
// RoPE frequency table, and the decode step used by the layer entry point.
#pragma once
#include "vx_common.h"

constexpr int VX_GQA_HD = 256;      // head dim of the gated GQA layers
constexpr int VX_GQA_VBLK = 32;     // positions per dim-major V block
constexpr int VX_ROPE_MAXH = 128;   // max rope_dim/2

// K: [B][n_kv][L][256]; V: [B][n_kv][L/32][256][32]
__device__ __forceinline__ size_t vx_k_index(int n_kv, int L, int b, int h, int p, int i) {
    return (((size_t)b * n_kv + h) * L + p) * VX_GQA_HD + i;
}
__device__ __forceinline__ size_t vx_v_index(int n_kv, int L, int b, int h, int p, int i) {
    return ((((size_t)b * n_kv + h) * (L / VX_GQA_VBLK) + p / VX_GQA_VBLK) * VX_GQA_HD + i) * VX_GQA_VBLK +
           (p % VX_GQA_VBLK);
}

// RoPE inverse frequencies freq_i = powf(theta, -2i/rope_dim) in the
// reference's float arithmetic (vx27_rope.c:11), computed on the host; the
// kernels form angle = ((float)pos / yarn) * freq_i in float as well.
struct vx_rope_tab {
    float freq[VX_ROPE_MAXH];
};
int vx_rope_fill(vx_rope_tab &t, int rope_dim, float theta);

// cos and sin of frequency i at position pos: angle = ((float)pos / yarn) *
// freq_i in float, then the device's float cosf/sinf (vx27_rope.c:11-14).
// Every kernel that rotates (decode prep, prefill k/v and query prologues
// through the prefill's table, vx27_hip_rope_table) evaluates it here.
__device__ __forceinline__ float vx_rope_angle(float freq, int pos, float yarn) {
    return ((float)pos / yarn) * freq;
}
__device__ __forceinline__ float2 vx_rope_cs_angle(float ang) {
    float sn, cs;
    sincosf(ang, &sn, &cs);   // (one argument reduction for both)
    return make_float2(cs, sn);
}
__device__ __forceinline__ float2 vx_rope_cs_f(float freq, int pos, float yarn) {
    return vx_rope_cs_angle(vx_rope_angle(freq, pos, yarn));
}
__device__ __forceinline__ float2 vx_rope_cs(const vx_rope_tab &t, int pos, float yarn, int i) {
    return vx_rope_cs_f(t.freq[i], pos, yarn);
}

size_t vx_gqa_scratch_bytes(const vx27_gqa_desc *d);
// The decode step with caller-provided scratch of vx_gqa_scratch_bytes(d);
// out_packed (optional) receives the gated attention as the packed operand of
// the output projection.
int vx_gqa_decode_into(vx27_hip_ctx *ctx, const vx27_gqa_desc *d, void *scr, uint16_t *out_packed,
                       float *zero = nullptr, size_t zero_n = 0);

// Looks up the per-device address of the no-allocation decode scratch
// (vx_gqa_decode.hip); called by vx27_hip_open with the device current.
int vx_noalloc_init(int device);
// The prefill on caller-provided scratch (vx_gqa_prefill.hip).
size_t vx_gqa_prefill_scratch(const vx27_gqa_prefill_desc *d);
int vx_gqa_prefill_into(vx27_hip_ctx *ctx, const vx27_gqa_prefill_desc *d, void *scr);
