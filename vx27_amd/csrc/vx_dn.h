// Internal interface of the DeltaNet recurrence kernel (vx_dn_decode.hip),
// shared with the layer entry points (vx_layer.hip).
#pragma once
#include "vx_common.h"

namespace {
constexpr int HD = 128;

// silu1 of vx27_qfwd.c:48 / vx27_deltanet.c:104
__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

// softplus with the reference's tails (vx27_deltanet.c:58-63)
__device__ __forceinline__ double softplus_d(double x) {
    if (x > 20.0) return x;
    if (x < -20.0) return exp(x);
    return log(1.0 + exp(x));
}

// one causal-conv step of a channel (vx27_deltanet.c:106-122): window
// (c0 oldest, c1, c2, x), products summed left to right, then SiLU
__device__ __forceinline__ float conv_step(float c[3], const float w[4], float x) {
    float acc = w[0] * c[0];
    acc = acc + w[1] * c[1];
    acc = acc + w[2] * c[2];
    acc = acc + w[3] * x;
    c[0] = c[1];
    c[1] = c[2];
    c[2] = x;
    return silu_f(acc);
}

__device__ __forceinline__ void load_conv_w(const void *w, int bf16, size_t ch, float out[4]) {
    if (bf16) {
        const uint16_t *p = (const uint16_t *)w + ch * 4;
#pragma unroll
        for (int t = 0; t < 4; t++) out[t] = vx_bf16_to_f32(p[t]);
    } else {
        const float *p = (const float *)w + ch * 4;
#pragma unroll
        for (int t = 0; t < 4; t++) out[t] = p[t];
    }
}
// Conv weights held as raw words (bf16: the 4 values in r[0..1]; f32:
// r[0..3]), converted after the load so that the load's wait falls at the
// first use of the values.
__device__ __forceinline__ void conv_w_decode(int bf16, const uint32_t r[4], float out[4]) {
    if (bf16) {
        out[0] = __uint_as_float(r[0] << 16);
        out[1] = __uint_as_float(r[0] & 0xffff0000u);
        out[2] = __uint_as_float(r[1] << 16);
        out[3] = __uint_as_float(r[1] & 0xffff0000u);
    } else {
#pragma unroll
        for (int t = 0; t < 4; t++) out[t] = __uint_as_float(r[t]);
    }
}
// Sum of two per-lane doubles over all NW waves of the block (wave partials
// added in wave order); every thread must call it (barrier inside).  slot is
// private to one call site.
template <int NW>
__device__ __forceinline__ void block_sum2(double &u, double &v, double (*slot)[2]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const double su = vx_wave_sum_f64_dpp(u), sv = vx_wave_sum_f64_dpp(v);
    if (lane == 0) {
        slot[wave][0] = su;
        slot[wave][1] = sv;
    }
    __syncthreads();
    double a0 = slot[0][0], a1 = slot[0][1];
#pragma unroll
    for (int w = 1; w < NW; w++) {
        a0 = a0 + slot[w][0];
        a1 = a1 + slot[w][1];
    }
    u = a0;
    v = a1;
}

// Sum over the R adjacent lanes that share a state column (butterfly; every
// lane of the group ends with the same bits since each add is commutative).
}  // namespace

// Internal flag: q and k are final (normalised and scaled as step_exact
// leaves them); the recurrence skips every q/k normalisation.
constexpr unsigned VX_DN_QK_READY = 1u << 16;

struct DnArgs {
    int B, nqk, nv, steps;
    // per-token arrays (x, q, k, v, gates, ga/gb, z, out) hold token t of
    // sequence b at index t * t_step + b * b_step (times the array's own
    // stride): t_step = B, b_step = 1 is the decode layout [steps][B];
    // t_step = 1, b_step = T the prefill layout [B][T].  0 means the decode
    // layout.
    int t_step, b_step;
    unsigned flags;
    int fused_conv;
    float *S;
    float *conv_state;
    const void *conv_w;
    int conv_bf16;
    // activations: either x (fused conv) or q/k/v (already convolved or given)
    const float *x;
    const float *q, *k, *v;
    size_t q_tok, k_tok, v_tok;   // per-(t,b) stride of q, k, v in floats
    const double2 *gates;         // [steps][B][nv] (beta, decay); NULL: the step kernel
                                  // maps ga, gb (one step) itself
    const float *ga, *gb;         // raw gate inputs [B][nv] (vx27_deltanet_gate_params's a, b)
    const float *A_log, *dt_bias; // [nv]
    const float *norm_w, *z;
    size_t z_tok;                 // per-(t,b) stride of z
    float *out;                   // may be NULL when out_packed is set
    size_t out_tok;               // per-(t,b) stride of out
    uint16_t *out_packed;         // optional: out as the packed GEMV operand (steps == 1)
    // optional scratch [B][nv][128] for pre-norm outputs: lets a single-step
    // call with VX27_DN_OUT_GATE split each head's columns over workgroups
    // (the output norm then runs in a separate finish kernel)
    float *o_pre;
    // optional scratch of vx_dn_qk_bytes(a) bytes: a multi-step call (no fused
    // conv) then normalises every token's q and k up front, in parallel, and
    // the recurrence's per-token chain skips the q/k normalisation
    float *qk_buf;
};
// bytes of DnArgs::qk_buf: q and k of every (token, sequence), [steps*B][nqk][128] each
inline size_t vx_dn_qk_bytes(int steps, int B, int nqk) { return (size_t)2 * steps * B * nqk * HD * sizeof(float); }

// Channel-parallel causal conv over `steps` tokens (dn_conv_kernel): one
// thread per (b, c), the state carried in registers; act receives silu(conv).
struct ConvArgs {
    int B, C, steps, w_bf16;
    float *state;         // [B][C][3], oldest first; left as after the last token
    const void *w;
    const float *x;
    float *act;
    int t_step, b_step;   // token (t, b) of x and act at row t * t_step + b * b_step
    float *ckpt;          // optional: the state after each token, [rows][C][3] in the same row order
};
int vx_dn_conv(vx27_hip_ctx *ctx, const ConvArgs &ca);
// (beta, exp(g_log)) of n gate inputs (vx27_deltanet_gate_params), value head e % nv
int vx_dn_gates(vx27_hip_ctx *ctx, size_t n, int nv, const float *ga, const float *gb, const float *A_log,
                const float *dt_bias, double2 *gates);

// Launch the recurrence (one or more workgroups per (sequence, value head)).
int vx_dn_recurrence(vx27_hip_ctx *ctx, const DnArgs &a);
// Whether vx_dn_recurrence runs a call as one single-step kernel (which can
// also map the gates itself, with gates == NULL).
bool vx_dn_single_step(const DnArgs &a);

// The DeltaNet prefill on caller-provided scratch (vx_dn_prefill.hip), for
// entry points that hold other scratch of their own at the same time.
size_t vx_dn_prefill_scratch(const vx27_dn_prefill_desc *d);
// out_packed: the gated output written instead as the long-prompt GEMM's
// packed tokens (vx_gemm_pack_unit, K = nv 128) for a projection that takes
// it next; the chunked form with VX27_DN_OUT_GATE only (d->out then holds
// the ungated output).
int vx_dn_prefill_into(vx27_hip_ctx *ctx, const vx27_dn_prefill_desc *d, void *scr, char *out_packed = nullptr);
