// Whole-mixer layer steps (projections + mixer core + output projection),
// device-side synthetic fills and HIP-graph capture.
//
// DeltaNet layer (vx27_qfwd.c:102-153), one decode token of B sequences:
//   gemv_dn_in               [qkv | z | a | b] projection with its epilogue
//                            (DnInEpi): causal conv/SiLU on qkv (state in
//                            place), z, a and b copied out
//   dn_step_kernel           gates (decay from a, beta from b), q/k
//                            normalisation chain, exact step, gated output
//                            norm, output written as the packed operand of
//                            W_out
//   gemv_wk_store(W_out)     -> out
// Gated GQA layer (vx27_qfwd.c:162-213):
//   gemv_wk_store(W_qkv)     -> [q|gate interleaved | k | v]
//   gqa_prep / gqa_split / gqa_combine (vx_gqa_decode.hip; the combine
//                            writes the packed operand of W_o)
//   gemv_wk_store(W_o)       -> out
// (the GEMVs are whole-K workgroups with the reduction in LDS:
// vx_gemv_body.h)
#include <math.h>

#include <algorithm>

#include "vx_dn.h"
#include "vx_gemv_body.h"
#include "vx_gqa.h"


namespace {

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct DnInArgs {
    int B, C, vd, nv;
    float *conv_state;
    const void *conv_w;
    int conv_bf16;
    float *act, *z;
    float *ga, *gb;   // the a and b rows, [B][nv] each (the step kernel maps them to the gates)
    int b0;   // first vector of this pass (the pass's B vectors are b0 .. b0+B-1)
    float *zero;    // optional: zero_n floats cleared (the output out_proj adds its halves into)
    size_t zero_n;
};

// Epilogue of the stacked DeltaNet input projection [qkv | z | a | b]
// (vx27_qfwd.c:102-117): one thread per row for all vectors of a pass of up
// to DN_PREB vectors, one thread per (row, vector) for larger passes:
//   q|k|v rows: causal conv + SiLU (conv state in place) -> act; the q/k
//               normalisation chain runs in the recurrence kernel, which
//               has whole heads
//   z, a, b rows: copied out (the step kernel maps a and b to decay and
//               beta, after its state loads are issued: no WG of this
//               kernel waits on transcendental code)
// For passes of up to DN_PREB vectors the conv weights (raw bits, converted
// after the loop so that nothing waits on them) and the conv state of a
// q|k|v row are loaded before the projection's K loop.
constexpr int DN_PREB = 5;
struct DnInEpi {
    DnInArgs a;
    struct Pre {
        uint32_t w[4];   // bf16: 4 values in w[0..1]; f32: 4 values
        float st[DN_PREB][3];
    };
    __device__ __forceinline__ Pre prefetch(int row0, int rows, int tid) const {
        Pre p;
        const int n = row0 + tid;
        if (a.B <= DN_PREB && tid < rows && n < a.C) {
            if (a.conv_bf16) {
                const uint2 u = *((const uint2 *)a.conv_w + n);
                p.w[0] = u.x;
                p.w[1] = u.y;
            } else {
                const uint4 u = *((const uint4 *)a.conv_w + n);
                p.w[0] = u.x;
                p.w[1] = u.y;
                p.w[2] = u.z;
                p.w[3] = u.w;
            }
#pragma unroll
            for (int b = 0; b < DN_PREB; b++)
                if (b < a.B) {
                    const float *sp = a.conv_state + ((size_t)(a.b0 + b) * a.C + n) * 3;
                    p.st[b][0] = sp[0];
                    p.st[b][1] = sp[1];
                    p.st[b][2] = sp[2];
                }
        }
        return p;
    }
    // conv taps of channel n from their raw words (bf16 pairs or fp32)
    __device__ __forceinline__ void taps(const uint32_t u[4], float w[4]) const {
        if (a.conv_bf16) {
            w[0] = __uint_as_float(u[0] << 16);
            w[1] = __uint_as_float(u[0] & 0xffff0000u);
            w[2] = __uint_as_float(u[1] << 16);
            w[3] = __uint_as_float(u[1] & 0xffff0000u);
        } else {
#pragma unroll
            for (int t = 0; t < 4; t++) w[t] = __uint_as_float(u[t]);
        }
    }
    // one (row n, vector b) result y
    __device__ __forceinline__ void item(int n, int b, float y) const {
        if (n < a.C) {
            uint32_t u[4] = {0u, 0u, 0u, 0u};
            if (a.conv_bf16) {
                const uint2 v = *((const uint2 *)a.conv_w + n);
                u[0] = v.x;
                u[1] = v.y;
            } else {
                const uint4 v = *((const uint4 *)a.conv_w + n);
                u[0] = v.x;
                u[1] = v.y;
                u[2] = v.z;
                u[3] = v.w;
            }
            float w[4];
            taps(u, w);
            float *sp = a.conv_state + ((size_t)(a.b0 + b) * a.C + n) * 3;
            float st[3] = {sp[0], sp[1], sp[2]};
            a.act[(size_t)(a.b0 + b) * a.C + n] = conv_step(st, w, y);
            sp[0] = st[0]; sp[1] = st[1]; sp[2] = st[2];
        } else if (n < a.C + a.vd) {
            a.z[(size_t)(a.b0 + b) * a.vd + (n - a.C)] = y;
        } else if (n < a.C + a.vd + a.nv) {
            a.ga[(size_t)(a.b0 + b) * a.nv + (n - a.C - a.vd)] = y;
        } else {
            a.gb[(size_t)(a.b0 + b) * a.nv + (n - a.C - a.vd - a.nv)] = y;
        }
    }
    template <int RB, int G>
    __device__ __forceinline__ void operator()(int row0, int rows, const WkRows<RB, G> &c, int tid,
                                               const Pre &p) const {
        if (a.zero) {   // this workgroup's share of the range to clear
            const size_t nwg = gridDim.x, wg = blockIdx.x;
            const size_t lo = a.zero_n * wg / nwg, hi = a.zero_n * (wg + 1) / nwg;
            for (size_t i = lo + tid; i < hi; i += blockDim.x) a.zero[i] = 0.0f;
        }
        if (a.B > DN_PREB) {   // more vectors: one thread per (row, vector)
            for (int t = tid; t < rows * a.B; t += blockDim.x) {
                const int r = t % rows, b = t / rows;
                item(row0 + r, b, c.y(r, b));
            }
            return;
        }
        if (tid >= rows) return;   // up to DN_PREB vectors: one thread per row, prefetched state
        const int n = row0 + tid;
        if (n < a.C) {                       // q, k or v channel: causal conv + SiLU
            float w[4];
            taps(p.w, w);
            auto step = [&](int b, float st[3]) {
                float *sp = a.conv_state + ((size_t)(a.b0 + b) * a.C + n) * 3;
                a.act[(size_t)(a.b0 + b) * a.C + n] = conv_step(st, w, c.y(tid, b));
                sp[0] = st[0]; sp[1] = st[1]; sp[2] = st[2];
            };
#pragma unroll
            for (int b = 0; b < DN_PREB; b++)   // the prefetched states
                if (b < a.B) {
                    float st[3] = {p.st[b][0], p.st[b][1], p.st[b][2]};
                    step(b, st);
                }
        } else if (n < a.C + a.vd) {         // z
            for (int b = 0; b < a.B; b++) a.z[(size_t)(a.b0 + b) * a.vd + (n - a.C)] = c.y(tid, b);
        } else if (n < a.C + a.vd + a.nv) {  // a
            const int vh = n - a.C - a.vd;
            for (int b = 0; b < a.B; b++) a.ga[(size_t)(a.b0 + b) * a.nv + vh] = c.y(tid, b);
        } else {                             // b
            const int vh = n - a.C - a.vd - a.nv;
            for (int b = 0; b < a.B; b++) a.gb[(size_t)(a.b0 + b) * a.nv + vh] = c.y(tid, b);
        }
    }
};

template <int RB, int G>
__global__ __launch_bounds__(VX_WK_NW * 64) void gemv_dn_in(WkWeights wt, int N, int K, const uint16_t *xp, int Gt,
                                                           int g0, int B, DnInEpi epi) {
    vx_gemv_wk_body<RB, G>(wt, N, K, xp, Gt, g0, B, 1, epi);   // whole rows (the conv needs them)
}

__global__ void advance_pos_kernel(int *pos, int B) {
    const int b = threadIdx.x;
    if (b < B) pos[b] += 1;
}

// splitmix64 finaliser
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ float normal_at(uint64_t seed, size_t i) {
    const uint64_t h1 = mix64(seed + 0x9e3779b97f4a7c15ull * (2 * (uint64_t)i + 1));
    const uint64_t h2 = mix64(seed + 0x9e3779b97f4a7c15ull * (2 * (uint64_t)i + 2));
    const float u1 = ((float)(h1 >> 40) + 1.0f) * (1.0f / 16777216.0f);   // (0, 1]
    const float u2 = (float)(h2 >> 40) * (1.0f / 16777216.0f);            // [0, 1)
    return sqrtf(-2.0f * __logf(u1)) * __cosf(6.2831853071795864f * u2);
}
__global__ void fill_f32_kernel(float *p, size_t n, uint64_t seed, float mean, float std) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = mean + std * normal_at(seed, i);
}
__global__ void fill_bf16_kernel(uint16_t *p, size_t n, uint64_t seed, float mean, float std) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = vx_f32_to_bf16(mean + std * normal_at(seed, i));
}

// q|gate|k|v projection rows [R][Nq + 2 kvd] fp32 -> bf16 operands of the
// GQA prefill: qg [R][Nq] (q_proj's interleaved layout kept), k, v [R][kvd].
// grid (R, ceil((Nq + 2 kvd) / 256)), block 256.
__global__ __launch_bounds__(256) void qkv_to_bf16(const float *y, int Nq, int kvd, uint16_t *qg, uint16_t *k,
                                                   uint16_t *v) {
    const size_t r = blockIdx.x;
    const int j = blockIdx.y * 256 + threadIdx.x, N = Nq + 2 * kvd;
    if (j >= N) return;
    const uint16_t h = vx_f32_to_bf16(y[r * N + j]);
    if (j < Nq) qg[r * Nq + j] = h;
    else if (j < Nq + kvd) k[r * kvd + (j - Nq)] = h;
    else v[r * kvd + (j - Nq - kvd)] = h;
}

}  // namespace

extern "C" size_t vx27_hip_pack_bytes(int K, int B) { return vx_pack_bytes(K, B); }

extern "C" int vx27_hip_pack_x(vx27_hip_ctx *ctx, const float *x, int B, int K, uint16_t *packed) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(x && packed && B >= 1, "vx27_hip_pack_x: bad arguments");
    return vx_pack(ctx, x, (size_t)K, B, K, packed);
}

extern "C" int vx27_hip_dn_layer_decode(vx27_hip_ctx *ctx, const vx27_dn_layer_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d != nullptr, "vx27_hip_dn_layer_decode: null descriptor");
    VX_REQUIRE(d->hd == HD, "vx27_hip_dn_layer_decode: hd must be 128");
    VX_REQUIRE(d->B >= 1, "vx27_hip_dn_layer_decode: B must be >= 1 (got %d)", d->B);
    VX_REQUIRE(d->nqk >= 1 && d->nv % d->nqk == 0 && d->nv % 8 == 0,
               "vx27_hip_dn_layer_decode: nv must be a multiple of nqk and of 8 (nqk=%d nv=%d)", d->nqk, d->nv);
    VX_REQUIRE(d->hidden > 0 && d->hidden % 32 == 0, "vx27_hip_dn_layer_decode: hidden must be a multiple of 32");
    VX_REQUIRE(d->x && d->w_in && d->w_out && d->conv_w && d->A_log && d->dt_bias && d->norm_w && d->S &&
                   d->conv_state && d->out,
               "vx27_hip_dn_layer_decode: null pointer in descriptor");
    VX_REQUIRE(d->conv_w_dtype == VX27_F32 || d->conv_w_dtype == VX27_BF16,
               "vx27_hip_dn_layer_decode: conv_w_dtype must be VX27_F32 or VX27_BF16");
    VX_REQUIRE(((uintptr_t)d->conv_w & 15) == 0, "vx27_hip_dn_layer_decode: conv_w must be 16-byte aligned");
    const int B = d->B, nv = d->nv, qd = d->nqk * HD, vd = nv * HD, C = 2 * qd + vd, H = d->hidden;
    const int Nin = C + vd + 2 * nv;
    const size_t pk_x = d->x_packed ? 0 : align256(vx_pack_bytes(H, B));
    const size_t act_b = align256((size_t)B * C * 4), z_b = align256((size_t)B * vd * 4);
    const size_t g_b = align256((size_t)B * nv * sizeof(float));
    const size_t gm_b = align256((size_t)B * nv * sizeof(double2));
    const size_t pk_o = align256(vx_pack_bytes(vd, B));
    void *scr;
    if (vx_ctx_scratch(ctx, pk_x + act_b + z_b + 2 * g_b + gm_b + pk_o, &scr)) return -1;
    char *p = (char *)scr;
    uint16_t *xp = d->x_packed ? (uint16_t *)d->x_packed : (uint16_t *)p;
    p += pk_x;
    float *act = (float *)p; p += act_b;
    float *z = (float *)p; p += z_b;
    float *ga = (float *)p; p += g_b;
    float *gb = (float *)p; p += g_b;
    double2 *gates = (double2 *)p; p += gm_b;
    uint16_t *op = (uint16_t *)p;

    if (!d->x_packed && vx_pack(ctx, d->x, (size_t)H, B, H, xp)) return -1;
    const int Gt = vx_pack_groups(B);
    for (int g0 = 0; g0 < Gt; g0 += VX_PASS_G) {   // one pass over W_in up to 13 groups (65 vectors)
        const int b0 = g0 * VX_PACK_GV, G = vx_pass_groups(B, b0);
        const int Bp = B - b0 < G * VX_PACK_GV ? B - b0 : G * VX_PACK_GV;
        // the first pass clears out, so that out_proj may add its two halves
        // into it (the same bits as whole rows)
        const DnInArgs ea = {Bp, C, vd, nv, d->conv_state, d->conv_w, d->conv_w_dtype == VX27_BF16, act, z, ga, gb,
                             b0, g0 == 0 ? d->out : nullptr, (size_t)B * H};
        const WkPlan wp = vx_gemv_wk_plan(Nin, H, ctx->n_cu, G);
        VX_WK_DISPATCH(ctx, gemv_dn_in, wp, (WkWeights{d->w_in, 0}), Nin, H, xp, Gt, g0, Bp, (DnInEpi{ea}));
    }

    DnArgs ra = {};
    ra.B = B; ra.nqk = d->nqk; ra.nv = nv; ra.steps = 1;
    ra.flags = VX27_DN_PRE_RMS | VX27_DN_PRE_L2 | VX27_DN_OUT_GATE;
    ra.S = d->S;
    ra.q = act; ra.k = act + qd; ra.v = act + 2 * qd;
    ra.q_tok = ra.k_tok = ra.v_tok = (size_t)C;
    ra.ga = ga; ra.gb = gb; ra.A_log = d->A_log; ra.dt_bias = d->dt_bias;   // mapped by the step kernel
    ra.norm_w = d->norm_w; ra.z = z; ra.z_tok = (size_t)vd;
    ra.out = nullptr; ra.out_tok = (size_t)vd; ra.out_packed = op;
    if (!vx_dn_single_step(ra)) {   // (the multi-step kernel takes mapped gates)
        if (vx_dn_gates(ctx, (size_t)B * nv, nv, ga, gb, d->A_log, d->dt_bias, gates)) return -1;
        ra.gates = gates;
    }
    if (vx_dn_recurrence(ctx, ra)) return -1;

    return vx_gemv_store(ctx, d->w_out, H, vd, op, B, d->out, (size_t)H, true);
}

extern "C" int vx27_hip_gqa_layer_decode(vx27_hip_ctx *ctx, const vx27_gqa_layer_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d != nullptr, "vx27_hip_gqa_layer_decode: null descriptor");
    VX_REQUIRE(d->B >= 1, "vx27_hip_gqa_layer_decode: B must be >= 1 (got %d)", d->B);
    VX_REQUIRE(d->hidden > 0 && d->hidden % 32 == 0 && d->hd == 256,
               "vx27_hip_gqa_layer_decode: hidden must be a multiple of 32 and hd 256");
    VX_REQUIRE(d->x && d->w_qkv && d->w_o && d->out, "vx27_hip_gqa_layer_decode: null pointer in descriptor");
    const int B = d->B, H = d->hidden, hd = d->hd;
    const int Nq = d->n_q * 2 * hd, Nqkv = Nq + 2 * d->n_kv * hd, Ka = d->n_q * hd;

    vx27_gqa_desc g = {};
    g.B = B; g.n_q = d->n_q; g.n_kv = d->n_kv; g.hd = hd; g.rope_dim = d->rope_dim;
    g.rope_theta = d->rope_theta; g.rope_yarn = d->rope_yarn; g.L = d->L; g.flags = 0; g.pos = d->pos;
    g.q_seq_stride = (size_t)Nqkv; g.q_head_stride = (size_t)2 * hd;
    g.gate_seq_stride = (size_t)Nqkv; g.gate_head_stride = (size_t)2 * hd;
    g.kv_seq_stride = (size_t)Nqkv;
    g.q_norm_w = d->q_norm_w; g.k_norm_w = d->k_norm_w;
    g.k_cache = d->k_cache; g.v_cache = d->v_cache; g.n_split = d->n_split;

    const size_t pk_x = d->x_packed ? 0 : align256(vx_pack_bytes(H, B));
    const size_t y_b = align256((size_t)B * Nqkv * 4);
    const size_t pk_a = align256(vx_pack_bytes(Ka, B));
    // placeholders so the scratch size of the attention step can be planned
    g.q = g.gate = g.k_new = g.v_new = (const float *)1;
    const size_t gq_b = align256(vx_gqa_scratch_bytes(&g));
    void *scr;
    if (vx_ctx_scratch(ctx, pk_x + y_b + pk_a + gq_b, &scr)) return -1;
    char *p = (char *)scr;
    uint16_t *xp = d->x_packed ? (uint16_t *)d->x_packed : (uint16_t *)p;
    p += pk_x;
    float *y = (float *)p; p += y_b;
    uint16_t *ap = (uint16_t *)p; p += pk_a;
    void *gscr = p;

    if (!d->x_packed && vx_pack(ctx, d->x, (size_t)H, B, H, xp)) return -1;
    if (vx_gemv_store(ctx, d->w_qkv, Nqkv, H, xp, B, y, (size_t)Nqkv)) return -1;
    g.q = y; g.gate = y + hd; g.k_new = y + Nq; g.v_new = y + Nq + (size_t)d->n_kv * hd;
    g.out = nullptr;
    // the combine kernel clears out for o_proj's two halves
    if (vx_gqa_decode_into(ctx, &g, gscr, ap, d->out, (size_t)B * H)) return -1;
    return vx_gemv_store(ctx, d->w_o, H, Ka, ap, B, d->out, (size_t)H, true);
}

extern "C" int vx27_hip_advance_pos(vx27_hip_ctx *ctx, int *pos, int B) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(pos && B >= 1 && B <= 1024, "vx27_hip_advance_pos: bad arguments");
    VX_LAUNCH(ctx, advance_pos_kernel, dim3(1), dim3(B), pos, B);
    return 0;
}

extern "C" int vx27_hip_fill_normal_f32(vx27_hip_ctx *ctx, float *p, size_t n, uint64_t seed, float mean,
                                        float std) {
    if (vx_ctx_enter(ctx)) return -1;
    if (n == 0) return 0;
    VX_REQUIRE(p != nullptr, "vx27_hip_fill_normal_f32: null pointer");
    VX_LAUNCH(ctx, fill_f32_kernel, dim3(8192), dim3(256), p, n, seed, mean, std);
    return 0;
}

extern "C" int vx27_hip_fill_normal_bf16(vx27_hip_ctx *ctx, uint16_t *p, size_t n, uint64_t seed, float mean,
                                         float std) {
    if (vx_ctx_enter(ctx)) return -1;
    if (n == 0) return 0;
    VX_REQUIRE(p != nullptr, "vx27_hip_fill_normal_bf16: null pointer");
    VX_LAUNCH(ctx, fill_bf16_kernel, dim3(8192), dim3(256), p, n, seed, mean, std);
    return 0;
}

extern "C" int vx27_hip_dn_layer_prefill(vx27_hip_ctx *ctx, const vx27_dn_layer_prefill_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d != nullptr, "vx27_hip_dn_layer_prefill: null descriptor");
    VX_REQUIRE(d->hd == HD && d->B >= 1 && d->T >= 1 && d->nqk >= 1 && d->nv % d->nqk == 0 && d->hidden > 0 &&
                   d->hidden % 32 == 0,
               "vx27_hip_dn_layer_prefill: bad sizes (B=%d T=%d nqk=%d nv=%d hd=%d hidden=%d)", d->B, d->T, d->nqk,
               d->nv, d->hd, d->hidden);
    VX_REQUIRE((d->flags & ~(VX27_DN_EXACT | VX27_DN_BF16)) == 0,
               "vx27_hip_dn_layer_prefill: flags may only be VX27_DN_EXACT, VX27_DN_BF16");
    VX_REQUIRE(d->x && d->w_in && d->w_out && d->conv_w && d->A_log && d->dt_bias && d->norm_w && d->S &&
                   d->conv_state && d->out,
               "vx27_hip_dn_layer_prefill: null pointer in descriptor");
    const int R = d->B * d->T, nv = d->nv, qd = d->nqk * HD, vd = nv * HD, C = 2 * qd + vd, H = d->hidden;
    const int Nin = C + vd + 2 * nv;
    vx27_dn_prefill_desc pd = {};
    pd.B = d->B; pd.T = d->T; pd.nqk = d->nqk; pd.nv = nv; pd.hd = HD;
    pd.flags = VX27_DN_CONV | VX27_DN_PRE_RMS | VX27_DN_PRE_L2 | VX27_DN_OUT_GATE | d->flags;
    pd.S = d->S; pd.A_log = d->A_log; pd.dt_bias = d->dt_bias;
    pd.conv_state = d->conv_state; pd.conv_w = d->conv_w; pd.conv_w_dtype = d->conv_w_dtype;
    pd.norm_w = d->norm_w; pd.S_ckpt = d->S_ckpt; pd.conv_ckpt = d->conv_ckpt;
    const size_t pk_x = align256(vx_pack_bytes(H, R)), y_b = align256((size_t)R * Nin * 4);
    const size_t x_b = align256((size_t)R * C * 4), z_b = align256((size_t)R * vd * 4);
    const size_t g_b = align256((size_t)R * nv * 4), o_b = align256((size_t)R * vd * 4);
    const size_t pk_o = align256(vx_pack_bytes(vd, R));
    const size_t inner = vx_dn_prefill_scratch(&pd);
    // [qkv | z | a | b] = W_in x for all B*T tokens: a long prompt of the
    // chunked form in the GEMM (W_in read once per 256 tokens, x as two bf16
    // parts, as precise as the chunked products); otherwise one pass over W_in
    // per 65 tokens with each row summed in the same order as in a decode step
    // (the exact form is bit-identical to T decode calls)
    const bool exact = (d->flags & VX27_DN_EXACT) || d->S_ckpt || d->conv_ckpt;
    const bool gemm = !exact && R >= VX_GEMM_MIN_ROWS;
    // (the long-prompt GEMMs' workspace, one region for both)
    const size_t ws_b =
        gemm ? align256(std::max(vx_gemm_ws_bytes(Nin, H, R, ctx->n_cu), vx_gemm_ws_bytes(H, vd, R, ctx->n_cu))) : 0;
    const size_t opk_b = gemm ? align256(vx_gemm_pack_bytes(vd, R)) : 0;   // the gated output, packed for out_proj
    void *scr;
    if (vx_ctx_scratch(ctx, pk_x + y_b + x_b + z_b + 2 * g_b + o_b + pk_o + ws_b + opk_b + inner, &scr)) return -1;
    char *p = (char *)scr;
    uint16_t *xp = (uint16_t *)p; p += pk_x;
    float *y = (float *)p; p += y_b;
    float *xq = (float *)p; p += x_b;
    float *z = (float *)p; p += z_b;
    float *ga = (float *)p; p += g_b;
    float *gb = (float *)p; p += g_b;
    float *o = (float *)p; p += o_b;
    uint16_t *op = (uint16_t *)p; p += pk_o;
    void *gws = p; p += ws_b;
    char *opk = p; p += opk_b;
    GemmOut seg = {};   // (the GEMM writes qkv, z, a and b straight into their buffers)
    seg.n = 4;
    seg.s[0] = GemmSeg{0, 0, (size_t)C, xq};
    seg.s[1] = GemmSeg{C / 16, 0, (size_t)vd, z};
    seg.s[2] = GemmSeg{(C + vd) / 16, 0, (size_t)nv, ga};
    seg.s[3] = GemmSeg{(C + vd + nv) / 16, 0, (size_t)nv, gb};
    if (gemm && nv % 16 == 0 && vx_gemm_fits_seg(Nin, H, R, d->x, (size_t)H, seg)) {
        if (vx_gemm_store_seg(ctx, d->w_in, Nin, H, d->x, (size_t)H, R, seg, gws)) return -1;
    } else {
        if (gemm && vx_gemm_fits(Nin, H, R, d->x, (size_t)H, y, (size_t)Nin)) {
            if (vx_gemm_store(ctx, d->w_in, Nin, H, d->x, (size_t)H, R, y, (size_t)Nin, gws)) return -1;
        } else {
            if (vx_pack(ctx, d->x, (size_t)H, R, H, xp)) return -1;
            if (vx_gemv_store(ctx, d->w_in, Nin, H, xp, R, y, (size_t)Nin)) return -1;
        }
        const size_t ys = (size_t)Nin * 4;
        VX_HIP(hipMemcpy2DAsync(xq, (size_t)C * 4, y, ys, (size_t)C * 4, (size_t)R, hipMemcpyDeviceToDevice,
                                ctx->stream));
        VX_HIP(hipMemcpy2DAsync(z, (size_t)vd * 4, y + C, ys, (size_t)vd * 4, (size_t)R, hipMemcpyDeviceToDevice,
                                ctx->stream));
        VX_HIP(hipMemcpy2DAsync(ga, (size_t)nv * 4, y + C + vd, ys, (size_t)nv * 4, (size_t)R,
                                hipMemcpyDeviceToDevice, ctx->stream));
        VX_HIP(hipMemcpy2DAsync(gb, (size_t)nv * 4, y + C + vd + nv, ys, (size_t)nv * 4, (size_t)R,
                                hipMemcpyDeviceToDevice, ctx->stream));
    }
    pd.x = xq; pd.z = z; pd.a = ga; pd.b = gb; pd.out = o;
    // out_proj in the GEMM takes the gated output straight in its packed
    // form (the gated norm writes it, in place of fp32 rows to pack)
    GemmOut oseg = {};
    oseg.n = 1;
    oseg.s[0] = GemmSeg{0, 0, (size_t)H, d->out};
    const bool gemm_out = gemm && vx_gemm_fits_seg(H, vd, R, o, (size_t)vd, oseg);
    if (vx_dn_prefill_into(ctx, &pd, p, gemm_out ? opk : nullptr)) return -1;
    if (gemm_out) return vx_gemm_store_packed(ctx, d->w_out, H, vd, opk, R, oseg, gws);
    if (vx_pack(ctx, o, (size_t)vd, R, vd, op)) return -1;
    return vx_gemv_store(ctx, d->w_out, H, vd, op, R, d->out, (size_t)H);
}

extern "C" int vx27_hip_gqa_layer_prefill(vx27_hip_ctx *ctx, const vx27_gqa_layer_prefill_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d != nullptr, "vx27_hip_gqa_layer_prefill: null descriptor");
    VX_REQUIRE(d->B >= 1 && d->T >= 1 && d->hd == 256 && d->hidden > 0 && d->hidden % 32 == 0 && d->n_kv >= 1 &&
                   d->n_q % d->n_kv == 0,
               "vx27_hip_gqa_layer_prefill: bad sizes (B=%d T=%d n_q=%d n_kv=%d hd=%d hidden=%d)", d->B, d->T,
               d->n_q, d->n_kv, d->hd, d->hidden);
    VX_REQUIRE(d->x && d->w_qkv && d->w_o && d->q_norm_w && d->k_norm_w && d->k_cache && d->v_cache && d->out,
               "vx27_hip_gqa_layer_prefill: null pointer in descriptor");
    const int R = d->B * d->T, H = d->hidden, hd = d->hd, kvd = d->n_kv * hd;
    const int Nq = d->n_q * 2 * hd, Nqkv = Nq + 2 * kvd, Ka = d->n_q * hd;
    vx27_gqa_prefill_desc gp = {};
    gp.B = d->B; gp.T = d->T; gp.n_q = d->n_q; gp.n_kv = d->n_kv; gp.hd = hd; gp.rope_dim = d->rope_dim;
    gp.rope_theta = d->rope_theta; gp.rope_yarn = d->rope_yarn; gp.L = d->L; gp.pos0 = d->pos0; gp.flags = d->flags;
    gp.q_tok_stride = (size_t)Nq; gp.q_head_stride = (size_t)2 * hd;
    gp.gate_tok_stride = (size_t)Nq; gp.gate_head_stride = (size_t)2 * hd;
    gp.q_norm_w = d->q_norm_w; gp.k_norm_w = d->k_norm_w; gp.k_cache = d->k_cache; gp.v_cache = d->v_cache;
    const size_t pk_x = align256(vx_pack_bytes(H, R)), y_b = align256((size_t)R * Nqkv * 4);
    const size_t qg_b = align256((size_t)R * Nq * 2), kv_b = align256((size_t)R * kvd * 2);
    const size_t at_b = align256((size_t)R * Ka * 4), pk_a = align256(vx_pack_bytes(Ka, R));
    const size_t inner = vx_gqa_prefill_scratch(&gp);
    // a long prompt's projections in the GEMM (weights once per 256 tokens),
    // rounded to bf16 straight into q|gate, k and v
    const bool gemm = R >= VX_GEMM_MIN_ROWS;
    const size_t ws_b =
        gemm ? align256(std::max(vx_gemm_ws_bytes(Nqkv, H, R, ctx->n_cu), vx_gemm_ws_bytes(H, Ka, R, ctx->n_cu))) : 0;
    void *scr;
    if (vx_ctx_scratch(ctx, pk_x + y_b + qg_b + 2 * kv_b + at_b + pk_a + ws_b + inner, &scr)) return -1;
    char *p = (char *)scr;
    uint16_t *xp = (uint16_t *)p; p += pk_x;
    float *y = (float *)p; p += y_b;
    uint16_t *qg = (uint16_t *)p; p += qg_b;
    uint16_t *kb = (uint16_t *)p; p += kv_b;
    uint16_t *vb = (uint16_t *)p; p += kv_b;
    float *att = (float *)p; p += at_b;
    uint16_t *ap = (uint16_t *)p; p += pk_a;
    void *gws = p; p += ws_b;
    GemmOut seg = {};
    seg.n = 3;
    seg.s[0] = GemmSeg{0, 1, (size_t)Nq, qg};
    seg.s[1] = GemmSeg{Nq / 16, 1, (size_t)kvd, kb};
    seg.s[2] = GemmSeg{(Nq + kvd) / 16, 1, (size_t)kvd, vb};
    if (gemm && vx_gemm_fits_seg(Nqkv, H, R, d->x, (size_t)H, seg)) {
        if (vx_gemm_store_seg(ctx, d->w_qkv, Nqkv, H, d->x, (size_t)H, R, seg, gws)) return -1;
    } else {
        if (vx_pack(ctx, d->x, (size_t)H, R, H, xp)) return -1;
        if (vx_gemv_store(ctx, d->w_qkv, Nqkv, H, xp, R, y, (size_t)Nqkv)) return -1;
        VX_LAUNCH(ctx, qkv_to_bf16, dim3((unsigned)R, (unsigned)((Nqkv + 255) / 256)), dim3(256), y, Nq, kvd, qg, kb,
                  vb);
    }
    gp.q = qg; gp.gate = qg + hd; gp.k_new = kb; gp.v_new = vb; gp.out = att;
    if (vx_gqa_prefill_into(ctx, &gp, p)) return -1;
    // (written packed by the attention epilogue, the output measured slower
    // there than the pack it saves: its scattered stores hold up the next
    // item's loads)
    if (gemm && vx_gemm_fits(H, Ka, R, att, (size_t)Ka, d->out, (size_t)H))
        return vx_gemm_store(ctx, d->w_o, H, Ka, att, (size_t)Ka, R, d->out, (size_t)H, gws);
    if (vx_pack(ctx, att, (size_t)Ka, R, Ka, ap)) return -1;
    return vx_gemv_store(ctx, d->w_o, H, Ka, ap, R, d->out, (size_t)H);
}
