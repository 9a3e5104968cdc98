// Whole-mixer layer steps (projections + mixer core + output projection),
// device-side synthetic fills and HIP-graph capture.
//
// DeltaNet layer (vx27_qfwd.c:102-153), one decode token of B sequences:
//   gemv_part(W_in)          [qkv | z | a | b] partial sums
//   dn_in_epilogue           reduce + causal conv/SiLU on qkv (state in place),
//                            the q/k normalisation chain, z, decay from a,
//                            beta from b
//   dn_decode_kernel         exact step on the final q/k, gated output norm,
//                            output written as the packed operand of W_out
//   gemv_part(W_out) + reduce   -> out
// Gated GQA layer (vx27_qfwd.c:162-213):
//   gemv_part(W_qkv) + reduce  -> [q|gate interleaved | k | v]
//   gqa_prep / gqa_split / gqa_combine (vx_gqa_decode.hip)
//   pack_x(att) + gemv_part(W_o) + reduce   -> out
#include <math.h>

#include "vx_dn.h"
#include "vx_gemv.h"
#include "vx_gqa.h"


namespace {

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct DnInArgs {
    const float *part;
    int N, B, n_pseg, C, vd, nv, nqk;
    float *conv_state;
    const void *conv_w;
    int conv_bf16;
    const float *A_log, *dt_bias, *norm_w;
    float *act, *z;
    double2 *gates;
};

// One block of 128 lanes per 128-row group of the stacked input projection
// (one row per lane, all sequences): the split-K sum, then
//   q|k|v rows: causal conv + SiLU (conv state in place); the q and k groups
//               are whole heads, and run the normalisation chain of
//               vx27_qfwd.c:119-130 plus step_exact's own (vx27_deltanet.c:
//               77-80): rmsn(1+w), l2norm (q /= sqrt(hd)), l2norm (q /= sqrt(hd))
//   z rows:     copied out; a rows: decay = exp(g_log); b rows: beta
__global__ __launch_bounds__(HD) void dn_in_epilogue(DnInArgs a) {
    const int n = blockIdx.x * HD + threadIdx.x;
    const bool live = n < a.N;
    float v[5];
    if (live) vx_gemv_sum_row(a.part, a.N, a.B, a.n_pseg, live ? n : 0, v);
    const int qd = a.nqk * HD;
    if ((int)blockIdx.x < 2 * a.nqk) {   // a q or k head: conv, then the norm chain per sequence
        __shared__ double s_red[3][2][2];
        float w[4];
        load_conv_w(a.conv_w, a.conv_bf16, (size_t)n, w);
        const bool is_q = n < qd;
        const float nw = a.norm_w[threadIdx.x] + 1.0f;
        const float qs = 1.0f / sqrtf((float)HD);
        for (int b = 0; b < a.B; b++) {
            float st[3];
            float *sp = a.conv_state + ((size_t)b * a.C + n) * 3;
            st[0] = sp[0]; st[1] = sp[1]; st[2] = sp[2];
            float x = conv_step(st, w, v[b]);
            sp[0] = st[0]; sp[1] = st[1]; sp[2] = st[2];
            double unused = 0.0, ss = (double)x * (double)x;
            block_sum2<2>(ss, unused, s_red[0]);
            x = (x * (1.0f / sqrtf((float)(ss / HD) + 1e-6f))) * nw;
            ss = (double)x * (double)x;
            block_sum2<2>(ss, unused, s_red[1]);
            x = x * (1.0f / sqrtf((float)ss + 1e-6f));
            if (is_q) x = x * qs;
            ss = (double)x * (double)x;
            block_sum2<2>(ss, unused, s_red[2]);
            x = x * (1.0f / sqrtf((float)ss + 1e-6f));
            if (is_q) x = x * qs;
            a.act[(size_t)b * a.C + n] = x;
        }
        return;
    }
    if (!live) return;
    if (n < a.C) {                       // v channel: causal conv + SiLU
        float w[4];
        load_conv_w(a.conv_w, a.conv_bf16, (size_t)n, w);
        for (int b = 0; b < a.B; b++) {
            float st[3];
            float *sp = a.conv_state + ((size_t)b * a.C + n) * 3;
            st[0] = sp[0]; st[1] = sp[1]; st[2] = sp[2];
            a.act[(size_t)b * a.C + n] = conv_step(st, w, v[b]);
            sp[0] = st[0]; sp[1] = st[1]; sp[2] = st[2];
        }
    } else if (n < a.C + a.vd) {         // z
        for (int b = 0; b < a.B; b++) a.z[(size_t)b * a.vd + (n - a.C)] = v[b];
    } else if (n < a.C + a.vd + a.nv) {  // a -> decay = exp(g_log), vx27_deltanet.c:68,82
        const int vh = n - a.C - a.vd;
        const double eA = exp((double)a.A_log[vh]), dtb = (double)a.dt_bias[vh];
        for (int b = 0; b < a.B; b++)
            a.gates[(size_t)b * a.nv + vh].y = exp(-eA * softplus_d((double)v[b] + dtb));
    } else {                             // b -> beta = sigmoid(b), vx27_deltanet.c:67
        const int vh = n - a.C - a.vd - a.nv;
        for (int b = 0; b < a.B; b++) a.gates[(size_t)b * a.nv + vh].x = 1.0 / (1.0 + exp(-(double)v[b]));
    }
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

}  // namespace

extern "C" size_t vx27_hip_pack_bytes(int K) { return vx_pack_bytes(K); }

extern "C" int vx27_hip_pack_x(vx27_hip_ctx *ctx, const float *x, int B, int K, uint16_t *packed) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(x && packed && B >= 1 && B <= 5, "vx27_hip_pack_x: bad arguments");
    return vx_pack(ctx, x, (size_t)K, B, K, packed);
}

extern "C" int vx27_hip_dn_layer_decode(vx27_hip_ctx *ctx, const vx27_dn_layer_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d != nullptr, "vx27_hip_dn_layer_decode: null descriptor");
    VX_REQUIRE(d->hd == HD, "vx27_hip_dn_layer_decode: hd must be 128");
    VX_REQUIRE(d->B >= 1 && d->B <= 5, "vx27_hip_dn_layer_decode: B must be 1..5 (got %d)", d->B);
    VX_REQUIRE(d->nqk >= 1 && d->nv % d->nqk == 0 && d->nv % 8 == 0,
               "vx27_hip_dn_layer_decode: nv must be a multiple of nqk and of 8 (nqk=%d nv=%d)", d->nqk, d->nv);
    VX_REQUIRE(d->hidden > 0 && d->hidden % 32 == 0, "vx27_hip_dn_layer_decode: hidden must be a multiple of 32");
    VX_REQUIRE(d->x && d->w_in && d->w_out && d->conv_w && d->A_log && d->dt_bias && d->norm_w && d->S &&
                   d->conv_state && d->out,
               "vx27_hip_dn_layer_decode: null pointer in descriptor");
    VX_REQUIRE(d->conv_w_dtype == VX27_F32 || d->conv_w_dtype == VX27_BF16,
               "vx27_hip_dn_layer_decode: conv_w_dtype must be VX27_F32 or VX27_BF16");
    const int B = d->B, nv = d->nv, qd = d->nqk * HD, vd = nv * HD, C = 2 * qd + vd, H = d->hidden;
    const int Nin = C + vd + 2 * nv;
    int seg_in, per_in, seg_out, per_out;
    if (vx_gemv_plan(Nin, H, &seg_in, &per_in) || vx_gemv_plan(H, vd, &seg_out, &per_out)) return -1;
    const size_t pk_x = d->x_packed ? 0 : align256(vx_pack_bytes(H));
    size_t part_b = vx_gemv_part_bytes(Nin, seg_in);
    if (vx_gemv_part_bytes(H, seg_out) > part_b) part_b = vx_gemv_part_bytes(H, seg_out);
    part_b = align256(part_b);
    const size_t act_b = align256((size_t)B * C * 4), z_b = align256((size_t)B * vd * 4);
    const size_t g_b = align256((size_t)B * nv * sizeof(double2));
    const size_t pk_o = align256(vx_pack_bytes(vd));
    void *scr;
    if (vx_ctx_scratch(ctx, pk_x + part_b + act_b + z_b + g_b + pk_o, &scr)) return -1;
    char *p = (char *)scr;
    uint16_t *xp = d->x_packed ? (uint16_t *)d->x_packed : (uint16_t *)p;
    p += pk_x;
    float *part = (float *)p; p += part_b;
    float *act = (float *)p; p += act_b;
    float *z = (float *)p; p += z_b;
    double2 *gates = (double2 *)p; p += g_b;
    uint16_t *op = (uint16_t *)p;

    if (!d->x_packed && vx_pack(ctx, d->x, (size_t)H, B, H, xp)) return -1;
    if (vx_gemv_part(ctx, d->w_in, 1, Nin, H, xp, seg_in, per_in, part)) return -1;
    DnInArgs ea = {part, Nin, B, vx_gemv_pseg(seg_in), C, vd, nv, d->nqk, d->conv_state, d->conv_w,
                   d->conv_w_dtype == VX27_BF16, d->A_log, d->dt_bias, d->norm_w, act, z, gates};
    VX_LAUNCH(ctx, dn_in_epilogue, dim3((unsigned)((Nin + HD - 1) / HD)), dim3(HD), ea);

    DnArgs ra = {};
    ra.B = B; ra.nqk = d->nqk; ra.nv = nv; ra.steps = 1;
    ra.flags = VX_DN_QK_READY | VX27_DN_OUT_GATE;
    ra.S = d->S;
    ra.q = act; ra.k = act + qd; ra.v = act + 2 * qd;
    ra.q_tok = ra.k_tok = ra.v_tok = (size_t)C;
    ra.gates = gates; ra.norm_w = d->norm_w; ra.z = z; ra.z_tok = (size_t)vd;
    ra.out = nullptr; ra.out_tok = (size_t)vd; ra.out_packed = op;
    if (vx_dn_recurrence(ctx, ra)) return -1;

    if (vx_gemv_part(ctx, d->w_out, 1, H, vd, op, seg_out, per_out, part)) return -1;
    return vx_gemv_reduce_store(ctx, part, H, B, seg_out, d->out, (size_t)H);
}

extern "C" int vx27_hip_gqa_layer_decode(vx27_hip_ctx *ctx, const vx27_gqa_layer_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d != nullptr, "vx27_hip_gqa_layer_decode: null descriptor");
    VX_REQUIRE(d->B >= 1 && d->B <= 5, "vx27_hip_gqa_layer_decode: B must be 1..5 (got %d)", d->B);
    VX_REQUIRE(d->hidden > 0 && d->hidden % 32 == 0 && d->hd == 256,
               "vx27_hip_gqa_layer_decode: hidden must be a multiple of 32 and hd 256");
    VX_REQUIRE(d->x && d->w_qkv && d->w_o && d->out, "vx27_hip_gqa_layer_decode: null pointer in descriptor");
    const int B = d->B, H = d->hidden, hd = d->hd;
    const int Nq = d->n_q * 2 * hd, Nqkv = Nq + 2 * d->n_kv * hd, Ka = d->n_q * hd;
    int seg_in, per_in, seg_out, per_out;
    if (vx_gemv_plan(Nqkv, H, &seg_in, &per_in) || vx_gemv_plan(H, Ka, &seg_out, &per_out)) return -1;

    vx27_gqa_desc g = {};
    g.B = B; g.n_q = d->n_q; g.n_kv = d->n_kv; g.hd = hd; g.rope_dim = d->rope_dim;
    g.rope_theta = d->rope_theta; g.rope_yarn = d->rope_yarn; g.L = d->L; g.flags = 0; g.pos = d->pos;
    g.q_seq_stride = (size_t)Nqkv; g.q_head_stride = (size_t)2 * hd;
    g.gate_seq_stride = (size_t)Nqkv; g.gate_head_stride = (size_t)2 * hd;
    g.kv_seq_stride = (size_t)Nqkv;
    g.q_norm_w = d->q_norm_w; g.k_norm_w = d->k_norm_w;
    g.k_cache = d->k_cache; g.v_cache = d->v_cache; g.n_split = d->n_split;

    const size_t pk_x = d->x_packed ? 0 : align256(vx_pack_bytes(H));
    size_t part_b = vx_gemv_part_bytes(Nqkv, seg_in);
    if (vx_gemv_part_bytes(H, seg_out) > part_b) part_b = vx_gemv_part_bytes(H, seg_out);
    part_b = align256(part_b);
    const size_t y_b = align256((size_t)B * Nqkv * 4);
    const size_t pk_a = align256(vx_pack_bytes(Ka));
    // placeholders so the scratch size of the attention step can be planned
    g.q = g.gate = g.k_new = g.v_new = (const float *)1;
    const size_t gq_b = align256(vx_gqa_scratch_bytes(&g));
    void *scr;
    if (vx_ctx_scratch(ctx, pk_x + part_b + y_b + pk_a + gq_b, &scr)) return -1;
    char *p = (char *)scr;
    uint16_t *xp = d->x_packed ? (uint16_t *)d->x_packed : (uint16_t *)p;
    p += pk_x;
    float *part = (float *)p; p += part_b;
    float *y = (float *)p; p += y_b;
    uint16_t *ap = (uint16_t *)p; p += pk_a;
    void *gscr = p;

    if (!d->x_packed && vx_pack(ctx, d->x, (size_t)H, B, H, xp)) return -1;
    if (vx_gemv_part(ctx, d->w_qkv, 1, Nqkv, H, xp, seg_in, per_in, part)) return -1;
    if (vx_gemv_reduce_store(ctx, part, Nqkv, B, seg_in, y, (size_t)Nqkv)) return -1;
    g.q = y; g.gate = y + hd; g.k_new = y + Nq; g.v_new = y + Nq + (size_t)d->n_kv * hd;
    g.out = nullptr;
    if (vx_gqa_decode_into(ctx, &g, gscr, ap)) return -1;
    if (vx_gemv_part(ctx, d->w_o, 1, H, Ka, ap, seg_out, per_out, part)) return -1;
    return vx_gemv_reduce_store(ctx, part, H, B, seg_out, d->out, (size_t)H);
}

extern "C" int vx27_hip_advance_pos(vx27_hip_ctx *ctx, int *pos, int B) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(pos && B >= 1 && B <= 1024, "vx27_hip_advance_pos: bad arguments");
    VX_LAUNCH(ctx, advance_pos_kernel, dim3(1), dim3(B), pos, B);
    return 0;
}

extern "C" int vx27_hip_graph_begin(vx27_hip_ctx *ctx) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(!ctx->prof_on, "vx27_hip_graph_begin: disable the profiler before capturing");
    VX_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return 0;
}

extern "C" int vx27_hip_graph_end(vx27_hip_ctx *ctx, void **graph_exec) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(graph_exec != nullptr, "vx27_hip_graph_end: null output");
    hipGraph_t g = nullptr;
    VX_HIP(hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t e = nullptr;
    const hipError_t rc = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    VX_HIP(rc);
    *graph_exec = (void *)e;
    return 0;
}

extern "C" int vx27_hip_graph_launch(vx27_hip_ctx *ctx, void *graph_exec) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(graph_exec != nullptr, "vx27_hip_graph_launch: null graph");
    VX_HIP(hipGraphLaunch((hipGraphExec_t)graph_exec, ctx->stream));
    return 0;
}

extern "C" int vx27_hip_graph_destroy(void *graph_exec) {
    if (graph_exec) VX_HIP(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
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
