// Gated GQA prefill on gfx950: causal flash attention over T new tokens per
// sequence, bf16 MFMA, online softmax in fp32, keys read from the bf16 KV
// cache that the same call fills.
//
// Reference semantics: vx27_qlayer_batch (vx27_qfwd.c:314-376) runs the
// decode glue of vx27_qlayer (vx27_qfwd.c:172-211) token by token: rmsn(q),
// rmsn(k) with (1+w), RoPE at the token's position, append k,v, attend over
// positions 0..pos inclusive with scores q.k/sqrt(256) and a float softmax,
// then multiply by sigmoid(gate).  Processing the T tokens in order is the
// same as causal attention of all T queries over the cache.
//
// Kernels per call:
//   gqp_prep   one workgroup per (head, token, sequence): norm + RoPE of q
//              (bf16, head-major scratch) and of k; k,v rounded to bf16 and
//              stored at positions pos0..pos0+T-1 of the cache.
//   gqp_attn   one workgroup per (128-query tile, Q head, sequence), heaviest
//              tiles first; 4 waves of 32 queries.  Per 64-key tile staged in
//              LDS:  S^T[key][q] = K . Q^T (v_mfma_f32_16x16x32_bf16, 4 key
//              blocks x 2 query blocks x 8 k-steps), causal mask, online
//              softmax; the C layout of S^T (lane (g,n): keys 4g..4g+3 of a
//              16-key block, query n) is, for key blocks 2s and 2s+1, the A
//              operand of O += P V with the keys of k-step s in the order
//              (4g..4g+3, 16+4g..16+4g+3); the V operand takes the keys in
//              the same order from the dim-major V tile.
#include <math.h>

#include "vx_gqa.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int HDG = VX_GQA_HD;
constexpr int QT = 128;     // queries per workgroup
constexpr int KT = 64;      // keys per tile
constexpr int KROW = HDG + 8;   // padded LDS row of the K tile (bf16)
constexpr int VROW = KT + 8;    // padded LDS row of the dim-major V tile (bf16)

struct PrepArgs {
    int T, n_q, n_kv, rope_dim, L, pos0;
    unsigned flags;
    float yarn;
    const uint16_t *q, *k, *v;
    size_t q_ts, q_hs, kv_ts;     // token / head strides (elements); k,v head stride 256
    const float *q_norm_w, *k_norm_w;
    uint16_t *k_cache, *v_cache;
    uint16_t *q_rot;              // [B][n_q][T][256]
    vx_rope_tab rope;
};

// grid (n_q + n_kv, T, B), block 256 (thread = dim)
__global__ __launch_bounds__(256) void gqp_prep(PrepArgs a) {
    const int h = blockIdx.x, t = blockIdx.y, b = blockIdx.z, i = threadIdx.x;
    const int wave = i >> 6, lane = i & 63;
    __shared__ double red[4];
    __shared__ float row[HDG];
    __shared__ float cs[VX_ROPE_MAXH], sn[VX_ROPE_MAXH];
    const int pos = a.pos0 + t;
    const int half = a.rope_dim / 2;
    if (i < half) {
        const float ang = ((float)pos / a.yarn) * a.rope.freq[i];
        cs[i] = cosf(ang);
        sn[i] = sinf(ang);
    }
    const bool is_q = h < a.n_q;
    const int hk = h - a.n_q;
    const size_t tok = (size_t)b * a.T + t;
    const float x = vx_bf16_to_f32(is_q ? a.q[tok * a.q_ts + (size_t)h * a.q_hs + i]
                                        : a.k[tok * a.kv_ts + (size_t)hk * HDG + i]);
    const float w = is_q ? a.q_norm_w[i] : a.k_norm_w[i];
    const double ws = vx_wave_sum_f64((double)x * (double)x);
    if (lane == 0) red[wave] = ws;
    __syncthreads();
    const double ss = ((red[0] + red[1]) + red[2]) + red[3];
    const float s = 1.0f / sqrtf((float)(ss / HDG) + 1e-6f);
    const float y = (a.flags & VX27_GQA_NORM_W) ? (x * s) * w : (x * s) * (w + 1.0f);
    row[i] = y;
    __syncthreads();
    float r = y;
    if (i < half)
        r = row[i] * cs[i] - row[i + half] * sn[i];
    else if (i < 2 * half)
        r = row[i - half] * sn[i - half] + row[i] * cs[i - half];
    if (is_q) {
        a.q_rot[(((size_t)b * a.n_q + h) * a.T + t) * HDG + i] = vx_f32_to_bf16(r);
    } else {
        a.k_cache[vx_k_index(a.n_kv, a.L, b, hk, pos, i)] = vx_f32_to_bf16(r);
        a.v_cache[vx_v_index(a.n_kv, a.L, b, hk, pos, i)] = a.v[tok * a.kv_ts + (size_t)hk * HDG + i];
    }
}

struct AttnArgs {
    int T, n_q, n_kv, L, pos0;
    float scale_log2;             // log2(e) / sqrt(256)
    const uint16_t *q_rot;        // [B][n_q][T][256]
    const uint16_t *k_cache, *v_cache;
    const uint16_t *gate;
    size_t g_ts, g_hs;
    float *out;                   // [B][T][n_q][256]
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) {
    bf16x8_t r;
    __builtin_memcpy(&r, &u, 16);
    return r;
}
__device__ __forceinline__ uint32_t pack2(float x, float y) {
    return (uint32_t)vx_f32_to_bf16(x) | ((uint32_t)vx_f32_to_bf16(y) << 16);
}

// grid (ceil(T/128), n_q, B), block 256
__global__ __launch_bounds__(256) void gqp_attn(AttnArgs a) {
    const int qt = gridDim.x - 1 - blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (a.n_q / a.n_kv);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int r0 = qt * QT + wave * 32;                 // this wave's first query (token index)

    __shared__ uint16_t K_l[KT][KROW];
    __shared__ uint16_t V_l[HDG][VROW];

    // Q^T operands of the two 16-query blocks (rows past T clamped; never stored)
    bf16x8_t qb[2][8];
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const int t = min(r0 + rb * 16 + n, a.T - 1);
        const uint16_t *qp = a.q_rot + (((size_t)b * a.n_q + h) * a.T + t) * HDG + 8 * g;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) qb[rb][ks] = as_bf16x8(*(const uint4 *)(qp + 32 * ks));
    }
    floatx4_t O[2][16];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int db = 0; db < 16; db++) O[rb][db] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    float mrow[2] = {-INFINITY, -INFINITY}, lrow[2] = {0.f, 0.f};

    const int n_keys = a.pos0 + a.T;                           // valid cache positions
    const int wg_last = a.pos0 + min(qt * QT + QT, a.T) - 1;   // last key any row here sees
    const int n_tiles = wg_last / KT + 1;
    const int wave_last = a.pos0 + min(r0 + 31, a.T - 1);
    const uint16_t *Kc = a.k_cache + vx_k_index(a.n_kv, a.L, b, kvh, 0, 0);
    const uint16_t *Vc = a.v_cache + vx_v_index(a.n_kv, a.L, b, kvh, 0, 0);

    for (int kt = 0; kt < n_tiles; kt++) {
        const int k0 = kt * KT;
        __syncthreads();   // the previous tile's readers are done
        // stage K rows k0..k0+63 and the two dim-major V blocks; V of
        // positions past the valid keys is zeroed (masked P is 0, and 0 * a
        // stale NaN would not be)
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int idx = it * 256 + tid;
            const int kr = idx >> 5, c16 = idx & 31;
            *(uint4 *)&K_l[kr][c16 * 8] = *(const uint4 *)(Kc + (size_t)(k0 + kr) * HDG + c16 * 8);
        }
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int idx = it * 256 + tid;
            const int blk = idx >> 10, w = idx & 1023, dim = w >> 2, c = w & 3;
            const int p = k0 + blk * 32 + c * 8;
            uint4 v = *(const uint4 *)(Vc + ((size_t)(k0 / 32 + blk) * HDG + dim) * 32 + c * 8);
            if (p + 8 > n_keys) {
                uint16_t *e = (uint16_t *)&v;
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (p + j >= n_keys) e[j] = 0;
            }
            *(uint4 *)&V_l[dim][blk * 32 + c * 8] = v;
        }
        __syncthreads();
        if (k0 > wave_last) continue;   // wave-uniform: every key here is masked for this wave

        floatx4_t s[4][2];
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int rb = 0; rb < 2; rb++) s[kb][rb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const bf16x8_t ka = as_bf16x8(*(const uint4 *)&K_l[kb * 16 + n][32 * ks + 8 * g]);
#pragma unroll
                for (int rb = 0; rb < 2; rb++)
                    s[kb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[rb][ks], s[kb][rb], 0, 0, 0);
            }
        }
        const bool need_mask = k0 + KT - 1 > a.pos0 + r0;
        bf16x8_t pa[2][2];
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
            const int qpos = a.pos0 + r0 + rb * 16 + n;
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float x = s[kb][rb][i] * a.scale_log2;
                    if (need_mask && k0 + kb * 16 + 4 * g + i > qpos) x = -INFINITY;
                    s[kb][rb][i] = x;
                    mx = fmaxf(mx, x);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(mrow[rb], mx);
            const float alpha = exp2f(mrow[rb] - mnew);
            mrow[rb] = mnew;
            float sum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float pv = exp2f(s[kb][rb][i] - mnew);
                    s[kb][rb][i] = pv;
                    sum += pv;
                }
            sum += __shfl_xor(sum, 16, 64);
            sum += __shfl_xor(sum, 32, 64);
            lrow[rb] = lrow[rb] * alpha + sum;
            // O rows 4g+i of this block take the factor of query 4g+i
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; i++) al[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int i = 0; i < 4; i++) O[rb][db][i] *= al[i];
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const uint4 u = make_uint4(pack2(s[2 * ks][rb][0], s[2 * ks][rb][1]),
                                           pack2(s[2 * ks][rb][2], s[2 * ks][rb][3]),
                                           pack2(s[2 * ks + 1][rb][0], s[2 * ks + 1][rb][1]),
                                           pack2(s[2 * ks + 1][rb][2], s[2 * ks + 1][rb][3]));
                pa[rb][ks] = as_bf16x8(u);
            }
        }
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
#pragma unroll
            for (int db = 0; db < 16; db++) {
                const uint2 lo = *(const uint2 *)&V_l[db * 16 + n][32 * ks + 4 * g];
                const uint2 hi = *(const uint2 *)&V_l[db * 16 + n][32 * ks + 16 + 4 * g];
                const bf16x8_t vb = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int rb = 0; rb < 2; rb++)
                    O[rb][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[rb][ks], vb, O[rb][db], 0, 0, 0);
            }
        }
    }

    // out = O / l * sigmoid(gate)
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        float il[4];
#pragma unroll
        for (int i = 0; i < 4; i++) il[i] = 1.0f / __shfl(lrow[rb], 4 * g + i, 64);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = r0 + rb * 16 + 4 * g + i;
            if (t >= a.T) continue;
            const size_t tok = (size_t)b * a.T + t;
            float *op = a.out + (tok * a.n_q + h) * HDG;
            const uint16_t *gp = a.gate + tok * a.g_ts + (size_t)h * a.g_hs;
#pragma unroll
            for (int db = 0; db < 16; db++) {
                const int dim = db * 16 + n;
                const float gl = vx_bf16_to_f32(gp[dim]);
                op[dim] = (O[rb][db][i] * il[i]) * (1.0f / (1.0f + expf(-gl)));
            }
        }
    }
}

}  // namespace

extern "C" int vx27_hip_gqa_prefill(vx27_hip_ctx *ctx, const vx27_gqa_prefill_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d, "vx27_hip_gqa_prefill: null descriptor");
    VX_REQUIRE(d->hd == HDG, "vx27_hip_gqa_prefill: hd must be 256 (got %d)", d->hd);
    VX_REQUIRE(d->B >= 1 && d->T >= 1 && d->n_kv >= 1 && d->n_q >= d->n_kv && d->n_q % d->n_kv == 0,
               "vx27_hip_gqa_prefill: bad sizes B=%d T=%d n_q=%d n_kv=%d", d->B, d->T, d->n_q, d->n_kv);
    VX_REQUIRE(d->L >= 64 && d->L % 64 == 0, "vx27_hip_gqa_prefill: L must be a positive multiple of 64");
    VX_REQUIRE(d->pos0 >= 0 && (long long)d->pos0 + d->T <= d->L,
               "vx27_hip_gqa_prefill: positions [%d, %d) outside the cache (L=%d)", d->pos0, d->pos0 + d->T, d->L);
    VX_REQUIRE(d->rope_dim >= 0 && d->rope_dim <= HDG, "vx27_hip_gqa_prefill: bad rope_dim");
    VX_REQUIRE(d->q && d->gate && d->k_new && d->v_new && d->q_norm_w && d->k_norm_w && d->k_cache &&
                   d->v_cache && d->out,
               "vx27_hip_gqa_prefill: null pointer in descriptor");
    PrepArgs pa = {};
    if (d->rope_dim > 0 && vx_rope_fill(pa.rope, d->rope_dim, d->rope_theta)) return -1;
    void *scr;
    if (vx_ctx_scratch(ctx, (size_t)d->B * d->n_q * d->T * HDG * sizeof(uint16_t), &scr)) return -1;
    pa.T = d->T; pa.n_q = d->n_q; pa.n_kv = d->n_kv; pa.rope_dim = d->rope_dim; pa.L = d->L;
    pa.pos0 = d->pos0; pa.flags = d->flags; pa.yarn = d->rope_yarn < 1.0f ? 1.0f : d->rope_yarn;
    pa.q = d->q; pa.k = d->k_new; pa.v = d->v_new;
    pa.q_ts = d->q_tok_stride ? d->q_tok_stride : (size_t)d->n_q * HDG;
    pa.q_hs = d->q_head_stride ? d->q_head_stride : HDG;
    pa.kv_ts = (size_t)d->n_kv * HDG;
    pa.q_norm_w = d->q_norm_w; pa.k_norm_w = d->k_norm_w;
    pa.k_cache = d->k_cache; pa.v_cache = d->v_cache; pa.q_rot = (uint16_t *)scr;
    VX_LAUNCH(ctx, gqp_prep, dim3((unsigned)(d->n_q + d->n_kv), (unsigned)d->T, (unsigned)d->B), dim3(256), pa);

    AttnArgs aa;
    aa.T = d->T; aa.n_q = d->n_q; aa.n_kv = d->n_kv; aa.L = d->L; aa.pos0 = d->pos0;
    aa.scale_log2 = 1.4426950408889634f / 16.0f;
    aa.q_rot = (const uint16_t *)scr; aa.k_cache = d->k_cache; aa.v_cache = d->v_cache;
    aa.gate = d->gate;
    aa.g_ts = d->gate_tok_stride ? d->gate_tok_stride : (size_t)d->n_q * HDG;
    aa.g_hs = d->gate_head_stride ? d->gate_head_stride : HDG;
    aa.out = d->out;
    VX_LAUNCH(ctx, gqp_attn, dim3((unsigned)((d->T + QT - 1) / QT), (unsigned)d->n_q, (unsigned)d->B), dim3(256), aa);
    return 0;
}
