// Gated GQA decode over a bf16 KV cache for gfx950 (split-K flash decode).
//
// Reference semantics (vx27_qfwd.c:172-211): rmsn(q)*(1+w) and rmsn(k)*(1+w)
// per head, NeoX RoPE on the first rope_dim dims, append k,v at position pos,
// softmax(q.k / sqrt(hd)) over positions 0..pos, P.V, then * sigmoid(gate)
// (no gate with VX27_GQA_NO_GATE, as the MTP drafter's use_gate = 0).
//
// Kernels per call:
//   gqa_prep     one workgroup per (sequence, head): norm + RoPE of q (kept
//                fp32 in scratch) and of the new k; k,v rounded to bf16 and
//                appended to the cache.
//   gqa_split    one wave per (split, KV head, sequence): streams its share of
//                the cache once for all n_q/n_kv query heads of the group with
//                v_mfma_f32_16x16x32_bf16, online softmax in fp32, writes a
//                partial (m, l, O) per query head.
//   gqa_combine  merges the partials, divides by l, applies sigmoid(gate)
//                (unless there is no gate).
//
// Tile algebra (32 keys per tile, query heads padded to 16):
//   S^T[key][q] = K[key][:] . Q^T[:][q]    two 16-row MFMA blocks r=0,1 over
//                                           8 k-steps of 32 dims.  Row m of
//                                           block r loads key 8(m/4)+4r+m%4, so
//                                           the C layout (lane (g,n) holds rows
//                                           4g..4g+3) leaves lane (g,n) with keys
//                                           8g..8g+7 of query head n.
//   O^T[dim][q] += V^T[dim][key] . P^T[key][q]   16 MFMAs (16 dims each); the
//                                           B operand of lane (g,n) is exactly
//                                           its 8 probabilities, the A operand
//                                           is 16 contiguous bytes of the
//                                           dim-major V block.
#include <math.h>

#include <algorithm>
#include <mutex>

#include "vx_gemv.h"
#include "vx_gqa.h"

namespace {

constexpr int HDG = VX_GQA_HD;
constexpr int TILE = VX_GQA_VBLK;    // keys per tile (V block size)
constexpr int MAXR = VX_ROPE_MAXH;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

typedef vx_rope_tab RopeTab;

__device__ __forceinline__ size_t k_index(int B_unused, int n_kv, int L, int b, int h, int p, int i) {
    (void)B_unused;
    return vx_k_index(n_kv, L, b, h, p, i);
}
__device__ __forceinline__ size_t v_index(int n_kv, int L, int b, int h, int p, int i) {
    return vx_v_index(n_kv, L, b, h, p, i);
}

// Block-wide double sum over 256 threads (4 waves, wave sums on the DPP
// paths, then in wave order); contains barriers.
__device__ __forceinline__ double block_sum256(double v, double *red) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    v = vx_wave_sum_f64_dpp(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

struct PrepArgs {
    int B, n_q, n_kv, rope_dim, L;
    unsigned flags;
    float yarn;
    const int *pos;
    const float *q;
    size_t q_ss, q_hs;
    const float *k_new, *v_new, *q_norm_w, *k_norm_w;
    size_t kv_ss;   // per-sequence stride of k_new / v_new
    uint16_t *k_cache, *v_cache;
    float *q_out;   // [B][n_q][256]
    int *err_flag;  // set to 1 when pos is outside [0, L)
    RopeTab rope;
};

// grid (n_q + n_kv, B), block 256
__global__ __launch_bounds__(256) void gqa_prep(PrepArgs a) {
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    __shared__ double red[4];
    __shared__ float row[HDG];
    __shared__ float cs[MAXR], sn[MAXR];
    // the row's loads first (one load each, from an address chosen per head
    // kind): they do not need the position, whose load and angles follow
    const bool is_q = h < a.n_q;
    const int hk = h - a.n_q;
    const float *xp = is_q ? a.q + (size_t)b * a.q_ss + (size_t)h * a.q_hs + i
                           : a.k_new + (size_t)b * a.kv_ss + (size_t)hk * HDG + i;
    const float *vp = is_q ? xp : a.v_new + (size_t)b * a.kv_ss + (size_t)hk * HDG + i;
    const float x = *xp;
    const float w = (is_q ? a.q_norm_w : a.k_norm_w)[i];
    const float vv = *vp;   // the new value row (k heads; q heads re-read x)
    const float fr = a.rope.freq[min(i, MAXR - 1)];
    // positions outside the cache are clamped so no access leaves the
    // buffers, and flagged for vx27_hip_sync to report (the host contract is
    // 0 <= pos < L)
    const int pos_in = a.pos[b];
    const int pos = min(max(pos_in, 0), a.L - 1);
    if (pos != pos_in && h == 0 && i == 0) *a.err_flag = 1;
    const int half = a.rope_dim / 2;
    if (i < half) {
        const float2 c = vx_rope_cs_f(fr, pos, a.yarn);
        cs[i] = c.x;
        sn[i] = c.y;
    }
    const double ss = block_sum256((double)x * (double)x, red);
    const float s = 1.0f / sqrtf((float)(ss / HDG) + 1e-6f);
    const float y = (a.flags & VX27_GQA_NORM_W) ? (x * s) * w : (x * s) * (w + 1.0f);
    row[i] = y;
    __syncthreads();
    float r = y;
    if (i < half) {
        r = row[i] * cs[i] - row[i + half] * sn[i];
    } else if (i < 2 * half) {
        r = row[i - half] * sn[i - half] + row[i] * cs[i - half];
    }
    if (is_q) {
        a.q_out[((size_t)b * a.n_q + h) * HDG + i] = r;
    } else {
        a.k_cache[k_index(a.B, a.n_kv, a.L, b, hk, pos, i)] = vx_f32_to_bf16(r);
        a.v_cache[v_index(a.n_kv, a.L, b, hk, pos, i)] = vx_f32_to_bf16(vv);
    }
}

struct SplitArgs {
    int B, n_q, n_kv, L, n_split;
    const int *pos;
    const float *q_rot;          // [B][n_q][256]
    const uint16_t *k_cache, *v_cache;
    float *part_o;               // [B][n_kv][n_split][qg][256]
    float *part_ml;              // [B][n_kv][n_split][qg][2]
};

#ifndef VX_SPLIT_NT
#define VX_SPLIT_NT 1        // streaming (nontemporal) loads of the KV cache
#endif
__device__ __forceinline__ bf16x8_t load_bf16x8(const uint16_t *p) {
    if (VX_SPLIT_NT) return __builtin_nontemporal_load((const bf16x8_t *)p);
    return *(const bf16x8_t *)p;
}

// grid (n_split, n_kv, B), block 64 (one wave)
#ifndef VX_SPLIT_WPE
#define VX_SPLIT_WPE 2       // waves per SIMD the split kernel is compiled for
#endif
#ifndef VX_SPLIT_WAVES
#define VX_SPLIT_WAVES 2048  // target split waves per launch
#endif
#ifndef VX_SPLIT_MINT
#define VX_SPLIT_MINT 2      // at least this many key tiles per split wave
#endif
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(VX_SPLIT_WPE))) void gqa_split(SplitArgs a) {
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x, g = lane >> 4, n = lane & 15;
    const int qg = a.n_q / a.n_kv;
    const int n_keys = min(max(a.pos[b], 0), a.L - 1) + 1;
    const int n_tiles = (n_keys + TILE - 1) / TILE;

    // Q^T operand: lane (g,n) holds dims 32s + 8g + 0..7 of query head n
    bf16x8_t qB[8];
    {
        // every lane loads (lanes past the group's heads re-read head 0 and
        // zero it), as 16-byte loads all in flight at once: a load under the
        // lane condition would be a branch with its own wait per element
        const bool live = n < qg;
        const float4 *qp = (const float4 *)(a.q_rot + ((size_t)b * a.n_q + (size_t)kvh * qg + (live ? n : 0)) * HDG);
        float4 qv[16];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            qv[2 * s] = qp[(32 * s + 8 * g) / 4];
            qv[2 * s + 1] = qp[(32 * s + 8 * g) / 4 + 1];
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const float f[8] = {qv[2 * s].x, qv[2 * s].y, qv[2 * s].z, qv[2 * s].w,
                                qv[2 * s + 1].x, qv[2 * s + 1].y, qv[2 * s + 1].z, qv[2 * s + 1].w};
#pragma unroll
            for (int e = 0; e < 8; e++) qB[s][e] = (__bf16)(live ? f[e] : 0.0f);
        }
    }
    floatx4_t acc[16];
#pragma unroll
    for (int t = 0; t < 16; t++) acc[t] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;
    const float scale_log2 = 0.0625f * 1.4426950408889634f;   // 1/sqrt(256) * log2(e)

    const uint16_t *Kb = a.k_cache + ((size_t)b * a.n_kv + kvh) * (size_t)a.L * HDG;
    const uint16_t *Vb = a.v_cache + ((size_t)b * a.n_kv + kvh) * (size_t)a.L * HDG;
    // A-operand row m of block r holds key 8(m/4) + 4r + m%4
    const int krow0 = 8 * (n >> 2) + (n & 3);

    // split s takes tiles s, s + n_split, ...: at any moment the splits in
    // flight read one contiguous window of the cache (rather than n_split
    // streams a fixed distance apart, which land on the same HBM channels)
    for (int tile = split; tile < n_tiles; tile += a.n_split) {
        const int key0 = tile * TILE;
        // ---- scores S^T (two 16-key blocks)
        floatx4_t sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
        const uint16_t *kr0 = Kb + (size_t)(key0 + krow0) * HDG + 8 * g;
        const uint16_t *kr1 = kr0 + 4 * HDG;
        bf16x8_t ka[8], kb[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            ka[s] = load_bf16x8(kr0 + 32 * s);
            kb[s] = load_bf16x8(kr1 + 32 * s);
        }
        // V^T operand for this tile: 16 dims x 32 keys per MFMA
        const uint16_t *vt = Vb + (size_t)tile * HDG * TILE + (size_t)n * TILE + 8 * g;
        bf16x8_t va[16];
#pragma unroll
        for (int t = 0; t < 16; t++) va[t] = load_bf16x8(vt + (size_t)t * 16 * TILE);
#pragma unroll
        for (int s = 0; s < 8; s++) {
            sc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[s], qB[s], sc0, 0, 0, 0);
            sc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb[s], qB[s], sc1, 0, 0, 0);
        }
        // lane (g,n): keys key0 + 8g + 0..3 (sc0) and + 4..7 (sc1), query head n
        float sv[8];
        const int kbase = key0 + 8 * g;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            sv[e] = (kbase + e < n_keys) ? sc0[e] * scale_log2 : -INFINITY;
            sv[4 + e] = (kbase + 4 + e < n_keys) ? sc1[e] * scale_log2 : -INFINITY;
        }
        float mt = sv[0];
#pragma unroll
        for (int e = 1; e < 8; e++) mt = fmaxf(mt, sv[e]);
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt);
        const float alpha = (m_new == -INFINITY) ? 1.0f : exp2f(m_run - m_new);
        bf16x8_t pB;
        float lsum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = (m_new == -INFINITY) ? 0.0f : exp2f(sv[e] - m_new);
            lsum += p;
            pB[e] = (__bf16)p;
        }
        l_run = l_run * alpha + lsum;
        m_run = m_new;
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int t = 0; t < 16; t++) acc[t] *= alpha;
        }
        // masked keys of the last tile: zero their V so cache garbage cannot leak
        if (key0 + TILE > n_keys) {
#pragma unroll
            for (int t = 0; t < 16; t++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (kbase + e >= n_keys) va[t][e] = (__bf16)0.0f;
        }
#pragma unroll
        for (int t = 0; t < 16; t++)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[t], pB, acc[t], 0, 0, 0);
    }
    // ---- partials: lane (g,n) holds O^T[16t + 4g + i][n]
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    const size_t pidx = (((size_t)b * a.n_kv + kvh) * a.n_split + split) * qg;
    if (n < qg) {
        float *po = a.part_o + (pidx + n) * HDG;
#pragma unroll
        for (int t = 0; t < 16; t++) *(floatx4_t *)(po + 16 * t + 4 * g) = acc[t];
        if (g == 0) {
            a.part_ml[(pidx + n) * 2 + 0] = m_run;
            a.part_ml[(pidx + n) * 2 + 1] = l_run;
        }
    }
}

struct CombArgs {
    int B, n_q, n_kv, n_split;
    const float *part_o, *part_ml;
    const float *gate;           // NULL: no output gate
    size_t g_ss, g_hs;
    float *out;                  // [B][n_q][256] or NULL
    uint16_t *out_packed;        // optional packed GEMV operand of out (K = n_q*256)
    float *zero;                 // optional: zero_n floats cleared (the next projection's output)
    size_t zero_n;
};

// grid (n_q, B), block 64 nw (nw <= 16 waves, enough for 12 splits a wave):
// wave w merges splits w, w + nw, ... over all 256 dims (four per lane, one
// 16-byte load per split), against its own running maximum, with the loads
// of 12 splits in flight at once; the nw wave results are then merged in LDS
// in wave order.  One pass over the partials.
constexpr int CB_W = 16, CB_N = 12;
__global__ __launch_bounds__(1024) void gqa_combine(CombArgs a) {
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), nw = blockDim.x >> 6;
    if (a.zero) {   // this workgroup's share of the range
        const size_t nwg = (size_t)gridDim.x * gridDim.y, wg = (size_t)b * gridDim.x + h;
        const size_t lo = a.zero_n * wg / nwg, hi = a.zero_n * (wg + 1) / nwg;
        for (size_t i = lo + tid; i < hi; i += blockDim.x) a.zero[i] = 0.0f;
    }
    const int qg = a.n_q / a.n_kv, kvh = h / qg, n = h % qg;
    const size_t base = ((size_t)b * a.n_kv + kvh) * a.n_split;
    __shared__ float4 s_o[CB_W][64];
    __shared__ float s_m[CB_W], s_l[CB_W];
    float gl = 0.0f;   // the gate of dim tid, loaded first
    if (a.gate && tid < HDG) gl = a.gate[(size_t)b * a.g_ss + (size_t)h * a.g_hs + tid];
    float M = -INFINITY, L = 0.0f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = wave; s0 < a.n_split; s0 += nw * CB_N) {
        // (m, l) of split s0 + nw j by lane j (lanes repeat j mod 16), then
        // the CB_N partial rows; past n_split the last split is re-read,
        // weighed 0
        const float2 ml = ((const float2 *)a.part_ml)[(base + min(s0 + nw * (lane & 15), a.n_split - 1)) * qg + n];
        float4 o[CB_N];
#pragma unroll
        for (int j = 0; j < CB_N; j++) {
            const size_t pi = (base + min(s0 + nw * j, a.n_split - 1)) * qg + n;
            o[j] = ((const float4 *)(a.part_o + pi * HDG))[lane];
        }
        __builtin_amdgcn_sched_barrier(0);   // every load issued before the first wait
        float m[CB_N], l[CB_N];
        float mb = M;
#pragma unroll
        for (int j = 0; j < CB_N; j++) {
            m[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml.x), j));
            l[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml.y), j));
            if (s0 + nw * j >= a.n_split) m[j] = -INFINITY;
            mb = fmaxf(mb, m[j]);
        }
        // no branch here (the partial rows' loads would sink into it): with
        // every maximum still -inf the sums stay 0
        const bool none = mb == -INFINITY;
        const float sc = none ? 1.0f : exp2f(M - mb);   // 0 while M is -inf
        L *= sc;
        O.x *= sc; O.y *= sc; O.z *= sc; O.w *= sc;
#pragma unroll
        for (int j = 0; j < CB_N; j++) {
            const float w = none ? 0.0f : exp2f(m[j] - mb);
            L += l[j] * w;
            O.x += o[j].x * w; O.y += o[j].y * w; O.z += o[j].z * w; O.w += o[j].w * w;
        }
        M = mb;
    }
    s_o[wave][lane] = O;
    if (lane == 0) {
        s_m[wave] = M;
        s_l[wave] = L;
    }
    __syncthreads();
    for (int d = tid; d < HDG; d += blockDim.x) {
        float Mt = s_m[0];
        for (int w = 1; w < nw; w++) Mt = fmaxf(Mt, s_m[w]);
        float Lt = 0.0f, Ot = 0.0f;
        for (int w = 0; w < nw; w++) {
            const float sc = (s_m[w] == -INFINITY) ? 0.0f : exp2f(s_m[w] - Mt);
            Lt += s_l[w] * sc;
            Ot += ((const float *)s_o[w])[d] * sc;
        }
        float r = Ot / Lt;
        if (a.gate) {
            if (d != tid) gl = a.gate[(size_t)b * a.g_ss + (size_t)h * a.g_hs + d];
            r = r * (1.0f / (1.0f + expf(-gl)));
        }
        if (a.out) a.out[((size_t)b * a.n_q + h) * HDG + d] = r;
        if (a.out_packed) vx_pack_store(a.out_packed, a.B, b, h * HDG + d, r);
    }
}

struct KvMoveArgs {
    int n_kv, L, b, p0, n;
    uint16_t *kc, *vc;
    const uint16_t *kc_r, *vc_r;
    const float *k_in, *v_in;
    float *k_out, *v_out;
};

// grid (n, n_kv), block 256: write rows into the cache format
__global__ __launch_bounds__(256) void kv_write_kernel(KvMoveArgs a) {
    const int r = blockIdx.x, h = blockIdx.y, i = threadIdx.x, p = a.p0 + r;
    const size_t src = ((size_t)r * a.n_kv + h) * HDG + i;
    a.kc[k_index(0, a.n_kv, a.L, a.b, h, p, i)] = vx_f32_to_bf16(a.k_in[src]);
    a.vc[v_index(a.n_kv, a.L, a.b, h, p, i)] = vx_f32_to_bf16(a.v_in[src]);
}
__global__ __launch_bounds__(256) void kv_read_kernel(KvMoveArgs a) {
    const int r = blockIdx.x, h = blockIdx.y, i = threadIdx.x, p = a.p0 + r;
    const size_t dst = ((size_t)r * a.n_kv + h) * HDG + i;
    if (a.k_out) a.k_out[dst] = vx_bf16_to_f32(a.kc_r[k_index(0, a.n_kv, a.L, a.b, h, p, i)]);
    if (a.v_out) a.v_out[dst] = vx_bf16_to_f32(a.vc_r[v_index(a.n_kv, a.L, a.b, h, p, i)]);
}

struct RopeTabArgs {
    const int *pos;
    int n, half;
    float yarn;
    float *cosv, *sinv;
    RopeTab rope;
};
__global__ void rope_table_kernel(RopeTabArgs a) {
    const int r = blockIdx.x, i = threadIdx.x;
    if (i >= a.half) return;
    const float2 c = vx_rope_cs(a.rope, a.pos[r], a.yarn, i);
    a.cosv[(size_t)r * a.half + i] = c.x;
    a.sinv[(size_t)r * a.half + i] = c.y;
}

}  // namespace

// freq_i = powf(theta, -2i/rope_dim) on the host, as vx27_rope.c:11
int vx_rope_fill(vx_rope_tab &t, int rope_dim, float theta) {
    VX_REQUIRE(rope_dim >= 2 && rope_dim % 2 == 0 && rope_dim / 2 <= MAXR,
               "rope_dim must be even and <= %d (got %d)", 2 * MAXR, rope_dim);
    for (int i = 0; i < rope_dim / 2; i++) {
        const float expo = (-2.0f * (float)i) / (float)rope_dim;
        t.freq[i] = powf(theta, expo);
    }
    return 0;
}

static int gqa_check(const vx27_gqa_desc *d) {
    VX_REQUIRE(d != nullptr, "vx27_hip_gqa_decode: null descriptor");
    VX_REQUIRE(d->hd == HDG, "vx27_hip_gqa_decode: hd must be 256 (got %d)", d->hd);
    VX_REQUIRE(d->B >= 1 && d->n_kv >= 1 && d->n_q >= d->n_kv && d->n_q % d->n_kv == 0 &&
                   d->n_q / d->n_kv <= 16,
               "vx27_hip_gqa_decode: need n_q = k*n_kv with k <= 16 (n_q=%d n_kv=%d)", d->n_q, d->n_kv);
    VX_REQUIRE(d->L >= 64 && d->L % 64 == 0, "vx27_hip_gqa_decode: L must be a positive multiple of 64");
    VX_REQUIRE(d->rope_dim >= 0 && d->rope_dim <= HDG, "vx27_hip_gqa_decode: bad rope_dim");
    VX_REQUIRE(d->pos && d->q && (d->gate || (d->flags & VX27_GQA_NO_GATE)) && d->k_new && d->v_new &&
                   d->q_norm_w && d->k_norm_w &&
                   d->k_cache && d->v_cache,
               "vx27_hip_gqa_decode: null pointer in descriptor");
    return 0;
}

static int gqa_n_split(const vx27_gqa_desc *d) {
    int n_split = d->n_split;
    if (n_split <= 0) {
        // ~VX_SPLIT_WAVES waves over all (sequence, KV head) pairs, at least
        // VX_SPLIT_MINT tiles per wave
        const int tiles = d->L / TILE;
        n_split = (VX_SPLIT_WAVES + d->B * d->n_kv - 1) / (d->B * d->n_kv);
        if (n_split > (tiles + VX_SPLIT_MINT - 1) / VX_SPLIT_MINT) n_split = (tiles + VX_SPLIT_MINT - 1) / VX_SPLIT_MINT;
        if (n_split < 1) n_split = 1;
    }
    return n_split;
}

size_t vx_gqa_scratch_bytes(const vx27_gqa_desc *d) {
    const size_t n_part = (size_t)d->B * d->n_kv * gqa_n_split(d) * (d->n_q / d->n_kv);
    return ((size_t)d->B * d->n_q * HDG + n_part * HDG + n_part * 2) * sizeof(float);
}

// The decode step with caller-provided scratch of vx_gqa_scratch_bytes(d);
// out_packed (optional) receives the output as the packed GEMV operand;
// zero (optional) is cleared by the combine kernel.
int vx_gqa_decode_into(vx27_hip_ctx *ctx, const vx27_gqa_desc *d, void *scr, uint16_t *out_packed, float *zero,
                       size_t zero_n) {
    if (gqa_check(d)) return -1;
    RopeTab rt = {};
    if (d->rope_dim > 0 && vx_rope_fill(rt, d->rope_dim, d->rope_theta)) return -1;
    const float yarn = d->rope_yarn < 1.0f ? 1.0f : d->rope_yarn;
    const int qg = d->n_q / d->n_kv;
    const int n_split = gqa_n_split(d);
    const size_t n_part = (size_t)d->B * d->n_kv * n_split * qg;
    float *q_rot = (float *)scr;
    float *part_o = q_rot + (size_t)d->B * d->n_q * HDG;
    float *part_ml = part_o + n_part * HDG;

    PrepArgs pa;
    pa.B = d->B; pa.n_q = d->n_q; pa.n_kv = d->n_kv; pa.rope_dim = d->rope_dim; pa.L = d->L;
    pa.flags = d->flags; pa.yarn = yarn; pa.pos = d->pos; pa.q = d->q;
    pa.q_ss = d->q_seq_stride; pa.q_hs = d->q_head_stride;
    pa.k_new = d->k_new; pa.v_new = d->v_new; pa.q_norm_w = d->q_norm_w; pa.k_norm_w = d->k_norm_w;
    pa.kv_ss = d->kv_seq_stride ? d->kv_seq_stride : (size_t)d->n_kv * HDG;
    pa.k_cache = d->k_cache; pa.v_cache = d->v_cache; pa.q_out = q_rot; pa.rope = rt;
    pa.err_flag = ctx->err_flag;
    VX_LAUNCH(ctx, gqa_prep, dim3(d->n_q + d->n_kv, d->B), dim3(256), pa);

    SplitArgs sa;
    sa.B = d->B; sa.n_q = d->n_q; sa.n_kv = d->n_kv; sa.L = d->L; sa.n_split = n_split;
    sa.pos = d->pos; sa.q_rot = q_rot; sa.k_cache = d->k_cache; sa.v_cache = d->v_cache;
    sa.part_o = part_o; sa.part_ml = part_ml;
    VX_LAUNCH(ctx, gqa_split, dim3(n_split, d->n_kv, d->B), dim3(64), sa);

    CombArgs ca;
    ca.B = d->B; ca.n_q = d->n_q; ca.n_kv = d->n_kv; ca.n_split = n_split;
    ca.part_o = part_o; ca.part_ml = part_ml; ca.gate = (d->flags & VX27_GQA_NO_GATE) ? nullptr : d->gate;
    ca.g_ss = d->gate_seq_stride; ca.g_hs = d->gate_head_stride; ca.out = d->out;
    ca.out_packed = out_packed;
    ca.zero = zero; ca.zero_n = zero_n;
    const int cb_waves = std::min(CB_W, (n_split + CB_N - 1) / CB_N);
    VX_LAUNCH(ctx, gqa_combine, dim3(d->n_q, d->B), dim3(64 * cb_waves), ca);
    return 0;
}

extern "C" int vx27_hip_gqa_decode(vx27_hip_ctx *ctx, const vx27_gqa_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    if (gqa_check(d)) return -1;
    VX_REQUIRE(d->out != nullptr, "vx27_hip_gqa_decode: null output");
    void *scr;
    if (vx_ctx_scratch(ctx, vx_gqa_scratch_bytes(d), &scr)) return -1;
    return vx_gqa_decode_into(ctx, d, scr, nullptr);
}

// ---- the decode step without allocation ----------------------------------
// Scratch of vx27_hip_gqa_decode_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the
// symbol): vx_noalloc_init looks up each device's address once, with that
// device current, and the entry point passes that address.
#define VX_NOALLOC_SCRATCH_BYTES (16u << 20)
static __device__ __align__(256) char scratch[VX_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int VX_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;
void *g_noalloc_ptr[VX_MAX_DEVICES];
}  // namespace

// Called by vx27_hip_open (the device is current): the device address of
// `scratch` on `device`, looked up once per device.
int vx_noalloc_init(int device) {
    VX_REQUIRE(device >= 0 && device < VX_MAX_DEVICES, "vx27_hip_open: device %d beyond %d", device, VX_MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (g_noalloc_ptr[device]) return 0;
    void *ptr = nullptr;
    VX_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    VX_REQUIRE(ptr != nullptr, "vx27_hip_open: no device address for the decode scratch on device %d", device);
    g_noalloc_ptr[device] = ptr;
    return 0;
}

extern "C" int vx27_hip_gqa_decode_noalloc(vx27_hip_ctx *ctx, const vx27_gqa_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    if (gqa_check(d)) return -1;
    VX_REQUIRE(d->out != nullptr, "vx27_hip_gqa_decode_noalloc: null output");
    const size_t need = vx_gqa_scratch_bytes(d);
    VX_REQUIRE(need <= VX_NOALLOC_SCRATCH_BYTES,
               "vx27_hip_gqa_decode_noalloc: needs %zu bytes of scratch, the static buffer holds %u "
               "(lower B or n_split, or use vx27_hip_gqa_decode)",
               need, VX_NOALLOC_SCRATCH_BYTES);
    void *scr = g_noalloc_ptr[ctx->device];
    VX_REQUIRE(scr != nullptr, "vx27_hip_gqa_decode_noalloc: scratch not set up on device %d", ctx->device);
    // every scratch element a kernel reads was written earlier in the same
    // call (q, then the split partials), so nothing needs clearing; the
    // profiler (host event records) is bypassed
    const int prof = ctx->prof_on;
    ctx->prof_on = 0;
    const int rc = vx_gqa_decode_into(ctx, d, scr, nullptr);
    ctx->prof_on = prof;
    return rc;
}

extern "C" int vx27_hip_kv_write(vx27_hip_ctx *ctx, uint16_t *k_cache, uint16_t *v_cache, int B_total,
                                 int n_kv, int hd, int L, int b, int p0, int n,
                                 const float *k_rows, const float *v_rows) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(hd == HDG, "vx27_hip_kv_write: hd must be 256");
    VX_REQUIRE(L % 64 == 0 && b >= 0 && b < B_total && p0 >= 0 && n >= 0 && p0 + n <= L,
               "vx27_hip_kv_write: rows [%d,%d) of sequence %d outside cache (L=%d, B=%d)", p0, p0 + n, b, L, B_total);
    if (n == 0) return 0;
    KvMoveArgs a = {n_kv, L, b, p0, n, k_cache, v_cache, nullptr, nullptr, k_rows, v_rows, nullptr, nullptr};
    VX_LAUNCH(ctx, kv_write_kernel, dim3(n, n_kv), dim3(256), a);
    return 0;
}

extern "C" int vx27_hip_kv_read(vx27_hip_ctx *ctx, const uint16_t *k_cache, const uint16_t *v_cache,
                                int B_total, int n_kv, int hd, int L, int b, int p0, int n,
                                float *k_rows, float *v_rows) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(hd == HDG, "vx27_hip_kv_read: hd must be 256");
    VX_REQUIRE(L % 64 == 0 && b >= 0 && b < B_total && p0 >= 0 && n >= 0 && p0 + n <= L,
               "vx27_hip_kv_read: rows [%d,%d) of sequence %d outside cache (L=%d, B=%d)", p0, p0 + n, b, L, B_total);
    if (n == 0) return 0;
    KvMoveArgs a = {n_kv, L, b, p0, n, nullptr, nullptr, k_cache, v_cache, nullptr, nullptr, k_rows, v_rows};
    VX_LAUNCH(ctx, kv_read_kernel, dim3(n, n_kv), dim3(256), a);
    return 0;
}

extern "C" int vx27_hip_rope_table(vx27_hip_ctx *ctx, const int *pos, int n, int rope_dim, float theta,
                                   float yarn, float *cosv, float *sinv) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(pos && cosv && sinv && n >= 0, "vx27_hip_rope_table: bad arguments");
    RopeTab rt = {};
    if (vx_rope_fill(rt, rope_dim, theta)) return -1;
    if (n == 0) return 0;
    RopeTabArgs a = {pos, n, rope_dim / 2, yarn < 1.0f ? 1.0f : yarn, cosv, sinv, rt};
    VX_LAUNCH(ctx, rope_table_kernel, dim3(n), dim3(MAXR), a);
    return 0;
}
