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
//   gqp_kv       one workgroup per 32-position V block of one KV head: rmsn +
//                RoPE of k; k,v rounded to bf16 and stored (streaming) at
//                positions pos0..pos0+T-1 of the cache; the (cos, sin) table
//                of the new positions for the query prologue.
//   gqp_attn_pp  items of (128-query tile, Q head, sequence): one
//                workgroup per CU walking a balanced per-XCD list built on
//                the host (or, inside a stream capture for a shape not yet
//                scheduled, one workgroup per item, heaviest first); 4 waves
//                of 32 queries (one wave per SIMD).  Each wave's query rows
//                of an item are staged in LDS by direct-to-LDS loads while
//                the previous item's epilogue runs; the wave normalises,
//                rotates and scales them into MFMA operand registers (the B operand layout
//                puts both halves of a RoPE pair in one lane when rope_dim is
//                a multiple of 64).  64-key K and V tiles arrive in LDS by
//                direct-to-LDS loads.  Per tile: S^T[key][q] = K . Q^T
//                (v_mfma_f32_16x16x32_bf16, 4 key blocks x 2 query blocks x
//                8 k-steps), causal mask, softmax.  Row m of key block kb
//                holds key 32(kb/2) + 8(m/4) + 4(kb%2) + m%4, so in the C
//                layout of S^T lane (g,n) of key blocks 2s and 2s+1 holds
//                keys 32s + 8g + 0..7 of query n: that is the A operand of
//                O += P V for k-step s as it stands, and the matching V
//                operand is one 16-byte unit (8 consecutive keys) of a dim
//                row of the dim-major V tile.  The S of tile kt+1 runs on the
//                MFMA pipe while the VALU does the softmax of tile kt (see
//                the kernel's comment for the schedule and the softmax
//                reference).
#include <math.h>

#include <algorithm>
#include <type_traits>
#include <utility>
#include <vector>

#include "vx_gqa.h"
#include "vx_lds.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int HDG = VX_GQA_HD;
constexpr int KT = 64;      // keys per tile

struct KvArgs {
    int T, n_kv, rope_dim, L, pos0;
    unsigned flags;
    float yarn;
    const uint16_t *k, *v;        // [B][T][n_kv][256] (16-byte aligned rows)
    size_t kv_ts;                 // token stride (elements); head stride 256
    const float *k_norm_w;
    uint16_t *k_cache, *v_cache;
    float2 *cs_tab;               // [T][rope_dim/2] (cos, sin) of each token's angles, for gqp_attn
    vx_rope_tab rope;
};

// grid (32-position blocks touched, n_kv, B), block 256: one workgroup per
// 32-position block of one KV head (the V cache's block: written as whole
// 16-byte runs, element by element only at partial blocks, so positions
// outside [pos0, pos0+T) keep their contents).  k: wave w takes the block's
// tokens w, w+4, ..., w+28; lane l holds dims 4l..4l+3 of each, so the two
// halves of a RoPE pair (dims i and i+half, half = 32 or 64) sit in lanes l
// and l ^ (half/4).  Every global load is issued before any of the work, and
// the eight tokens' sums of squares are reduced side by side.
constexpr int VB = VX_GQA_VBLK;
constexpr int KV_VLD = VB * (HDG / 8) / 256;   // 16-byte v loads per thread
#ifndef GQP_KV_NT
#define GQP_KV_NT 1         // streaming (nontemporal) stores of the new cache rows
#endif
constexpr bool KV_NT = GQP_KV_NT;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__global__ __launch_bounds__(256) void gqp_kv(KvArgs a) {
    const int hk = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int p0 = (a.pos0 / VB + (int)blockIdx.x) * VB;        // first position of the block
    const int lo = max(p0, a.pos0), hi = min(p0 + VB, a.pos0 + a.T);   // valid positions [lo, hi)
    const int half = a.rope_dim / 2;
    __shared__ float2 csn[VB][VX_ROPE_MAXH / 2];                          // rope_dim <= 128 here
    __shared__ __attribute__((aligned(16))) uint16_t vt[VB][HDG];         // the block's v rows

    // Every load is unconditional, from a position clamped into [lo, hi):
    // a load under the position test would be a branch with its own wait.
    // The frequency of this thread's (position, frequency) pairs goes first,
    // so that the angles wait for it alone (half is 32 or 64, so every pair
    // of thread tid has frequency tid % half).
    constexpr int NCS = VB * (VX_ROPE_MAXH / 2) / 256;
    const int hm = max(half, 1);
    const float fr = a.rope.freq[tid % hm];
    __builtin_amdgcn_sched_barrier(0);
    u32x4_t vr[KV_VLD];
#pragma unroll
    for (int r = 0; r < KV_VLD; r++) {
        const int e = tid + 256 * r, j = e / (HDG / 8), c = e % (HDG / 8), pos = min(max(p0 + j, lo), hi - 1);
        vr[r] = *(const u32x4_t *)(a.v + ((size_t)b * a.T + (pos - a.pos0)) * a.kv_ts + (size_t)hk * HDG + c * 8);
    }
    uint2 kr[VB / 4];
#pragma unroll
    for (int jj = 0; jj < VB / 4; jj++) {
        const int pos = min(max(p0 + wave + 4 * jj, lo), hi - 1);
        kr[jj] = *(const uint2 *)(a.k + ((size_t)b * a.T + (pos - a.pos0)) * a.kv_ts + (size_t)hk * HDG + 4 * lane);
    }
    float w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) w[e] = a.k_norm_w[4 * lane + e];
    // the angles of this thread's pairs, for clamped positions: computed
    // unconditionally, so the frequency load is not moved under the tests
    // below (with a wait of its own)
    __builtin_amdgcn_sched_barrier(0);
    float ang[NCS];
#pragma unroll
    for (int it = 0; it < NCS; it++) ang[it] = vx_rope_angle(fr, min(max(p0 + (tid + 256 * it) / hm, lo), hi - 1), a.yarn);

    // the v rows into LDS (rows outside [lo, hi) hold a clamped row, never
    // stored), before the cos/sin code, whose temporaries would push them
    // out of registers
#pragma unroll
    for (int r = 0; r < KV_VLD; r++) {
        const int e = tid + 256 * r, j = e / (HDG / 8), c = e % (HDG / 8);
        *(u32x4_t *)&vt[j][c * 8] = vr[r];
    }

    // cos/sin of every (position, frequency) of the block
#pragma unroll
    for (int it = 0; it < NCS; it++) {
        const int e = tid + 256 * it;
        if (e < VB * half) {
            const int j = e / half, i = e % half, pos = p0 + j;
            if (pos >= lo && pos < hi) {
                const float2 v = vx_rope_cs_angle(ang[it]);
                csn[j][i] = v;
                if (b == 0 && hk == 0) a.cs_tab[(size_t)(pos - a.pos0) * half + i] = v;
            }
        }
    }

    // k: rmsn (sum of squares in double) of the wave's 8 tokens
    float x[VB / 4][4];
    double ss[VB / 4];
#pragma unroll
    for (int jj = 0; jj < VB / 4; jj++) {
        const int pos = p0 + wave + 4 * jj;
        ss[jj] = 0.0;
        if (pos < lo || pos >= hi) continue;   // wave-uniform
        const uint32_t u[2] = {kr[jj].x, kr[jj].y};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[jj][e] = vx_bf16_to_f32((uint16_t)(u[e >> 1] >> (16 * (e & 1))));
            ss[jj] += (double)x[jj][e] * (double)x[jj][e];
        }
    }
    // (wave sums on the DPP paths: no LDS round trips)
#pragma unroll
    for (int jj = 0; jj < VB / 4; jj++) ss[jj] = vx_wave_sum_f64_dpp(ss[jj]);
    __syncthreads();   // csn and vt complete

    // V block [256 dims][32 positions]: thread -> (dim, 8 positions)
    {
        uint16_t *vb = a.v_cache + vx_v_index(a.n_kv, a.L, b, hk, p0, 0);
        for (int e = tid; e < HDG * (VB / 8); e += 256) {
            const int d = e / (VB / 8), c = e % (VB / 8);
            const int q0 = p0 + c * 8;
            if (q0 >= lo && q0 + 8 <= hi) {
                uint16_t v8[8];
#pragma unroll
                for (int k = 0; k < 8; k++) v8[k] = vt[c * 8 + k][d];
                const uint4 w = make_uint4(v8[0] | ((uint32_t)v8[1] << 16), v8[2] | ((uint32_t)v8[3] << 16),
                                           v8[4] | ((uint32_t)v8[5] << 16), v8[6] | ((uint32_t)v8[7] << 16));
                u32x4_t *dst = (u32x4_t *)(vb + (size_t)d * VB + c * 8);
                const u32x4_t wv = {w.x, w.y, w.z, w.w};
                if (KV_NT) __builtin_nontemporal_store(wv, dst); else *dst = wv;
            } else {
                for (int k = 0; k < 8; k++)
                    if (q0 + k >= lo && q0 + k < hi) vb[(size_t)d * VB + c * 8 + k] = vt[c * 8 + k][d];
            }
        }
    }

    // k: scale, RoPE with the partner lane's values, one 8-byte store per lane
    const int partner = lane ^ (half / 4);
#pragma unroll
    for (int jj = 0; jj < VB / 4; jj++) {
        const int j = wave + 4 * jj, pos = p0 + j;
        if (pos < lo || pos >= hi) continue;   // wave-uniform
        const float sc = 1.0f / sqrtf((float)(ss[jj] / HDG) + 1e-6f);
        float xn[4], xp[4], r[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            xn[e] = (a.flags & VX27_GQA_NORM_W) ? (x[jj][e] * sc) * w[e] : (x[jj][e] * sc) * (w[e] + 1.0f);
#pragma unroll
        for (int e = 0; e < 4; e++) xp[e] = __shfl(xn[e], partner, 64);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int i = 4 * lane + e;
            r[e] = xn[e];
            if (i < half) {
                const float2 t = csn[j][i];
                r[e] = xn[e] * t.x - xp[e] * t.y;
            } else if (i < 2 * half) {
                const float2 t = csn[j][i - half];
                r[e] = xp[e] * t.y + xn[e] * t.x;
            }
        }
        const uint2 kw = make_uint2((uint32_t)vx_f32_to_bf16(r[0]) | ((uint32_t)vx_f32_to_bf16(r[1]) << 16),
                                    (uint32_t)vx_f32_to_bf16(r[2]) | ((uint32_t)vx_f32_to_bf16(r[3]) << 16));
        u32x2_t *kdst = (u32x2_t *)(a.k_cache + vx_k_index(a.n_kv, a.L, b, hk, pos, 4 * lane));
        const u32x2_t kv2 = {kw.x, kw.y};
        if (KV_NT) __builtin_nontemporal_store(kv2, kdst); else *kdst = kv2;
    }
}

struct AttnArgs {
    int T, n_q, n_kv, L, pos0, xcd_map, rope_dim;
    unsigned flags;
    float yarn;
    const uint16_t *q;            // raw q: q[(b*T + t)*q_ts + h*q_hs + i]
    size_t q_ts, q_hs;
    const float *q_norm_w;
    const uint16_t *k_cache, *v_cache;
    const uint16_t *gate;         // NULL: no output gate
    size_t g_ts, g_hs;
    float *out;                   // [B][T][n_q][256]
    const float2 *cs_tab;         // [T][rope_dim/2] (cos, sin), written by gqp_kv
    // gqp_attn_pp with a schedule: workgroup w runs items sched[w*sched_len ..]
    // in order (item = (b * n_q + h) * n_qt + qt; -1 ends the list)
    const int *sched;
    int sched_len, n_qt;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) {
    bf16x8_t r;
    __builtin_memcpy(&r, &u, 16);
    return r;
}
// hardware round-to-nearest-even pack (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = (bf16x2_t){(__bf16)x, (__bf16)y};
    return __builtin_bit_cast(uint32_t, v);
}


// LDS tile buffers: K [64 keys][256 dims] and V [256 dims][64 keys], bf16,
// 16-byte units XOR-swizzled so the MFMA operand reads are conflict-free:
//   K unit u of key r at r*32 + (u ^ kswz(r)), kswz(r) = (r & 3) | ((r >> 1) & 12)
//     (the 16 rows one key block reads are distinct in kswz)
//   V unit u (8 keys) of dim d at d*8 + (u ^ ((d >> 1) & 7))
constexpr int KBUF = KT * HDG * 2;          // bytes of the K part
constexpr int TBUF = 2 * KBUF;              // bytes of one K+V tile buffer

// Direct-to-LDS loads of one 64-key tile, K and V separately: 4 waves x 8
// instructions of 64 lanes x 16 bytes each; every lane loads the global unit
// that belongs at its swizzled LDS slot.
// XOR swizzle of K row r's 16-byte units in the LDS tile.
__device__ __forceinline__ int kswz(int r) { return (r & 3) | ((r >> 1) & 12); }

// NB 16-query blocks as the B operand of S^T = K Q^T: lane (g,n) of k-step
// ks gets dims 32ks + 8g + 0..7 of token row t[blk] (the block's row n).
// rmsn (1+w, or w with VX27_GQA_NORM_W), RoPE (pair (i, i + half) sits in
// one lane: k-steps ks and ks + half/32; cos and sin from the table gqp_kv
// wrote) and the log2(e)/sqrt(256) score scale, so scores come out in the
// exp2 domain.  The scale commutes with the rotation, so it is folded into
// the per-dim norm factor (1+w) log2(e)/16, computed once for both blocks.
// The squares of the bf16 inputs are exact in fp32; the sum of squares is
// fp32 per lane and double across the row's 4 lanes.  Every global load
// (rows, norm weights, cos/sin) is issued before any of them is used: one
// round trip.  The raw rows come in as u (the attention kernel stages them
// in LDS).
constexpr int HQ_MAX = VX_ROPE_MAXH / 64;   // k-steps holding the first half of the pairs, at most
template <int NB>
__device__ __forceinline__ void q_prep_rows(const AttnArgs &a, const int (&t)[NB], int g, const uint4 (&u)[NB][8],
                                            bf16x8_t (&qv)[NB][8]) {
    const int hq = a.rope_dim / 64;
    float4 w[8][2];
    float4 cs[NB][HQ_MAX][4];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        w[ks][0] = *(const float4 *)(a.q_norm_w + 32 * ks + 8 * g);
        w[ks][1] = *(const float4 *)(a.q_norm_w + 32 * ks + 8 * g + 4);
    }
#pragma unroll
    for (int blk = 0; blk < NB; blk++) {
        const float4 *ct = (const float4 *)(a.cs_tab + (size_t)t[blk] * (32 * hq) + 8 * g);
#pragma unroll
        for (int ks = 0; ks < HQ_MAX; ks++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                cs[blk][ks][e] = ks < hq ? ct[16 * ks + e] : make_float4(1.f, 0.f, 1.f, 0.f);
    }
    constexpr float QS = 1.4426950408889634f / 16.0f;   // scores in the exp2 domain
    const bool wdirect = (a.flags & VX27_GQA_NORM_W) != 0;
    float wq[8][8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        const float wv[8] = {w[ks][0].x, w[ks][0].y, w[ks][0].z, w[ks][0].w,
                             w[ks][1].x, w[ks][1].y, w[ks][1].z, w[ks][1].w};
#pragma unroll
        for (int e = 0; e < 8; e++) wq[ks][e] = (wdirect ? wv[e] : wv[e] + 1.0f) * QS;
    }
#pragma unroll
    for (int blk = 0; blk < NB; blk++) {
        float x[8][8];
        float ssf = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            const uint32_t w4[4] = {u[blk][ks].x, u[blk][ks].y, u[blk][ks].z, u[blk][ks].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[ks][2 * e] = __uint_as_float(w4[e] << 16);
                x[ks][2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) ssf += x[ks][e] * x[ks][e];
        }
        double ss = (double)ssf;
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        const float sc = 1.0f / sqrtf((float)(ss / HDG) + 1e-6f);
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int e = 0; e < 8; e++) x[ks][e] = (x[ks][e] * sc) * wq[ks][e];
        // the pair offset as a constant, so x stays in registers
        auto rope = [&](auto hqc) {
            constexpr int HQ = decltype(hqc)::value;
#pragma unroll
            for (int ks = 0; ks < HQ; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float4 c4 = cs[blk][ks][e >> 1];
                    const float cx = (e & 1) ? c4.z : c4.x, cy = (e & 1) ? c4.w : c4.y;
                    const float x0 = x[ks][e], x1 = x[ks + HQ][e];
                    x[ks][e] = x0 * cx - x1 * cy;
                    x[ks + HQ][e] = x0 * cy + x1 * cx;
                }
        };
        static_assert(HQ_MAX == 2, "RoPE cases below cover rope_dim 64 and 128");
        switch (hq) {
            case 1: rope(std::integral_constant<int, 1>{}); break;
            case 2: rope(std::integral_constant<int, 2>{}); break;
            default: break;
        }
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            qv[blk][ks] = as_bf16x8(make_uint4(pack2(x[ks][0], x[ks][1]), pack2(x[ks][2], x[ks][3]),
                                               pack2(x[ks][4], x[ks][5]), pack2(x[ks][6], x[ks][7])));
    }
}

// Software-pipelined attention: 4 waves of 32 queries (two 16-query blocks,
// so every K and V operand read from LDS feeds two MFMAs).  The stretch
// between two barriers, interval kt, runs the S MFMAs of tile kt+1 with the
// softmax of tile kt interleaved on the VALU, then O += P V of tile kt; row
// sums come out of the MFMA pipe as P times a ones operand, in the C layout
// of O.  Two K and two V tile buffers: interval kt streams K(kt+2) and
// V(kt+1) into the buffers that K(kt) and V(kt-1) left (a clamped tile index
// past the end reloads a valid tile into a buffer nobody reads again, so the
// loads carry no branch).
//
// Softmax reference: each query's max over its first tile, fixed for the
// whole pass, so P = exp2(s - m0) needs no running max and O no rescale.
// That is exact in fp32 (the reference cancels in O / l) unless a later
// score exceeds m0 by more than fp32 range allows: then O or l is no longer
// finite, and the wave redoes its queries with the online (rescaling)
// softmax, reading K and V straight from the cache.  grid (ceil(T/128) *
// n_q, B), block 256.
// 4 waves x 2 blocks of 16 queries (measured: 8 waves x 16 queries 3% slower,
// 4 x 48 spills and runs 25% slower)
constexpr int PP_NW = 4, PP_RB = 2, PP_QT = PP_NW * PP_RB * 16, PP_PER = 32 / PP_NW;
// The epilogue stages the next item's query rows in LDS (about 4% off the
// kernel against loading them in the prologue): a wave's 16 RB query rows
// fill its two V-buffer slots exactly, and the epilogue's transposition,
// 16 KiB per wave, stays in the K buffers.
static_assert(PP_RB * 8 == 2 * PP_PER && PP_NW * 16 * HDG * 4 <= 2 * (int)KBUF, "query staging layout");
#ifndef GQP_OUT_NT
#define GQP_OUT_NT 1        // streaming (nontemporal) stores of the attention output
#endif
constexpr bool OUT_NT = GQP_OUT_NT;

__global__ __launch_bounds__(PP_NW * 64) void gqp_attn_pp(AttnArgs a) {
    constexpr int RB = PP_RB, QT = PP_QT, PER = PP_PER;
    const int n_items = a.sched ? a.sched_len : 1;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // K tile buffers, then V tile buffers, in one array (the epilogue reuses
    // all 128 KiB)
    __shared__ __attribute__((aligned(16))) char smem[4 * KBUF];

    // (qt, h, b) of this workgroup's item `it`; false past the end of its list
    auto item_of = [&](int it, int &qt, int &h, int &b) -> bool {
        if (a.sched) {   // persistent: this workgroup's list (wave-uniform scalar loads)
            const int code = a.sched[blockIdx.x * a.sched_len + it];
            if (code < 0) return false;
            qt = code % a.n_qt;
            h = (code / a.n_qt) % a.n_q;
            b = code / (a.n_qt * a.n_q);
        } else if (a.xcd_map) {   // one item per workgroup: one KV head's query heads per XCD group, heaviest first
            const int n_qt = gridDim.x / a.n_q, id = blockIdx.x, xcd = id & 7, slot = id >> 3;
            const int xpk = 8 / a.n_kv, hpx = a.n_q / 8;
            b = blockIdx.y;
            qt = n_qt - 1 - slot / hpx;
            h = (xcd / xpk) * (a.n_q / a.n_kv) + (xcd % xpk) * hpx + slot % hpx;
        } else {
            const int n_qt = gridDim.x / a.n_q;
            b = blockIdx.y;
            qt = n_qt - 1 - (int)blockIdx.x / a.n_q;
            h = blockIdx.x % a.n_q;
        }
        return true;
    };
    // Stage this wave's 16 RB query rows of item (sqt, sh, sb) in its slots
    // of the V buffers, by direct-to-LDS loads: rows 0 .. 8 RB - 1 in its
    // PER KiB of V buffer 0, the rest in its PER KiB of V buffer 1 (exactly
    // the slots its own loads of V(0) and V(1) fill later), 16-byte unit u
    // of row q at position u ^ (q % 16) so that the reads of 16 rows at one
    // unit fall on distinct banks.
    auto stage_q = [&](int sqt, int sh, int sb) {
        const int nr0 = sqt * QT + wave * (RB * 16), tf = min(nr0, a.T - 1);
        const uint16_t *qb = vx_uniform_ptr(a.q + ((size_t)sb * a.T + tf) * a.q_ts + (size_t)sh * a.q_hs);
        // (an opaque copy of the lane index: the per-lane offsets below are
        // the same for every item, and hoisted out of the item loop they
        // would hold registers through the main loop)
        int ln = lane;
        __asm__ volatile("" : "+v"(ln));
        const uint32_t vb = vx_lds_addr(smem + 2 * KBUF) + wave * PER * 1024;
#pragma unroll
        for (int j = 0; j < RB * 8; j++) {   // rows 2j and 2j + 1
            const int q = 2 * j + (ln >> 5), t = min(nr0 + q, a.T - 1);
            const uint32_t off = (uint32_t)((t - tf) * a.q_ts * 2) + (uint32_t)(((ln & 31) ^ (q & 15)) << 4);
            vx_dma16(qb, off, vb + ((2 * j) / (RB * 8)) * KBUF + ((2 * j) % (RB * 8)) * 512);
        }
    };
    {
        int qt0, h0, b0;
        if (item_of(0, qt0, h0, b0)) stage_q(qt0, h0, b0);
    }

    for (int item = 0; item < n_items; item++) {
    int qt, h, b;
    if (!item_of(item, qt, h, b)) break;
    if (item > 0) vx_lds_barrier();   // the previous item's epilogue is done with LDS
    const int kvh = h / (a.n_q / a.n_kv);
    const int r0 = qt * QT + wave * (RB * 16);

    char (*Kl)[KBUF] = (char (*)[KBUF])smem;
    char (*Vl)[KBUF] = (char (*)[KBUF])(smem + 2 * KBUF);

    const int n_keys = a.pos0 + a.T;
    const int wg_last = a.pos0 + min(qt * QT + QT, a.T) - 1;
    const int n_tiles = wg_last / KT + 1;
    const int wave_tiles = (a.pos0 + min(r0 + RB * 16 - 1, a.T - 1)) / KT + 1;   // tiles with a key this wave sees
    // tiles with no key past any query of this wave (a wave wholly past the T
    // new tokens counts as the last one: its main tiles then end before the
    // partial last tile, which every wave takes as a tail interval, with the
    // barrier of its V zeroing)
    const int n_main = min((a.pos0 + min(r0, a.T - 1) + 1) / KT, n_tiles);
    const char *Kc = (const char *)(a.k_cache + vx_k_index(a.n_kv, a.L, b, kvh, 0, 0));
    const char *Vc = (const char *)(a.v_cache + vx_v_index(a.n_kv, a.L, b, kvh, 0, 0));

    // this wave's share of a tile: PER 1 KiB units of K and of V; per-lane
    // source offsets of the swizzled LDS slots (loop-invariant)
    uint32_t ko[PER], vo[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int r = (wave * PER + j) * 2 + (lane >> 5), u = (lane & 31) ^ kswz(r);
        ko[j] = (uint32_t)(r * HDG + u * 8) * 2;
        const int d = (wave * PER + j) * 8 + (lane >> 3), w = (lane & 7) ^ ((d >> 1) & 7);
        vo[j] = (uint32_t)((((w >> 2) * HDG + d) * 32) + (w & 3) * 8) * 2;
    }
    const uint32_t kl0 = vx_lds_addr(Kl[0]), vl0 = vx_lds_addr(Vl[0]);
    // (tile and buf are wave-uniform; vx_uniform_ptr keeps the source base
    // in scalar registers where the compiler would not know it)
    auto dma_k = [&](int tile, int buf, int j) {
        vx_dma16(vx_uniform_ptr(Kc + (size_t)tile * KBUF), ko[j], kl0 + buf * KBUF + (wave * PER + j) * 1024);
    };
    auto dma_v = [&](int tile, int buf, int j) {
        vx_dma16(vx_uniform_ptr(Vc + (size_t)tile * KBUF), vo[j], vl0 + buf * KBUF + (wave * PER + j) * 1024);
    };
    // Prologue: K(0) and K(1) into LDS; the query rows (staged in this
    // wave's V-buffer slots before the item loop or by the previous item's
    // epilogue) read out; then V(0) into those slots, and the rows' norm and
    // rotation, whose loads are L2 hits.
    bf16x8_t qv[RB][8];
    {
        int tq[RB];   // rows past T repeat row T-1
#pragma unroll
        for (int rb = 0; rb < RB; rb++) tq[rb] = min(r0 + 16 * rb + n, a.T - 1);
        uint4 u[RB][8];
#pragma unroll
        for (int j = 0; j < PER; j++) dma_k(0, 0, j);
#pragma unroll
        for (int j = 0; j < PER; j++) dma_k(min(1, n_tiles - 1), 1, j);
        // the staging loads and everything issued before K(0) have landed
        __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PER) : "memory");
        int ln = lane;   // (opaque, as in stage_q)
        __asm__ volatile("" : "+v"(ln));
        const int gg = ln >> 4, nn = ln & 15;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            const int q = 16 * rb + nn;
            const char *rp = smem + (2 + q / (RB * 8)) * KBUF + wave * PER * 1024 + (q % (RB * 8)) * 512;
#pragma unroll
            for (int ks = 0; ks < 8; ks++) u[rb][ks] = *(const uint4 *)(rp + (((4 * ks + gg) ^ (q & 15)) << 4));
        }
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // read out before V(0) lands there
#pragma unroll
        for (int j = 0; j < PER; j++) dma_v(0, 0, j);
        q_prep_rows<RB>(a, tq, g, u, qv);
    }

    floatx4_t O[RB][16], Ol[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        Ol[rb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int db = 0; db < 16; db++) O[rb][db] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    }
    const bf16x8_t ones = as_bf16x8(make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u));

    // key row held by row n of key block kb (see kswz): in the C layout of
    // S^T, lane (g,n) of blocks 2s, 2s+1 holds keys 32s + 8g + 0..7
    auto key_of = [&](int kb, int i) { return 32 * (kb >> 1) + 8 * g + 4 * (kb & 1) + i; };
    auto kload = [&](const char *Kt, int ks, bf16x8_t *dst) {
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            const int kr = 32 * (kb >> 1) + 8 * (n >> 2) + 4 * (kb & 1) + (n & 3);
            const int uo = ((4 * ks + g) ^ kswz(kr)) << 4;
            dst[kb] = as_bf16x8(*(const uint4 *)(Kt + kr * 512 + uo));
        }
    };
    auto zero_s = [&](floatx4_t (&x)[4][RB]) {
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++) x[kb][rb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    };
    auto s_tile = [&](const char *Kt, floatx4_t (&x)[4][RB]) {   // S without interleaved work
        bf16x8_t kf[2][4];
        kload(Kt, 0, kf[0]);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            if (ks + 1 < 8) kload(Kt, ks + 1, kf[(ks + 1) & 1]);
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
                    x[kb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks & 1][kb], qv[rb][ks], x[kb][rb], 0, 0, 0);
        }
    };
    // causal: keys past the query's position.  Rows past the T new tokens
    // (the last query block's padding, never stored) are masked as the last
    // token: keys past the cache's valid ones hold stale data, and an
    // overflow there would send the wave's valid rows down the fallback.
    auto mask = [&](int k0, floatx4_t (&x)[4][RB]) {
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            const int qpos = min(a.pos0 + r0 + rb * 16 + n, n_keys - 1);
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (k0 + key_of(kb, i) > qpos) x[kb][rb][i] = -INFINITY;
        }
    };
    auto row_max = [&](floatx4_t (&x)[4][RB], int rb) {   // over the 4 lanes of query n
        float m = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++) m = fmaxf(m, x[kb][rb][i]);
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        return fmaxf(m, __shfl_xor(m, 32, 64));
    };

    // softmax of one tile in 8 pieces (piece p runs beside k-step p of the
    // next tile's S): P = exp2(s - m0) for one key block of one query block,
    // packed to bf16 as the A operand of P V once both blocks of a k-step
    // are done.  The main intervals start the S accumulators at -m0 (mq),
    // so their S already is s - m0 (sub = false).
    float m0[RB];
    floatx4_t mq[RB];
    bf16x8_t pa[RB][2];
    auto sm_piece = [&](int piece, floatx4_t (&x)[4][RB], bool sub) {
        const int rb = piece >> 2, kb = piece & 3;
#pragma unroll
        for (int i = 0; i < 4; i++) x[kb][rb][i] = __builtin_amdgcn_exp2f(sub ? x[kb][rb][i] - m0[rb] : x[kb][rb][i]);
        if (kb & 1)
            pa[rb][kb >> 1] = as_bf16x8(make_uint4(pack2(x[kb - 1][rb][0], x[kb - 1][rb][1]),
                                                   pack2(x[kb - 1][rb][2], x[kb - 1][rb][3]),
                                                   pack2(x[kb][rb][0], x[kb][rb][1]), pack2(x[kb][rb][2], x[kb][rb][3])));
    };
    // O += P V: groups of 4 dim blocks, the V operands of group j+1 read while
    // the MFMAs of group j run; row sums from P times ones
    auto pv_tile = [&](const char *Vt) {
        const int vsw = (n >> 1) & 7;
        bf16x8_t vf[2][4];
        auto vload = [&](int grp, bf16x8_t *dst) {
            const int ks = grp >> 2, db0 = (grp & 3) * 4;
            const int uo = ((4 * ks + g) ^ vsw) << 4;
#pragma unroll
            for (int j = 0; j < 4; j++) dst[j] = as_bf16x8(*(const uint4 *)(Vt + ((db0 + j) * 16 + n) * (KT * 2) + uo));
        };
        vload(0, vf[0]);
#pragma unroll
        for (int grp = 0; grp < 8; grp++) {
            if (grp + 1 < 8) vload(grp + 1, vf[(grp + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            const int ks = grp >> 2, db0 = (grp & 3) * 4;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
                    O[rb][db0 + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[rb][ks], vf[grp & 1][j], O[rb][db0 + j], 0, 0, 0);
            if ((grp & 3) == 3)
#pragma unroll
                for (int rb = 0; rb < RB; rb++) Ol[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[rb][ks], ones, Ol[rb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // wait for K(kt+1) and V(kt) (every wave's share), then one barrier:
    // every wave is done with interval kt-1, whose buffers take K(kt+2) and
    // V(kt+1); sources clamped to a valid tile
    auto enter = [&](int kt, int &tk, int &tv) {
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        vx_lds_barrier();
        tk = min(kt + 2, n_tiles - 1);
        tv = min(kt + 1, n_tiles - 1);
    };

    // S(kt) as VGPRs for the softmax, copied out of the MFMA result registers
    // at the start of an interval, so S(kt+1) accumulates in the same ones
    auto take_s = [&](floatx4_t (&x)[4][RB], floatx4_t (&sc)[4][RB]) {
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                sc[kb][rb] = x[kb][rb];
                __asm__ volatile("" : "+v"(sc[kb][rb]));
            }
    };
    // Main interval: tile kt has no key past any query of this wave (no
    // mask); S(kt+1) on the MFMA pipe, the softmax of tile kt beside it,
    // this wave's loads of K(kt+2) and V(kt+1) spread over the k-steps, then
    // P V(kt).  One straight-line body; sn holds S(kt) on entry and S(kt+1)
    // on exit.
    auto main_iv = [&](int kt, floatx4_t (&sn)[4][RB]) {
        int tk, tv;
        enter(kt, tk, tv);
        floatx4_t sc[4][RB];
        take_s(sn, sc);
        const int bk = kt & 1, bv = bk ^ 1;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++) sn[kb][rb] = mq[rb];
        const char *Kt = Kl[(kt + 1) & 1];
        bf16x8_t kf[2][4];
        kload(Kt, 0, kf[0]);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            if (ks + 1 < 8) kload(Kt, ks + 1, kf[(ks + 1) & 1]);
            if (ks < PER) {
                dma_k(tk, bk, ks);
                dma_v(tv, bv, ks);
            }
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
                    sn[kb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks & 1][kb], qv[rb][ks], sn[kb][rb], 0, 0, 0);
#pragma unroll
            for (int p = ks; p < 4 * RB; p += 8) sm_piece(p, sc, false);
#pragma unroll
            for (int x = 0; x < 8; x++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // up to two VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        pv_tile(Vl[kt & 1]);
    };
    // Tail interval (the few tiles that straddle this wave's queries, and
    // those past them): causal mask; the last tile's V past the valid keys
    // zeroed (masked P is 0, and 0 * a stale NaN would not be); tiles past
    // this wave's last query only take part in the loads.
    auto tail_iv = [&](int kt, floatx4_t (&sn)[4][RB]) {
        int tk, tv;
        enter(kt, tk, tv);
        floatx4_t sc[4][RB];
        take_s(sn, sc);
        const int k0 = kt * KT;
#pragma unroll
        for (int j = 0; j < PER; j++) dma_k(tk, kt & 1, j);
#pragma unroll
        for (int j = 0; j < PER; j++) dma_v(tv, (kt & 1) ^ 1, j);
        if (k0 + KT > n_keys) {
            uint16_t *V = (uint16_t *)Vl[kt & 1];
            for (int e = tid; e < HDG * KT; e += 256) {
                const int d = e >> 6, key = e & 63;
                if (k0 + key >= n_keys) V[d * KT + (((key >> 3) ^ ((d >> 1) & 7)) * 8) + (key & 7)] = 0;
            }
            vx_lds_barrier();   // (workgroup-uniform)
        }
        if (kt < wave_tiles) {
            mask(k0, sc);
#pragma unroll
            for (int piece = 0; piece < 4 * RB; piece++) sm_piece(piece, sc, false);
            if (kt + 1 < wave_tiles) {
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int rb = 0; rb < RB; rb++) sn[kb][rb] = mq[rb];
                s_tile(Kl[(kt + 1) & 1], sn);
            }
            pv_tile(Vl[kt & 1]);
        }
    };

    // S(0) and the reference maxima, then the main intervals, then the tail
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    vx_lds_barrier();
    floatx4_t sS[4][RB];
    zero_s(sS);
    s_tile(Kl[0], sS);
    if (KT - 1 > min(a.pos0 + r0, n_keys - 1)) mask(0, sS);
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        m0[rb] = row_max(sS, rb);
        mq[rb] = (floatx4_t){-m0[rb], -m0[rb], -m0[rb], -m0[rb]};
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++) sS[kb][rb][i] -= m0[rb];   // tile 0 relative to m0, as the others
    }
    int kt = 0;
    for (; kt < n_main; kt++) main_iv(kt, sS);
    for (; kt < n_tiles; kt++) tail_iv(kt, sS);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the last (unused) tile loads

    // Overflow past the fixed reference: redo this wave's queries with the
    // online softmax (running max per query, O and l rescaled when it moves
    // by more than 16), K and V operands read from the cache.
    // (x * 0 is 0 for a finite x and NaN for an infinite or NaN one, so a sum
    // of such products is NaN exactly when some O or l is not finite: four
    // independent chains of fma(x, 0, acc), two VALU operations a value,
    // where a per-value class test ran as one serial chain through the
    // scalar unit)
    float zc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            zc[i] = __builtin_fmaf(Ol[rb][i], 0.f, zc[i]);
#pragma unroll
            for (int db = 0; db < 16; db++) zc[i] = __builtin_fmaf(O[rb][db][i], 0.f, zc[i]);
        }
    const bool bad = !((zc[0] + zc[1]) + (zc[2] + zc[3]) == 0.f);
    if (__any(bad)) {
        float mrow[RB];
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            mrow[rb] = -INFINITY;
            Ol[rb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int db = 0; db < 16; db++) O[rb][db] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
        }
        for (int t = 0; t < wave_tiles; t++) {
            const int k0 = t * KT;
            floatx4_t x[4][RB];
            zero_s(x);
#pragma unroll
            for (int ks = 0; ks < 8; ks++)
#pragma unroll
                for (int kb = 0; kb < 4; kb++) {
                    const int kr = 32 * (kb >> 1) + 8 * (n >> 2) + 4 * (kb & 1) + (n & 3);
                    const bf16x8_t kf = as_bf16x8(*(const uint4 *)(Kc + ((size_t)(k0 + kr) * HDG + 32 * ks + 8 * g) * 2));
#pragma unroll
                    for (int rb = 0; rb < RB; rb++) x[kb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qv[rb][ks], x[kb][rb], 0, 0, 0);
                }
            mask(k0, x);
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                const float m = row_max(x, rb);
                const float mnew = m > mrow[rb] + 16.0f ? m : mrow[rb];
                const float alpha = __builtin_amdgcn_exp2f(mrow[rb] - mnew);   // 0 on the first tile
                mrow[rb] = mnew;
                m0[rb] = mnew;
                float al[4];
#pragma unroll
                for (int i = 0; i < 4; i++) al[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    Ol[rb][i] *= al[i];
#pragma unroll
                    for (int db = 0; db < 16; db++) O[rb][db][i] *= al[i];
                }
            }
#pragma unroll
            for (int piece = 0; piece < 4 * RB; piece++) sm_piece(piece, x, true);
            // V operands: keys 32ks + 8g .. +7 of dim 16db + n, zero past the valid keys
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const int key = k0 + 32 * ks + 8 * g;
#pragma unroll
                for (int db = 0; db < 16; db++) {
                    const int d = db * 16 + n;
                    uint4 u = *(const uint4 *)(Vc + ((((size_t)(key / 32) * HDG + d) * 32) + (key % 32)) * 2);
                    uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        if (key + 2 * e >= n_keys) w4[e] &= 0xffff0000u;
                        if (key + 2 * e + 1 >= n_keys) w4[e] &= 0x0000ffffu;
                    }
                    const bf16x8_t vf = as_bf16x8(make_uint4(w4[0], w4[1], w4[2], w4[3]));
#pragma unroll
                    for (int rb = 0; rb < RB; rb++) O[rb][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[rb][ks], vf, O[rb][db], 0, 0, 0);
                }
#pragma unroll
                for (int rb = 0; rb < RB; rb++) Ol[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[rb][ks], ones, Ol[rb], 0, 0, 0);
            }
        }
    }

    // out = O / l * sigmoid(gate), one query row (256 dims) per instruction:
    // this wave's O rows, scaled by 1/l, go 16 at a time through its 16 KiB
    // of the (now idle) tile buffers, so every gate load and output store is
    // one whole row across the wave (lane L: dims 4L..4L+3).  Row r's 16-dim groups are
    // XOR-swizzled by (r / 4) % 4, so the four rows one C-layout store
    // touches fall on distinct banks.  The gate rows are loaded first, to
    // overlap their latency with the transposition.
    uint2 gv[RB * 16];
    const bool gated = a.gate != nullptr;
#pragma unroll
    for (int q = 0; q < RB * 16; q++) {
        const int t = min(r0 + q, a.T - 1);
        gv[q] = gated ? *(const uint2 *)(a.gate + ((size_t)b * a.T + t) * a.g_ts + (size_t)h * a.g_hs + 4 * lane)
                      : make_uint2(0u, 0u);
    }
    vx_lds_barrier();   // every wave is done with the tile buffers
    float *Ow = (float *)smem + wave * (16 * HDG);   // 16 rows at a time
    constexpr float L2E = 1.4426950408889634f;
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float il = __builtin_amdgcn_rcpf(Ol[rb][i]);
#pragma unroll
            for (int db = 0; db < 16; db++) Ow[(4 * g + i) * HDG + ((db ^ g) * 16) + n] = O[rb][db][i] * il;
        }
        __builtin_amdgcn_wave_barrier();   // (one wave's LDS operations complete in order)
        // each row's LDS read is issued one row ahead, so that it lands while
        // the previous row's gate factors are computed
        auto orow = [&](int qq) {
            const int sw = (qq >> 2) & 3;
            return *(const float4 *)&Ow[qq * HDG + (((lane >> 2) ^ sw) * 16) + 4 * (lane & 3)];
        };
        float4 on = orow(0);
#pragma unroll
        for (int qq = 0; qq < 16; qq++) {
            const int q = rb * 16 + qq, t = r0 + q;
            const float4 o = on;
            if (qq + 1 < 16) on = orow(qq + 1);
            const float g0 = __uint_as_float(gv[q].x << 16), g1 = __uint_as_float(gv[q].x & 0xffff0000u);
            const float g2 = __uint_as_float(gv[q].y << 16), g3 = __uint_as_float(gv[q].y & 0xffff0000u);
            float4 r = o;
            if (gated) {
                r.x = o.x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g0 * L2E));
                r.y = o.y * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g1 * L2E));
                r.z = o.z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g2 * L2E));
                r.w = o.w * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g3 * L2E));
            }
            if (t < a.T) {
                floatx4_t *dst = (floatx4_t *)(a.out + (((size_t)b * a.T + t) * a.n_q + h) * HDG + 4 * lane);
                const floatx4_t rv = {r.x, r.y, r.z, r.w};
                if (OUT_NT) __builtin_nontemporal_store(rv, dst); else *dst = rv;
            }
        }
        __builtin_amdgcn_wave_barrier();   // this pass's reads before the next pass's writes
        // the next item's query rows go into this wave's V-buffer slots while
        // the second pass runs (the transposition uses only the K buffers).
        // Not before the first pass: its first gate value would then wait
        // for these loads too, vmcnt counting in issue order.
        if (rb == 0 && item + 1 < n_items) {
            int nqt, nh, nb;
            if (item_of(item + 1, nqt, nh, nb)) stage_q(nqt, nh, nb);
        }
    }
    }   // items
}

}  // namespace

// ---- host: the prefill attention work schedule ----------------------------
// gqp_attn_pp runs as one workgroup per CU over precomputed lists of items
// (b, h, qt).  An item costs its key tiles plus a fixed overhead of about
// nine tiles' time (its prologue and epilogue, measured by wall-clock
// stamps: about 16 us against 1.75 us per 64-key tile).
// Workgroup w runs on XCD w % 8 (the dispatcher deals workgroups round-robin
// over the XCDs).  With the XCD grouping, XCD x owns the query heads of one
// KV head, so its L2 holds that head's K and V, and its items are packed
// into the XCD's n_cu/8 lists: heaviest first onto the lightest list, then
// single moves and pairwise swaps while they lower the heaviest list, then
// re-splits of the heaviest list with another.
// Hardware dispatch of one workgroup per item gives the heaviest-first
// greedy packing alone, about 8% above the mean for a 4096-token prompt.
namespace {
constexpr int GQP_ITEM_OVERHEAD = 9;   // tile-times of an item's prologue and epilogue
struct GqpSched {
    int key[7];
    int *dev;
    int len, n_wg;
    bool captured;   // launched inside a stream capture: a graph may hold dev
};
typedef std::pair<int, int> CostItem;   // (cost, item code)

void gqp_pack(std::vector<CostItem> items, int nb, std::vector<std::vector<CostItem>> &bins) {
    std::sort(items.begin(), items.end(), [](const CostItem &x, const CostItem &y) { return x.first > y.first; });
    bins.assign(nb, {});
    std::vector<long> load(nb, 0);
    for (const CostItem &it : items) {
        const int j = (int)(std::min_element(load.begin(), load.end()) - load.begin());
        bins[j].push_back(it);
        load[j] += it.first;
    }
    for (int iter = 0; iter < 4096; iter++) {
        const int m = (int)(std::max_element(load.begin(), load.end()) - load.begin());
        long best = 0;
        int bj = -1, ba = -1, bb = -1;   // move item ba of bin m to bin bj (bb < 0) or swap it with item bb of bj
        for (int j = 0; j < nb; j++) {
            if (j == m) continue;
            for (int ia = 0; ia < (int)bins[m].size(); ia++) {
                const long ca = bins[m][ia].first;
                long nm = load[m] - ca, nj = load[j] + ca;
                if (load[m] - std::max(nm, nj) > best) { best = load[m] - std::max(nm, nj); bj = j; ba = ia; bb = -1; }
                for (int ib = 0; ib < (int)bins[j].size(); ib++) {
                    const long d = ca - bins[j][ib].first;
                    if (d <= 0) continue;
                    nm = load[m] - d; nj = load[j] + d;
                    if (load[m] - std::max(nm, nj) > best) { best = load[m] - std::max(nm, nj); bj = j; ba = ia; bb = ib; }
                }
            }
        }
        if (bj < 0) break;
        const CostItem a = bins[m][ba];
        if (bb < 0) {
            bins[m].erase(bins[m].begin() + ba);
            bins[bj].push_back(a);
            load[m] -= a.first; load[bj] += a.first;
        } else {
            const CostItem bi = bins[bj][bb];
            bins[m][ba] = bi; bins[bj][bb] = a;
            load[m] += bi.first - a.first; load[bj] += a.first - bi.first;
        }
    }
    // Then the heaviest list and another one re-split: any distribution of
    // the union of their items (up to 8) over the two, while that lowers the
    // heaviest list.  (Single moves and swaps stop short at 4096 tokens: 129
    // tile-times against 127 here and a mean of 126.)
    for (int iter = 0; iter < 4096; iter++) {
        const int m = (int)(std::max_element(load.begin(), load.end()) - load.begin());
        long best = load[m];
        int bj = -1;
        unsigned bmask = 0;
        for (int j = 0; j < nb; j++) {
            const int nu = (int)(bins[m].size() + bins[j].size());
            if (j == m || nu > 8) continue;
            const long tot = load[m] + load[j];
            for (unsigned mask = 0; mask < (1u << nu); mask++) {
                long sm = 0;
                for (int i = 0; i < nu; i++)
                    if (mask >> i & 1) sm += (i < (int)bins[m].size() ? bins[m][i] : bins[j][i - bins[m].size()]).first;
                if (std::max(sm, tot - sm) < best) {
                    best = std::max(sm, tot - sm);
                    bj = j;
                    bmask = mask;
                }
            }
        }
        if (bj < 0) break;
        std::vector<CostItem> u(bins[m]), nm, nj;
        u.insert(u.end(), bins[bj].begin(), bins[bj].end());
        for (size_t i = 0; i < u.size(); i++) (bmask >> i & 1 ? nm : nj).push_back(u[i]);
        bins[m] = nm; bins[bj] = nj;
        load[m] = 0; load[bj] = 0;
        for (const CostItem &c : nm) load[m] += c.first;
        for (const CostItem &c : nj) load[bj] += c.first;
    }
    for (auto &bn : bins)
        std::sort(bn.begin(), bn.end(), [](const CostItem &x, const CostItem &y) { return x.first > y.first; });
}

// The schedule for this call's shape, built and uploaded once per shape and
// cached; nullptr when the items fit the CUs (one workgroup per item needs no
// list) or when it would have to be uploaded inside a stream capture.  After
// 64 shapes the cache starts afresh: a schedule that a capture launched is
// retired (kept while a captured graph may hold its address), the others are
// freed at once.  A verify window that moves pos0 every step has at most one
// 128-query tile per head, so it never builds a schedule.
const GqpSched *gqp_schedule(vx27_hip_ctx *ctx, const vx27_gqa_prefill_desc *d, int xcd_map) {
    const int n_qt = (d->T + PP_QT - 1) / PP_QT;
    if ((long long)d->B * d->n_q * n_qt <= ctx->n_cu) return nullptr;
    const bool capturing = vx_ctx_capturing(ctx);
    const int key[7] = {d->T, d->pos0, d->n_q, d->n_kv, d->B, ctx->n_cu, xcd_map};
    for (void *p : ctx->gqp_scheds) {
        GqpSched *c = (GqpSched *)p;
        if (std::equal(key, key + 7, c->key)) {
            if (capturing) c->captured = true;
            return c;
        }
    }
    if (capturing) return nullptr;
    if (ctx->gqp_scheds.size() >= 64) {
        if (hipStreamSynchronize(ctx->stream) != hipSuccess) return nullptr;
        for (void *p : ctx->gqp_scheds) {
            GqpSched *old = (GqpSched *)p;
            if (old->captured)
                vx_ctx_release(ctx, old->dev);
            else
                (void)hipFree(old->dev);
            free(old);
        }
        ctx->gqp_scheds.clear();
    }
    const int n_groups = xcd_map ? 8 : 1;
    const int per = xcd_map ? std::max(1, ctx->n_cu / 8) : std::max(1, ctx->n_cu);
    std::vector<std::vector<CostItem>> group(n_groups);
    for (int b = 0; b < d->B; b++)
        for (int h = 0; h < d->n_q; h++) {
            int g = 0;
            if (xcd_map) {   // the XCD whose head set holds h (inverse of the one-item-per-workgroup map)
                const int gq = d->n_q / d->n_kv, hpx = d->n_q / 8, xpk = 8 / d->n_kv;
                g = (h / gq) * xpk + (h % gq) / hpx;
            }
            for (int qt = 0; qt < n_qt; qt++) {
                const int last = d->pos0 + std::min(qt * PP_QT + PP_QT, d->T) - 1;
                group[g].push_back(CostItem(last / KT + 1 + GQP_ITEM_OVERHEAD, (b * d->n_q + h) * n_qt + qt));
            }
        }
    std::vector<std::vector<std::vector<CostItem>>> bins(n_groups);
    int len = 1;
    for (int g = 0; g < n_groups; g++) {
        gqp_pack(group[g], per, bins[g]);
        for (auto &bn : bins[g]) len = std::max(len, (int)bn.size());
    }
    const int n_wg = per * n_groups;
    std::vector<int> tab((size_t)n_wg * len, -1);
    for (int w = 0; w < n_wg; w++) {
        const auto &bn = bins[w % n_groups][w / n_groups];
        for (size_t i = 0; i < bn.size(); i++) tab[(size_t)w * len + i] = bn[i].second;
    }
    GqpSched *sc = (GqpSched *)calloc(1, sizeof(GqpSched));
    if (!sc) return nullptr;
    if (hipMalloc(&sc->dev, tab.size() * sizeof(int)) != hipSuccess) { free(sc); return nullptr; }
    if (hipMemcpy(sc->dev, tab.data(), tab.size() * sizeof(int), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(sc->dev);
        free(sc);
        return nullptr;
    }
    std::copy(key, key + 7, sc->key);
    sc->len = len;
    sc->n_wg = n_wg;
    ctx->gqp_scheds.push_back(sc);
    return sc;
}
}  // namespace

void vx_gqp_sched_free(vx27_hip_ctx *ctx) {
    for (void *p : ctx->gqp_scheds) {
        GqpSched *sc = (GqpSched *)p;
        (void)hipFree(sc->dev);
        free(sc);
    }
    ctx->gqp_scheds.clear();
}

static int gqa_prefill_check(const vx27_gqa_prefill_desc *d) {
    VX_REQUIRE(d, "vx27_hip_gqa_prefill: null descriptor");
    VX_REQUIRE(d->hd == HDG, "vx27_hip_gqa_prefill: hd must be 256 (got %d)", d->hd);
    VX_REQUIRE(d->B >= 1 && d->T >= 1 && d->n_kv >= 1 && d->n_q >= d->n_kv && d->n_q % d->n_kv == 0,
               "vx27_hip_gqa_prefill: bad sizes B=%d T=%d n_q=%d n_kv=%d", d->B, d->T, d->n_q, d->n_kv);
    VX_REQUIRE(d->L >= 64 && d->L % 64 == 0, "vx27_hip_gqa_prefill: L must be a positive multiple of 64");
    VX_REQUIRE(d->pos0 >= 0 && (long long)d->pos0 + d->T <= d->L,
               "vx27_hip_gqa_prefill: positions [%d, %d) outside the cache (L=%d)", d->pos0, d->pos0 + d->T, d->L);
    VX_REQUIRE(d->rope_dim >= 0 && d->rope_dim <= VX_ROPE_MAXH && d->rope_dim % 64 == 0,
               "vx27_hip_gqa_prefill: rope_dim must be a multiple of 64 in [0, %d] (got %d)", VX_ROPE_MAXH, d->rope_dim);
    VX_REQUIRE((d->q_tok_stride == 0 || d->q_tok_stride % 8 == 0) && (d->q_head_stride == 0 || d->q_head_stride % 8 == 0) &&
                   ((uintptr_t)d->q & 15) == 0,
               "vx27_hip_gqa_prefill: q must be 16-byte aligned with strides that are multiples of 8 elements");
    VX_REQUIRE(((uintptr_t)d->v_new & 15) == 0, "vx27_hip_gqa_prefill: v_new must be 16-byte aligned");
    VX_REQUIRE(((uintptr_t)d->k_new & 7) == 0, "vx27_hip_gqa_prefill: k_new must be 8-byte aligned");
    VX_REQUIRE((((uintptr_t)d->k_cache | (uintptr_t)d->v_cache) & 15) == 0,
               "vx27_hip_gqa_prefill: k_cache and v_cache must be 16-byte aligned");
    const bool gated = !(d->flags & VX27_GQA_NO_GATE);
    VX_REQUIRE(!gated || ((d->gate_tok_stride == 0 || d->gate_tok_stride % 4 == 0) &&
                          (d->gate_head_stride == 0 || d->gate_head_stride % 4 == 0) && ((uintptr_t)d->gate & 7) == 0),
               "vx27_hip_gqa_prefill: gate must be 8-byte aligned with strides that are multiples of 4 elements");
    VX_REQUIRE(((uintptr_t)d->out & 15) == 0, "vx27_hip_gqa_prefill: out must be 16-byte aligned");
    VX_REQUIRE(((uintptr_t)d->q_norm_w & 15) == 0, "vx27_hip_gqa_prefill: q_norm_w must be 16-byte aligned");
    VX_REQUIRE(d->q && (d->gate || !gated) && d->k_new && d->v_new && d->q_norm_w && d->k_norm_w && d->k_cache &&
                   d->v_cache && d->out,
               "vx27_hip_gqa_prefill: null pointer in descriptor");
    return 0;
}

size_t vx_gqa_prefill_scratch(const vx27_gqa_prefill_desc *d) {
    return (size_t)d->T * (d->rope_dim / 2 + 1) * sizeof(float2);
}

// The prefill on caller-provided scratch of vx_gqa_prefill_scratch(d) bytes.
int vx_gqa_prefill_into(vx27_hip_ctx *ctx, const vx27_gqa_prefill_desc *d, void *scr) {
    if (gqa_prefill_check(d)) return -1;
    const bool gated = !(d->flags & VX27_GQA_NO_GATE);
    KvArgs ka = {};
    if (d->rope_dim > 0 && vx_rope_fill(ka.rope, d->rope_dim, d->rope_theta)) return -1;
    ka.T = d->T; ka.n_kv = d->n_kv; ka.rope_dim = d->rope_dim; ka.L = d->L; ka.pos0 = d->pos0;
    ka.flags = d->flags; ka.yarn = d->rope_yarn < 1.0f ? 1.0f : d->rope_yarn;
    ka.k = d->k_new; ka.v = d->v_new; ka.kv_ts = (size_t)d->n_kv * HDG;
    ka.k_norm_w = d->k_norm_w; ka.k_cache = d->k_cache; ka.v_cache = d->v_cache;
    ka.cs_tab = (float2 *)scr;
    {
        const int nblk = (d->pos0 + d->T - 1) / VX_GQA_VBLK - d->pos0 / VX_GQA_VBLK + 1;
        VX_LAUNCH(ctx, gqp_kv, dim3((unsigned)nblk, (unsigned)d->n_kv, (unsigned)d->B), dim3(256), ka);
    }

    AttnArgs aa;
    aa.T = d->T; aa.n_q = d->n_q; aa.n_kv = d->n_kv; aa.L = d->L; aa.pos0 = d->pos0;
    aa.rope_dim = d->rope_dim; aa.flags = d->flags; aa.yarn = ka.yarn; aa.cs_tab = ka.cs_tab;
    aa.q = d->q;
    aa.q_ts = d->q_tok_stride ? d->q_tok_stride : (size_t)d->n_q * HDG;
    aa.q_hs = d->q_head_stride ? d->q_head_stride : HDG;
    aa.q_norm_w = d->q_norm_w;
    aa.k_cache = d->k_cache; aa.v_cache = d->v_cache;
    aa.gate = gated ? d->gate : nullptr;
    aa.g_ts = d->gate_tok_stride ? d->gate_tok_stride : (size_t)d->n_q * HDG;
    aa.g_hs = d->gate_head_stride ? d->gate_head_stride : HDG;
    aa.out = d->out;
    // XCD grouping needs whole KV heads per XCD pair set: n_kv | 8 and 8 | n_q
    aa.xcd_map = (8 % d->n_kv == 0) && (d->n_q % 8 == 0) && ((d->n_q / 8) * (8 / d->n_kv) == d->n_q / d->n_kv);
    const int n_qt = (d->T + PP_QT - 1) / PP_QT;
    aa.n_qt = n_qt;
    aa.sched = nullptr;
    aa.sched_len = 0;
    const GqpSched *sc = gqp_schedule(ctx, d, aa.xcd_map);
    if (sc) {   // persistent: one workgroup per CU over its list
        aa.sched = sc->dev;
        aa.sched_len = sc->len;
        VX_LAUNCH_NAMED(ctx, "gqp_attn", gqp_attn_pp, dim3((unsigned)sc->n_wg), dim3(PP_NW * 64), aa);
    } else {    // few items, or a capture's first call of a shape: one workgroup per item
        VX_LAUNCH_NAMED(ctx, "gqp_attn", gqp_attn_pp, dim3((unsigned)(n_qt * d->n_q), (unsigned)d->B), dim3(PP_NW * 64), aa);
    }
    return 0;
}

extern "C" int vx27_hip_gqa_prefill(vx27_hip_ctx *ctx, const vx27_gqa_prefill_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    if (gqa_prefill_check(d)) return -1;
    void *scr;
    if (vx_ctx_scratch(ctx, vx_gqa_prefill_scratch(d), &scr)) return -1;
    return vx_gqa_prefill_into(ctx, d, scr);
}

