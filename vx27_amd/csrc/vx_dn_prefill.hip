// Gated DeltaNet prefill on gfx950: the chunked (WY) form of the exact delta
// rule, bf16 MFMA for the chunk products, fp32 state carried across chunks.
//
// Per token the reference (vx27_deltanet_step_exact, vx27_deltanet.c:71-102,
// applied token by token by vx27_qlayer_batch, vx27_qfwd.c:249-313) does
//   kn = l2norm(k), qn = l2norm(q)/sqrt(128), S <- e^g S,
//   u = beta (v - S^T kn), S <- S + kn u^T, o = S^T qn.
// Over a chunk of C = 64 tokens with state S0 at its start and cumulative
// log-decay gam_t = g_1 + ... + g_t this is exactly
//   U  = T (beta V) - T (beta e^gam K) S0 = Ut + NW S0,     T = (I + A)^-1,
//   A[s][r] = beta_s e^(gam_s - gam_r) kn_s.kn_r   (r < s),
//   O  = (e^gam Q) S0 + P U,   P[t][s] = e^(gam_t - gam_s) qn_t.kn_s (s <= t),
//   S  = e^gam_C S0 + Kt^T U,  Kt[t] = e^(gam_C - gam_t) kn_t,
// where every exponent is <= 0.  Only S0 couples the chunks.
//
// dnp_prep  (grid chunks x value heads x sequences, fully parallel): gates,
//           norms, K K^T and Q K^T on MFMA, the triangular solve for Ut and
//           NW = -T (beta e^gam K) by forward substitution in fp32 (one lane
//           per column), and the chunk's MFMA operand tiles written to a
//           record in scratch.
// dnp_scan  (grid value heads x 8 column slices x sequences): walks the
//           chunks in order; a workgroup owns 16 value columns of one head's
//           state (columns are independent in all three products), keeps
//           them in MFMA accumulators and runs 14 MFMAs per wave per chunk.
//           Each wave loads its own operand tiles straight into registers,
//           a chunk ahead.  The 8 slices of a head are placed on one XCD so
//           the records they share are read from HBM once.
//
// Operand tiles ([rows/16][k/32][64 lanes][8] bf16) follow the MFMA operand
// layout of v_mfma_f32_16x16x32_bf16: lane (g = l/16, m = l%16) of an A tile
// holds A[m][8g..8g+7]; a wave's tile is 1 KiB of contiguous memory.
#include <algorithm>

#include "vx_dn.h"
#include "vx_gemv.h"
#include "vx_lds.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int CH = 64;            // chunk length
constexpr int NSLICE = 8;         // 16-column slices of a head's state


// chunk record (bytes)
constexpr size_t R_NW = 0;                       // -W   [4][4][64][8] bf16
constexpr size_t R_QE = R_NW + 4 * 4 * 512 * 2;  // e^gam qn  [4][4][64][8] bf16
constexpr size_t R_KT = R_QE + 4 * 4 * 512 * 2;  // Kt^T [8][2][64][8] bf16
constexpr size_t R_P = R_KT + 8 * 2 * 512 * 2;   // P    [4][2][64][8] bf16
constexpr size_t R_UT = R_P + 4 * 2 * 512 * 2;   // Ut   [4 rb][8 cs][64][4] fp32
constexpr size_t R_GC = R_UT + 4 * 8 * 64 * 4 * 4; // e^gam_C, one float
constexpr size_t REC = R_GC + 256;

struct PrepArgs {
    int T, nqk, nv, NC;
    const uint16_t *q, *k, *v;       // [B][T][nqk|nqk|nv][128] bf16
    const float *a, *b;              // [B][T][nv]
    const float *A_log, *dt_bias;    // [nv]
    char *rec;                       // [B][nv][NC] records
    float *gC;                       // [B][nv][NC] e^gam_C
};

// round-to-nearest-even pair (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = (bf16x2_t){(__bf16)x, (__bf16)y};
    uint32_t r;
    __builtin_memcpy(&r, &v, 4);
    return r;
}
__device__ __forceinline__ uint4 pack8(const float *f) {
    return make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
}
__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) {
    bf16x8_t r;
    __builtin_memcpy(&r, &u, 16);
    return r;
}

// LDS of dnp_prep, one byte array carved into regions whose contents change
// with the phase:
//   R1: raw q rows [64][RP] bf16  -> P staging [64][TP] bf16 -> T [64][64] fp32
//   R2: raw k rows [64][RP] bf16  -> V^T [128][TP] bf16     -> -W staging [64][RP] bf16
//   KTR: K^T [128][TP] bf16 (raw k, dims x tokens)
//   AS: A [64][AP] fp32; MT: level products [3][16][16] fp32; then per-token scalars
constexpr int RP = HD + 8;     // padded bf16 row of 128 elements
constexpr int TP = CH + 8;     // padded bf16 row of 64 elements
constexpr int AP = CH + 4;     // padded fp32 row of A
constexpr int L_R1 = 0;
constexpr int L_R2 = L_R1 + CH * RP * 2;
constexpr int L_KT = L_R2 + HD * TP * 2;
constexpr int L_AS = L_KT + HD * TP * 2;
constexpr int L_MT = L_AS + CH * AP * 4;
constexpr int L_GAM = L_MT + 3 * 256 * 4;
constexpr int L_SC = L_GAM + CH * 8;            // 5 float[64]: beta, e^gam, e^(gamC-gam), 1/|q|, 1/|k|
constexpr int L_TOTAL = L_SC + 5 * CH * 4;
static_assert(CH * 64 * 4 <= CH * RP * 2, "T fits region R1");

// One workgroup per (chunk of 64 tokens, value head, sequence):
//   phase 1  gates and the cumulative log-decay (wave 0); raw k rows, K^T and
//            1/|k| (wave 1); raw q rows and 1/|q| (wave 2); v rows (wave 3)
//   phase 2  K K^T and Q K^T on MFMA (raw bf16 rows, norms applied after);
//            e^gam Q and Kt^T operand tiles
//   phase 3  A = beta e^(gam_s - gam_r) kn_s.kn_r (r < s), P operand tiles;
//            V^T in LDS
//   phase 4  T = (I + A)^-1, blocked: the four 16x16 diagonal blocks by
//            forward substitution, then T_ij = -T_ii sum_k A_ik T_kj level by
//            level (fp32)
//   phase 5  [Ut | W] = T [beta V | beta e^gam kn] on MFMA, as
//            (T diag(beta)) V and (T diag(beta e^gam /|k|)) K with V, K the
//            raw bf16 inputs (exact operands) and the scaled T split into
//            bf16 hi + lo (a 16-bit-significand product, fp32 sums)
__global__ __launch_bounds__(256) void dnp_prep(PrepArgs p) {
    const int c = blockIdx.x, vh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, m = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qh = vh * p.nqk / p.nv;
    const int t0 = c * CH;
    const int nvalid = min(CH, p.T - t0);

    __shared__ __attribute__((aligned(16))) char smem[L_TOTAL];
    uint16_t *q_rows = (uint16_t *)(smem + L_R1);   // [64][RP]
    uint16_t *P_b = (uint16_t *)(smem + L_R1);      // [64][TP]
    float *T_s = (float *)(smem + L_R1);            // [64][64]
    uint16_t *k_rows = (uint16_t *)(smem + L_R2);   // [64][RP]
    uint16_t *V_t = (uint16_t *)(smem + L_R2);      // [128][TP]
    uint16_t *W_b = (uint16_t *)(smem + L_R2);      // [64][RP]
    uint16_t *K_t = (uint16_t *)(smem + L_KT);      // [128][TP]
    float *A_s = (float *)(smem + L_AS);            // [64][AP]
    float *M_t = (float *)(smem + L_MT);            // [3][16][16]
    double *gam_s = (double *)(smem + L_GAM);
    float *beta_s = (float *)(smem + L_SC), *eg_s = beta_s + CH, *egc_s = eg_s + CH;
    float *iq_s = egc_s + CH, *ik_s = iq_s + CH;

    // ---- phase 1
    // gates and the cumulative log-decay (wave 0, lane = token); masked
    // tokens get beta = 0 and g = 0, which leaves U and S unchanged
    if (wave == 0) {
        double beta = 0.0, glog = 0.0;
        if (lane < nvalid) {
            const size_t e = ((size_t)b * p.T + t0 + lane) * p.nv + vh;
            beta = 1.0 / (1.0 + exp(-(double)p.b[e]));
            glog = -exp((double)p.A_log[vh]) * softplus_d((double)p.a[e] + (double)p.dt_bias[vh]);
        }
        double sc = glog;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(sc, off, 64);
            if (lane >= off) sc += o;
        }
        const double sC = __shfl(sc, 63, 64);
        gam_s[lane] = sc;
        beta_s[lane] = (float)beta;
        eg_s[lane] = (float)exp(sc);
        egc_s[lane] = (float)exp(sC - sc);
    }
    // rows of one token per lane (wave 1: k, wave 2: q, wave 3: v); the lane
    // sums its own squares (double), so no cross-lane reduction is needed
    uint4 raw[16];
    if (wave >= 1) {
        const uint16_t *src = wave == 1 ? p.k + (((size_t)b * p.T + t0 + lane) * p.nqk + qh) * HD
                            : wave == 2 ? p.q + (((size_t)b * p.T + t0 + lane) * p.nqk + qh) * HD
                                        : p.v + (((size_t)b * p.T + t0 + lane) * p.nv + vh) * HD;
        if (lane < nvalid) {
#pragma unroll
            for (int j = 0; j < 16; j++) raw[j] = *(const uint4 *)(src + 8 * j);
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) raw[j] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    if (wave == 1 || wave == 2) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const double lo = (double)vx_bf16_to_f32((uint16_t)w4[e]);
                const double hi = (double)vx_bf16_to_f32((uint16_t)(w4[e] >> 16));
                ss = ss + lo * lo;
                ss = ss + hi * hi;
            }
        }
        const float inv = 1.0f / sqrtf((float)ss + 1e-6f);   // l2norm, vx27_deltanet.c:51-56
        uint16_t *rows = wave == 1 ? k_rows : q_rows;
#pragma unroll
        for (int j = 0; j < 16; j++) *(uint4 *)&rows[lane * RP + 8 * j] = raw[j];
        if (wave == 1) {
            ik_s[lane] = inv;
            // K^T: dim d of every token, one 128-byte row per instruction
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    K_t[(8 * j + 2 * e) * TP + lane] = (uint16_t)w4[e];
                    K_t[(8 * j + 2 * e + 1) * TP + lane] = (uint16_t)(w4[e] >> 16);
                }
            }
        } else {
            iq_s[lane] = inv;
        }
    }
    __syncthreads();

    char *rec = p.rec + (((size_t)b * p.nv + vh) * p.NC + c) * REC;
    const double gamC = gam_s[CH - 1];
    if (tid == 0) *(float *)(rec + R_GC) = (float)exp(gamC);
    const float qscale = 1.0f / sqrtf((float)HD);

    // ---- phase 2: raw K K^T and Q K^T for row block `wave`; e^gam qn tiles
    floatx4_t acck[4], accq[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
        acck[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
        accq[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    }
    const int rowA = wave * 16 + m;
    const float qeA = eg_s[rowA] * (iq_s[rowA] * qscale);
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const int d0 = 32 * ks + 8 * g;
        const uint4 qa = *(const uint4 *)&q_rows[rowA * RP + d0];
        const bf16x8_t aq = as_bf16x8(qa);
        const bf16x8_t ak = as_bf16x8(*(const uint4 *)&k_rows[rowA * RP + d0]);
        {   // e^gam qn tile (row block wave, k-step ks)
            const uint16_t *qs = (const uint16_t *)&qa;
            float f[8];
#pragma unroll
            for (int e = 0; e < 8; e++) f[e] = qeA * vx_bf16_to_f32(qs[e]);
            *(uint4 *)(rec + R_QE + ((size_t)(wave * 4 + ks) * 64 + lane) * 16) = pack8(f);
        }
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
            const bf16x8_t bk = as_bf16x8(*(const uint4 *)&k_rows[(nb * 16 + m) * RP + d0]);
            acck[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, bk, acck[nb], 0, 0, 0);
            accq[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq, bk, accq[nb], 0, 0, 0);
        }
    }
    // Kt^T tiles: rows = key dims (8 blocks), k = tokens (2 steps); 4 per wave
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int tile = wave * 4 + j, rb = tile >> 1, ks = tile & 1;
        const int i = rb * 16 + m, tb = 32 * ks + 8 * g;
        const uint4 kr = *(const uint4 *)&K_t[i * TP + tb];
        const uint16_t *kv = (const uint16_t *)&kr;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; e++) f[e] = (egc_s[tb + e] * ik_s[tb + e]) * vx_bf16_to_f32(kv[e]);
        *(uint4 *)(rec + R_KT + ((size_t)tile * 64 + lane) * 16) = pack8(f);
    }
    __syncthreads();   // q and k rows are no longer read

    // ---- phase 3: A (fp32, for the inverse), P (bf16 staging), V^T
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int s = wave * 16 + 4 * g + i, r = nb * 16 + m;
            const float ed = r <= s ? expf((float)(gam_s[s] - gam_s[r])) : 0.0f;
            A_s[s * AP + r] = r < s ? beta_s[s] * ed * ((ik_s[s] * ik_s[r]) * acck[nb][i]) : 0.0f;
            P_b[s * TP + r] = vx_f32_to_bf16(ed * (((iq_s[s] * qscale) * ik_s[r]) * accq[nb][i]));
        }
    }
    if (wave == 3) {   // V^T: dim d of every token
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                V_t[(8 * j + 2 * e) * TP + lane] = (uint16_t)w4[e];
                V_t[(8 * j + 2 * e + 1) * TP + lane] = (uint16_t)(w4[e] >> 16);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const uint4 v = *(const uint4 *)&P_b[rowA * TP + 32 * ks + 8 * g];
        *(uint4 *)(rec + R_P + ((size_t)(wave * 2 + ks) * 64 + lane) * 16) = v;
    }
    __syncthreads();   // P staging is read out; R1 takes T

    // ---- phase 4: T = (I + A)^-1
    if (tid < 64) {   // diagonal blocks: thread (block bi, column cc)
        const int bi = tid >> 4, cc = tid & 15, o = 16 * bi;
        float t[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float acc = r == cc ? 1.0f : 0.0f;
#pragma unroll
            for (int k = 0; k < r; k++) acc -= A_s[(o + r) * AP + o + k] * t[k];
            t[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) T_s[(o + r) * 64 + o + cc] = t[r];
    }
    __syncthreads();
    // off-diagonal blocks, level by level: T[j+lev][j] = -T[i][i] M,
    // M = sum_{kb=j}^{i-1} A[i][kb] T[kb][j] (i = j + lev), one block per wave
    // on the fp32 MFMA (v_mfma_f32_16x16x4_f32: lane l holds A[l%16][k0 + l/16]
    // and B[k0 + l/16][l%16]; exact fp32 products)
    float *Mw = M_t + (wave < 3 ? wave : 0) * 256;   // this wave's 16x16 scratch
#pragma unroll
    for (int lev = 1; lev < 4; lev++) {
        if (wave < 4 - lev) {
            const int j = wave, i = j + lev;
            floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
            for (int kb = j; kb < i; kb++) {
#pragma unroll
                for (int k0 = 0; k0 < 16; k0 += 4) {
                    const float av = A_s[(16 * i + m) * AP + 16 * kb + k0 + g];
                    const float bv = T_s[(16 * kb + k0 + g) * 64 + 16 * j + m];
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
                }
            }
#pragma unroll
            for (int ii = 0; ii < 4; ii++) Mw[(4 * g + ii) * 16 + m] = acc[ii];
            asm volatile("" ::: "memory");   // LDS ops of one wave stay in order
            floatx4_t tacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k0 = 0; k0 < 16; k0 += 4) {
                const float av = T_s[(16 * i + m) * 64 + 16 * i + k0 + g];
                const float bv = Mw[(k0 + g) * 16 + m];
                tacc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, tacc, 0, 0, 0);
            }
#pragma unroll
            for (int ii = 0; ii < 4; ii++) T_s[(16 * i + 4 * g + ii) * 64 + 16 * j + m] = -tacc[ii];
        }
        __syncthreads();
    }

    // ---- phase 5: [Ut | W] rows of block `wave` = T_V V | T_K K (MFMA)
    bf16x8_t tv[2][2], tk[2][2];   // [k-step][hi, lo]
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const int s = wave * 16 + m, r0 = 32 * ks + 8 * g;
        float fv[8], fk[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int r = r0 + e;
            const float tsr = r <= s ? T_s[s * 64 + r] : 0.0f;   // upper blocks are never written
            fv[e] = tsr * beta_s[r];
            fk[e] = tsr * ((beta_s[r] * eg_s[r]) * ik_s[r]);
        }
        float lv[8], lk[8];
        const uint4 hv = pack8(fv), hk = pack8(fk);
        const uint16_t *hvs = (const uint16_t *)&hv, *hks = (const uint16_t *)&hk;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            lv[e] = fv[e] - vx_bf16_to_f32(hvs[e]);
            lk[e] = fk[e] - vx_bf16_to_f32(hks[e]);
        }
        tv[ks][0] = as_bf16x8(hv);
        tv[ks][1] = as_bf16x8(pack8(lv));
        tk[ks][0] = as_bf16x8(hk);
        tk[ks][1] = as_bf16x8(pack8(lk));
    }
    floatx4_t wacc[8];
    float *ut = (float *)(rec + R_UT);
#pragma unroll
    for (int cb = 0; cb < 16; cb++) {
        const bool isv = cb < 8;
        const uint16_t *src = isv ? V_t : K_t;
        const int col = (cb & 7) * 16 + m;
        floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const bf16x8_t bop = as_bf16x8(*(const uint4 *)&src[col * TP + 32 * ks + 8 * g]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(isv ? tv[ks][0] : tk[ks][0], bop, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(isv ? tv[ks][1] : tk[ks][1], bop, acc, 0, 0, 0);
        }
        if (isv) {   // Ut: C layout tile (rb = wave, cs = cb), as the scan reads it
            *(floatx4_t *)&ut[(((size_t)wave * 8 + cb) * 64 + lane) * 4] = acc;
        } else {
            wacc[cb - 8] = acc;
        }
    }
    __syncthreads();   // every read of V^T is done: R2 takes the -W staging
    // -W rows (token 16 wave + 4g + i, dim 16 cb + m) -> bf16 staging
#pragma unroll
    for (int cb = 0; cb < 8; cb++)
#pragma unroll
        for (int i = 0; i < 4; i++) W_b[(wave * 16 + 4 * g + i) * RP + cb * 16 + m] = vx_f32_to_bf16(-wacc[cb][i]);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
        *(uint4 *)(rec + R_NW + ((size_t)(wave * 4 + ks) * 64 + lane) * 16) = *(const uint4 *)&W_b[rowA * RP + 32 * ks + 8 * g];
}

struct ScanArgs {
    int T, nv, NC, xcd_map;
    const char *rec;
    const float *gC;
    float *S;        // [B][nv][128][128]
    float *out;      // [B][T][nv][128]
};

// A wave's operands of one chunk: 15 tiles of 1 KiB in its record -- -W
// (rows 16w..16w+15, 4 k-steps), e^gam Q (same rows), Kt^T (row blocks 2w,
// 2w+1, 2 k-steps each), P (rows 16w.., 2 k-steps) and the wave's Ut block
// of the slice -- and e^gam_C.  They come straight from the record into
// registers, and each group takes the next chunk's loads as soon as its
// MFMAs have read it (as in dnp_scant, below).
constexpr int OPS_TILES = 15;

__device__ __forceinline__ uint32_t ops_src(int j, int wave, int slice) {
    return j < 4    ? (uint32_t)(R_NW + (wave * 4 + j) * 1024)
           : j < 8  ? (uint32_t)(R_QE + (wave * 4 + j - 4) * 1024)
           : j < 12 ? (uint32_t)(R_KT + (wave * 4 + j - 8) * 1024)
           : j < 14 ? (uint32_t)(R_P + (wave * 2 + j - 12) * 1024)
                    : (uint32_t)(R_UT + (wave * 8 + slice) * 1024);
}
// (global address space: a generic pointer would make these flat loads,
// which count on the LDS counter too, so every LDS wait would drain them)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4_t g_u32x4;
typedef const __attribute__((address_space(1))) float g_float;
template <int J0, int J1>
__device__ __forceinline__ void ops_load(const char *rec, int wave, int slice, int lane, uint4 *op) {
#pragma unroll
    for (int j = J0; j < J1; j++) {
        const u32x4_t v = *(g_u32x4 *)(rec + ops_src(j, wave, slice) + (uint32_t)lane * 16);
        op[j] = make_uint4(v.x, v.y, v.z, v.w);
    }
}

__global__ __launch_bounds__(256) void dnp_scan(ScanArgs p) {
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.y, bid = blockIdx.x;
    int vh, slice;
    if (p.xcd_map) {   // the 8 slices of a head on one XCD (workgroups go round-robin over 8)
        const int xcd = bid & 7, idx = bid >> 3;
        slice = idx % NSLICE;
        vh = (idx / NSLICE) * 8 + xcd;
    } else {
        vh = bid / NSLICE;
        slice = bid % NSLICE;
    }
    const int col = slice * 16 + n;

    __shared__ uint16_t S_l[16][HD + 8];   // S slice, bf16, [column][key dim]
    __shared__ uint16_t U_l[16][CH + 8];   // U slice, bf16, [column][token]

    const char *rec0 = vx_uniform_ptr(p.rec + ((size_t)b * p.nv + vh) * p.NC * REC);
    uint4 op[OPS_TILES];
    ops_load<0, OPS_TILES>(rec0, wave, slice, lane, op);
    float gc = *(g_float *)(rec0 + R_GC);

    // state rows 32w .. 32w+31 (row blocks 2w, 2w+1) of the slice, C layout
    float *Sg = p.S + ((size_t)b * p.nv + vh) * HD * HD;
    floatx4_t S[2];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) S[r][i] = Sg[(size_t)((2 * wave + r) * 16 + 4 * g + i) * HD + col];

    for (int c = 0; c < p.NC; c++) {
        const char *rec1 = rec0 + (size_t)min(c + 1, p.NC - 1) * REC;   // the last one again after the end
        // S (bf16) -> LDS as [column][key dim]
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int d = (2 * wave + r) * 16 + 4 * g;
            *(uint2 *)&S_l[n][d] = make_uint2(pack2(S[r][0], S[r][1]), pack2(S[r][2], S[r][3]));
        }
        __syncthreads();   // S_l complete
        bf16x8_t sb[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) sb[ks] = as_bf16x8(*(const uint4 *)&S_l[n][32 * ks + 8 * g]);
        // U = Ut - W S for tokens 16w .. 16w+15, and the e^gam Q S part of O,
        // as independent two-MFMA chains; then -W, e^gam Q and Ut take chunk c+1
        const uint4 utu = op[14];
        floatx4_t U0 = (floatx4_t){__uint_as_float(utu.x), __uint_as_float(utu.y), __uint_as_float(utu.z), __uint_as_float(utu.w)};
        floatx4_t U1 = {0.f, 0.f, 0.f, 0.f};
        floatx4_t O0 = {0.f, 0.f, 0.f, 0.f}, O1 = {0.f, 0.f, 0.f, 0.f};
        U0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[0]), sb[0], U0, 0, 0, 0);
        U1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[1]), sb[1], U1, 0, 0, 0);
        O0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[4]), sb[0], O0, 0, 0, 0);
        O1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[5]), sb[1], O1, 0, 0, 0);
        U0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[2]), sb[2], U0, 0, 0, 0);
        U1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[3]), sb[3], U1, 0, 0, 0);
        O0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[6]), sb[2], O0, 0, 0, 0);
        O1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[7]), sb[3], O1, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        ops_load<0, 8>(rec1, wave, slice, lane, op);
        ops_load<14, 15>(rec1, wave, slice, lane, op);
        __builtin_amdgcn_sched_barrier(0);
        const floatx4_t U = U0 + U1;
        *(uint2 *)&U_l[n][wave * 16 + 4 * g] = make_uint2(pack2(U[0], U[1]), pack2(U[2], U[3]));
        __syncthreads();   // U_l complete
        bf16x8_t ub[2];
#pragma unroll
        for (int ks = 0; ks < 2; ks++) ub[ks] = as_bf16x8(*(const uint4 *)&U_l[n][32 * ks + 8 * g]);
        // O += P U (two more independent MFMAs); S = e^gam_C S + Kt^T U (per
        // row block, two independent MFMAs); then P, Kt^T, e^gam_C take chunk c+1
        O0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[12]), ub[0], O0, 0, 0, 0);
        O1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[13]), ub[1], O1, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 2; r++) {
            floatx4_t Sa = S[r] * gc, Sb = {0.f, 0.f, 0.f, 0.f};
            Sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[8 + 2 * r]), ub[0], Sa, 0, 0, 0);
            Sb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(op[9 + 2 * r]), ub[1], Sb, 0, 0, 0);
            S[r] = Sa + Sb;
        }
        __builtin_amdgcn_sched_barrier(0);
        ops_load<8, 14>(rec1, wave, slice, lane, op);
        gc = *(g_float *)(rec1 + R_GC);
        __builtin_amdgcn_sched_barrier(0);
        const floatx4_t O = O0 + O1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tt = c * CH + wave * 16 + 4 * g + i;
            if (tt < p.T) p.out[(((size_t)b * p.T + tt) * p.nv + vh) * HD + col] = O[i];
        }
    }
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) Sg[(size_t)((2 * wave + r) * 16 + 4 * g + i) * HD + col] = S[r][i];
}

// ---- split precision, T records (the default chunked form) ----------------
// Every product of the chunk form enters the MFMAs as bf16 pairs, hi =
// bf16(x) and lo = bf16(x - hi), summed as hi*hi + lo*hi + hi*lo (the lo*lo
// term, ~2^-16 of the product, is dropped): about 16 significand bits per
// operand, so the result stays within ~1e-5 of the fp32 recurrence instead
// of bf16's ~1e-2.  Inputs that are exact in bf16 (no lo part) take two.
//
// With K, Q the raw k, q rows of a chunk and kn = diag(1/|k|) K,
//   T' = (I + A)^-1 diag(beta),  Ut = T' V,  T'' = T' diag(sk),
//   sk_t = e^gam_t / |k_t|,  skc_t = e^(gam_C - gam_t) / |k_t|,
//   sq_t = e^gam_t / (|q_t| sqrt(128)),
// the chunk step is
//   U = Ut - T'' (K S0),
//   O = diag(sq) Q S0 + P U,
//   S = e^gam_C S0 + K^T diag(skc) U,
// so the chunk record (dnp_prept) holds -T'' and P as hi/lo operand tiles,
// Ut and the scales skc, sq, e^gam_C (65 KiB), and the raw K, Q and K^T
// operand tiles are kept once per QK head.  This is the form of the glue's
// inputs (q, k split into hi/lo pairs, v in fp32, nv = 3 nqk at the real
// layer): its records are less than half the full form's and the QK head's
// Gram products are shared by its value heads.  Masked tokens past the prompt have
// beta = 0 and g = 0: their columns of T' (and rows, since their row of A is
// zero) vanish, so whatever finite values their K, Q rows hold never reach
// U, S or a stored output.
constexpr size_t T_TH = 0;                 // -T'' hi: [4 rb][2 ks][64][8] bf16
constexpr size_t T_TL = 8192;              // -T'' lo
constexpr size_t T_PH = 16384;             // P hi
constexpr size_t T_PL = 24576;             // P lo
constexpr size_t T_UT = 32768;             // Ut fp32, C layout [4 rb][8 column blocks][64][4]
constexpr size_t T_SC = 65536;             // float skc[64], sq[64], e^gam_C
constexpr size_t TREC = T_SC + 1024;
// K record of (sequence, QK head, chunk): the raw k, q rows as MFMA operand
// tiles, 16 KiB each, hi parts then (with lo parts) lo parts:
constexpr size_t K_KT = 0;                 // K^T [8 rb (key dims)][2 ks (tokens)][64][8] bf16
constexpr size_t K_KA = 16384;             // K [4 rb (tokens)][4 dim blocks of 32][64][8]
constexpr size_t K_QA = 32768;             // Q, as K
constexpr size_t K_LO = 49152;             // offset of the lo parts

struct PrepTArgs {
    int T, nqk, nv, NC;
    const uint16_t *q, *k;          // hi parts [B][T][nqk][128] bf16
    const uint16_t *ql, *kl;        // lo parts as rows
    const float *v;                 // [B][T][nv][128] fp32 (unless XIN)
    const float *a, *b;             // [B][T][nv]
    const float *A_log, *dt_bias;   // [nv]
    char *rec;                      // [B][nv][NC] records of TREC bytes
    char *krec;                     // [B][nqk][NC] K records of krec_bytes
    int krec_bytes;
    // XIN: q, k and v formed here from x [B][T][C]: the causal conv + SiLU
    // (state before token 0 in conv_state [B][C][3], taps conv_w [C][4]),
    // then for q and k the pre-norms of `flags` (norm_w [128])
    int C, w_bf16;
    const float *x, *conv_state;
    const void *conv_w;
    unsigned flags;
    const float *norm_w;
};

// bf16 hi and lo of 8 floats
__device__ __forceinline__ void split8(const float *f, uint4 &hi, uint4 &lo) {
    hi = pack8(f);
    const uint16_t *h = (const uint16_t *)&hi;
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = f[e] - vx_bf16_to_f32(h[e]);
    lo = pack8(r);
}
// bf16 hi, lo of 4 floats, as two packed uint2
__device__ __forceinline__ void split4(const floatx4_t v, uint2 &h, uint2 &l) {
    h = make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
    const uint16_t *hs = (const uint16_t *)&h;
    l = make_uint2(pack2(v[0] - vx_bf16_to_f32(hs[0]), v[1] - vx_bf16_to_f32(hs[1])),
                   pack2(v[2] - vx_bf16_to_f32(hs[2]), v[3] - vx_bf16_to_f32(hs[3])));
}

// One causal-conv step of a channel as conv_step (window c0 oldest, c1, c2,
// x; products summed left to right), with SiLU as v / (1 + e^-v) from the
// hardware exp2 and reciprocal: a few ulp from the correctly rounded
// quotient, at a fifth of its instructions (prept's v channels)
__device__ __forceinline__ float conv_step_fast(float c[3], const float w[4], float x) {
    float acc = w[0] * c[0];
    acc = acc + w[1] * c[1];
    acc = acc + w[2] * c[2];
    acc = acc + w[3] * x;
    c[0] = c[1];
    c[1] = c[2];
    c[2] = x;
    return acc * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(acc * -1.4426950408889634f));
}

#define MFMA1(acc, a, b) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0)
#define MFMA3(acc, ah, al, bh, bl) \
    do {                           \
        MFMA1(acc, ah, bh);        \
        MFMA1(acc, al, bh);        \
        MFMA1(acc, ah, bl);        \
    } while (0)

// Transpose a row-major [64 tokens][RP] bf16 tile (128 dims) into
// [128 dims][TP] (64 tokens) with all 256 threads: thread (wave w, half h,
// pair q) takes tokens 2q, 2q+1 and dims 32w + 2i + h (i < 16), and packs the
// two tokens of a dim into one 32-bit LDS store (the halves of a wave write
// neighbouring dims, whose rows start 36 banks apart).
__device__ __forceinline__ void tr_rows(const uint16_t *src, uint16_t *dst, int tid) {
    const int w = tid >> 6, h = (tid >> 5) & 1, q = tid & 31;
    uint32_t r0[16], r1[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint4 a0 = *(const uint4 *)&src[(2 * q) * RP + 32 * w + 8 * k];
        const uint4 a1 = *(const uint4 *)&src[(2 * q + 1) * RP + 32 * w + 8 * k];
        r0[4 * k] = a0.x; r0[4 * k + 1] = a0.y; r0[4 * k + 2] = a0.z; r0[4 * k + 3] = a0.w;
        r1[4 * k] = a1.x; r1[4 * k + 1] = a1.y; r1[4 * k + 2] = a1.z; r1[4 * k + 3] = a1.w;
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t x = h ? r0[i] >> 16 : r0[i] & 0xffffu, y = h ? r1[i] >> 16 : r1[i] & 0xffffu;
        *(uint32_t *)&dst[(32 * w + 2 * i + h) * TP + 2 * q] = x | (y << 16);
    }
}

// Sum of a double over the 16 lanes of each 16-lane row (a fixed butterfly).
__device__ __forceinline__ double row16_sum(double v) {
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}
// The same sum on the DPP paths (no LDS round trips): quad exchanges 1 and 2,
// row rotations by 4 and 8 (a fixed tree), then lane 0's total broadcast to
// its row, so that every lane of a row holds the same bits.
__device__ __forceinline__ double row16_sum_dpp(double v) {
    v = v + vx_dpp_f64<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = v + vx_dpp_f64<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = v + vx_dpp_f64<0x124, 0xF>(v);   // row_ror:4
    v = v + vx_dpp_f64<0x128, 0xF>(v);   // row_ror:8
    return vx_dpp_f64<0x150, 0xF>(v);    // row_newbcast:0
}

// LDS of dnp_prept, 77 KiB (two workgroups a CU), four regions whose
// contents change with the phase (XIN, phase 1 first: the x windows of the
// QK head's q channels in R0-R1 and k channels in R2-R3, [68 tokens][128]
// fp32; then q and k after the conv as fp32 rows [64][128] in R0-R1 and
// R2-R3; then the lo rows of q in R2 and k in R3 beside the hi rows):
//   R0: q rows [64][RP] bf16 -> K^T lo [128][TP] -> A [64][AP] fp32 -> V hi rows
//       (XIN: V^T hi [128][TP])
//   R1: k rows [64][RP] bf16 -> k lo rows -> T [64][64] fp32 -> V^T lo [128][TP]
//   R2: K^T hi [128][TP] -> P hi, lo staging 2 x [64][TP] -> V^T hi [128][TP]
//       (XIN: the x window of v channels 64-127, [68 tokens][64] fp32)
//   R3: V lo rows [64][RP] (XIN: the x window of v channels 0-63)
constexpr int TN_REG = HD * TP * 2;
constexpr int TN_R0 = 0;
constexpr int TN_R1 = TN_R0 + TN_REG;
constexpr int TN_R2 = TN_R1 + TN_REG;
constexpr int TN_R3 = TN_R2 + TN_REG;
constexpr int TN_MT = TN_R3 + TN_REG;              // level products [3][16][16] fp32
constexpr int TN_GAM = TN_MT + 3 * 256 * 4;        // double gam[64]
constexpr int TN_SC = TN_GAM + CH * 8;             // float beta, e^gam, e^(gamC-gam), 1/|q|, 1/|k| [64]
constexpr int TN_TOTAL = TN_SC + 5 * CH * 4;
static_assert(CH * RP * 2 <= TN_REG && CH * AP * 4 <= TN_REG && CH * 64 * 4 <= TN_REG && 2 * CH * TP * 2 <= TN_REG,
              "regions hold rows, A, T and the P staging");
static_assert(2 * TN_TOTAL <= 160 * 1024, "two workgroups per CU");

// One workgroup per (chunk of 64 tokens, QK head, sequence); the value
// heads that share the QK head (nv / nqk of them) reuse its Gram products:
//   phase 1  q, k rows (hi to LDS; the lo parts from global memory where a
//            product needs them), four rows per instruction (thread: row
//            t/16 + 16 j, 8 dims), and 1/|q|, 1/|k| (double sums)
//   phase 2  K K^T and Q K^T on MFMA (raw rows, norms applied after); the
//            K^T operand tiles (hi, lo) into the K record
//   then per value head:
//   phase 3  gates and the cumulative log-decay (wave 0); the scales skc,
//            sq; A = beta e^(gam_s - gam_r) kn_s.kn_r (r < s) in LDS;
//            P = e^(gam_t - gam_s) qn_t.kn_s (s <= t) as hi/lo tiles
//   phase 4  T = (I + A)^-1, blocked: the four 16x16 diagonal blocks by
//            forward substitution, then T_ij = -T_ii sum_k A_ik T_kj level
//            by level (fp32 MFMA)
//   phase 5  T' = T diag(beta) (hi/lo in registers); -T'' = -T' diag(sk)
//            as hi/lo tiles; V through LDS transposed, Ut = T' V on MFMA
//            (with XIN q, k and v are formed here from x: phase 1 runs the
//            q/k conv and pre-norms, phase 5 the v conv; there is no glue
//            kernel)
template <bool XIN>
__global__ __launch_bounds__(256, 2) void dnp_prept(PrepTArgs p) {   // (two workgroups a CU: 256 registers)
    constexpr bool LO = true;   // (the glue's q, k, v always come with lo parts)
    const int c = blockIdx.x, qh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, m = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool w2 = wave >= 2;
    const int nr = p.nv / p.nqk;
    const int t0 = c * CH;
    const int nvalid = min(CH, p.T - t0);

    __shared__ __attribute__((aligned(16))) char smem[TN_TOTAL];
    uint16_t *q_rows = (uint16_t *)(smem + TN_R0), *kT_l = (uint16_t *)(smem + TN_R0);
    float *A_s = (float *)(smem + TN_R0);
    uint16_t *vh_rows = (uint16_t *)(smem + TN_R0);
    uint16_t *k_rows = (uint16_t *)(smem + TN_R1), *vl_rows = (uint16_t *)(smem + TN_R3);
    float *T_s = (float *)(smem + TN_R1);
    uint16_t *kT_h = (uint16_t *)(smem + TN_R2);
    uint16_t *P_h = (uint16_t *)(smem + TN_R2), *P_l = P_h + CH * TP;
    uint16_t *vT_h = (uint16_t *)(smem + TN_R2), *vT_l = (uint16_t *)(smem + TN_R1);
    float *M_t = (float *)(smem + TN_MT);
    double *gam_s = (double *)(smem + TN_GAM);
    float *beta_s = (float *)(smem + TN_SC), *eg_s = beta_s + CH, *egc_s = eg_s + CH;
    float *iq_s = egc_s + CH, *ik_s = iq_s + CH;
    const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
    const int seg = tid & 15;   // 8-dim segment of a row (phase 1, V rows)

    // ---- phase 1: k and q rows, thread (row tid/16 + 16 j, dims 8 seg ..)
    uint4 kh[4], kl[4], qhv[4], qlv[4];
    float xq[2][4], xk[2][4];   // (XIN) conv taps
    if (XIN) {
        // the x windows of the QK head's q and k channels (tokens t0-3 ..
        // t0+64, clamped to the prompt; 512-byte rows) into R0-R1 and R2-R3
        // by direct loads, 2 rows a wave instruction; the taps of channels
        // lane and lane + 64 of q and of k
        const float *xb = p.x + (size_t)b * p.T * p.C + (size_t)qh * HD;
        for (int i = wave; i < 34; i += 4) {
            const int row0 = min(max(t0 - 3 + 2 * i, 0), p.T - 1);
            const int row = min(max(t0 - 3 + 2 * i + (lane >> 5), 0), p.T - 1);
            const uint32_t off = (uint32_t)(((row - row0) * p.C + 4 * (lane & 31)) * 4);
            vx_dma16(vx_uniform_ptr(xb + (size_t)row0 * p.C), off, vx_lds_addr(smem + TN_R0) + 1024 * i);
            vx_dma16(vx_uniform_ptr(xb + (size_t)p.nqk * HD + (size_t)row0 * p.C), off, vx_lds_addr(smem + TN_R2) + 1024 * i);
        }
#pragma unroll
        for (int hc = 0; hc < 2; hc++) {
            const size_t chq = (size_t)qh * HD + lane + 64 * hc, chk = chq + (size_t)p.nqk * HD;
            load_conv_w(p.conv_w, p.w_bf16, chq, xq[hc]);
            load_conv_w(p.conv_w, p.w_bf16, chk, xk[hc]);
        }
        if (tid < HD) M_t[tid] = p.norm_w ? p.norm_w[tid] : 1.0f;   // (M_t is free until phase 4)
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = (tid >> 4) + 16 * j;
            const size_t off = (((size_t)b * p.T + t0 + r) * p.nqk + qh) * HD + 8 * seg;
            const bool ok = r < nvalid;
            kh[j] = ok ? *(const uint4 *)(p.k + off) : z4;
            qhv[j] = ok ? *(const uint4 *)(p.q + off) : z4;
            kl[j] = (LO && ok) ? *(const uint4 *)(p.kl + off) : z4;
            qlv[j] = (LO && ok) ? *(const uint4 *)(p.ql + off) : z4;
        }
    }
    // the gates of value head jv < 4 by wave jv, while the rows arrive (lane =
    // token; masked tokens get beta = 0 and g = 0): beta, the cumulative
    // log-decay gam and e^gam, e^(gam_C - gam), written to LDS in its phase 3
    double g_gam = 0.0;
    float g_beta = 0.f, g_eg = 0.f, g_egc = 0.f;
    auto gates = [&](int vh, double &gam, float &bt, float &eg, float &egc) {
        double beta = 0.0, glog = 0.0;
        if (lane < nvalid) {
            const size_t e = ((size_t)b * p.T + t0 + lane) * p.nv + vh;
            beta = 1.0 / (1.0 + exp(-(double)p.b[e]));
            glog = -exp((double)p.A_log[vh]) * softplus_d((double)p.a[e] + (double)p.dt_bias[vh]);
        }
        double sc = glog;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(sc, off, 64);
            if (lane >= off) sc += o;
        }
        const double sC = __shfl(sc, 63, 64);
        gam = sc;
        bt = (float)beta;
        eg = (float)exp(sc);
        egc = (float)exp(sC - sc);
    };
    if (wave < nr) gates(qh * nr + wave, g_gam, g_beta, g_eg, g_egc);
    if (XIN) {
        // q and k from x as the glue's operations (vx27_qfwd.c:118-131): the
        // conv + SiLU, thread (tokens 16 wave .. +15, channels lane and
        // lane + 64) out of the LDS windows (row r: token t0 - 3 + r) ...
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's window loads
        __syncthreads();
        float yq[2][16], yk[2][16];
        const float *wq = (const float *)(smem + TN_R0), *wk = (const float *)(smem + TN_R2);
#pragma unroll
        for (int hc = 0; hc < 2; hc++) {
            const int ch = lane + 64 * hc;
            float cq[3], ck[3];
#pragma unroll
            for (int t = 0; t < 3; t++) {
                cq[t] = wq[(16 * wave + t) * HD + ch];
                ck[t] = wk[(16 * wave + t) * HD + ch];
            }
            if (t0 == 0 && wave == 0) {   // tokens -3 .. -1: the conv state (oldest first)
                const size_t chq = (size_t)qh * HD + ch, chk = chq + (size_t)p.nqk * HD;
#pragma unroll
                for (int t = 0; t < 3; t++) {
                    cq[t] = p.conv_state[((size_t)b * p.C + chq) * 3 + t];
                    ck[t] = p.conv_state[((size_t)b * p.C + chk) * 3 + t];
                }
            }
#pragma unroll
            for (int k = 0; k < 16; k++) {
                yq[hc][k] = conv_step_fast(cq, xq[hc], wq[(16 * wave + 3 + k) * HD + ch]);
                yk[hc][k] = conv_step_fast(ck, xk[hc], wk[(16 * wave + 3 + k) * HD + ch]);
            }
        }
        __syncthreads();   // the windows are read out: the fp32 rows take R0-R1 and R2-R3
        float *fq = (float *)(smem + TN_R0), *fk = (float *)(smem + TN_R2);
#pragma unroll
        for (int hc = 0; hc < 2; hc++)
#pragma unroll
            for (int k = 0; k < 16; k++) {
                fq[(16 * wave + k) * HD + lane + 64 * hc] = yq[hc][k];
                fk[(16 * wave + k) * HD + lane + 64 * hc] = yk[hc][k];
            }
        __syncthreads();
        // ... then per row (thread: rows tid/16 + 16 j, dims 8 seg) the
        // (1+w) RMS pre-norm and l2norm with q/sqrt(128) (double sums over
        // the row's 16 lanes), rows past the prompt zero, and the bf16 hi/lo
        // split of the values
        float nw[8];
        *(float4 *)&nw[0] = *(const float4 *)&M_t[8 * seg];
        *(float4 *)&nw[4] = *(const float4 *)&M_t[8 * seg + 4];
        const float qs = 1.0f / sqrtf((float)HD);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = (tid >> 4) + 16 * j;
            float vq[8], vk[8];
            *(float4 *)&vq[0] = *(const float4 *)&fq[r * HD + 8 * seg];
            *(float4 *)&vq[4] = *(const float4 *)&fq[r * HD + 8 * seg + 4];
            *(float4 *)&vk[0] = *(const float4 *)&fk[r * HD + 8 * seg];
            *(float4 *)&vk[4] = *(const float4 *)&fk[r * HD + 8 * seg + 4];
            if (p.flags & VX27_DN_PRE_RMS) {   // rmsn(x)*(1+w), vx27_qfwd.c:32-39,123
                double ssq = 0.0, ssk = 0.0;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    ssq = ssq + (double)vq[e] * (double)vq[e];
                    ssk = ssk + (double)vk[e] * (double)vk[e];
                }
                ssq = row16_sum_dpp(ssq);
                ssk = row16_sum_dpp(ssk);
                const float iq = 1.0f / sqrtf((float)(ssq / HD) + 1e-6f), ik = 1.0f / sqrtf((float)(ssk / HD) + 1e-6f);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    vq[e] = (vq[e] * iq) * (nw[e] + 1.0f);
                    vk[e] = (vk[e] * ik) * (nw[e] + 1.0f);
                }
            }
            if (p.flags & VX27_DN_PRE_L2) {    // l2norm + q/sqrt(hd), vx27_qfwd.c:124-130
                double ssq = 0.0, ssk = 0.0;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    ssq = ssq + (double)vq[e] * (double)vq[e];
                    ssk = ssk + (double)vk[e] * (double)vk[e];
                }
                ssq = row16_sum_dpp(ssq);
                ssk = row16_sum_dpp(ssk);
                const float iq = 1.0f / sqrtf((float)ssq + 1e-6f), ik = 1.0f / sqrtf((float)ssk + 1e-6f);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    vq[e] = vq[e] * iq;
                    vk[e] = vk[e] * ik;
                    vq[e] = vq[e] * qs;
                }
            }
            const bool ok = r < nvalid;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                vq[e] = ok ? vq[e] : 0.0f;
                vk[e] = ok ? vk[e] : 0.0f;
            }
            split8(vq, qhv[j], qlv[j]);
            split8(vk, kh[j], kl[j]);
        }
        __syncthreads();   // the fp32 rows are read out
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = (tid >> 4) + 16 * j;
        if (XIN) {   // lo rows beside the hi rows: q in R2, k in R3 (phase 2's lo operands)
            *(uint4 *)&((uint16_t *)(smem + TN_R2))[r * RP + 8 * seg] = qlv[j];
            *(uint4 *)&((uint16_t *)(smem + TN_R3))[r * RP + 8 * seg] = kl[j];
        }
        *(uint4 *)&k_rows[r * RP + 8 * seg] = kh[j];
        *(uint4 *)&q_rows[r * RP + 8 * seg] = qhv[j];
        double sk = 0.0, sq = 0.0;   // of the values hi + lo (exact in double)
        const uint32_t kw[4] = {kh[j].x, kh[j].y, kh[j].z, kh[j].w}, klw[4] = {kl[j].x, kl[j].y, kl[j].z, kl[j].w};
        const uint32_t qw[4] = {qhv[j].x, qhv[j].y, qhv[j].z, qhv[j].w},
                       qlw[4] = {qlv[j].x, qlv[j].y, qlv[j].z, qlv[j].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const double k0 = (double)vx_bf16_to_f32((uint16_t)kw[e]) + (double)vx_bf16_to_f32((uint16_t)klw[e]);
            const double k1 = (double)vx_bf16_to_f32((uint16_t)(kw[e] >> 16)) +
                              (double)vx_bf16_to_f32((uint16_t)(klw[e] >> 16));
            const double q0 = (double)vx_bf16_to_f32((uint16_t)qw[e]) + (double)vx_bf16_to_f32((uint16_t)qlw[e]);
            const double q1 = (double)vx_bf16_to_f32((uint16_t)(qw[e] >> 16)) +
                              (double)vx_bf16_to_f32((uint16_t)(qlw[e] >> 16));
            sk = sk + k0 * k0;
            sk = sk + k1 * k1;
            sq = sq + q0 * q0;
            sq = sq + q1 * q1;
        }
        sk = row16_sum_dpp(sk);
        sq = row16_sum_dpp(sq);
        if (seg == 0) {   // l2norm, vx27_deltanet.c:51-56
            ik_s[r] = 1.0f / sqrtf((float)sk + 1e-6f);
            iq_s[r] = 1.0f / sqrtf((float)sq + 1e-6f);
        }
    }
    __syncthreads();
    // the lo operands of the Gram products (global memory, issued now so that
    // they arrive during the transposition): this wave's q and k rows (A) and
    // the chunk's k rows (B) for every k-step; rows past the prompt give zeros
    const int rowA = wave * 16 + m;
    auto lo_row = [&](const uint16_t *base, int r, int d0) -> uint4 {
        const size_t row = ((size_t)b * p.T + t0 + (r < nvalid ? r : 0)) * p.nqk + qh;
        const u32x4_t v = *(g_u32x4 *)(base + row * HD + d0);
        // masked by AND with an opaque mask: a select would let the compiler
        // move the load under a branch, with a wait at its end
        uint32_t mk = r < nvalid ? 0xffffffffu : 0u;
        __asm__("" : "+v"(mk));
        return make_uint4(v.x & mk, v.y & mk, v.z & mk, v.w & mk);
    };
    uint4 qal[4], kal[4], bkl[4][4];
    if (XIN) {   // from the lo rows in LDS (rows past the prompt are zero there)
        const uint16_t *qlr = (const uint16_t *)(smem + TN_R2), *klr = (const uint16_t *)(smem + TN_R3);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            qal[ks] = *(const uint4 *)&qlr[rowA * RP + 32 * ks + 8 * g];
            kal[ks] = *(const uint4 *)&klr[rowA * RP + 32 * ks + 8 * g];
#pragma unroll
            for (int nb = 0; nb < 4; nb++) bkl[nb][ks] = *(const uint4 *)&klr[(nb * 16 + m) * RP + 32 * ks + 8 * g];
        }
        __syncthreads();   // the lo rows are read out: R2 takes K^T hi
    } else if (LO) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            qal[ks] = lo_row(p.ql, rowA, 32 * ks + 8 * g);
            kal[ks] = lo_row(p.kl, rowA, 32 * ks + 8 * g);
#pragma unroll
            for (int nb = 0; nb < 4; nb++) bkl[nb][ks] = lo_row(p.kl, nb * 16 + m, 32 * ks + 8 * g);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    tr_rows(k_rows, kT_h, tid);   // K^T hi by all waves
    __syncthreads();

    // ---- phase 2: K K^T and Q K^T (hi*hi + lo*hi + hi*lo)
    floatx4_t acck[4], accq[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
        acck[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
        accq[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const int d0 = 32 * ks + 8 * g;
        const bf16x8_t qa = as_bf16x8(*(const uint4 *)&q_rows[rowA * RP + d0]);
        const bf16x8_t ka = as_bf16x8(*(const uint4 *)&k_rows[rowA * RP + d0]);
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
            const bf16x8_t bk = as_bf16x8(*(const uint4 *)&k_rows[(nb * 16 + m) * RP + d0]);
            MFMA1(acck[nb], ka, bk);
            MFMA1(accq[nb], qa, bk);
            if (LO) {
                const bf16x8_t bklo = as_bf16x8(bkl[nb][ks]);
                MFMA1(acck[nb], as_bf16x8(kal[ks]), bk);
                MFMA1(acck[nb], ka, bklo);
                MFMA1(accq[nb], as_bf16x8(qal[ks]), bk);
                MFMA1(accq[nb], qa, bklo);
            }
        }
    }
    // the K record: K^T operand tiles (rows = key dims in 8 blocks, k =
    // tokens in 2 steps) and the K and Q operand tiles (rows = tokens, k =
    // one 32-dim block), four of each a wave
    char *kr = p.krec + (((size_t)b * p.nqk + qh) * p.NC + c) * p.krec_bytes;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int tile = wave * 4 + j, rb = tile >> 1, ks = tile & 1;
        const int tr = tile >> 2, db = tile & 3;
        const size_t o = ((size_t)tile * 64 + lane) * 16;
        *(uint4 *)(kr + K_KT + o) = *(const uint4 *)&kT_h[(rb * 16 + m) * TP + 32 * ks + 8 * g];
        *(uint4 *)(kr + K_KA + o) = *(const uint4 *)&k_rows[(tr * 16 + m) * RP + 32 * db + 8 * g];
        *(uint4 *)(kr + K_QA + o) = *(const uint4 *)&q_rows[(tr * 16 + m) * RP + 32 * db + 8 * g];
    }
    __syncthreads();   // the rows and K^T hi are read out
    if (LO) {          // the lo parts: k lo rows through R1 (K^T lo transposed into R0), then q lo rows
#pragma unroll
        for (int j = 0; j < 4; j++) *(uint4 *)&k_rows[((tid >> 4) + 16 * j) * RP + 8 * seg] = kl[j];
        __syncthreads();
        tr_rows(k_rows, kT_l, tid);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int tile = wave * 4 + j, tr = tile >> 2, db = tile & 3;
            *(uint4 *)(kr + K_LO + K_KA + ((size_t)tile * 64 + lane) * 16) =
                *(const uint4 *)&k_rows[(tr * 16 + m) * RP + 32 * db + 8 * g];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int tile = wave * 4 + j, rb = tile >> 1, ks = tile & 1;
            *(uint4 *)(kr + K_LO + K_KT + ((size_t)tile * 64 + lane) * 16) =
                *(const uint4 *)&kT_l[(rb * 16 + m) * TP + 32 * ks + 8 * g];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) *(uint4 *)&k_rows[((tid >> 4) + 16 * j) * RP + 8 * seg] = qlv[j];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int tile = wave * 4 + j, tr = tile >> 2, db = tile & 3;
            *(uint4 *)(kr + K_LO + K_QA + ((size_t)tile * 64 + lane) * 16) =
                *(const uint4 *)&k_rows[(tr * 16 + m) * RP + 32 * db + 8 * g];
        }
        __syncthreads();   // R0 and R1 are free
    }

    const float qscale = 1.0f / sqrtf((float)HD);
    // XIN: the x window of one value head's v channels (tokens t0-3 ..
    // t0+64, clamped to the prompt; 64 channels, 256-byte rows) streamed
    // into LDS region `lds` by direct loads, 4 rows a wave instruction, while
    // the phases before phase 5 run (waited for before phase 5's conv)
    auto x_window = [&](int vh, int half, uint32_t lds) {
        const float *xb = p.x + (size_t)b * p.T * p.C + (size_t)2 * p.nqk * HD + (size_t)vh * HD + 64 * half;
        for (int i = wave; i < 17; i += 4) {
            const int row0 = min(max(t0 - 3 + 4 * i, 0), p.T - 1);
            const int row = min(max(t0 - 3 + 4 * i + (lane >> 4), 0), p.T - 1);
            const float *base = vx_uniform_ptr(xb + (size_t)row0 * p.C);
            vx_dma16(base, (uint32_t)(((row - row0) * p.C + 4 * (lane & 15)) * 4), lds + 1024 * i);
        }
    };
    for (int jv = 0; jv < nr; jv++) {
        const int vh = qh * nr + jv;
        if (XIN) x_window(vh, 0, vx_lds_addr(smem + TN_R3));
        // ---- phase 3: the gates to LDS (computed in phase 1 by wave jv for
        // jv < 4, else here by wave 0)
        if (jv < 4 ? wave == jv : wave == 0) {
            if (jv >= 4) gates(vh, g_gam, g_beta, g_eg, g_egc);
            gam_s[lane] = g_gam;
            beta_s[lane] = g_beta;
            eg_s[lane] = g_eg;
            egc_s[lane] = g_egc;
        }
        __syncthreads();
        char *rec = p.rec + (((size_t)b * p.nv + vh) * p.NC + c) * TREC;
        if (wave == 1) {   // the walk's per-token scales
            float *sc = (float *)(rec + T_SC);
            sc[lane] = egc_s[lane] * ik_s[lane];
            sc[64 + lane] = eg_s[lane] * (iq_s[lane] * qscale);
            if (lane == 0) sc[128] = (float)exp(gam_s[CH - 1]);
        }
        // A (fp32) and P hi/lo staging: the per-token scalars of this lane's
        // rows s and columns r in one batch of LDS reads, then 16 elements
        // with no branch (the masked ones selected away)
        double gs[4], gr[4];
        float bs[4], iks[4], iqs[4], ikr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int s = wave * 16 + 4 * g + i, r = i * 16 + m;
            gs[i] = gam_s[s];
            bs[i] = beta_s[s];
            iks[i] = ik_s[s];
            iqs[i] = iq_s[s] * qscale;
            gr[i] = gam_s[r];
            ikr[i] = ik_s[r];
        }
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int s = wave * 16 + 4 * g + i, r = nb * 16 + m;
                const float e = expf((float)(gs[i] - gr[nb]));   // masked when r > s (may be inf there)
                const float ed = r <= s ? e : 0.0f;
                const float av = bs[i] * ed * ((iks[i] * ikr[nb]) * acck[nb][i]);
                A_s[s * AP + r] = r < s ? av : 0.0f;
                const float pv = ed * ((iqs[i] * ikr[nb]) * accq[nb][i]);
                const uint16_t ph = vx_f32_to_bf16(pv);
                P_h[s * TP + r] = ph;
                P_l[s * TP + r] = vx_f32_to_bf16(pv - vx_bf16_to_f32(ph));
            }
        }
        __syncthreads();
        // P operand tiles (row block wave, 2 k-steps) out of the staging
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const size_t o = ((size_t)(wave * 2 + ks) * 64 + lane) * 16;
            *(uint4 *)(rec + T_PH + o) = *(const uint4 *)&P_h[rowA * TP + 32 * ks + 8 * g];
            *(uint4 *)(rec + T_PL + o) = *(const uint4 *)&P_l[rowA * TP + 32 * ks + 8 * g];
        }
        // ---- phase 4: T = (I + A)^-1; the diagonal blocks, one lane per column
        // (with XIN waves 1 and 2, idle here, load the conv taps of the
        // head's 128 v channels, stored in the last level below)
        float w4[4];
        if (XIN && (wave == 1 || wave == 2))
            load_conv_w(p.conv_w, p.w_bf16, (size_t)2 * p.nqk * HD + (size_t)vh * HD + (tid - 64), w4);
        if (tid < 64) {
            const int bi = tid >> 4, cc = tid & 15, o = 16 * bi;
            float t[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float acc = r == cc ? 1.0f : 0.0f;
#pragma unroll
                for (int k = 0; k < r; k++) acc -= A_s[(o + r) * AP + o + k] * t[k];
                t[r] = acc;
            }
#pragma unroll
            for (int r = 0; r < 16; r++) T_s[(o + r) * 64 + o + cc] = t[r];
        }
        __syncthreads();   // (and the P staging in R2 is read out)
        if (XIN) x_window(vh, 1, vx_lds_addr(smem + TN_R2));
        float *Mw = M_t + (wave < 3 ? wave : 0) * 256;
#pragma unroll
        for (int lev = 1; lev < 4; lev++) {
            if (XIN && lev == 3 && (wave == 1 || wave == 2))   // (wave 0 alone uses its scratch, M_t[0, 256))
                *(float4 *)&M_t[256 + (tid - 64) * 4] = make_float4(w4[0], w4[1], w4[2], w4[3]);
            if (wave < 4 - lev) {
                const int j = wave, i = j + lev;
                floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
                for (int kb = j; kb < i; kb++) {
#pragma unroll
                    for (int k0 = 0; k0 < 16; k0 += 4) {
                        const float av = A_s[(16 * i + m) * AP + 16 * kb + k0 + g];
                        const float bv = T_s[(16 * kb + k0 + g) * 64 + 16 * j + m];
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
                    }
                }
#pragma unroll
                for (int ii = 0; ii < 4; ii++) Mw[(4 * g + ii) * 16 + m] = acc[ii];
                asm volatile("" ::: "memory");
                floatx4_t tacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k0 = 0; k0 < 16; k0 += 4) {
                    const float av = T_s[(16 * i + m) * 64 + 16 * i + k0 + g];
                    const float bv = Mw[(k0 + g) * 16 + m];
                    tacc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, tacc, 0, 0, 0);
                }
#pragma unroll
                for (int ii = 0; ii < 4; ii++) T_s[(16 * i + 4 * g + ii) * 64 + 16 * j + m] = -tacc[ii];
            }
            __syncthreads();
        }
        // ---- phase 5: T' = T diag(beta) of row block wave in registers (the
        // upper blocks of T hold stale bytes: selected away) and the -T''
        // tiles; V^T hi/lo: without XIN from the fp32 v rows (hi to R0, lo
        // to R3, thread (row tid/16 + 16 j, 8 columns)) transposed into R2
        // and R1; with XIN the causal conv + SiLU of the x window in LDS,
        // thread (tokens 16 wave .. +15, channels lane and lane + 64), written
        // transposed straight into R0 and R1 (vx27_qfwd.c:118-131)
        if (!XIN) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r = (tid >> 4) + 16 * j;
                const bool ok = r < nvalid;
                const size_t off = (((size_t)b * p.T + t0 + r) * p.nv + vh) * HD + 8 * seg;
                const float *vf = p.v + off;
                const float4 a0 = ok ? *(const float4 *)vf : make_float4(0.f, 0.f, 0.f, 0.f);
                const float4 a1 = ok ? *(const float4 *)(vf + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                const float f[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                uint4 h, l;
                split8(f, h, l);
                *(uint4 *)&vh_rows[r * RP + 8 * seg] = h;
                *(uint4 *)&vl_rows[r * RP + 8 * seg] = l;
            }
        }
        bf16x8_t tph[2], tpl[2];
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const int s = wave * 16 + m, r0 = 32 * ks + 8 * g;
            float tr[8], bt[8], eg[8], ik[8];
            *(float4 *)&tr[0] = *(const float4 *)&T_s[s * 64 + r0];
            *(float4 *)&tr[4] = *(const float4 *)&T_s[s * 64 + r0 + 4];
            *(float4 *)&bt[0] = *(const float4 *)&beta_s[r0];
            *(float4 *)&bt[4] = *(const float4 *)&beta_s[r0 + 4];
            *(float4 *)&eg[0] = *(const float4 *)&eg_s[r0];
            *(float4 *)&eg[4] = *(const float4 *)&eg_s[r0 + 4];
            *(float4 *)&ik[0] = *(const float4 *)&ik_s[r0];
            *(float4 *)&ik[4] = *(const float4 *)&ik_s[r0 + 4];
            float f[8], f2[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                f[e] = (r0 + e <= s ? tr[e] : 0.0f) * bt[e];
                f2[e] = -(f[e] * (eg[e] * ik[e]));
            }
            uint4 h, l;
            split8(f, h, l);
            tph[ks] = as_bf16x8(h);
            tpl[ks] = as_bf16x8(l);
            split8(f2, h, l);
            const size_t o = ((size_t)(wave * 2 + ks) * 64 + lane) * 16;
            *(uint4 *)(rec + T_TH + o) = h;
            *(uint4 *)(rec + T_TL + o) = l;
        }
        uint16_t *vTh = XIN ? (uint16_t *)(smem + TN_R0) : vT_h;
        if (XIN) {
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's window loads
            __syncthreads();   // every wave's window is in LDS, and T is read out
            const float *win[2] = {(const float *)(smem + TN_R3), (const float *)(smem + TN_R2)};
#pragma unroll
            for (int hc = 0; hc < 2; hc++) {
                const int ch = lane + 64 * hc;
                const float4 wv = *(const float4 *)&M_t[256 + ch * 4];
                const float w[4] = {wv.x, wv.y, wv.z, wv.w};
                const float *xw = win[hc] + lane;   // row r: token t0 - 3 + r
                float cs[3] = {xw[(16 * wave) * 64], xw[(16 * wave + 1) * 64], xw[(16 * wave + 2) * 64]};
                if (t0 == 0 && wave == 0) {   // tokens -3 .. -1: the conv state (oldest first)
                    const float *sp = p.conv_state + ((size_t)b * p.C + (size_t)2 * p.nqk * HD + (size_t)vh * HD + ch) * 3;
                    cs[0] = sp[0]; cs[1] = sp[1]; cs[2] = sp[2];
                }
                float f[16];
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    const float y = conv_step_fast(cs, w, xw[(16 * wave + 3 + k) * 64]);
                    f[k] = 16 * wave + k < nvalid ? y : 0.0f;
                }
                uint4 h0, l0, h1, l1;
                split8(f, h0, l0);
                split8(f + 8, h1, l1);
                *(uint4 *)&vTh[ch * TP + 16 * wave] = h0;
                *(uint4 *)&vTh[ch * TP + 16 * wave + 8] = h1;
                *(uint4 *)&vT_l[ch * TP + 16 * wave] = l0;
                *(uint4 *)&vT_l[ch * TP + 16 * wave + 8] = l1;
            }
            __syncthreads();
        } else {
            __syncthreads();   // the V rows are complete and T is read out
            tr_rows(vh_rows, vT_h, tid);
            tr_rows(vl_rows, vT_l, tid);
            __syncthreads();
        }
        // Ut = T' V, row block wave, as C-layout tiles per 16-column block
#pragma unroll
        for (int cb = 0; cb < 8; cb++) {
            floatx4_t u0 = {0.f, 0.f, 0.f, 0.f}, u1 = {0.f, 0.f, 0.f, 0.f};
            const int col = cb * 16 + m;
            {
                const bf16x8_t vb = as_bf16x8(*(const uint4 *)&vTh[col * TP + 8 * g]);
                MFMA1(u0, tph[0], vb);
                MFMA1(u0, tpl[0], vb);
                if (LO) MFMA1(u0, tph[0], as_bf16x8(*(const uint4 *)&vT_l[col * TP + 8 * g]));
            }
            if (w2) {
                const bf16x8_t vb = as_bf16x8(*(const uint4 *)&vTh[col * TP + 32 + 8 * g]);
                MFMA1(u1, tph[1], vb);
                MFMA1(u1, tpl[1], vb);
                if (LO) MFMA1(u1, tph[1], as_bf16x8(*(const uint4 *)&vT_l[col * TP + 32 + 8 * g]));
            }
            *(floatx4_t *)(rec + T_UT + ((size_t)(wave * 8 + cb) * 64 + lane) * 16) = u0 + u1;
        }
        __syncthreads();   // before the next value head rewrites the LDS
    }
}

struct ScanTArgs {
    int T, nqk, nv, NC, xcd_map;
    const uint16_t *q, *k;          // hi parts [B][T][nqk][128] bf16
    const uint16_t *ql, *kl;        // lo parts as rows (LO)
    const char *rec, *krec;
    int krec_bytes;
    float *S;                       // [B][nv][128][128]
    float *out;                     // [B][T][nv][128]
};

// dnp_scant: the walk over the chunks of one value head.  A workgroup owns
// NCB blocks of 16 state columns (columns are independent in every
// product), wave w the state rows 32w .. 32w+31 of each block.  Per chunk:
//   the wave's S rows become the MFMA operand of its 32 key dims by two
//   lane swaps (no LDS); partial K S and (Q S)^T over those dims for all 64
//   tokens go to LDS;
//   [barrier] U = Ut - T'' sum(K S) for the wave's tokens 16w .. 16w+15,
//   and skc U, to LDS (hi/lo); the wave's rows of sum (Q S)^T are read now;
//   [barrier] S = e^gam_C S + K^T (skc U) for the wave's rows, and
//   O^T = sq (Q S)^T + U^T P^T for its tokens, stored 16 bytes a lane.
// Each wave loads its operands straight into registers (K and Q from the
// inputs, the rest from the records); each group takes the next chunk's
// loads as soon as its last MFMA has read it.  T'' and P vanish above the
// diagonal, so waves 0 and 1 skip their second k-step of both.
typedef const __attribute__((address_space(1))) floatx4_t g_floatx4;
template <int NCB>
__global__ __launch_bounds__(256) void dnp_scant(ScanTArgs p) {
    constexpr bool LO = true;
    constexpr int NSL = NSLICE / NCB;
    constexpr int KR = CH + 4, QR = 20;   // padded rows of the partial sums (floats)
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool w2 = wave >= 2;
    const int b = blockIdx.y, bid = blockIdx.x;
    const int nr = p.nv / p.nqk;
    int vh, slice;
    if (p.xcd_map) {   // the value heads of a QK head, all their slices, on one XCD
        const int xcd = bid & 7, idx = bid >> 3, per = nr * NSL;
        const int qh = (idx / per) * 8 + xcd, rem = idx % per;
        vh = qh * nr + rem / NSL;
        slice = rem % NSL;
    } else {
        vh = bid / NSL;
        slice = bid % NSL;
    }
    const int qh = vh / nr;
    const int cb0 = slice * NCB;

    __shared__ __attribute__((aligned(16))) float KSp[4][NCB][16][KR];   // partial K S [wave][block][column][token]
    __shared__ __attribute__((aligned(16))) float QSp[4][NCB][CH][QR];   // partial (Q S)^T [wave][block][token][column]
    __shared__ __attribute__((aligned(16))) uint16_t U_h[NCB][16][CH + 8], U_l[NCB][16][CH + 8];
    __shared__ __attribute__((aligned(16))) uint16_t W_h[NCB][16][CH + 8], W_l[NCB][16][CH + 8];

    const char *rec0 = vx_uniform_ptr(p.rec + ((size_t)b * p.nv + vh) * p.NC * TREC);
    const char *krec0 = vx_uniform_ptr(p.krec + ((size_t)b * p.nqk + qh) * p.NC * p.krec_bytes);

    // operand registers of one chunk
    uint4 kA[4], qA[4], kAl[4], qAl[4];     // K, Q tiles: rows 16 rb + n, dims 32w + 8g .. (4 row blocks)
    uint4 tp[2][2], pp[2][2];               // -T'', P row block w [k-step][hi, lo]
    uint4 kt[2][2], ktl[2][2];              // K^T row blocks 2w, 2w+1 [rb][k-step], hi and lo
    floatx4_t ut[NCB], skc4;
    float sqv, gc;
    // Buffer loads: the head's records as one resource each, the chunk and
    // tile offsets in scalar registers, the lane's offset one VGPR, so an
    // operand load costs no vector instruction (the sizes are checked on
    // the host: below 2^31 bytes)
    const __amdgpu_buffer_rsrc_t Rr = __builtin_amdgcn_make_buffer_rsrc((void *)rec0, 0, (int)(p.NC * TREC), 0x00020000);
    const __amdgpu_buffer_rsrc_t Rk = __builtin_amdgcn_make_buffer_rsrc((void *)krec0, 0, p.NC * p.krec_bytes, 0x00020000);
    const int lo16 = lane * 16;
    auto ld_r = [&](int cc, int off) -> uint4 {   // a T-record tile
        const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(Rr, lo16, cc * (int)TREC + off, 0));
        return make_uint4(v.x, v.y, v.z, v.w);
    };
    auto ld_k = [&](int cc, int off) -> uint4 {   // a K-record tile
        const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(Rk, lo16, cc * p.krec_bytes + off, 0));
        return make_uint4(v.x, v.y, v.z, v.w);
    };
    auto ld_kq = [&](int cc) {
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            const int o = (rb * 4 + wave) * 1024;
            kA[rb] = ld_k(cc, (int)K_KA + o);
            qA[rb] = ld_k(cc, (int)K_QA + o);
            if (LO) {
                kAl[rb] = ld_k(cc, (int)(K_LO + K_KA) + o);
                qAl[rb] = ld_k(cc, (int)(K_LO + K_QA) + o);
            }
        }
    };
    auto ld_u = [&](int cc) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
            if (ks == 0 || w2) {
                tp[ks][0] = ld_r(cc, (int)T_TH + (wave * 2 + ks) * 1024);
                tp[ks][1] = ld_r(cc, (int)T_TL + (wave * 2 + ks) * 1024);
            }
#pragma unroll
        for (int cb = 0; cb < NCB; cb++)
            ut[cb] = __builtin_bit_cast(floatx4_t, ld_r(cc, (int)T_UT + (wave * 8 + cb0 + cb) * 1024));
        skc4 = __builtin_bit_cast(floatx4_t, __builtin_amdgcn_raw_buffer_load_b128(Rr, (16 * wave + 4 * g) * 4, cc * (int)TREC + (int)T_SC, 0));
    };
    auto ld_s = [&](int cc) {
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                kt[r][ks] = ld_k(cc, (int)K_KT + ((2 * wave + r) * 2 + ks) * 1024);
                if (LO) ktl[r][ks] = ld_k(cc, (int)(K_LO + K_KT) + ((2 * wave + r) * 2 + ks) * 1024);
            }
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
            if (ks == 0 || w2) {
                pp[ks][0] = ld_r(cc, (int)T_PH + (wave * 2 + ks) * 1024);
                pp[ks][1] = ld_r(cc, (int)T_PL + (wave * 2 + ks) * 1024);
            }
        sqv = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(Rr, (16 * wave + n) * 4, cc * (int)TREC + (int)T_SC + 256, 0));
        gc = *(g_float *)(rec0 + (size_t)cc * TREC + T_SC + 512);
    };
    // The state first, waited for here: the loop head joins this path and the
    // loop's back edge, and a load still pending on either path would make
    // every iteration wait there for the loads of the step before.
    float *Sg = p.S + ((size_t)b * p.nv + vh) * HD * HD;
    floatx4_t S[NCB][2];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                S[cb][r][i] = Sg[(size_t)((2 * wave + r) * 16 + 4 * g + i) * HD + (cb0 + cb) * 16 + n];
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    ld_kq(0);
    ld_u(0);
    ld_s(0);

    const floatx4_t z = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < p.NC; c++) {
        const int nx = min(c + 1, p.NC - 1);   // (the last chunk again after the end: never used)
        // the wave's S rows as the B operand of its 32 dims: lane (g, n)
        // takes dims 8g .. 8g+7 of column n from the two C tiles (rows 4g'+i
        // of lane group g') by a 32-lane and a 16-lane swap
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            float e[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const auto r1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(S[cb][0][i]),
                                                                 __float_as_uint(S[cb][1][i]), false, false);
                const auto r2 = __builtin_amdgcn_permlane16_swap(r1[0], r1[1], false, false);
                e[i] = __uint_as_float(r2[0]);
                e[4 + i] = __uint_as_float(r2[1]);
            }
            uint4 h, l;
            split8(e, h, l);
            const bf16x8_t sh = as_bf16x8(h), sl = as_bf16x8(l);
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                floatx4_t ks = z, qs = z;
                MFMA1(ks, as_bf16x8(kA[rb]), sh);
                MFMA1(qs, sh, as_bf16x8(qA[rb]));
                MFMA1(ks, as_bf16x8(kA[rb]), sl);
                MFMA1(qs, sl, as_bf16x8(qA[rb]));
                if (LO) {
                    MFMA1(ks, as_bf16x8(kAl[rb]), sh);
                    MFMA1(qs, sh, as_bf16x8(qAl[rb]));
                }
                *(floatx4_t *)&KSp[wave][cb][n][16 * rb + 4 * g] = ks;
                *(floatx4_t *)&QSp[wave][cb][16 * rb + n][4 * g] = qs;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        ld_kq(nx);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        // U = Ut - T'' K S of the wave's tokens; skc U; the wave's (Q S)^T
        floatx4_t qsum[NCB];
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            bf16x8_t xh[2], xl[2];
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
                if (ks == 0 || w2) {
                    float f[8];
                    floatx4_t a0 = *(const floatx4_t *)&KSp[0][cb][n][32 * ks + 8 * g];
                    floatx4_t a1 = *(const floatx4_t *)&KSp[0][cb][n][32 * ks + 8 * g + 4];
#pragma unroll
                    for (int w = 1; w < 4; w++) {
                        a0 += *(const floatx4_t *)&KSp[w][cb][n][32 * ks + 8 * g];
                        a1 += *(const floatx4_t *)&KSp[w][cb][n][32 * ks + 8 * g + 4];
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        f[i] = a0[i];
                        f[4 + i] = a1[i];
                    }
                    uint4 h, l;
                    split8(f, h, l);
                    xh[ks] = as_bf16x8(h);
                    xl[ks] = as_bf16x8(l);
                }
            floatx4_t u0 = ut[cb], u1 = z;
            MFMA3(u0, as_bf16x8(tp[0][0]), as_bf16x8(tp[0][1]), xh[0], xl[0]);
            if (w2) MFMA3(u1, as_bf16x8(tp[1][0]), as_bf16x8(tp[1][1]), xh[1], xl[1]);
            const floatx4_t U = u0 + u1;
            uint2 h, l;
            split4(U, h, l);
            *(uint2 *)&U_h[cb][n][16 * wave + 4 * g] = h;
            *(uint2 *)&U_l[cb][n][16 * wave + 4 * g] = l;
            split4(U * skc4, h, l);
            *(uint2 *)&W_h[cb][n][16 * wave + 4 * g] = h;
            *(uint2 *)&W_l[cb][n][16 * wave + 4 * g] = l;
            floatx4_t qq = *(const floatx4_t *)&QSp[0][cb][16 * wave + n][4 * g];
#pragma unroll
            for (int w = 1; w < 4; w++) qq += *(const floatx4_t *)&QSp[w][cb][16 * wave + n][4 * g];
            qsum[cb] = qq;
        }
        __builtin_amdgcn_sched_barrier(0);
        ld_u(nx);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        // S = e^gam_C S + K^T (skc U);  O^T = sq (Q S)^T + U^T P^T
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            bf16x8_t uh[2], ul[2], wh[2], wl[2];
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                uh[ks] = as_bf16x8(*(const uint4 *)&U_h[cb][n][32 * ks + 8 * g]);
                ul[ks] = as_bf16x8(*(const uint4 *)&U_l[cb][n][32 * ks + 8 * g]);
                wh[ks] = as_bf16x8(*(const uint4 *)&W_h[cb][n][32 * ks + 8 * g]);
                wl[ks] = as_bf16x8(*(const uint4 *)&W_l[cb][n][32 * ks + 8 * g]);
            }
#pragma unroll
            for (int r = 0; r < 2; r++) {
                floatx4_t sa = S[cb][r] * gc, sb = z;
                MFMA1(sa, as_bf16x8(kt[r][0]), wh[0]);
                MFMA1(sb, as_bf16x8(kt[r][1]), wh[1]);
                MFMA1(sa, as_bf16x8(kt[r][0]), wl[0]);
                MFMA1(sb, as_bf16x8(kt[r][1]), wl[1]);
                if (LO) {
                    MFMA1(sa, as_bf16x8(ktl[r][0]), wh[0]);
                    MFMA1(sb, as_bf16x8(ktl[r][1]), wh[1]);
                }
                S[cb][r] = sa + sb;
            }
            floatx4_t o0 = qsum[cb] * sqv, o1 = z;
            MFMA3(o0, uh[0], ul[0], as_bf16x8(pp[0][0]), as_bf16x8(pp[0][1]));
            if (w2) MFMA3(o1, uh[1], ul[1], as_bf16x8(pp[1][0]), as_bf16x8(pp[1][1]));
            const int tt = c * CH + 16 * wave + n;
            if (tt < p.T)
                *(floatx4_t *)(p.out + (((size_t)b * p.T + tt) * p.nv + vh) * HD + (cb0 + cb) * 16 + 4 * g) = o0 + o1;
        }
        __builtin_amdgcn_sched_barrier(0);
        ld_s(nx);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                Sg[(size_t)((2 * wave + r) * 16 + 4 * g + i) * HD + (cb0 + cb) * 16 + n] = S[cb][r][i];
}

// ---- split precision, full records (bf16 inputs without the glue) --------
// The form for inputs that are exact in bf16: the preparation writes every
// operand of the walk (-W, e^gam Q, Kt^T, P as hi/lo tiles, Ut), 144 KiB per
// (chunk, value head), and the walk has two LDS hand-offs per chunk (S, U).
// With q, k, v exact in bf16 these records stay in L2 across the head's
// column slices, and the walk's lighter LDS traffic makes it the faster one;
// the T-record form above wins once the glue's lo parts and 48 value heads
// make the records large.
// The default chunked form: every operand of the chunk products enters the
// MFMAs as a pair of bf16 values, hi = bf16(x) and lo = bf16(x - hi), and
// each product is hi*hi + lo*hi + hi*lo (the lo*lo term, ~2^-16 of the
// product, is dropped): about 16 significand bits per operand, so the
// chunked result stays within ~1e-5 of the fp32 recurrence instead of
// bf16's ~1e-2.  Inputs q, k, v come as hi/lo pairs too (lo = NULL: the
// inputs are exact in bf16).  The record holds each operand tile as a hi
// tile and a lo tile.
constexpr size_t X_NW = 0;                    // -W        hi, lo: 2 x [4][4][64][8] bf16
constexpr size_t X_QE = X_NW + 2 * 16384;     // e^gam qn  hi, lo
constexpr size_t X_KT = X_QE + 2 * 16384;     // Kt^T      hi, lo: 2 x [8][2][64][8]
constexpr size_t X_P = X_KT + 2 * 16384;      // P         hi, lo: 2 x [4][2][64][8]
constexpr size_t X_UT = X_P + 2 * 8192;       // Ut fp32 [4 rb][8 cs][64][4]
constexpr size_t X_GC = X_UT + 32768;         // e^gam_C
constexpr size_t XREC = X_GC + 256;

struct Prep3Args {
    int T, nqk, nv, NC;
    const uint16_t *q, *k, *v;          // hi parts [B][T][nqk|nqk|nv][128] bf16
    const uint16_t *ql, *kl;            // lo parts of q, k as rows, or NULL
    const uint16_t *klT, *vlT;          // lo parts of k, v transposed, [B][nqk|nv][128][Tp]
    int Tp;
    const float *a, *b;
    const float *A_log, *dt_bias;
    char *rec;                          // [B][nv][NC] records of XREC bytes
};


// LDS of dnp_prep3 (phases as dnp_prep's), 76.5 KiB, so two workgroups
// share a CU: four regions whose contents change with the phase.  The lo
// parts of split inputs never enter it: each is read from global memory in
// the layout its use needs (rows, or transposed).
constexpr int XN_QH = 0;                        // q rows -> P hi staging -> v rows -> T fp32
constexpr int XN_KH = XN_QH + CH * RP * 2;      // k rows -> P lo staging -> V^T -> -W hi staging
constexpr int XN_TH = XN_KH + HD * TP * 2;      // K^T -> -W lo staging
constexpr int XN_AS = XN_TH + HD * TP * 2;      // A fp32
constexpr int XN_MT = XN_AS + CH * AP * 4;
constexpr int XN_GAM = XN_MT + 3 * 256 * 4;
constexpr int XN_SC = XN_GAM + CH * 8;
constexpr int XN_TOTAL = XN_SC + 5 * CH * 4;
static_assert(CH * 64 * 4 <= CH * RP * 2 && CH * TP * 2 <= HD * TP * 2 && CH * RP * 2 <= HD * TP * 2,
              "T, P and -W staging fit their regions");
static_assert(2 * XN_TOTAL <= 160 * 1024, "two workgroups per CU");


// LO: the inputs come with lo parts (the glue's fp32 values as bf16 pairs),
// read from global memory where a product or an operand tile takes them;
// without them they are zero and never read.
template <bool LO>
__global__ __launch_bounds__(256) void dnp_prep3(Prep3Args p) {
    const int c = blockIdx.x, vh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, m = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qh = vh * p.nqk / p.nv;
    const int t0 = c * CH;
    const int nvalid = min(CH, p.T - t0);
    constexpr bool has_lo = LO;

    __shared__ __attribute__((aligned(16))) char smem[XN_TOTAL];
    uint16_t *q_rows = (uint16_t *)(smem + XN_QH);
    uint16_t *P_h = (uint16_t *)(smem + XN_QH), *P_l = (uint16_t *)(smem + XN_KH);    // [64][TP]
    float *T_s = (float *)(smem + XN_QH);                                             // [64][64]
    uint16_t *k_rows = (uint16_t *)(smem + XN_KH);
    uint16_t *V_h = (uint16_t *)(smem + XN_KH);                                       // [128][TP]
    uint16_t *W_h = (uint16_t *)(smem + XN_KH), *W_l = (uint16_t *)(smem + XN_TH);    // [64][RP]
    uint16_t *K_h = (uint16_t *)(smem + XN_TH);                                       // [128][TP]
    float *A_s = (float *)(smem + XN_AS);
    float *M_t = (float *)(smem + XN_MT);
    double *gam_s = (double *)(smem + XN_GAM);
    float *beta_s = (float *)(smem + XN_SC), *eg_s = beta_s + CH, *egc_s = eg_s + CH;
    float *iq_s = egc_s + CH, *ik_s = iq_s + CH;
    // lo parts from global memory: 8 dims d0.. of row r of the chunk (q or
    // k; rows past the prompt read row 0 and give zeros), and 8 tokens t..
    // of dim d of the transposed k or v (zero past the prompt)
    const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
    auto lo_row = [&](const uint16_t *base, int r, int d0) -> uint4 {
        const size_t row = ((size_t)b * p.T + t0 + (r < nvalid ? r : 0)) * p.nqk + qh;
        const u32x4_t v = *(g_u32x4 *)(base + row * HD + d0);
        // masked by AND with an opaque mask: a select would let the compiler
        // move the load under a branch, with a wait at its end
        uint32_t mk = r < nvalid ? 0xffffffffu : 0u;
        __asm__("" : "+v"(mk));
        return make_uint4(v.x & mk, v.y & mk, v.z & mk, v.w & mk);
    };
    const uint16_t *klT = LO ? p.klT + ((size_t)b * p.nqk + qh) * HD * p.Tp + t0 : nullptr;
    const uint16_t *vlT = LO ? p.vlT + ((size_t)b * p.nv + vh) * HD * p.Tp + t0 : nullptr;
    auto lo_tr = [&](const uint16_t *base, int d, int t) -> uint4 {
        const u32x4_t v = *(g_u32x4 *)(base + (size_t)d * p.Tp + t);
        return make_uint4(v.x, v.y, v.z, v.w);
    };

    // ---- phase 1: gates (wave 0); k, q, v rows (waves 1, 2, 3), hi and lo
    if (wave == 0) {
        double beta = 0.0, glog = 0.0;
        if (lane < nvalid) {
            const size_t e = ((size_t)b * p.T + t0 + lane) * p.nv + vh;
            beta = 1.0 / (1.0 + exp(-(double)p.b[e]));
            glog = -exp((double)p.A_log[vh]) * softplus_d((double)p.a[e] + (double)p.dt_bias[vh]);
        }
        double sc = glog;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(sc, off, 64);
            if (lane >= off) sc += o;
        }
        const double sC = __shfl(sc, 63, 64);
        gam_s[lane] = sc;
        beta_s[lane] = (float)beta;
        eg_s[lane] = (float)exp(sc);
        egc_s[lane] = (float)exp(sC - sc);
    }
    uint4 raw[16], rawl[16];
    if (wave >= 1) {
        const size_t row = wave == 3 ? (((size_t)b * p.T + t0 + lane) * p.nv + vh) * HD
                                     : (((size_t)b * p.T + t0 + lane) * p.nqk + qh) * HD;
        const uint16_t *src = wave == 1 ? p.k : wave == 2 ? p.q : p.v;
        const uint16_t *srl = wave == 1 ? p.kl : p.ql;   // (v's lo part is read transposed, in phase 5)
#pragma unroll
        for (int j = 0; j < 16; j++) {
            raw[j] = lane < nvalid ? *(const uint4 *)(src + row + 8 * j) : make_uint4(0u, 0u, 0u, 0u);
            rawl[j] = (has_lo && wave < 3 && lane < nvalid) ? *(const uint4 *)(srl + row + 8 * j)
                                                            : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    if (wave == 1 || wave == 2) {
        double ss = 0.0;   // of the value hi + lo (exact in double)
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
            const uint32_t l4[4] = {rawl[j].x, rawl[j].y, rawl[j].z, rawl[j].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const double x0 = (double)vx_bf16_to_f32((uint16_t)w4[e]) + (double)vx_bf16_to_f32((uint16_t)l4[e]);
                const double x1 = (double)vx_bf16_to_f32((uint16_t)(w4[e] >> 16)) +
                                  (double)vx_bf16_to_f32((uint16_t)(l4[e] >> 16));
                ss = ss + x0 * x0;
                ss = ss + x1 * x1;
            }
        }
        const float inv = 1.0f / sqrtf((float)ss + 1e-6f);   // l2norm, vx27_deltanet.c:51-56
        uint16_t *rows = wave == 1 ? k_rows : q_rows;
#pragma unroll
        for (int j = 0; j < 16; j++) *(uint4 *)&rows[lane * RP + 8 * j] = raw[j];
        if (wave == 1) ik_s[lane] = inv;
        else iq_s[lane] = inv;
    }
    __syncthreads();
    // the lo operands of phase 2 (split inputs), all issued now so that they
    // arrive during the transposition: this wave's q and k rows (A) and the
    // chunk's k rows (B) for every k-step, and its Kt^T tiles' lo parts
    const int rowA = wave * 16 + m;
    uint4 qal[4], kal[4], bkl[4][4], krl[4];
    if (LO) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            qal[ks] = lo_row(p.ql, rowA, 32 * ks + 8 * g);
            kal[ks] = lo_row(p.kl, rowA, 32 * ks + 8 * g);
#pragma unroll
            for (int nb = 0; nb < 4; nb++) bkl[nb][ks] = lo_row(p.kl, nb * 16 + m, 32 * ks + 8 * g);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int tile = wave * 4 + j;
            krl[j] = lo_tr(klT, (tile >> 1) * 16 + m, 32 * (tile & 1) + 8 * g);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    tr_rows(k_rows, K_h, tid);   // K^T by all waves
    __syncthreads();

    char *rec = p.rec + (((size_t)b * p.nv + vh) * p.NC + c) * XREC;
    const double gamC = gam_s[CH - 1];
    if (tid == 0) *(float *)(rec + X_GC) = (float)exp(gamC);
    const float qscale = 1.0f / sqrtf((float)HD);

    // ---- phase 2: K K^T and Q K^T (hi*hi + lo*hi + hi*lo); e^gam qn tiles
    floatx4_t acck[4], accq[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
        acck[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
        accq[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    }
    const float qeA = eg_s[rowA] * (iq_s[rowA] * qscale);
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const int d0 = 32 * ks + 8 * g;
        const uint4 qa = *(const uint4 *)&q_rows[rowA * RP + d0], qlo = LO ? qal[ks] : z4;
        const uint4 ka = *(const uint4 *)&k_rows[rowA * RP + d0], klo = LO ? kal[ks] : z4;
        {   // e^gam qn tile (row block wave, k-step ks), hi and lo
            const uint16_t *qs = (const uint16_t *)&qa, *qsl = (const uint16_t *)&qlo;
            float f[8];
#pragma unroll
            for (int e = 0; e < 8; e++) f[e] = qeA * (vx_bf16_to_f32(qs[e]) + vx_bf16_to_f32(qsl[e]));
            uint4 h, l;
            split8(f, h, l);
            *(uint4 *)(rec + X_QE + ((size_t)(wave * 4 + ks) * 64 + lane) * 16) = h;
            *(uint4 *)(rec + X_QE + 16384 + ((size_t)(wave * 4 + ks) * 64 + lane) * 16) = l;
        }
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
            const bf16x8_t bk = as_bf16x8(*(const uint4 *)&k_rows[(nb * 16 + m) * RP + d0]);
            acck[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka), bk, acck[nb], 0, 0, 0);
            accq[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qa), bk, accq[nb], 0, 0, 0);
            if (has_lo) {
                const bf16x8_t bklo = as_bf16x8(bkl[nb][ks]);
                acck[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(klo), bk, acck[nb], 0, 0, 0);
                acck[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka), bklo, acck[nb], 0, 0, 0);
                accq[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qlo), bk, accq[nb], 0, 0, 0);
                accq[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qa), bklo, accq[nb], 0, 0, 0);
            }
        }
    }
    // Kt^T tiles (hi, lo): rows = key dims (8 blocks), k = tokens (2 steps); 4 per wave
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int tile = wave * 4 + j, rb = tile >> 1, ks = tile & 1;
        const int i = rb * 16 + m, tb = 32 * ks + 8 * g;
        const uint4 kr = *(const uint4 *)&K_h[i * TP + tb];
        const uint4 krlo = LO ? krl[j] : z4;
        const uint16_t *kv = (const uint16_t *)&kr, *kvl = (const uint16_t *)&krlo;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            f[e] = (egc_s[tb + e] * ik_s[tb + e]) * (vx_bf16_to_f32(kv[e]) + vx_bf16_to_f32(kvl[e]));
        uint4 h, l;
        split8(f, h, l);
        *(uint4 *)(rec + X_KT + ((size_t)tile * 64 + lane) * 16) = h;
        *(uint4 *)(rec + X_KT + 16384 + ((size_t)tile * 64 + lane) * 16) = l;
    }
    __syncthreads();   // q and k rows are no longer read

    // ---- phase 3: A (fp32), P hi/lo staging.  The per-token scalars of
    // this lane's rows s and columns r come first, in one batch of LDS
    // reads; the 16 elements then need no branch (the masked ones are
    // selected away), so no LDS round trip waits inside the loop.
    double gs[4], gr[4];
    float bs[4], iks[4], iqs[4], ikr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int s = wave * 16 + 4 * g + i, r = i * 16 + m;
        gs[i] = gam_s[s];
        bs[i] = beta_s[s];
        iks[i] = ik_s[s];
        iqs[i] = iq_s[s] * qscale;
        gr[i] = gam_s[r];
        ikr[i] = ik_s[r];
    }
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int s = wave * 16 + 4 * g + i, r = nb * 16 + m;
            const float e = expf((float)(gs[i] - gr[nb]));   // masked when r > s (may be inf there)
            const float ed = r <= s ? e : 0.0f;
            const float av = bs[i] * ed * ((iks[i] * ikr[nb]) * acck[nb][i]);
            A_s[s * AP + r] = r < s ? av : 0.0f;
            const float pv = ed * ((iqs[i] * ikr[nb]) * accq[nb][i]);
            const uint16_t ph = vx_f32_to_bf16(pv);
            P_h[s * TP + r] = ph;
            P_l[s * TP + r] = vx_f32_to_bf16(pv - vx_bf16_to_f32(ph));
        }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const size_t o = ((size_t)(wave * 2 + ks) * 64 + lane) * 16;
        *(uint4 *)(rec + X_P + o) = *(const uint4 *)&P_h[rowA * TP + 32 * ks + 8 * g];
        *(uint4 *)(rec + X_P + 8192 + o) = *(const uint4 *)&P_l[rowA * TP + 32 * ks + 8 * g];
    }
    __syncthreads();   // P staging is read out: the q region takes the v rows, then T
    if (wave == 3) {
#pragma unroll
        for (int j = 0; j < 16; j++) *(uint4 *)&q_rows[lane * RP + 8 * j] = raw[j];
    }
    __syncthreads();
    tr_rows(q_rows, V_h, tid);   // V^T by all waves
    __syncthreads();

    // the lo parts of phase 5's B operands (split inputs): V^T's now, to
    // arrive during the inversion; K^T's at the start of phase 5
    uint4 vlo[8][2], klo5[8][2];
    if (LO) {
#pragma unroll
        for (int cb = 0; cb < 8; cb++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++) vlo[cb][ks] = lo_tr(vlT, cb * 16 + m, 32 * ks + 8 * g);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- phase 4: T = (I + A)^-1 (as dnp_prep)
    if (tid < 64) {
        const int bi = tid >> 4, cc = tid & 15, o = 16 * bi;
        float t[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float acc = r == cc ? 1.0f : 0.0f;
#pragma unroll
            for (int k = 0; k < r; k++) acc -= A_s[(o + r) * AP + o + k] * t[k];
            t[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) T_s[(o + r) * 64 + o + cc] = t[r];
    }
    __syncthreads();
    float *Mw = M_t + (wave < 3 ? wave : 0) * 256;
#pragma unroll
    for (int lev = 1; lev < 4; lev++) {
        if (wave < 4 - lev) {
            const int j = wave, i = j + lev;
            floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
            for (int kb = j; kb < i; kb++) {
#pragma unroll
                for (int k0 = 0; k0 < 16; k0 += 4) {
                    const float av = A_s[(16 * i + m) * AP + 16 * kb + k0 + g];
                    const float bv = T_s[(16 * kb + k0 + g) * 64 + 16 * j + m];
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
                }
            }
#pragma unroll
            for (int ii = 0; ii < 4; ii++) Mw[(4 * g + ii) * 16 + m] = acc[ii];
            asm volatile("" ::: "memory");
            floatx4_t tacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k0 = 0; k0 < 16; k0 += 4) {
                const float av = T_s[(16 * i + m) * 64 + 16 * i + k0 + g];
                const float bv = Mw[(k0 + g) * 16 + m];
                tacc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, tacc, 0, 0, 0);
            }
#pragma unroll
            for (int ii = 0; ii < 4; ii++) T_s[(16 * i + 4 * g + ii) * 64 + 16 * j + m] = -tacc[ii];
        }
        __syncthreads();
    }

    // ---- phase 5: [Ut | W] rows of block `wave` = T_V V | T_K K, all pairs
    bf16x8_t tv[2][2], tk[2][2];   // [k-step][hi, lo]
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        // row s of T and the scalars of tokens r0..r0+7 as vector LDS reads
        // (the upper blocks of T hold stale bytes: selected away, never used)
        const int s = wave * 16 + m, r0 = 32 * ks + 8 * g;
        float tr[8], bt[8], ev[8], kv[8];
        *(float4 *)&tr[0] = *(const float4 *)&T_s[s * 64 + r0];
        *(float4 *)&tr[4] = *(const float4 *)&T_s[s * 64 + r0 + 4];
        *(float4 *)&bt[0] = *(const float4 *)&beta_s[r0];
        *(float4 *)&bt[4] = *(const float4 *)&beta_s[r0 + 4];
        *(float4 *)&ev[0] = *(const float4 *)&eg_s[r0];
        *(float4 *)&ev[4] = *(const float4 *)&eg_s[r0 + 4];
        *(float4 *)&kv[0] = *(const float4 *)&ik_s[r0];
        *(float4 *)&kv[4] = *(const float4 *)&ik_s[r0 + 4];
        float fv[8], fk[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float tsr = r0 + e <= s ? tr[e] : 0.0f;
            fv[e] = tsr * bt[e];
            fk[e] = tsr * ((bt[e] * ev[e]) * kv[e]);
        }
        uint4 hv, lv, hk, lk;
        split8(fv, hv, lv);
        split8(fk, hk, lk);
        tv[ks][0] = as_bf16x8(hv);
        tv[ks][1] = as_bf16x8(lv);
        tk[ks][0] = as_bf16x8(hk);
        tk[ks][1] = as_bf16x8(lk);
    }
    if (LO) {
#pragma unroll
        for (int cb = 0; cb < 8; cb++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++) klo5[cb][ks] = lo_tr(klT, cb * 16 + m, 32 * ks + 8 * g);
    }
    __builtin_amdgcn_sched_barrier(0);
    floatx4_t wacc[8];
    float *ut = (float *)(rec + X_UT);
#pragma unroll
    for (int cb = 0; cb < 16; cb++) {
        const bool isv = cb < 8;
        const uint16_t *src = isv ? V_h : K_h;
        const int col = (cb & 7) * 16 + m;
        floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const bf16x8_t bop = as_bf16x8(*(const uint4 *)&src[col * TP + 32 * ks + 8 * g]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(isv ? tv[ks][0] : tk[ks][0], bop, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(isv ? tv[ks][1] : tk[ks][1], bop, acc, 0, 0, 0);
            if (has_lo) {
                const bf16x8_t bol = as_bf16x8(isv ? vlo[cb & 7][ks] : klo5[cb & 7][ks]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(isv ? tv[ks][0] : tk[ks][0], bol, acc, 0, 0, 0);
            }
        }
        if (isv) {
            *(floatx4_t *)&ut[(((size_t)wave * 8 + cb) * 64 + lane) * 4] = acc;
        } else {
            wacc[cb - 8] = acc;
        }
    }
    __syncthreads();   // every read of V^T is done: the k region takes the -W staging
#pragma unroll
    for (int cb = 0; cb < 8; cb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float w = -wacc[cb][i];
            const uint16_t h = vx_f32_to_bf16(w);
            W_h[(wave * 16 + 4 * g + i) * RP + cb * 16 + m] = h;
            W_l[(wave * 16 + 4 * g + i) * RP + cb * 16 + m] = vx_f32_to_bf16(w - vx_bf16_to_f32(h));
        }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const size_t o = ((size_t)(wave * 4 + ks) * 64 + lane) * 16;
        *(uint4 *)(rec + X_NW + o) = *(const uint4 *)&W_h[rowA * RP + 32 * ks + 8 * g];
        *(uint4 *)(rec + X_NW + 16384 + o) = *(const uint4 *)&W_l[rowA * RP + 32 * ks + 8 * g];
    }
}

// dnp_scan3: the chunk walk of dnp_scan with every operand as a hi/lo pair.
// A wave's operands of one chunk are 28 tiles of 1 KiB, a Ut tile per
// 16-column block and e^gam_C; they
// come straight from the record into registers (no LDS staging: a CU's
// memory pipe, about 64 B per cycle, is what bounds a chunk step, and an LDS
// slot would add its write and read).  The operand groups are consumed in
// order -- -W and Ut by U = Ut - W S, e^gam Q by O, Kt^T and e^gam_C by the
// state update, P by O += P U -- and each group's registers take the next
// chunk's loads as soon as its MFMAs have read them, so every load has about
// a whole chunk step to land and only one chunk's operands are live.
// The output rows of a chunk are stored at the top of the next step.
__device__ __forceinline__ uint32_t x3_src(int j, int wave, int slice) {
    // operand order: NW hi 0-3, NW lo 4-7, QE hi 8-11, QE lo 12-15, KT hi 16-19,
    // KT lo 20-23, P hi 24-25, P lo 26-27, Ut 28
    return j < 8    ? (uint32_t)(X_NW + (j >> 2) * 16384 + (wave * 4 + (j & 3)) * 1024)
           : j < 16 ? (uint32_t)(X_QE + ((j - 8) >> 2) * 16384 + (wave * 4 + (j & 3)) * 1024)
           : j < 24 ? (uint32_t)(X_KT + ((j - 16) >> 2) * 16384 + (wave * 4 + (j & 3)) * 1024)
           : j < 28 ? (uint32_t)(X_P + ((j - 24) >> 1) * 8192 + (wave * 2 + (j & 1)) * 1024)
                    : (uint32_t)(X_UT + (wave * 8 + slice + (j - 28)) * 1024);   // Ut of column block slice + j - 28
}
// tiles J0 .. J1-1 of a wave's operands of one chunk record into op[J0 ..]
template <int J0, int J1>
__device__ __forceinline__ void x3_load(const char *rec, int wave, int slice, int lane, uint4 *op) {
#pragma unroll
    for (int j = J0; j < J1; j++) {
        const u32x4_t v = *(g_u32x4 *)(rec + x3_src(j, wave, slice) + (uint32_t)lane * 16);
        op[j] = make_uint4(v.x, v.y, v.z, v.w);
    }
}



// NCB column blocks of 16 per workgroup (NSLICE / NCB workgroups per head):
// the A operands (-W, e^gam Q, Kt^T, P) a wave loads serve all NCB blocks,
// each block adds its Ut tile and its own MFMAs.  NCB = 2 halves the
// workgroups (and the operand fetch) of a launch with more workgroups than
// CUs.
template <int NCB>
__global__ __launch_bounds__(256) void dnp_scan3(ScanArgs p) {
    constexpr int NSL = NSLICE / NCB, NT = 28 + NCB;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.y, bid = blockIdx.x;
    int vh, slice;
    if (p.xcd_map) {
        const int xcd = bid & 7, idx = bid >> 3;
        slice = idx % NSL;
        vh = (idx / NSL) * 8 + xcd;
    } else {
        vh = bid / NSL;
        slice = bid % NSL;
    }
    const int cb0 = slice * NCB;   // first 16-column block of the workgroup

    __shared__ uint16_t S_h[NCB][16][HD + 8], S_lo[NCB][16][HD + 8];   // S blocks hi/lo, [column][key dim]
    __shared__ uint16_t U_h[NCB][16][CH + 8], U_lo[NCB][16][CH + 8];   // U blocks hi/lo, [column][token]

    const char *rec0 = vx_uniform_ptr(p.rec + ((size_t)b * p.nv + vh) * p.NC * XREC);
    uint4 op[NT];
    x3_load<0, NT>(rec0, wave, cb0, lane, op);
    float gc = *(g_float *)(rec0 + X_GC);

    float *Sg = p.S + ((size_t)b * p.nv + vh) * HD * HD;
    floatx4_t S[NCB][2];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                S[cb][r][i] = Sg[(size_t)((2 * wave + r) * 16 + 4 * g + i) * HD + (cb0 + cb) * 16 + n];

    floatx4_t Oprev[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) Oprev[cb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < p.NC; c++) {
        // the next chunk's record (the last one again after the end: those
        // loads are never used)
        const char *rec1 = rec0 + (size_t)min(c + 1, p.NC - 1) * XREC;
        if (c > 0) {
#pragma unroll
            for (int cb = 0; cb < NCB; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int tt = (c - 1) * CH + wave * 16 + 4 * g + i;
                    if (tt < p.T) p.out[(((size_t)b * p.T + tt) * p.nv + vh) * HD + (cb0 + cb) * 16 + n] = Oprev[cb][i];
                }
        }
        // S -> bf16 hi/lo, [column][key dim]
#pragma unroll
        for (int cb = 0; cb < NCB; cb++)
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int d = (2 * wave + r) * 16 + 4 * g;
                uint2 h, l;
                split4(S[cb][r], h, l);
                *(uint2 *)&S_h[cb][n][d] = h;
                *(uint2 *)&S_lo[cb][n][d] = l;
            }
        __syncthreads();   // S hi/lo complete
        floatx4_t O0[NCB], O1[NCB];
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            bf16x8_t sbh[4], sbl[4];
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                sbh[ks] = as_bf16x8(*(const uint4 *)&S_h[cb][n][32 * ks + 8 * g]);
                sbl[ks] = as_bf16x8(*(const uint4 *)&S_lo[cb][n][32 * ks + 8 * g]);
            }
            // U = Ut - W S, in independent chains
            const uint4 utu = op[28 + cb];
            floatx4_t U0 = (floatx4_t){__uint_as_float(utu.x), __uint_as_float(utu.y), __uint_as_float(utu.z),
                                       __uint_as_float(utu.w)};
            floatx4_t U1 = {0.f, 0.f, 0.f, 0.f}, U2 = {0.f, 0.f, 0.f, 0.f}, U3 = {0.f, 0.f, 0.f, 0.f};
            MFMA3(U0, as_bf16x8(op[0]), as_bf16x8(op[4]), sbh[0], sbl[0]);
            MFMA3(U1, as_bf16x8(op[1]), as_bf16x8(op[5]), sbh[1], sbl[1]);
            MFMA3(U2, as_bf16x8(op[2]), as_bf16x8(op[6]), sbh[2], sbl[2]);
            MFMA3(U3, as_bf16x8(op[3]), as_bf16x8(op[7]), sbh[3], sbl[3]);
            if (cb == NCB - 1) {   // -W and Ut take chunk c+1
                __builtin_amdgcn_sched_barrier(0);
                x3_load<0, 8>(rec1, wave, cb0, lane, op);
                x3_load<28, NT>(rec1, wave, cb0, lane, op);
                __builtin_amdgcn_sched_barrier(0);
            }
            const floatx4_t U = (U0 + U1) + (U2 + U3);
            {
                uint2 h, l;
                split4(U, h, l);
                *(uint2 *)&U_h[cb][n][wave * 16 + 4 * g] = h;
                *(uint2 *)&U_lo[cb][n][wave * 16 + 4 * g] = l;
            }
            // the e^gam Q S part of O
            O0[cb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
            O1[cb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
            MFMA3(O0[cb], as_bf16x8(op[8]), as_bf16x8(op[12]), sbh[0], sbl[0]);
            MFMA3(O1[cb], as_bf16x8(op[9]), as_bf16x8(op[13]), sbh[1], sbl[1]);
            MFMA3(O0[cb], as_bf16x8(op[10]), as_bf16x8(op[14]), sbh[2], sbl[2]);
            MFMA3(O1[cb], as_bf16x8(op[11]), as_bf16x8(op[15]), sbh[3], sbl[3]);
        }
        // e^gam Q takes chunk c+1
        __builtin_amdgcn_sched_barrier(0);
        x3_load<8, 16>(rec1, wave, cb0, lane, op);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();   // U hi/lo complete
        bf16x8_t ubh[NCB][2], ubl[NCB][2];
#pragma unroll
        for (int cb = 0; cb < NCB; cb++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                ubh[cb][ks] = as_bf16x8(*(const uint4 *)&U_h[cb][n][32 * ks + 8 * g]);
                ubl[cb][ks] = as_bf16x8(*(const uint4 *)&U_lo[cb][n][32 * ks + 8 * g]);
            }
        // S = e^gam_C S + Kt^T U, per row block two chains; then Kt^T and
        // e^gam_C take chunk c+1
#pragma unroll
        for (int cb = 0; cb < NCB; cb++)
#pragma unroll
            for (int r = 0; r < 2; r++) {
                floatx4_t Sa = S[cb][r] * gc, Sb = {0.f, 0.f, 0.f, 0.f};
                MFMA3(Sa, as_bf16x8(op[16 + 2 * r]), as_bf16x8(op[20 + 2 * r]), ubh[cb][0], ubl[cb][0]);
                MFMA3(Sb, as_bf16x8(op[17 + 2 * r]), as_bf16x8(op[21 + 2 * r]), ubh[cb][1], ubl[cb][1]);
                S[cb][r] = Sa + Sb;
            }
        __builtin_amdgcn_sched_barrier(0);
        x3_load<16, 24>(rec1, wave, cb0, lane, op);
        gc = *(g_float *)(rec1 + X_GC);
        __builtin_amdgcn_sched_barrier(0);
        // O += P U; then P takes chunk c+1
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
            MFMA3(O0[cb], as_bf16x8(op[24]), as_bf16x8(op[26]), ubh[cb][0], ubl[cb][0]);
            MFMA3(O1[cb], as_bf16x8(op[25]), as_bf16x8(op[27]), ubh[cb][1], ubl[cb][1]);
        }
        __builtin_amdgcn_sched_barrier(0);
        x3_load<24, 28>(rec1, wave, cb0, lane, op);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) Oprev[cb] = O0[cb] + O1[cb];
    }
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tt = (p.NC - 1) * CH + wave * 16 + 4 * g + i;
            if (tt < p.T) p.out[(((size_t)b * p.T + tt) * p.nv + vh) * HD + (cb0 + cb) * 16 + n] = Oprev[cb][i];
        }
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                Sg[(size_t)((2 * wave + r) * 16 + 4 * g + i) * HD + (cb0 + cb) * 16 + n] = S[cb][r][i];
}

// ---- the glue of vx27_qlayer_batch around the chunked core --------------
// dnp_glue_in: one wave per (128-channel head of the q|k|v row, block of
// GT tokens): the head's conv weights and the prompt's x rows t0-3 .. t0+GT-1
// are loaded once (a lane holds two channels), then for each token the
// causal conv + SiLU from the prompt's x and the carried conv state
// (VX27_DN_CONV; else the bf16 q/k/v widened), on q and k heads the
// pre-norms the flags ask for -- rmsn(x)(1+w) (vx27_qfwd.c:32-39, 123) and
// l2norm with q/sqrt(128) (:124-130), sums in double -- and the result as
// bf16 hi (and lo) for the chunked products (whose prep applies step_exact's
// own l2norm and scale once more, as the reference does).  In the split
// form q and k also get their lo parts as rows, and v is kept in fp32 (the
// walk subtracts from it in fp32 and never multiplies it on MFMA).
// grid (ceil(T/GT/4), heads, B), block 256.
constexpr int GT = 8;
struct GlueInArgs {
    int B, T, nqk, nv, C;
    unsigned flags;
    int w_bf16;
    const float *x;            // [B][T][C] (VX27_DN_CONV)
    const float *conv_state;   // [B][C][3], the state before token 0
    const void *conv_w;
    const uint16_t *q, *k, *v; // bf16 inputs without VX27_DN_CONV
    const float *norm_w;       // [128]
    uint16_t *qo, *ko, *vo;    // bf16 [B][T][nqk|nqk|nv][128] (vo: without vo32)
    uint16_t *qol, *kol;       // lo parts (x - bf16(x)) of q, k as rows, or NULL
    float *vo32;               // v as fp32 rows [B][T][nv][128], or NULL
};
__global__ __launch_bounds__(256) void dnp_glue_in(GlueInArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hh = blockIdx.y, b = blockIdx.z, t0 = (blockIdx.x * 4 + wave) * GT;
    if (t0 >= a.T) return;
    const bool is_q = hh < a.nqk, is_k = !is_q && hh < 2 * a.nqk;
    __shared__ __attribute__((aligned(16))) uint16_t s_rows[4][2][GT][HD];   // [wave][hi, lo][token][channel]
    {
        const bool conv = (a.flags & VX27_DN_CONV) != 0;
        const float qs = 1.0f / sqrtf((float)HD);
        const int nt = min(GT, a.T - t0);
        // Every input of the block is loaded first, unconditionally, from
        // addresses clamped into the buffers, and the cases are selected after:
        // a load under a condition would wait for its data inside its branch.
        // With the conv: the x window of the two channels, tokens t0-3 ..
        // t0+GT-1 (older ones from the state, none past the prompt), and the
        // conv weights as raw words (two 8-byte words, the second one repeating
        // the first for bf16); without it, the block's q, k or v values.
        float xw[2][GT + 3], w[2][4];
        float nw[2] = {1.0f, 1.0f};
        uint2 wr[2][2];
        float cst[2][3];
        const uint16_t *src = is_q ? a.q + hh * HD : is_k ? a.k + (hh - a.nqk) * HD : a.v + (hh - 2 * a.nqk) * HD;
        const int hstride = (is_q || is_k) ? a.nqk * HD : a.nv * HD;
        if (conv) {   // (one branch around both channels' loads: they all stay in flight together)
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const size_t ch = (size_t)hh * HD + lane + 64 * e;
                const uint2 *wb = (const uint2 *)a.conv_w;
                const size_t w0 = a.w_bf16 ? ch : 2 * ch;
                wr[e][0] = wb[w0];
                wr[e][1] = wb[a.w_bf16 ? w0 : w0 + 1];
#pragma unroll
                for (int t = 0; t < 3; t++) cst[e][t] = a.conv_state[((size_t)b * a.C + ch) * 3 + t];
#pragma unroll
                for (int j = 0; j < GT + 3; j++) {
                    const int sc = min(max(t0 - 3 + j, 0), a.T - 1);
                    xw[e][j] = a.x[((size_t)b * a.T + sc) * a.C + ch];
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 2; e++)
#pragma unroll
                for (int j = 0; j < GT; j++) {
                    const size_t row = (size_t)b * a.T + min(t0 + j, a.T - 1);
                    xw[e][j] = vx_bf16_to_f32(src[row * hstride + lane + 64 * e]);
                }
        }
        if (a.norm_w && (is_q || is_k)) {
            nw[0] = a.norm_w[lane];
            nw[1] = a.norm_w[lane + 64];
        }
        if (conv) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t r[4] = {wr[e][0].x, wr[e][0].y, wr[e][1].x, wr[e][1].y};
                conv_w_decode(a.w_bf16, r, w[e]);
#pragma unroll
                for (int j = 0; j < GT + 3; j++) {
                    const int s = t0 - 3 + j;   // s < 0 only for j < 3 (t0 = 0): state slot j
                    xw[e][j] = s < 0 ? cst[e][j < 3 ? j : 0] : s < a.T ? xw[e][j] : 0.0f;
                }
            }
        }
        // Every token of the block first (tokens past nt come from clamped or
        // zero inputs and are never stored), then the pre-norms of all GT tokens
        // side by side: their wave sums are independent chains that the
        // scheduler interleaves, where one token at a time they ran back to back.
        // Each token's operations and their order are unchanged.
        float v2s[GT][2];
#pragma unroll
        for (int j = 0; j < GT; j++)
#pragma unroll
            for (int e = 0; e < 2; e++) {
                if (conv) {
                    float c[3] = {xw[e][j], xw[e][j + 1], xw[e][j + 2]};
                    v2s[j][e] = conv_step(c, w[e], xw[e][j + 3]);
                } else {
                    v2s[j][e] = xw[e][j];
                }
            }
        if ((is_q || is_k) && (a.flags & (VX27_DN_PRE_RMS | VX27_DN_PRE_L2))) {
            if (a.flags & VX27_DN_PRE_RMS) {
                double ss[GT];
#pragma unroll
                for (int j = 0; j < GT; j++)
                    ss[j] = vx_wave_sum_f64_dpp((double)v2s[j][0] * (double)v2s[j][0] + (double)v2s[j][1] * (double)v2s[j][1]);
#pragma unroll
                for (int j = 0; j < GT; j++) {
                    const float is = 1.0f / sqrtf((float)(ss[j] / HD) + 1e-6f);
#pragma unroll
                    for (int e = 0; e < 2; e++) v2s[j][e] = (v2s[j][e] * is) * (nw[e] + 1.0f);
                }
            }
            if (a.flags & VX27_DN_PRE_L2) {
                double ss[GT];
#pragma unroll
                for (int j = 0; j < GT; j++)
                    ss[j] = vx_wave_sum_f64_dpp((double)v2s[j][0] * (double)v2s[j][0] + (double)v2s[j][1] * (double)v2s[j][1]);
#pragma unroll
                for (int j = 0; j < GT; j++) {
                    const float il = 1.0f / sqrtf((float)ss[j] + 1e-6f);
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        v2s[j][e] = v2s[j][e] * il;
                        if (is_q) v2s[j][e] = v2s[j][e] * qs;
                    }
                }
            }
        }
        if (a.vo32 && !is_q && !is_k) {   // v in fp32: 256 contiguous bytes per channel half
#pragma unroll
            for (int j = 0; j < GT; j++) {
                if (j >= nt) break;
                float *dst = a.vo32 + (((size_t)b * a.T + t0 + j) * a.nv + (hh - 2 * a.nqk)) * HD;
                dst[lane] = v2s[j][0];
                dst[lane + 64] = v2s[j][1];
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < GT; j++) {
            if (j >= nt) break;
            const float v2[2] = {v2s[j][0], v2s[j][1]};
            const uint16_t h0 = vx_f32_to_bf16(v2[0]), h1 = vx_f32_to_bf16(v2[1]);
            s_rows[wave][0][j][lane] = h0;
            s_rows[wave][0][j][lane + 64] = h1;
            if (a.qol) {
                s_rows[wave][1][j][lane] = vx_f32_to_bf16(v2[0] - vx_bf16_to_f32(h0));
                s_rows[wave][1][j][lane + 64] = vx_f32_to_bf16(v2[1] - vx_bf16_to_f32(h1));
            }
        }
        // the block's rows out of the wave's own LDS slots, 16 bytes a lane
        // (lane: row (lane >> 4) + 4 i, channels 8 (lane & 15) ..): two stores
        // of hi rows (and of lo rows for q, k) instead of one 2-byte store per
        // row and channel half
        const int cg = lane & 15;
        __builtin_amdgcn_wave_barrier();   // (the slots are this wave's own: LDS runs its ops in order)
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int jr = (lane >> 4) + 4 * i;
            if (jr < nt) {
                const size_t row = (size_t)b * a.T + t0 + jr;
                uint16_t *dst = is_q ? a.qo + (row * a.nqk + hh) * HD
                              : is_k ? a.ko + (row * a.nqk + (hh - a.nqk)) * HD
                                     : a.vo + (row * a.nv + (hh - 2 * a.nqk)) * HD;
                *(uint4 *)(dst + 8 * cg) = *(const uint4 *)&s_rows[wave][0][jr][8 * cg];
                if (a.qol && (is_q || is_k)) {
                    uint16_t *dl = is_q ? a.qol + (row * a.nqk + hh) * HD : a.kol + (row * a.nqk + (hh - a.nqk)) * HD;
                    *(uint4 *)(dl + 8 * cg) = *(const uint4 *)&s_rows[wave][1][jr][8 * cg];
                }
            }
        }
    }
}

// The conv state after the prompt: the last three inputs of each channel
// (older ones from the state itself when T < 3).  One thread per (b, c); it
// runs after dnp_glue_in, which read the state before token 0.
__global__ __launch_bounds__(256) void dnp_conv_state(int B, int T, int C, const float *x, float *state) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)B * C) return;
    const int b = (int)(id / C), c = (int)(id % C);
    float *sp = state + id * 3;
    float n[3];
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int s = T - 3 + j;
        n[j] = s >= 0 ? x[((size_t)b * T + s) * C + c] : sp[3 + s];   // (T < 3: the old state shifted)
    }
    sp[0] = n[0]; sp[1] = n[1]; sp[2] = n[2];
}

// dnp_out_gate: the gated RMS norm rmsn_std(o) * norm_w * silu(z) of every
// (token, head) row of 128 (vx27_qfwd.c:145-151), in place.  One wave per 8
// rows, a half-wave per row (lane: 4 consecutive floats), every load of the
// 8 rows (o and z) issued before any is used; the sum of squares in double
// over the half-wave.  out, z and norm_w 16-byte aligned.
// grid ceil(rows / 32), block 256.
// One row's gated norm: rmsn_std(o) * norm_w * silu(z) for the 4 values a
// lane holds (the row's 128 values on the 32 lanes of a wave half).
__device__ __forceinline__ float4 out_gate_row(float4 o, float4 zz, float4 w) {
    double ss = (((double)o.x * (double)o.x + (double)o.y * (double)o.y) + (double)o.z * (double)o.z) +
                (double)o.w * (double)o.w;
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) ss += __shfl_xor(ss, off, 64);
    const float is = 1.0f / sqrtf((float)(ss / HD) + 1e-6f);
    float4 y;
    y.x = ((o.x * is) * w.x) * silu_f(zz.x);
    y.y = ((o.y * is) * w.y) * silu_f(zz.y);
    y.z = ((o.z * is) * w.z) * silu_f(zz.z);
    y.w = ((o.w * is) * w.w) * silu_f(zz.w);
    return y;
}

__global__ __launch_bounds__(256) void dnp_out_gate(int rows, const float *z, const float *norm_w, float *out) {
    const int lane = threadIdx.x & 63, hl = lane & 31, hr = lane >> 5;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 8;
    if (r0 >= rows) return;   // (wave-uniform)
    float4 o[4], zz[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {   // rows past the end re-read the last row
        const size_t r = (size_t)min(r0 + 2 * i + hr, rows - 1);
        o[i] = *(const float4 *)(out + r * HD + 4 * hl);
        zz[i] = *(const float4 *)(z + r * HD + 4 * hl);
    }
    const float4 w = *(const float4 *)(norm_w + 4 * hl);
    __builtin_amdgcn_sched_barrier(0);   // every load issued before the first wait
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 y = out_gate_row(o[i], zz[i], w);
        // (unconditional: rows past the end store the last row's own result
        // again; a store under the row test would take the loads into its
        // branch, with a wait for all of them)
        *(float4 *)(out + (size_t)min(r0 + 2 * i + hr, rows - 1) * HD + 4 * hl) = y;
    }
}

// The same gated norm written as the packed tokens of the long-prompt GEMM
// that takes it next (out_proj: K = nv 128, vx_gemm_pack_unit): hi =
// bf16(y), lo = bf16(y - hi), the split gemm_pack would make of the fp32
// rows, without writing and reading them back.  grid (token blocks of 16,
// nv), block 256: wave w takes tokens 4w .. 4w+3 of the block, for value
// head blockIdx.y.  The workgroup's share of the images (4 k-steps x hi,
// lo x one 1 KiB block) is assembled in LDS and stored as whole blocks, 16
// bytes a lane.  R: tokens (B T); rows t nv + h of o and z.
__global__ __launch_bounds__(256) void dnp_out_gate_packed(int R, int nv, const float *o, const float *z,
                                                           const float *norm_w, char *xp) {
    __shared__ __attribute__((aligned(16))) char img[8 * 1024];   // [k-step s of the head][hi, lo][1 KiB]
    const int tid = threadIdx.x, lane = tid & 63, hl = lane & 31, hr = lane >> 5;
    const int h = blockIdx.y, tb0 = blockIdx.x * 16, t0 = tb0 + (tid >> 6) * 4;
    float4 ov[2], zv[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {   // tokens past the end re-do the last token
        const size_t r = (size_t)min(t0 + 2 * i + hr, R - 1) * nv + h;
        ov[i] = *(const float4 *)(o + r * HD + 4 * hl);
        zv[i] = *(const float4 *)(z + r * HD + 4 * hl);
    }
    const float4 w = *(const float4 *)(norm_w + 4 * hl);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const float4 y = out_gate_row(ov[i], zv[i], w);
        const uint32_t h0 = pack2(y.x, y.y), h1 = pack2(y.z, y.w);
        const uint32_t l0 = pack2(y.x - __uint_as_float(h0 << 16), y.y - __uint_as_float(h0 & 0xffff0000u));
        const uint32_t l1 = pack2(y.z - __uint_as_float(h1 << 16), y.w - __uint_as_float(h1 & 0xffff0000u));
        // dims 4 hl .. of token n: k-step hl / 8 of the head, unit g = (hl / 2) % 4,
        // half hl % 2 (lanes hl, hl ^ 1 fill one unit)
        const int n = (t0 + 2 * i + hr) & 15, g = (hl >> 1) & 3;
        char *u = img + (hl >> 3) * 2048 + (g * 16 + (n ^ (g << 1))) * 16 + (hl & 1) * 8;
        *(uint2 *)u = make_uint2(h0, h1);
        *(uint2 *)(u + 1024) = make_uint2(l0, l1);
    }
    __syncthreads();
    // block (k-step sl, part) to its place: image (token tile, 4 h + sl),
    // block (token block within the tile) 2 + part
    const int K = nv * HD;
    const size_t base = vx_gemm_pack_unit(tb0, 4 * h * 32, K);   // hi unit 0 of (k-step 4h, token block tb0 / 16)
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int c = tid + 256 * q, blk = c >> 6, sl = blk >> 1, part = blk & 1;
        const uint4 v = *(const uint4 *)(img + c * 16);
        *(uint4 *)(xp + base + (size_t)sl * 32768 + part * 1024 + (c & 63) * 16) = v;
    }
}

// Widen bf16 q|k|v rows into one fp32 row per token (the exact path's input
// without the conv): act [B][T][C].
__global__ __launch_bounds__(256) void dnp_widen(int rows, int nqk, int nv, const uint16_t *q, const uint16_t *k,
                                                 const uint16_t *v, float *act) {
    const int qd = nqk * HD, vd = nv * HD, C = 2 * qd + vd;
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)rows * C) return;
    const size_t r = id / C;
    const int c = (int)(id % C);
    const uint16_t h = c < qd ? q[r * qd + c] : c < 2 * qd ? k[r * qd + (c - qd)] : v[r * vd + (c - 2 * qd)];
    act[id] = vx_bf16_to_f32(h);
}

// vx27_hip_dn_commit: checkpoint m[b] of sequence b into the live state.
// grid (chunks of 256 elements, B), block 256.
__global__ __launch_bounds__(256) void dn_commit_kernel(int T, size_t s_elems, size_t c_elems, const int *m,
                                                        const float *S_ckpt, const float *conv_ckpt, float *S,
                                                        float *conv, int *err_flag) {
    const int b = blockIdx.y;
    const int mb = m[b];
    if (mb < 0) return;
    if (mb >= T) {
        if (blockIdx.x == 0 && threadIdx.x == 0) *err_flag = 1;
        return;
    }
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (S_ckpt && i < s_elems) S[(size_t)b * s_elems + i] = S_ckpt[((size_t)b * T + mb) * s_elems + i];
    if (conv_ckpt && i < c_elems) conv[(size_t)b * c_elems + i] = conv_ckpt[((size_t)b * T + mb) * c_elems + i];
}

}  // namespace

// Scratch layout of one prefill call (sizes in bytes, 256-aligned pieces).
static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }
static bool dn_prefill_is_exact(const vx27_dn_prefill_desc *d) {
    return (d->flags & VX27_DN_EXACT) || d->S_ckpt || d->conv_ckpt;
}
// The glue's outputs: q, k hi rows and v as bf16 rows; the split form adds
// the q and k lo rows and keeps v in fp32 instead.
static size_t vx_dn_glue_bytes(int B, int T, int nqk, int nv, bool x3, bool xin) {
    const size_t rows = (size_t)B * T;
    const size_t qd = (size_t)nqk * HD, vd = (size_t)nv * HD;
    if (xin) return 0;   // prept forms q, k and v from x: no glue kernel
    return x3 ? al256(rows * 4 * qd * sizeof(uint16_t)) + rows * vd * sizeof(float)
              : rows * (2 * qd + vd) * sizeof(uint16_t);
}
// The T-record form with the conv forms q, k and v from x itself (prept),
// with no glue kernel: split products, the conv, and 16-byte aligned x rows.
static bool dn_prefill_xin(const vx27_dn_prefill_desc *d) {
    return !(d->flags & VX27_DN_BF16) && (d->flags & VX27_DN_CONV) && ((uintptr_t)d->x & 15) == 0;
}
// Bytes of one K record (K^T operand tiles, hi and, with lo parts, lo).
static size_t vx_dn_krec_bytes(bool lo) { return lo ? 2 * K_LO : K_LO; }

size_t vx_dn_prefill_scratch(const vx27_dn_prefill_desc *d) {
    const int qd = d->nqk * HD, vd = d->nv * HD, C = 2 * qd + vd;
    const size_t rows = (size_t)d->B * d->T;
    if (dn_prefill_is_exact(d))
        return al256(rows * d->nv * sizeof(double2)) + al256((size_t)d->B * vd * sizeof(float)) +
               al256(rows * C * sizeof(float)) + (d->S_ckpt ? 0 : vx_dn_qk_bytes(d->T, d->B, d->nqk));
    const int NC = (d->T + CH - 1) / CH;
    const bool x3 = !(d->flags & VX27_DN_BF16);
    const size_t n_rec = (size_t)d->B * d->nv * NC;
    const bool glue = (d->flags & (VX27_DN_CONV | VX27_DN_PRE_RMS | VX27_DN_PRE_L2)) != 0;
    const size_t glue_bytes = glue ? vx_dn_glue_bytes(d->B, d->T, d->nqk, d->nv, x3, dn_prefill_xin(d)) : 0;
    if (x3 && glue)
        return al256(n_rec * TREC) + al256((size_t)d->B * d->nqk * NC * vx_dn_krec_bytes(true)) + glue_bytes;
    return al256(n_rec * (x3 ? XREC : REC)) + al256(n_rec * sizeof(float)) + glue_bytes;
}

// The exact path: the decode kernels token by token (prefill layout).
static int dn_prefill_exact(vx27_hip_ctx *ctx, const vx27_dn_prefill_desc *d, void *scr) {
    const int qd = d->nqk * HD, vd = d->nv * HD, C = 2 * qd + vd;
    const bool conv = (d->flags & VX27_DN_CONV) != 0;
    const size_t rows = (size_t)d->B * d->T;
    const size_t gate_bytes = al256(rows * d->nv * sizeof(double2));
    const size_t opre_bytes = al256((size_t)d->B * vd * sizeof(float));
    double2 *gates = (double2 *)scr;
    float *act = (float *)((char *)scr + gate_bytes + opre_bytes);
    const size_t n_gate = rows * d->nv;
    if (vx_dn_gates(ctx, n_gate, d->nv, d->a, d->b, d->A_log, d->dt_bias, gates)) return -1;
    if (conv) {
        ConvArgs ca = {d->B, C, d->T, d->conv_w_dtype == VX27_BF16, d->conv_state, d->conv_w, d->x, act, 1, d->T,
                       d->conv_ckpt};
        if (vx_dn_conv(ctx, ca)) return -1;
    } else {
        const size_t n = rows * C;
        VX_LAUNCH(ctx, dnp_widen, dim3((unsigned)((n + 255) / 256)), dim3(256), (int)rows, d->nqk, d->nv, d->q, d->k,
                  d->v, act);
    }
    DnArgs a = {};
    a.B = d->B; a.nqk = d->nqk; a.nv = d->nv; a.flags = d->flags & (VX27_DN_PRE_RMS | VX27_DN_PRE_L2 | VX27_DN_OUT_GATE);
    a.t_step = 1; a.b_step = d->T;
    a.S = d->S; a.norm_w = d->norm_w; a.z = d->z; a.z_tok = (size_t)vd;
    a.q_tok = a.k_tok = a.v_tok = (size_t)C;
    a.out_tok = (size_t)vd;
    a.o_pre = (float *)((char *)scr + gate_bytes);
    if (!d->S_ckpt) {   // one launch, the state resident in registers
        a.steps = d->T;
        a.q = act; a.k = act + qd; a.v = act + 2 * qd;
        a.gates = gates; a.out = d->out;
        a.qk_buf = (float *)((char *)act + al256(rows * C * sizeof(float)));
        return vx_dn_recurrence(ctx, a);
    }
    // token by token, the state written out after each (single-step kernel)
    const size_t s_bytes = (size_t)d->nv * HD * HD * sizeof(float);
    for (int t = 0; t < d->T; t++) {
        DnArgs at = a;
        at.steps = 1;
        at.q = act + (size_t)t * C; at.k = at.q + qd; at.v = at.q + 2 * qd;
        at.gates = gates + (size_t)t * d->nv;
        at.z = d->z ? d->z + (size_t)t * vd : nullptr;
        at.out = d->out + (size_t)t * vd;
        if (vx_dn_recurrence(ctx, at)) return -1;
        VX_HIP(hipMemcpy2DAsync((char *)d->S_ckpt + (size_t)t * s_bytes, (size_t)d->T * s_bytes, d->S, s_bytes, s_bytes,
                                (size_t)d->B, hipMemcpyDeviceToDevice, ctx->stream));
    }
    return 0;
}

static int dn_prefill_check(const vx27_dn_prefill_desc *d) {
    VX_REQUIRE(d, "vx27_hip_dn_prefill: null descriptor");
    VX_REQUIRE(d->hd == HD, "vx27_hip_dn_prefill: head_dim must be 128 (got %d)", d->hd);
    VX_REQUIRE(d->B >= 1 && d->T >= 1 && d->nqk >= 1 && d->nv >= d->nqk && d->nv % d->nqk == 0 && d->nv <= 4096,
               "vx27_hip_dn_prefill: bad sizes B=%d T=%d nqk=%d nv=%d", d->B, d->T, d->nqk, d->nv);
    VX_REQUIRE((d->flags & ~63u) == 0, "vx27_hip_dn_prefill: unknown flags %#x", d->flags);
    VX_REQUIRE(d->S && d->a && d->b && d->A_log && d->dt_bias && d->out, "vx27_hip_dn_prefill: null pointer");
    const bool conv = (d->flags & VX27_DN_CONV) != 0;
    if (conv) {
        VX_REQUIRE(d->x && d->conv_state && d->conv_w, "vx27_hip_dn_prefill: VX27_DN_CONV needs x, conv_state, conv_w");
        VX_REQUIRE(d->conv_w_dtype == VX27_F32 || d->conv_w_dtype == VX27_BF16,
                   "vx27_hip_dn_prefill: conv_w_dtype must be VX27_F32 or VX27_BF16");
        VX_REQUIRE(((uintptr_t)d->conv_w & 15) == 0, "vx27_hip_dn_prefill: conv_w must be 16-byte aligned");
    } else {
        VX_REQUIRE(d->q && d->k && d->v, "vx27_hip_dn_prefill: q, k, v are required without VX27_DN_CONV");
        VX_REQUIRE((((uintptr_t)d->q | (uintptr_t)d->k | (uintptr_t)d->v) & 15) == 0,
                   "vx27_hip_dn_prefill: q, k and v must be 16-byte aligned");
        VX_REQUIRE(!d->conv_ckpt, "vx27_hip_dn_prefill: conv_ckpt needs VX27_DN_CONV");
    }
    VX_REQUIRE(((uintptr_t)d->out & 15) == 0, "vx27_hip_dn_prefill: out must be 16-byte aligned");
    if (d->flags & (VX27_DN_PRE_RMS | VX27_DN_OUT_GATE))
        VX_REQUIRE(d->norm_w != nullptr, "vx27_hip_dn_prefill: norm_w required by PRE_RMS/OUT_GATE");
    if (d->flags & VX27_DN_OUT_GATE) {
        VX_REQUIRE(d->z != nullptr, "vx27_hip_dn_prefill: z required by OUT_GATE");
        VX_REQUIRE((((uintptr_t)d->z | (uintptr_t)d->norm_w | (uintptr_t)d->out) & 15) == 0,
                   "vx27_hip_dn_prefill: OUT_GATE needs z, norm_w and out 16-byte aligned");
    }
    return 0;
}

// The prefill on caller-provided scratch of vx_dn_prefill_scratch(d) bytes.
int vx_dn_prefill_into(vx27_hip_ctx *ctx, const vx27_dn_prefill_desc *d, void *scr, char *out_packed) {
    if (dn_prefill_check(d)) return -1;
    VX_REQUIRE(!out_packed || (!dn_prefill_is_exact(d) && (d->flags & VX27_DN_OUT_GATE)),
               "internal: a packed output needs the chunked form with the output gate");
    if (dn_prefill_is_exact(d)) return dn_prefill_exact(ctx, d, scr);
    const bool conv = (d->flags & VX27_DN_CONV) != 0;
    const int NC = (d->T + CH - 1) / CH;
    const bool x3 = !(d->flags & VX27_DN_BF16);   // split (bf16x3) products unless asked for bf16
    const size_t n_rec = (size_t)d->B * d->nv * NC;
    const bool glue = conv || (d->flags & (VX27_DN_PRE_RMS | VX27_DN_PRE_L2));
    const int qd = d->nqk * HD, vd = d->nv * HD, C = 2 * qd + vd;
    const size_t rows = (size_t)d->B * d->T;
    // the T-record form for the glue's split inputs, the full records for
    // inputs exact in bf16 (and for the bf16 products)
    const bool trec = x3 && glue;
    const size_t rec_bytes = trec ? al256(n_rec * TREC) : al256(n_rec * (x3 ? XREC : REC)) + al256(n_rec * sizeof(float));
    const size_t krec_one = vx_dn_krec_bytes(true);
    const size_t krec_bytes = trec ? al256((size_t)d->B * d->nqk * NC * krec_one) : 0;
    // (the walk addresses one head's records with 32-bit offsets)
    VX_REQUIRE(!trec || (size_t)NC * krec_one < ((size_t)1 << 31),
               "vx27_hip_dn_prefill: T = %d exceeds the 1398080-token limit of one call", d->T);
    char *glue_buf = (char *)scr + rec_bytes + krec_bytes;
    const uint16_t *q = d->q, *k = d->k, *v = d->v;
    const uint16_t *ql = nullptr, *kl = nullptr;
    const float *v32 = nullptr;
    // the T form with the conv forms q, k and v itself from x (16-byte rows needed)
    const bool xin = trec && dn_prefill_xin(d);
    auto conv_state_update = [&]() -> int {   // after every reader of the old state
        const size_t nthr = (size_t)d->B * C;
        VX_LAUNCH(ctx, dnp_conv_state, dim3((unsigned)((nthr + 255) / 256)), dim3(256), d->B, d->T, C, d->x,
                  d->conv_state);
        return 0;
    };
    if (glue && !xin) {   // conv and pre-norms in fp32, then q, k as bf16 (hi, and lo for the split form), v
        uint16_t *qo = (uint16_t *)glue_buf, *ko = qo + rows * qd;
        uint16_t *qol = x3 ? ko + rows * qd : nullptr, *kol = x3 ? qol + rows * qd : nullptr;
        uint16_t *vo = x3 ? nullptr : ko + rows * qd;
        float *vo32 = x3 ? (float *)(glue_buf + al256(rows * 4 * qd * sizeof(uint16_t))) : nullptr;
        GlueInArgs ga{d->B, d->T, d->nqk, d->nv, C, d->flags, d->conv_w_dtype == VX27_BF16, d->x, d->conv_state,
                      d->conv_w, d->q, d->k, d->v, d->norm_w, qo, ko, vo, qol, kol, vo32};
        const int nh = 2 * d->nqk + d->nv;   // (q, k heads first)
        const int tblk = (d->T + GT - 1) / GT;
        VX_LAUNCH(ctx, dnp_glue_in, dim3((unsigned)((tblk + 3) / 4), (unsigned)nh, (unsigned)d->B), dim3(256), ga);
        if (conv && conv_state_update()) return -1;
        q = qo; k = ko; v = vo;
        ql = qol; kl = kol; v32 = vo32;
    }
    // two column blocks per walk workgroup once one each would exceed the CUs
    const bool two = d->nv * NSLICE * d->B > ctx->n_cu;
    if (trec) {
        char *rec = (char *)scr, *krec = (char *)scr + rec_bytes;
        PrepTArgs pa{d->T, d->nqk, d->nv, NC, q, k, ql, kl, v32, d->a, d->b, d->A_log, d->dt_bias, rec, krec,
                     (int)krec_one, C, d->conv_w_dtype == VX27_BF16, d->x, d->conv_state, d->conv_w, d->flags, d->norm_w};
        const dim3 pg((unsigned)NC, (unsigned)d->nqk, (unsigned)d->B);
        if (xin) VX_LAUNCH_NAMED(ctx, "dnp_prept", dnp_prept<true>, pg, dim3(256), pa);
        else VX_LAUNCH_NAMED(ctx, "dnp_prept", dnp_prept<false>, pg, dim3(256), pa);
        if (xin && conv_state_update()) return -1;   // prept read the state before token 0
        ScanTArgs sa{d->T, d->nqk, d->nv, NC, (d->nqk % 8) == 0, q, k, ql, kl, rec, krec, (int)krec_one, d->S, d->out};
        const dim3 sg((unsigned)(d->nv * NSLICE / (two ? 2 : 1)), (unsigned)d->B);
        if (two) VX_LAUNCH_NAMED(ctx, "dnp_scant", dnp_scant<2>, sg, dim3(256), sa);
        else VX_LAUNCH_NAMED(ctx, "dnp_scant", dnp_scant<1>, sg, dim3(256), sa);
    } else if (x3) {
        ScanArgs sa{d->T, d->nv, NC, (d->nv % 8) == 0, (const char *)scr,
                    (const float *)((char *)scr + al256(n_rec * XREC)), d->S, d->out};
        Prep3Args pa{d->T, d->nqk, d->nv, NC, q, k, v, nullptr, nullptr, nullptr, nullptr, NC * CH, d->a, d->b,
                     d->A_log, d->dt_bias, (char *)scr};
        VX_LAUNCH_NAMED(ctx, "dnp_prep3", dnp_prep3<false>, dim3((unsigned)NC, (unsigned)d->nv, (unsigned)d->B),
                        dim3(256), pa);
        if (two)
            VX_LAUNCH_NAMED(ctx, "dnp_scan3", dnp_scan3<2>, dim3((unsigned)(d->nv * NSLICE / 2), (unsigned)d->B),
                            dim3(256), sa);
        else
            VX_LAUNCH_NAMED(ctx, "dnp_scan3", dnp_scan3<1>, dim3((unsigned)(d->nv * NSLICE), (unsigned)d->B),
                            dim3(256), sa);
    } else {
        ScanArgs sa{d->T, d->nv, NC, (d->nv % 8) == 0, (const char *)scr, (const float *)((char *)scr + al256(n_rec * REC)),
                    d->S, d->out};
        PrepArgs pa{d->T, d->nqk, d->nv, NC, q, k, v, d->a, d->b, d->A_log, d->dt_bias,
                    (char *)scr, (float *)((char *)scr + al256(n_rec * REC))};
        VX_LAUNCH(ctx, dnp_prep, dim3((unsigned)NC, (unsigned)d->nv, (unsigned)d->B), dim3(256), pa);
        VX_LAUNCH(ctx, dnp_scan, dim3((unsigned)(d->nv * NSLICE), (unsigned)d->B), dim3(256), sa);
    }
    if (out_packed) {
        VX_LAUNCH(ctx, dnp_out_gate_packed, dim3((unsigned)((rows + 15) / 16), (unsigned)d->nv), dim3(256), (int)rows,
                  d->nv, d->out, d->z, d->norm_w, out_packed);
    } else if (d->flags & VX27_DN_OUT_GATE) {
        const int nrow = (int)(rows * d->nv);
        VX_LAUNCH(ctx, dnp_out_gate, dim3((unsigned)((nrow + 31) / 32)), dim3(256), nrow, d->z, d->norm_w, d->out);
    }
    return 0;
}

extern "C" int vx27_hip_dn_prefill(vx27_hip_ctx *ctx, const vx27_dn_prefill_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    if (dn_prefill_check(d)) return -1;
    void *scr;
    if (vx_ctx_scratch(ctx, vx_dn_prefill_scratch(d), &scr)) return -1;
    return vx_dn_prefill_into(ctx, d, scr);
}

extern "C" int vx27_hip_dn_commit(vx27_hip_ctx *ctx, int B, int T, int nv, int hd, int C, const int *m,
                                  const float *S_ckpt, const float *conv_ckpt, float *S, float *conv_state) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(hd == HD && B >= 1 && T >= 1 && nv >= 1 && C >= 0 && m,
               "vx27_hip_dn_commit: bad arguments (B=%d T=%d nv=%d hd=%d C=%d)", B, T, nv, hd, C);
    VX_REQUIRE(!S_ckpt || S, "vx27_hip_dn_commit: S_ckpt without S");
    VX_REQUIRE(!conv_ckpt || conv_state, "vx27_hip_dn_commit: conv_ckpt without conv_state");
    const size_t s_elems = (size_t)nv * HD * HD, c_elems = (size_t)C * 3;
    const size_t n = std::max(S_ckpt ? s_elems : 0, conv_ckpt ? c_elems : 0);
    if (n == 0) return 0;
    VX_LAUNCH(ctx, dn_commit_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)B), dim3(256), T, s_elems, c_elems, m,
              S_ckpt, conv_ckpt, S, conv_state, ctx->err_flag);
    return 0;
}
