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
//           Each wave streams its own operand tiles of the chunk two ahead
//           straight into LDS (two slots, explicit vmcnt waits, no barrier
//           for the hand-off).  The 8 slices of a head are placed on one XCD so the records they
//           share are read from HBM once.
//
// Operand tiles ([rows/16][k/32][64 lanes][8] bf16) follow the MFMA operand
// layout of v_mfma_f32_16x16x32_bf16: lane (g = l/16, m = l%16) of an A tile
// holds A[m][8g..8g+7]; a wave's tile is 1 KiB of contiguous memory.
#include "vx_dn.h"
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

// A wave's operands of one chunk: 15 tiles of 1 KiB in its record, staged in
// LDS in this order: -W (rows 16w..16w+15, 4 k-steps), e^gam Q (same rows),
// Kt^T (row blocks 2w, 2w+1, 2 k-steps each), P (rows 16w.., 2 k-steps) and
// the wave's Ut block of the slice; then the record's last 256 bytes, whose
// first float is e^gam_C.
constexpr int OPS_TILES = 15;
constexpr int OPS_LOADS = OPS_TILES + 1;   // load instructions per wave and chunk
constexpr uint32_t OPS_WAVE = OPS_TILES * 1024 + 256;
constexpr uint32_t OPS_BUF = 4 * OPS_WAVE;

__device__ __forceinline__ uint32_t ops_src(int j, int wave, int slice) {
    return j < 4    ? (uint32_t)(R_NW + (wave * 4 + j) * 1024)
           : j < 8  ? (uint32_t)(R_QE + (wave * 4 + j - 4) * 1024)
           : j < 12 ? (uint32_t)(R_KT + (wave * 4 + j - 8) * 1024)
           : j < 14 ? (uint32_t)(R_P + (wave * 2 + j - 12) * 1024)
                    : (uint32_t)(R_UT + (wave * 8 + slice) * 1024);
}

// Starts group q (0..3) of the wave's 16 direct-to-LDS loads of record
// `rec` into its slot at LDS address `lds` (tiles 4q .. 4q+3, the last
// group ending with the record's final 256 bytes).  Each wave reads back only
// what it loaded itself, so the hand-off needs this wave's vmcnt wait and no
// barrier.  The groups are issued at spread-out points of a chunk step: the
// load path drains 60 KiB per chunk per CU, and issuing all of it at once
// stalls the wave.
__device__ __forceinline__ void fetch_ops(const char *rec, uint32_t lds, int wave, int slice, int lane, int q) {
#pragma unroll
    for (int j = 4 * q; j < 4 * q + 4 && j < OPS_TILES; j++)
        vx_dma16(rec, ops_src(j, wave, slice) + (uint32_t)lane * 16, lds + (uint32_t)j * 1024);
    if (q == 3) vx_dma4(rec, (uint32_t)R_GC + (uint32_t)lane * 4, lds + OPS_TILES * 1024);
}
__device__ __forceinline__ void fetch_ops(const char *rec, uint32_t lds, int wave, int slice, int lane) {
#pragma unroll
    for (int q = 0; q < 4; q++) fetch_ops(rec, lds, wave, slice, lane, q);
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

    __shared__ __align__(16) char ops_l[2][OPS_BUF];   // chunk operands, two chunks in flight
    __shared__ uint16_t S_l[16][HD + 8];   // S slice, bf16, [column][key dim]
    __shared__ uint16_t U_l[16][CH + 8];   // U slice, bf16, [column][token]

    const char *rec0 = vx_uniform_ptr(p.rec + ((size_t)b * p.nv + vh) * p.NC * REC);
    const uint32_t ops_w = vx_lds_addr(ops_l) + (uint32_t)wave * OPS_WAVE;
    fetch_ops(rec0, ops_w, wave, slice, lane);
    if (p.NC > 1) fetch_ops(rec0 + REC, ops_w + OPS_BUF, wave, slice, lane);

    // state rows 32w .. 32w+31 (row blocks 2w, 2w+1) of the slice, C layout
    float *Sg = p.S + ((size_t)b * p.nv + vh) * HD * HD;
    floatx4_t S[2];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) S[r][i] = Sg[(size_t)((2 * wave + r) * 16 + 4 * g + i) * HD + col];
    // take the state loads' wait here, once, rather than inside the loop
    __asm__ volatile("" ::"v"(S[0]), "v"(S[1]));

    for (int c = 0; c < p.NC; c++) {
        // The chunk's dependent chain S -> U -> S' starts at once; the operand
        // reads go into its shadow (before the barrier whose far side needs
        // them), and chunk c+2's loads start once this slot is read out.
        // S (bf16) -> LDS as [column][key dim]
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int d = (2 * wave + r) * 16 + 4 * g;
            *(uint2 *)&S_l[n][d] = make_uint2(pack2(S[r][0], S[r][1]), pack2(S[r][2], S[r][3]));
        }
        // chunk c's loads have landed once at most the loads issued after its
        // last group are still outstanding: groups 0 and 1 of chunk c+1 (8
        // loads; loads complete in issue order)
        if (c + 1 < p.NC)
            __asm__ volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // groups 2 and 3 of chunk c+1 go out in this step's first half
        const bool fill1 = c >= 1 && c + 1 < p.NC;   // (chunks 0 and 1 are loaded whole up front)
        const char *rec1 = rec0 + (size_t)(c + 1) * REC;
        const uint32_t slot1 = ops_w + (uint32_t)((c + 1) & 1) * OPS_BUF;
        if (fill1) fetch_ops(rec1, slot1, wave, slice, lane, 2);
        const char *slot = &ops_l[c & 1][wave * OPS_WAVE];
        const uint4 *t = (const uint4 *)slot + lane;
        uint4 nw[4], qe[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            nw[ks] = t[ks * 64];
            qe[ks] = t[(4 + ks) * 64];
        }
        const uint4 utu = t[14 * 64];
        const float gc = *(const float *)(slot + OPS_TILES * 1024);
        vx_lds_barrier();   // S_l complete (and this wave's operand reads returned)
        if (fill1) fetch_ops(rec1, slot1, wave, slice, lane, 3);
        bf16x8_t sb[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) sb[ks] = as_bf16x8(*(const uint4 *)&S_l[n][32 * ks + 8 * g]);
        // U = Ut - W S for tokens 16w .. 16w+15, and the e^gam Q S part of O,
        // as independent two-MFMA chains (the dependent-MFMA latency, not the
        // issue rate, bounds this loop)
        floatx4_t U0 = (floatx4_t){__uint_as_float(utu.x), __uint_as_float(utu.y), __uint_as_float(utu.z), __uint_as_float(utu.w)};
        floatx4_t U1 = {0.f, 0.f, 0.f, 0.f};
        floatx4_t O0 = {0.f, 0.f, 0.f, 0.f}, O1 = {0.f, 0.f, 0.f, 0.f};
        U0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(nw[0]), sb[0], U0, 0, 0, 0);
        U1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(nw[1]), sb[1], U1, 0, 0, 0);
        O0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qe[0]), sb[0], O0, 0, 0, 0);
        O1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qe[1]), sb[1], O1, 0, 0, 0);
        U0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(nw[2]), sb[2], U0, 0, 0, 0);
        U1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(nw[3]), sb[3], U1, 0, 0, 0);
        O0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qe[2]), sb[2], O0, 0, 0, 0);
        O1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qe[3]), sb[3], O1, 0, 0, 0);
        const floatx4_t U = U0 + U1;
        *(uint2 *)&U_l[n][wave * 16 + 4 * g] = make_uint2(pack2(U[0], U[1]), pack2(U[2], U[3]));
        uint4 kt[4], pp[2];
#pragma unroll
        for (int j = 0; j < 4; j++) kt[j] = t[(8 + j) * 64];
        pp[0] = t[12 * 64];
        pp[1] = t[13 * 64];
        vx_lds_barrier();   // U_l complete; every read of this slot has returned
        // the slot is free: refill it with chunk c+2, groups 0 and 1 in this
        // step, 2 and 3 in the next
        const bool refill = c + 2 < p.NC;
        const char *rec2 = rec0 + (size_t)(c + 2) * REC;
        const uint32_t slot2 = ops_w + (uint32_t)(c & 1) * OPS_BUF;
        if (refill) fetch_ops(rec2, slot2, wave, slice, lane, 0);
        bf16x8_t ub[2];
#pragma unroll
        for (int ks = 0; ks < 2; ks++) ub[ks] = as_bf16x8(*(const uint4 *)&U_l[n][32 * ks + 8 * g]);
        // O += P U (two more independent MFMAs), then the two chains merge
        O0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(pp[0]), ub[0], O0, 0, 0, 0);
        O1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(pp[1]), ub[1], O1, 0, 0, 0);
        if (refill) fetch_ops(rec2, slot2, wave, slice, lane, 1);
        // S = e^gam_C S + Kt^T U: per row block, two independent MFMAs
#pragma unroll
        for (int r = 0; r < 2; r++) {
            floatx4_t Sa = S[r] * gc, Sb = {0.f, 0.f, 0.f, 0.f};
            Sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kt[2 * r]), ub[0], Sa, 0, 0, 0);
            Sb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kt[2 * r + 1]), ub[1], Sb, 0, 0, 0);
            S[r] = Sa + Sb;
        }
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

}  // namespace

extern "C" int vx27_hip_dn_prefill(vx27_hip_ctx *ctx, const vx27_dn_prefill_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d, "vx27_hip_dn_prefill: null descriptor");
    VX_REQUIRE(d->hd == HD, "vx27_hip_dn_prefill: head_dim must be 128 (got %d)", d->hd);
    VX_REQUIRE(d->B >= 1 && d->T >= 1 && d->nqk >= 1 && d->nv >= d->nqk && d->nv % d->nqk == 0 && d->nv <= 4096,
               "vx27_hip_dn_prefill: bad sizes B=%d T=%d nqk=%d nv=%d", d->B, d->T, d->nqk, d->nv);
    VX_REQUIRE(d->flags == 0, "vx27_hip_dn_prefill: flags must be 0");
    VX_REQUIRE(d->S && d->q && d->k && d->v && d->a && d->b && d->A_log && d->dt_bias && d->out,
               "vx27_hip_dn_prefill: null pointer");
    const int NC = (d->T + CH - 1) / CH;
    const size_t n_rec = (size_t)d->B * d->nv * NC;
    const size_t gc_off = (n_rec * REC + 255) & ~(size_t)255;
    void *scr;
    if (vx_ctx_scratch(ctx, gc_off + n_rec * sizeof(float), &scr)) return -1;
    PrepArgs pa{d->T, d->nqk, d->nv, NC, d->q, d->k, d->v, d->a, d->b, d->A_log, d->dt_bias,
                (char *)scr, (float *)((char *)scr + gc_off)};
    VX_LAUNCH(ctx, dnp_prep, dim3((unsigned)NC, (unsigned)d->nv, (unsigned)d->B), dim3(256), pa);
    ScanArgs sa{d->T, d->nv, NC, (d->nv % 8) == 0, (const char *)scr, (const float *)((char *)scr + gc_off),
                d->S, d->out};
    VX_LAUNCH(ctx, dnp_scan, dim3((unsigned)(d->nv * NSLICE), (unsigned)d->B), dim3(256), sa);
    return 0;
}
