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
constexpr int KP = HD + 4;        // padded fp32 row of kn in LDS
constexpr int QP = HD + 8;        // padded bf16 row of qn in LDS
constexpr int PP = CH + 8;        // padded bf16 row of P in LDS

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

__global__ __launch_bounds__(256) void dnp_prep(PrepArgs p) {
    const int c = blockIdx.x, vh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, m = lane & 15;
    const int qh = vh * p.nqk / p.nv;
    const int t0 = c * CH;
    const int nvalid = min(CH, p.T - t0);

    __shared__ float kn_f[CH][KP];        // kn (fp32); later -W
    __shared__ uint16_t qn_b[CH][QP];     // qn (bf16); later P (bf16, row stride PP); later v
    __shared__ float A_s[CH][CH];
    __shared__ double gam_s[CH];
    __shared__ float beta_s[CH], eg_s[CH], egc_s[CH];   // beta, e^gam_t, e^(gam_C - gam_t)

    // gates and the cumulative log-decay (wave 0, lane = token); masked
    // tokens get beta = 0 and g = 0, which leaves U and S unchanged
    if (wave == 0) {
        double beta = 0.0, glog = 0.0;
        if (lane < nvalid) {
            const size_t e = ((size_t)b * p.T + t0 + lane) * p.nv + vh;
            beta = 1.0 / (1.0 + exp(-(double)p.b[e]));
            glog = -exp((double)p.A_log[vh]) * softplus_d((double)p.a[e] + (double)p.dt_bias[vh]);
        }
        double s = glog;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const double o = __shfl_up(s, off, 64);
            if (lane >= off) s += o;
        }
        const double sC = __shfl(s, 63, 64);
        gam_s[lane] = s;
        beta_s[lane] = (float)beta;
        eg_s[lane] = (float)exp(s);
        egc_s[lane] = (float)exp(sC - s);
    }

    // q and k rows, one token per lane (wave 1: k, wave 2: q): the lane reads
    // its token's 256 bytes and sums the squares itself, so no cross-lane
    // reduction is needed
    const float qscale = 1.0f / sqrtf((float)HD);
    uint4 vrow[16];   // wave 3: v row of token `lane`, parked in LDS once qn_b is free
    if (wave == 3) {
        if (lane < nvalid) {
            const uint16_t *src = p.v + (((size_t)b * p.T + t0 + lane) * p.nv + vh) * HD;
#pragma unroll
            for (int j = 0; j < 16; j++) vrow[j] = *(const uint4 *)(src + 8 * j);
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) vrow[j] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    if (wave == 1 || wave == 2) {
        const int t = lane;
        uint4 raw[16];
        if (t < nvalid) {
            const uint16_t *src = (wave == 1 ? p.k : p.q) + (((size_t)b * p.T + t0 + t) * p.nqk + qh) * HD;
#pragma unroll
            for (int j = 0; j < 16; j++) raw[j] = *(const uint4 *)(src + 8 * j);
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) raw[j] = make_uint4(0u, 0u, 0u, 0u);
        }
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
        const float inv = 1.0f / sqrtf((float)ss + 1e-6f);
        if (wave == 1) {
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
                float f[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    f[2 * e] = vx_bf16_to_f32((uint16_t)w4[e]) * inv;
                    f[2 * e + 1] = vx_bf16_to_f32((uint16_t)(w4[e] >> 16)) * inv;
                }
                *(float4 *)&kn_f[t][8 * j] = make_float4(f[0], f[1], f[2], f[3]);
                *(float4 *)&kn_f[t][8 * j + 4] = make_float4(f[4], f[5], f[6], f[7]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
                uint32_t o4[4];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    o4[e] = pack2((vx_bf16_to_f32((uint16_t)w4[e]) * inv) * qscale,
                                  (vx_bf16_to_f32((uint16_t)(w4[e] >> 16)) * inv) * qscale);
                *(uint4 *)&qn_b[t][8 * j] = make_uint4(o4[0], o4[1], o4[2], o4[3]);
            }
        }
    }
    __syncthreads();

    char *rec = p.rec + (((size_t)b * p.nv + vh) * p.NC + c) * REC;
    const double gamC = gam_s[CH - 1];
    if (tid == 0) *(float *)(rec + R_GC) = (float)exp(gamC);

    // K K^T and Q K^T for row block `wave`; Qe tiles on the way
    floatx4_t acck[4], accq[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
        acck[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
        accq[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    }
    const int rowA = wave * 16 + m;
    const float egA = eg_s[rowA];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const int d0 = 32 * ks + 8 * g;
        const uint4 qa = *(const uint4 *)&qn_b[rowA][d0];
        const bf16x8_t aq = as_bf16x8(qa);
        const bf16x8_t ak = as_bf16x8(pack8(&kn_f[rowA][d0]));
        {   // Qe tile (row block wave, k-step ks): e^gam_t * qn
            const uint16_t *qs = (const uint16_t *)&qa;
            float f[8];
#pragma unroll
            for (int e = 0; e < 8; e++) f[e] = egA * vx_bf16_to_f32(qs[e]);
            *(uint4 *)(rec + R_QE + ((size_t)(wave * 4 + ks) * 64 + lane) * 16) = pack8(f);
        }
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
            const bf16x8_t bk = as_bf16x8(pack8(&kn_f[nb * 16 + m][d0]));
            acck[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, bk, acck[nb], 0, 0, 0);
            accq[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq, bk, accq[nb], 0, 0, 0);
        }
    }
    // Kt^T tiles: rows = key dims (8 blocks), k = tokens (2 steps); 4 per wave
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int tile = wave * 4 + j, rb = tile >> 1, ks = tile & 1;
        const int i = rb * 16 + m;
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int t = 32 * ks + 8 * g + e;
            f[e] = egc_s[t] * kn_f[t][i];
        }
        *(uint4 *)(rec + R_KT + ((size_t)tile * 64 + lane) * 16) = pack8(f);
    }
    __syncthreads();   // qn_b is reused for P below

    // A (fp32, for the solve) and P (bf16, staged for its operand tiles)
    uint16_t *P_b = &qn_b[0][0];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int s = wave * 16 + 4 * g + i, r = nb * 16 + m;
            const float ed = r <= s ? expf((float)(gam_s[s] - gam_s[r])) : 0.0f;
            A_s[s][r] = r < s ? beta_s[s] * ed * acck[nb][i] : 0.0f;
            P_b[s * PP + r] = vx_f32_to_bf16(ed * accq[nb][i]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const uint4 v = *(const uint4 *)&P_b[rowA * PP + 32 * ks + 8 * g];
        *(uint4 *)(rec + R_P + ((size_t)(wave * 2 + ks) * 64 + lane) * 16) = v;
    }
    __syncthreads();   // P is read out; qn_b now holds v (bf16 rows)
    if (wave == 3) {
#pragma unroll
        for (int j = 0; j < 16; j++) *(uint4 *)&qn_b[lane][8 * j] = vrow[j];
    }
    __syncthreads();

    // forward substitution x = (I + A)^-1 rhs, one column per thread:
    // columns 0..127 of beta V (-> Ut), 128..255 of beta e^gam K (-> W)
    float x[CH];
    if (tid < HD) {
#pragma unroll
        for (int t = 0; t < CH; t++) {
            x[t] = beta_s[t] * vx_bf16_to_f32(qn_b[t][tid]);
        }
    } else {
#pragma unroll
        for (int t = 0; t < CH; t++) x[t] = (beta_s[t] * eg_s[t]) * kn_f[t][tid - HD];
    }
    // blocked forward substitution over four 16-row blocks: first the rows of
    // a block against every earlier block (four independent partial sums per
    // row, so the rows proceed in parallel), then the 16-row triangle
#pragma unroll
    for (int blk = 0; blk < 4; blk++) {
        if (blk > 0) {
#pragma unroll
            for (int ii = 0; ii < 16; ii++) {
                const int i = 16 * blk + ii;
                float a0 = x[i], a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
                for (int k4 = 0; k4 < 16 * blk; k4 += 4) {
                    const float4 a4 = *(const float4 *)&A_s[i][k4];
                    a0 -= a4.x * x[k4];
                    a1 -= a4.y * x[k4 + 1];
                    a2 -= a4.z * x[k4 + 2];
                    a3 -= a4.w * x[k4 + 3];
                }
                x[i] = (a0 + a1) + (a2 + a3);
            }
        }
#pragma unroll
        for (int ii = 1; ii < 16; ii++) {
            const int i = 16 * blk + ii;
            float acc = x[i];
#pragma unroll
            for (int k = 16 * blk; k < i; k++) acc -= A_s[i][k] * x[k];
            x[i] = acc;
        }
    }
    if (tid < HD) {
        // Ut column tid in C-layout tiles [rb][cs][lane (g,n)][i]
        const int cs = tid >> 4, n = tid & 15;
        float *ut = (float *)(rec + R_UT);
#pragma unroll
        for (int t = 0; t < CH; t++) {
            const int rb = t >> 4, gg = (t & 15) >> 2, i = t & 3;
            ut[(((size_t)rb * 8 + cs) * 64 + gg * 16 + n) * 4 + i] = x[t];
        }
    }
    __syncthreads();   // every read of kn_f is done
    if (tid >= HD) {
#pragma unroll
        for (int t = 0; t < CH; t++) kn_f[t][tid - HD] = -x[t];
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
        *(uint4 *)(rec + R_NW + ((size_t)(wave * 4 + ks) * 64 + lane) * 16) = pack8(&kn_f[rowA][32 * ks + 8 * g]);
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
