// Gated DeltaNet recurrent decode for gfx950.
//
// Work decomposition: one workgroup per (sequence b, value head vh) with
// 128*R lanes.  Column j of the head's 128x128 state S[i][j] (i = key dim,
// j = value dim) is held by R adjacent lanes, 128/R rows each, in VGPRs for
// all steps of a call.  With R = 1 (large batches) kv[j] = sum_i S[i][j] kn[i]
// and o[j] = sum_i S[i][j] qn[i] are lane-local sums in the reference's row
// order (vx27_deltanet.c:84-101); with R = 2 or 4 (few heads, more lanes per
// head to fill the chip) the R row-block partial sums are added by a
// shuffle butterfly.  S is read and written once per call through a buffer
// resource (one lane offset, scalar row offsets).
//
// The causal conv (vx27_deltanet.c:106-122) is fused when every workgroup
// owns the conv channels it reads, i.e. nv == nqk (q_g, k_g, v_g all belong
// to head g).  With nv > nqk several value heads read the same q/k channels,
// so a channel-parallel conv kernel runs first and writes the activations.
//
// Arithmetic follows the reference op for op: this file is compiled with
// -ffp-contract=off, double accumulations stay double, and each float
// rounding of the reference happens at the same place.  Sums of squares over
// a head's 128 elements are wave trees in double (the reference sums them
// serially; the two can differ in the last bit of the double sum, far below
// the float rounding that follows).
#include "vx_dn.h"
#include "vx_gemv.h"
#include "vx_lds.h"

namespace {






// Gate mapping of vx27_deltanet.c:65-69 for every (token, sequence, value
// head): beta = sigmoid(b), decay = exp(g_log) with g_log = -exp(A_log) *
// softplus(a + dt_bias) (decay as vx27_deltanet.c:82).  A kernel of its own
// so the recurrence kernel carries no transcendental code in its registers.
__global__ __launch_bounds__(256) void dn_gate_kernel(int n, int nv, const float *a, const float *b,
                                                      const float *A_log, const float *dt_bias,
                                                      double2 *gates) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const int vh = e % nv;
    const double beta = 1.0 / (1.0 + exp(-(double)b[e]));
    const double glog = -exp((double)A_log[vh]) * softplus_d((double)a[e] + (double)dt_bias[vh]);
    gates[e] = make_double2(beta, exp(glog));
}



// Sum over the R (<= 16) adjacent lanes of a column, a butterfly on the
// VALU's DPP paths (no LDS crossbar): lane l ^ 1 and l ^ 2 by quad
// permutes, then, the quads being uniform, the other quad of the 8-lane
// half-row by row_half_mirror, and, the half-rows being uniform, the other
// half of the 16-lane row by row_mirror.  Each step adds two values that
// every lane of the pair sees in the same two roles, so all R lanes end with
// the same bits (the association of x + shfl_xor(x, 1), 2, 4, 8).
template <int R>
__device__ __forceinline__ double part_sum(double x) {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8 || R == 16, "part_sum: R lanes per column");
    if (R >= 2) x = x + vx_dpp_f64<0xB1, 0xF>(x);    // quad_perm [1,0,3,2]
    if (R >= 4) x = x + vx_dpp_f64<0x4E, 0xF>(x);    // quad_perm [2,3,0,1]
    if (R >= 8) x = x + vx_dpp_f64<0x141, 0xF>(x);   // row_half_mirror
    if (R >= 16) x = x + vx_dpp_f64<0x140, 0xF>(x);  // row_mirror
    return x;
}

// CS workgroups per (sequence, value head), each owning 128/CS state
// columns with R lanes per column (128/CS * R >= 128 lanes): lane (lcol,
// part) = (tid / R, tid % R) holds rows part*128/R .. of column
// slice*128/CS + lcol.  Lanes tid < 128 own q/k element tid (and its conv
// channels, CS == 1 only); the part-0 lane of a column owns the value channel
// and writes the column's output.  The columns of a head are independent in
// kv = S^T k, the rank-1 update and o = S^T q; the q/k normalisations are
// recomputed by every slice.  With CS > 1 and VX27_DN_OUT_GATE (one step),
// the pre-norm outputs go to o_pre and dn_out_gate finishes them.
template <int R, int CS>
__global__ __launch_bounds__(HD / CS * R) void dn_decode_kernel(DnArgs a) {
    constexpr int RR = HD / R;                 // state rows per lane
    constexpr int NT = HD / CS * R;            // lanes per block
    constexpr int NW = NT / 64;                // waves per block
    static_assert(NT >= HD && NT % 64 == 0, "a block needs a lane per q/k element");
    const int tid = threadIdx.x;
    const int part = tid % R, col = (blockIdx.x % CS) * (HD / CS) + tid / R;
    const int j = tid;                         // q/k element (qk lanes)
    const bool qk_lane = tid < HD;
    const bool v_lane = part == 0;
    const int head = blockIdx.x / CS;
    const int b = head / a.nv;
    const int vh = head % a.nv;
    const int g = vh * a.nqk / a.nv;           // QK head (vx27_qfwd.c:137)
    const int qd = a.nqk * HD, vd = a.nv * HD, C = 2 * qd + vd;

    __shared__ float s_qn[HD], s_kn[HD];
    __shared__ double s_red[4][NW][2];

    // ---- state rows of this lane into registers
    const __amdgpu_buffer_rsrc_t Sr = __builtin_amdgcn_make_buffer_rsrc(
        a.S + ((size_t)b * a.nv + vh) * HD * HD, 0, HD * HD * 4, 0x00020000);
    float Sc[RR];
#pragma unroll
    for (int u = 0; u < RR; u++)
        Sc[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(Sr, col * 4, (part * RR + u) * HD * 4, 0));

    // ---- owned conv channels (fused conv: nv == nqk, so g == vh; CS == 1)
    const bool conv = CS == 1 && a.fused_conv != 0;
    float cq[3] = {0, 0, 0}, ck[3] = {0, 0, 0}, cv[3] = {0, 0, 0};
    float wq[4] = {0, 0, 0, 0}, wk[4] = {0, 0, 0, 0}, wv[4] = {0, 0, 0, 0};
    const size_t chq = (size_t)g * HD + j, chk = (size_t)qd + g * HD + j,
                 chv = (size_t)2 * qd + (size_t)vh * HD + col;
    float *cst = conv ? a.conv_state + (size_t)b * C * 3 : nullptr;
    if (conv) {
        if (qk_lane) {
            load_conv_w(a.conv_w, a.conv_bf16, chq, wq);
            load_conv_w(a.conv_w, a.conv_bf16, chk, wk);
#pragma unroll
            for (int t = 0; t < 3; t++) {
                cq[t] = cst[chq * 3 + t];
                ck[t] = cst[chk * 3 + t];
            }
        }
        if (v_lane) {
            load_conv_w(a.conv_w, a.conv_bf16, chv, wv);
#pragma unroll
            for (int t = 0; t < 3; t++) cv[t] = cst[chv * 3 + t];
        }
    }
    const float nwj = (a.norm_w && qk_lane) ? a.norm_w[j] : 1.0f;     // q/k element weight
    const float nwc = a.norm_w ? a.norm_w[col] : 1.0f;                // output column weight
    const float qs = 1.0f / sqrtf((float)HD);

    // The inputs of step t+1 (gates, and x or q/k/v) are loaded while step t
    // runs: nothing in them depends on the state, so their memory latency
    // leaves the step's dependent chain.
    auto fetch = [&](int t, float &xq, float &xk, float &xv, double2 &gg) {
        const size_t sb = (size_t)t * a.t_step + (size_t)b * a.b_step;
        gg = a.gates[sb * a.nv + vh];   // uniform address: scalar load
        if (conv) {
            const float *x = a.x + sb * C;
            if (qk_lane) {
                xq = x[chq];
                xk = x[chk];
            }
            if (v_lane) xv = x[chv];
        } else {
            if (qk_lane) {
                xq = a.q[sb * a.q_tok + (size_t)g * HD + j];
                xk = a.k[sb * a.k_tok + (size_t)g * HD + j];
            }
            if (v_lane) xv = a.v[sb * a.v_tok + (size_t)vh * HD + col];
        }
    };
    float nq = 0.0f, nk = 0.0f, nvx = 0.0f;
    double2 ng;
    fetch(0, nq, nk, nvx, ng);
    for (int t = 0; t < a.steps; t++) {
        const size_t sb = (size_t)t * a.t_step + (size_t)b * a.b_step;
        const double2 gt = ng;
        const float xq = nq, xk = nk, xv = nvx;
        if (t + 1 < a.steps) fetch(t + 1, nq, nk, nvx, ng);
        // ---- activations of this token
        float qa = 0.0f, ka = 0.0f, va = 0.0f;
        if (conv) {
            if (qk_lane) {
                qa = conv_step(cq, wq, xq);
                ka = conv_step(ck, wk, xk);
            }
            if (v_lane) va = conv_step(cv, wv, xv);
        } else {
            if (qk_lane) {
                qa = xq;
                ka = xk;
            }
            if (v_lane) va = xv;
        }
        if (R > 1) va = __shfl(va, (tid & 63) - part, 64);   // from the column's part-0 lane
        // ---- q/k normalisation chain (skipped when q, k arrive final)
        if (a.flags & VX_DN_QK_READY) {
            if (qk_lane) {
                s_qn[j] = qa;
                s_kn[j] = ka;
            }
        } else {
            if (a.flags & VX27_DN_PRE_RMS) {       // rmsn(x)*(1+w), vx27_qfwd.c:32-39,123
                double sq = (double)qa * (double)qa, sk = (double)ka * (double)ka;
                block_sum2<NW>(sq, sk, s_red[0]);
                const float iq = 1.0f / sqrtf((float)(sq / HD) + 1e-6f);
                const float ik = 1.0f / sqrtf((float)(sk / HD) + 1e-6f);
                qa = (qa * iq) * (nwj + 1.0f);
                ka = (ka * ik) * (nwj + 1.0f);
            }
            if (a.flags & VX27_DN_PRE_L2) {        // l2norm + q/sqrt(hd), vx27_qfwd.c:124-130
                double sq = (double)qa * (double)qa, sk = (double)ka * (double)ka;
                block_sum2<NW>(sq, sk, s_red[1]);
                qa = qa * (1.0f / sqrtf((float)sq + 1e-6f));
                ka = ka * (1.0f / sqrtf((float)sk + 1e-6f));
                qa = qa * qs;
            }
            {                                       // inside step_exact, vx27_deltanet.c:77-80
                double sq = (double)qa * (double)qa, sk = (double)ka * (double)ka;
                block_sum2<NW>(sq, sk, s_red[2]);
                if (qk_lane) {
                    const float qn = qa * (1.0f / sqrtf((float)sq + 1e-6f));
                    s_qn[j] = qn * qs;
                    s_kn[j] = ka * (1.0f / sqrtf((float)sk + 1e-6f));
                }
            }
        }
        __syncthreads();
        const double beta = gt.x, decay = gt.y;
        // ---- S *= decay ; kv = S^T kn   (double, rows in order within the lane)
        double kv = 0.0;
#pragma unroll
        for (int u = 0; u < RR; u += 4) {
            const float4 kn4 = *(const float4 *)&s_kn[part * RR + u];
            const float knv[4] = {kn4.x, kn4.y, kn4.z, kn4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float sd = (float)((double)Sc[u + e] * decay);
                Sc[u + e] = sd;
                kv = kv + (double)sd * (double)knv[e];
            }
        }
        kv = part_sum<R>(kv);
        // ---- S += kn (x) (v - kv)*beta ; o = S^T qn
        // (compiler barrier: kn is re-read from LDS instead of held in registers)
        __asm__ volatile("" ::: "memory");
        const double dl = ((double)va - kv) * beta;
        double o = 0.0;
#pragma unroll
        for (int u = 0; u < RR; u += 4) {
            const float4 kn4 = *(const float4 *)&s_kn[part * RR + u];
            const float4 qn4 = *(const float4 *)&s_qn[part * RR + u];
            const float knv[4] = {kn4.x, kn4.y, kn4.z, kn4.w};
            const float qnv[4] = {qn4.x, qn4.y, qn4.z, qn4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float su = (float)((double)Sc[u + e] + (double)knv[e] * dl);
                Sc[u + e] = su;
                o = o + (double)su * (double)qnv[e];
            }
        }
        o = part_sum<R>(o);
        float of = (float)o;
        // ---- gated output norm (vx27_qfwd.c:147-151)
        if (CS > 1 && (a.flags & VX27_DN_OUT_GATE)) {   // finished by dn_out_gate
            if (v_lane) a.o_pre[((size_t)b * a.nv + vh) * HD + col] = of;
            __syncthreads();   // s_qn/s_kn are rewritten by the next step
            continue;
        }
        if (a.flags & VX27_DN_OUT_GATE) {
            double so = v_lane ? (double)of * (double)of : 0.0, unused = 0.0;
            block_sum2<NW>(so, unused, s_red[3]);
            const float is = 1.0f / sqrtf((float)(so / HD) + 1e-6f);
            const float zz = a.z[sb * a.z_tok + (size_t)vh * HD + col];
            of = ((of * is) * nwc) * silu_f(zz);
        } else {
            __syncthreads();   // s_qn/s_kn are rewritten by the next step
        }
        if (v_lane) {
            if (a.out) a.out[sb * a.out_tok + (size_t)vh * HD + col] = of;
            if (a.out_packed) vx_pack_store(a.out_packed, a.B, b, vh * HD + col, of);
        }
    }

    // ---- write back state and conv state
#pragma unroll
    for (int u = 0; u < RR; u++)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(Sc[u]), Sr, col * 4, (part * RR + u) * HD * 4, 0);
    if (conv) {
        if (qk_lane) {
#pragma unroll
            for (int t = 0; t < 3; t++) {
                cst[chq * 3 + t] = cq[t];
                cst[chk * 3 + t] = ck[t];
            }
        }
        if (v_lane) {
#pragma unroll
            for (int t = 0; t < 3; t++) cst[chv * 3 + t] = cv[t];
        }
    }
}

// One step (q, k given or, with the fused conv (nv == nqk), convolved here
// from x; final with VX_DN_QK_READY, else normalised here per the flags;
// gates given, or mapped here from a, b): one block of 512 lanes per
// (sequence, value head).  Lane (part = tid / 32, c4 = tid % 32)
// holds state rows 8 part .. 8 part + 7 of columns 4 c4 .. 4 c4 + 3, so each
// wave reads and writes two whole 512-byte state rows per instruction, and
// all of a lane's state loads are in flight before any other work.  The
// per-element arithmetic is the general kernel's (decay and the rank-1
// update through double, float state); kv and o are summed in double per
// lane over its rows, then over the 16 parts.  Wave 0 runs the q/k
// normalisation chain for the whole head (two elements per lane, wave sums
// on the DPP paths, no barrier) while the state loads are in flight, and
// finishes the gated output norm (vx27_qfwd.c:147-151).
#ifndef DN_STATE_NT_LD
#define DN_STATE_NT_LD 1    // streaming loads of the state (read once per step)
#endif
#ifndef DN_STATE_NT_ST
#define DN_STATE_NT_ST 1    // streaming stores of the state
#endif
template <bool FC>   // FC: the fused conv (a.fused_conv)
__global__ __launch_bounds__(512) void dn_step_kernel(DnArgs a) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: wave 0's work is a scalar branch
    const int part = tid >> 5, c4 = tid & 31;
    const int head = blockIdx.x, b = head / a.nv, vh = head % a.nv;
    const int g = vh * a.nqk / a.nv;           // QK head (vx27_qfwd.c:137)

    __shared__ float s_qn[HD], s_kn[HD], s_v[HD];
    __shared__ double s_red[8][HD];           // per-wave partial kv, then o
    __shared__ double s_dl[HD];

    // the state rows are loaded first, ahead of every other load and of any
    // wait (the conv's inputs and the gates' scalar loads would otherwise hold
    // them back by a round trip); wave 0's q/k chain waits for its own rows
    float *Sg = a.S + ((size_t)b * a.nv + vh) * HD * HD + (size_t)(8 * part) * HD + 4 * c4;
    float4 S4[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v *sp = (const f4v *)(Sg + (size_t)r * HD);
        const f4v v = DN_STATE_NT_LD ? __builtin_nontemporal_load(sp) : *sp;
        S4[r] = make_float4(v.x, v.y, v.z, v.w);
    }
    // waves 0, 1 and 2 own the head's q, k and v (elements lane and
    // lane + 64 each), so the three chains run side by side; wave 3 maps the
    // gates.  With the fused conv (nv == nqk: g == vh) a wave loads the
    // conv's inputs for its 128 channels, branch-free (each channel's weights
    // as two 8-byte words: the second one repeats the first for bf16), and
    // runs the conv below.
    const int qd = a.nqk * HD, Cc = 2 * qd + a.nv * HD;
    const int own = wave < 3 ? wave : -1;   // 0: q, 1: k, 2: v
    float xa[2] = {0.f, 0.f};
    uint2 cw[2][2];
    float cs[2][3], cx[2];
    if (own >= 0) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int i = lane + 64 * h;
            const size_t ch = own == 0 ? (size_t)g * HD + i : own == 1 ? (size_t)qd + g * HD + i
                                                                       : (size_t)2 * qd + (size_t)vh * HD + i;
            if (FC) {
                const float *x = a.x + (size_t)b * a.b_step * Cc;
                const float *cst = a.conv_state + (size_t)b * Cc * 3;
                const uint2 *wb = (const uint2 *)a.conv_w;
                const size_t w0 = a.conv_bf16 ? ch : 2 * ch;
                cw[h][0] = wb[w0];
                cw[h][1] = wb[a.conv_bf16 ? w0 : w0 + 1];
#pragma unroll
                for (int t = 0; t < 3; t++) cs[h][t] = cst[ch * 3 + t];
                cx[h] = x[ch];
            } else {
                const size_t bs = (size_t)b * a.b_step;
                xa[h] = own == 0 ? a.q[bs * a.q_tok + (size_t)g * HD + i]
                      : own == 1 ? a.k[bs * a.k_tok + (size_t)g * HD + i]
                                 : a.v[bs * a.v_tok + (size_t)vh * HD + i];
            }
        }
    }
    const bool gate = (a.flags & VX27_DN_OUT_GATE) != 0;
    float z0 = 0.f, z1 = 0.f, w0 = 1.f, w1 = 1.f;
    if ((wave == 0 && gate) || (own >= 0 && own < 2 && !(a.flags & VX_DN_QK_READY))) {
        if (wave == 0 && gate) {
            z0 = a.z[(size_t)b * a.b_step * a.z_tok + (size_t)vh * HD + lane];
            z1 = a.z[(size_t)b * a.b_step * a.z_tok + (size_t)vh * HD + lane + 64];
        }
        if (a.norm_w) {
            w0 = a.norm_w[lane];
            w1 = a.norm_w[lane + 64];
        }
    }
    // gates: given (double2), or mapped by wave 3 (vx27_deltanet_gate_params,
    // vx27_deltanet.c:65-69, decay = exp(g_log)) and passed on in LDS
    __shared__ double s_gt[2];
    const size_t ge = (size_t)b * a.b_step * a.nv + vh;
    double beta = 0.0, decay = 0.0;
    if (a.gates) {
        const double2 gt = a.gates[ge];
        beta = gt.x;
        decay = gt.y;
    } else if (wave == 3) {
        const float gbv = a.gb[ge], gav = a.ga[ge], alog = a.A_log[vh], dtb = a.dt_bias[vh];
        const double bt = 1.0 / (1.0 + exp(-(double)gbv));
        const double dc = exp(-exp((double)alog) * softplus_d((double)gav + (double)dtb));
        if (lane == 0) {
            s_gt[0] = bt;
            s_gt[1] = dc;
        }
    }
    if (FC && own >= 0) {   // causal conv + SiLU, the wave's conv state written back
        float *cst = a.conv_state + (size_t)b * Cc * 3;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int i = lane + 64 * h;
            const size_t ch = own == 0 ? (size_t)g * HD + i : own == 1 ? (size_t)qd + g * HD + i
                                                                       : (size_t)2 * qd + (size_t)vh * HD + i;
            float w[4];
            const uint32_t r[4] = {cw[h][0].x, cw[h][0].y, cw[h][1].x, cw[h][1].y};
            conv_w_decode(a.conv_bf16, r, w);
            xa[h] = conv_step(cs[h], w, cx[h]);
#pragma unroll
            for (int t = 0; t < 3; t++) cst[ch * 3 + t] = cs[h][t];
        }
    }
    if (own >= 0 && own < 2 && !(a.flags & VX_DN_QK_READY)) {
        // the q (wave 0) or k (wave 1) normalisation chain (vx27_qfwd.c:119-130
        // per flags, then step_exact's own l2norm, vx27_deltanet.c:77-80):
        // sums of squares in double, each lane's two elements, then the
        // wave's DPP tree; no barriers, and the state loads stay in flight.
        const float qs = 1.0f / sqrtf((float)HD);
        const float nw[2] = {w0, w1};
        const bool isq = own == 0;
        auto sum = [&]() { return vx_wave_sum_f64_dpp((double)xa[0] * (double)xa[0] + (double)xa[1] * (double)xa[1]); };
        if (a.flags & VX27_DN_PRE_RMS) {       // rmsn(x)*(1+w), vx27_qfwd.c:32-39,123
            const double ss = sum();
            const float is = 1.0f / sqrtf((float)(ss / HD) + 1e-6f);
#pragma unroll
            for (int h = 0; h < 2; h++) xa[h] = (xa[h] * is) * (nw[h] + 1.0f);
        }
        if (a.flags & VX27_DN_PRE_L2) {        // l2norm + q/sqrt(hd), vx27_qfwd.c:124-130
            const double ss = sum();
            const float il = 1.0f / sqrtf((float)ss + 1e-6f);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                xa[h] = xa[h] * il;
                if (isq) xa[h] = xa[h] * qs;
            }
        }
        {                                       // inside step_exact, vx27_deltanet.c:77-80
            const double ss = sum();
            const float il = 1.0f / sqrtf((float)ss + 1e-6f);
#pragma unroll
            for (int h = 0; h < 2; h++) xa[h] = isq ? (xa[h] * il) * qs : xa[h] * il;
        }
    }
    if (own >= 0) {   // v goes through LDS too, so its use waits on nothing late
        float *dst = own == 0 ? s_qn : own == 1 ? s_kn : s_v;
#pragma unroll
        for (int h = 0; h < 2; h++) dst[lane + 64 * h] = xa[h];
    }
    __syncthreads();
    if (!a.gates) {
        beta = s_gt[0];
        decay = s_gt[1];
    }

    float kn[8], qn[8];
    {
        const float4 k0 = *(const float4 *)&s_kn[8 * part], k1 = *(const float4 *)&s_kn[8 * part + 4];
        const float4 q0 = *(const float4 *)&s_qn[8 * part], q1 = *(const float4 *)&s_qn[8 * part + 4];
        kn[0] = k0.x; kn[1] = k0.y; kn[2] = k0.z; kn[3] = k0.w;
        kn[4] = k1.x; kn[5] = k1.y; kn[6] = k1.z; kn[7] = k1.w;
        qn[0] = q0.x; qn[1] = q0.y; qn[2] = q0.z; qn[3] = q0.w;
        qn[4] = q1.x; qn[5] = q1.y; qn[6] = q1.z; qn[7] = q1.w;
    }
    // ---- S *= decay ; kv = S^T kn
    double kv[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float *e = (float *)&S4[r];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float sd = (float)((double)e[c] * decay);
            e[c] = sd;
            // (a product of two floats is exact in double: the fused form rounds once, like mul + add)
            kv[c] = __builtin_fma((double)sd, (double)kn[r], kv[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) kv[c] = kv[c] + vx_xor32_f64(kv[c]);
    if (lane < 32) {
#pragma unroll
        for (int c = 0; c < 4; c++) s_red[wave][4 * c4 + c] = kv[c];
    }
    __syncthreads();
    if (tid < HD) {
        double s = s_red[0][tid];
#pragma unroll
        for (int w = 1; w < 8; w++) s = s + s_red[w][tid];
        s_dl[tid] = ((double)s_v[tid] - s) * beta;
    }
    __syncthreads();
    // ---- S += kn (x) dl ; o = S^T qn
    double dl[4];
#pragma unroll
    for (int c = 0; c < 4; c++) dl[c] = s_dl[4 * c4 + c];
    double o[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float *e = (float *)&S4[r];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float su = (float)((double)e[c] + (double)kn[r] * dl[c]);
            e[c] = su;
            o[c] = __builtin_fma((double)su, (double)qn[r], o[c]);
        }
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        f4v *sp = (f4v *)(Sg + (size_t)r * HD);
        const f4v v = {S4[r].x, S4[r].y, S4[r].z, S4[r].w};
        if (DN_STATE_NT_ST) __builtin_nontemporal_store(v, sp); else *sp = v;
    }
#pragma unroll
    for (int c = 0; c < 4; c++) o[c] = o[c] + vx_xor32_f64(o[c]);
    if (lane < 32) {
#pragma unroll
        for (int c = 0; c < 4; c++) s_red[wave][4 * c4 + c] = o[c];
    }
    __syncthreads();
    if (wave != 0) return;
    // ---- wave 0: columns lane and lane + 64
    double oa = s_red[0][lane], ob = s_red[0][lane + 64];
#pragma unroll
    for (int w = 1; w < 8; w++) {
        oa = oa + s_red[w][lane];
        ob = ob + s_red[w][lane + 64];
    }
    float f0 = (float)oa, f1 = (float)ob;
    if (gate) {
        const double so = vx_wave_sum_f64_dpp((double)f0 * (double)f0 + (double)f1 * (double)f1);
        const float is = 1.0f / sqrtf((float)(so / HD) + 1e-6f);
        f0 = ((f0 * is) * w0) * silu_f(z0);
        f1 = ((f1 * is) * w1) * silu_f(z1);
    }
    if (a.out) {
        a.out[(size_t)b * a.b_step * a.out_tok + (size_t)vh * HD + lane] = f0;
        a.out[(size_t)b * a.b_step * a.out_tok + (size_t)vh * HD + lane + 64] = f1;
    }
    if (a.out_packed) {
        vx_pack_store(a.out_packed, a.B, b, vh * HD + lane, f0);
        vx_pack_store(a.out_packed, a.B, b, vh * HD + lane + 64, f1);
    }
}

// One step with a head's columns split over CS workgroups of 128 lanes, for
// few heads (B * nv * CS workgroups spread the state over more of the chip
// than one block per head).  Workgroup (head, slice) owns columns
// slice*128/CS ..; lane (c4, pw) = (lane / PW, lane % PW) of wave w holds
// rows RPL*(w*PW + pw) .. of columns 4 c4 .. 4 c4 + 3 of the slice, so the
// PW lanes sharing columns are adjacent and their kv and o partial sums add
// on the DPP paths (part_sum), then the two waves in LDS.  Wave 0 forms the
// whole head's q, k and v as dn_step_kernel does (each slice recomputes
// them).  Not with the output gate (its norm spans all 128 columns) nor the
// fused conv (the slices would share the q/k channels' conv state, which one
// of them must advance only after all have read it).
template <int CS>
__global__ __launch_bounds__(128) void dn_step_split(DnArgs a) {
    constexpr int NCOL = HD / CS, CG = NCOL / 4, PW = 64 / CG, RPL = HD / (2 * PW);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c4 = lane / PW, pw = lane % PW, part = wave * PW + pw;
    const int head = blockIdx.x / CS, slice = blockIdx.x % CS;
    const int b = head / a.nv, vh = head % a.nv;
    const int g = vh * a.nqk / a.nv;           // QK head (vx27_qfwd.c:137)

    __shared__ float s_qn[HD], s_kn[HD], s_v[HD];
    __shared__ double s_red[2][NCOL];
    __shared__ double s_dl[NCOL];

    float *Sg = a.S + ((size_t)b * a.nv + vh) * HD * HD + (size_t)(RPL * part) * HD + slice * NCOL + 4 * c4;
    float4 S4[RPL];
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v *sp = (const f4v *)(Sg + (size_t)r * HD);
        const f4v v = DN_STATE_NT_LD ? __builtin_nontemporal_load(sp) : *sp;
        S4[r] = make_float4(v.x, v.y, v.z, v.w);
    }
    float qa[2] = {0.f, 0.f}, ka[2] = {0.f, 0.f}, va[2] = {0.f, 0.f};
    if (wave == 0) {
        const size_t bs = (size_t)b * a.b_step;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int i = lane + 64 * h;
            qa[h] = a.q[bs * a.q_tok + (size_t)g * HD + i];
            ka[h] = a.k[bs * a.k_tok + (size_t)g * HD + i];
            va[h] = a.v[bs * a.v_tok + (size_t)vh * HD + i];
        }
    }
    float w0 = 1.f, w1 = 1.f;
    if (wave == 0 && !(a.flags & VX_DN_QK_READY) && a.norm_w) {
        w0 = a.norm_w[lane];
        w1 = a.norm_w[lane + 64];
    }
    const size_t ge = (size_t)b * a.b_step * a.nv + vh;
    double beta, decay;
    if (a.gates) {
        const double2 gt = a.gates[ge];
        beta = gt.x;
        decay = gt.y;
    } else {   // vx27_deltanet_gate_params (vx27_deltanet.c:65-69), decay = exp(g_log)
        const float gbv = a.gb[ge], gav = a.ga[ge], alog = a.A_log[vh], dtb = a.dt_bias[vh];
        beta = 1.0 / (1.0 + exp(-(double)gbv));
        decay = exp(-exp((double)alog) * softplus_d((double)gav + (double)dtb));
    }
    if (wave == 0 && !(a.flags & VX_DN_QK_READY)) {
        // q/k normalisation chain (vx27_qfwd.c:119-130 per flags, then
        // step_exact's own l2norm, vx27_deltanet.c:77-80), as dn_step_kernel
        const float qs = 1.0f / sqrtf((float)HD);
        const float nw[2] = {w0, w1};
        auto sums = [&](double &sq, double &sk) {
            sq = vx_wave_sum_f64_dpp((double)qa[0] * (double)qa[0] + (double)qa[1] * (double)qa[1]);
            sk = vx_wave_sum_f64_dpp((double)ka[0] * (double)ka[0] + (double)ka[1] * (double)ka[1]);
        };
        double sq, sk;
        if (a.flags & VX27_DN_PRE_RMS) {       // rmsn(x)*(1+w), vx27_qfwd.c:32-39,123
            sums(sq, sk);
            const float iq = 1.0f / sqrtf((float)(sq / HD) + 1e-6f);
            const float ik = 1.0f / sqrtf((float)(sk / HD) + 1e-6f);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                qa[h] = (qa[h] * iq) * (nw[h] + 1.0f);
                ka[h] = (ka[h] * ik) * (nw[h] + 1.0f);
            }
        }
        if (a.flags & VX27_DN_PRE_L2) {        // l2norm + q/sqrt(hd), vx27_qfwd.c:124-130
            sums(sq, sk);
            const float iq = 1.0f / sqrtf((float)sq + 1e-6f), ik = 1.0f / sqrtf((float)sk + 1e-6f);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                qa[h] = qa[h] * iq;
                ka[h] = ka[h] * ik;
                qa[h] = qa[h] * qs;
            }
        }
        {                                       // inside step_exact, vx27_deltanet.c:77-80
            sums(sq, sk);
            const float iq = 1.0f / sqrtf((float)sq + 1e-6f), ik = 1.0f / sqrtf((float)sk + 1e-6f);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                qa[h] = (qa[h] * iq) * qs;
                ka[h] = ka[h] * ik;
            }
        }
    }
    if (wave == 0) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            s_qn[lane + 64 * h] = qa[h];
            s_kn[lane + 64 * h] = ka[h];
            s_v[lane + 64 * h] = va[h];
        }
    }
    __syncthreads();

    float kn[RPL], qn[RPL];
#pragma unroll
    for (int r = 0; r < RPL; r += 4) {
        const float4 k4 = *(const float4 *)&s_kn[RPL * part + r], q4 = *(const float4 *)&s_qn[RPL * part + r];
        kn[r] = k4.x; kn[r + 1] = k4.y; kn[r + 2] = k4.z; kn[r + 3] = k4.w;
        qn[r] = q4.x; qn[r + 1] = q4.y; qn[r + 2] = q4.z; qn[r + 3] = q4.w;
    }
    // ---- S *= decay ; kv = S^T kn
    double kv[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        float *e = (float *)&S4[r];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float sd = (float)((double)e[c] * decay);
            e[c] = sd;
            kv[c] = __builtin_fma((double)sd, (double)kn[r], kv[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) kv[c] = part_sum<PW>(kv[c]);
    if (pw == 0) {
#pragma unroll
        for (int c = 0; c < 4; c++) s_red[wave][4 * c4 + c] = kv[c];
    }
    __syncthreads();
    if (tid < NCOL) s_dl[tid] = ((double)s_v[slice * NCOL + tid] - (s_red[0][tid] + s_red[1][tid])) * beta;
    __syncthreads();
    // ---- S += kn (x) dl ; o = S^T qn
    double dl[4];
#pragma unroll
    for (int c = 0; c < 4; c++) dl[c] = s_dl[4 * c4 + c];
    double o[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        float *e = (float *)&S4[r];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float su = (float)((double)e[c] + (double)kn[r] * dl[c]);
            e[c] = su;
            o[c] = __builtin_fma((double)su, (double)qn[r], o[c]);
        }
    }
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        f4v *sp = (f4v *)(Sg + (size_t)r * HD);
        const f4v v = {S4[r].x, S4[r].y, S4[r].z, S4[r].w};
        if (DN_STATE_NT_ST) __builtin_nontemporal_store(v, sp); else *sp = v;
    }
#pragma unroll
    for (int c = 0; c < 4; c++) o[c] = part_sum<PW>(o[c]);
    __syncthreads();   // (s_red's kv values are read out)
    if (pw == 0) {
#pragma unroll
        for (int c = 0; c < 4; c++) s_red[wave][4 * c4 + c] = o[c];
    }
    __syncthreads();
    if (tid < NCOL) {
        const float f = (float)(s_red[0][tid] + s_red[1][tid]);
        const int j = slice * NCOL + tid;
        if (a.out) a.out[(size_t)b * a.b_step * a.out_tok + (size_t)vh * HD + j] = f;
        if (a.out_packed) vx_pack_store(a.out_packed, a.B, b, vh * HD + j, f);
    }
}

// Gated output norm of one step for column-split heads: one block of 128
// lanes per (sequence, value head); out = rmsn_std(o)*norm_w * silu(z)
// (vx27_qfwd.c:147-151) from the pre-norm outputs in o_pre.
__global__ __launch_bounds__(HD) void dn_out_gate(DnArgs a) {
    const int head = blockIdx.x, col = threadIdx.x;
    const int b = head / a.nv, vh = head % a.nv;
    __shared__ double s_red[2][2];
    float of = a.o_pre[(size_t)head * HD + col];
    double so = (double)of * (double)of, unused = 0.0;
    block_sum2<2>(so, unused, s_red);
    const float is = 1.0f / sqrtf((float)(so / HD) + 1e-6f);
    const float zz = a.z[(size_t)b * a.b_step * a.z_tok + (size_t)vh * HD + col];
    of = ((of * is) * a.norm_w[col]) * silu_f(zz);
    if (a.out) a.out[(size_t)b * a.b_step * a.out_tok + (size_t)vh * HD + col] = of;
    if (a.out_packed) vx_pack_store(a.out_packed, a.B, b, vh * HD + col, of);
}

// Channel-parallel causal conv over `steps` tokens: one thread per (b, c),
// state carried in registers; act [steps][B][C] receives silu(conv).
__global__ __launch_bounds__(256) void dn_conv_kernel(ConvArgs a) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)a.B * a.C) return;
    const int b = (int)(id / a.C), c = (int)(id % a.C);
    float w[4], st[3];
    load_conv_w(a.w, a.w_bf16, (size_t)c, w);
    float *sp = a.state + ((size_t)b * a.C + c) * 3;
    st[0] = sp[0]; st[1] = sp[1]; st[2] = sp[2];
    for (int t = 0; t < a.steps; t++) {
        const size_t row = (size_t)t * a.t_step + (size_t)b * a.b_step;
        const size_t e = row * a.C + c;
        a.act[e] = conv_step(st, w, a.x[e]);
        if (a.ckpt) {
            float *ck = a.ckpt + e * 3;
            ck[0] = st[0]; ck[1] = st[1]; ck[2] = st[2];
        }
    }
    sp[0] = st[0]; sp[1] = st[1]; sp[2] = st[2];
}

}  // namespace

// The q/k normalisation chain of dn_decode_kernel for every token up front:
// grid (rows, nqk), block 128 (lane j = element j), row r = t * t_step +
// b * b_step as in the recurrence.  The same operations and the same
// two-wave sums (block_sum2), so the values equal those the recurrence would
// form in its own chain; written as final (q scaled by 1/sqrt(128)).
__global__ __launch_bounds__(HD) void dn_qk_norm_kernel(DnArgs a, float *qo, float *ko) {
    const size_t r = blockIdx.x;
    const int g = blockIdx.y, j = threadIdx.x;
    __shared__ double s_red[3][2][2];
    float qa = a.q[r * a.q_tok + (size_t)g * HD + j];
    float ka = a.k[r * a.k_tok + (size_t)g * HD + j];
    const float qs = 1.0f / sqrtf((float)HD);
    if (a.flags & VX27_DN_PRE_RMS) {       // rmsn(x)*(1+w), vx27_qfwd.c:32-39,123
        const float nwj = a.norm_w[j];
        double sq = (double)qa * (double)qa, sk = (double)ka * (double)ka;
        block_sum2<2>(sq, sk, s_red[0]);
        const float iq = 1.0f / sqrtf((float)(sq / HD) + 1e-6f);
        const float ik = 1.0f / sqrtf((float)(sk / HD) + 1e-6f);
        qa = (qa * iq) * (nwj + 1.0f);
        ka = (ka * ik) * (nwj + 1.0f);
    }
    if (a.flags & VX27_DN_PRE_L2) {        // l2norm + q/sqrt(hd), vx27_qfwd.c:124-130
        double sq = (double)qa * (double)qa, sk = (double)ka * (double)ka;
        block_sum2<2>(sq, sk, s_red[1]);
        qa = qa * (1.0f / sqrtf((float)sq + 1e-6f));
        ka = ka * (1.0f / sqrtf((float)sk + 1e-6f));
        qa = qa * qs;
    }
    {                                       // inside step_exact, vx27_deltanet.c:77-80
        double sq = (double)qa * (double)qa, sk = (double)ka * (double)ka;
        block_sum2<2>(sq, sk, s_red[2]);
        const float qn = qa * (1.0f / sqrtf((float)sq + 1e-6f));
        qo[(r * a.nqk + g) * HD + j] = qn * qs;
        ko[(r * a.nqk + g) * HD + j] = ka * (1.0f / sqrtf((float)sk + 1e-6f));
    }
}

bool vx_dn_single_step(const DnArgs &a) {
#ifndef VX_DN_STEP
#define VX_DN_STEP 1
#endif
    return VX_DN_STEP && a.steps == 1 && ((uintptr_t)a.S & 15) == 0;
}

int vx_dn_recurrence(vx27_hip_ctx *ctx, const DnArgs &a_in) {
    DnArgs a = a_in;
    if (a.t_step == 0 && a.b_step == 0) {   // decode layout [steps][B]
        a.t_step = a.B;
        a.b_step = 1;
    }
    VX_REQUIRE(!a.fused_conv || a.nv == a.nqk, "dn recurrence: fused conv needs nv == nqk");
    // Spread few heads over the 256 CUs: split each head's columns over CS
    // workgroups (not with the fused conv, whose q/k channels one block owns,
    // nor with a per-step output norm over several steps), else split each
    // column's rows over R lanes of one workgroup.
    const int heads = a.B * a.nv;
    const bool gate = (a.flags & VX27_DN_OUT_GATE) != 0;
    if (vx_dn_single_step(a)) {
        // few heads, no fused conv and no output gate: columns split over CS workgroups
        const int CS = (gate || a.fused_conv || heads > 128) ? 1 : heads <= 32 ? 8 : heads <= 64 ? 4 : 2;
        if (CS > 1) {
            const dim3 grid((unsigned)(heads * CS));
            if (CS == 8) VX_LAUNCH_NAMED(ctx, "dn_step_split", dn_step_split<8>, grid, dim3(128), a);
            else if (CS == 4) VX_LAUNCH_NAMED(ctx, "dn_step_split", dn_step_split<4>, grid, dim3(128), a);
            else VX_LAUNCH_NAMED(ctx, "dn_step_split", dn_step_split<2>, grid, dim3(128), a);
            return 0;
        }
        if (a.fused_conv)
            VX_LAUNCH_NAMED(ctx, "dn_step_kernel", dn_step_kernel<true>, dim3((unsigned)heads), dim3(512), a);
        else
            VX_LAUNCH_NAMED(ctx, "dn_step_kernel", dn_step_kernel<false>, dim3((unsigned)heads), dim3(512), a);
        return 0;
    }
    VX_REQUIRE(a.gates != nullptr, "internal: the multi-step recurrence needs mapped gates");
    if (a.qk_buf && !a.fused_conv && !(a.flags & VX_DN_QK_READY)) {
        const size_t rows = (size_t)a.steps * a.B;
        float *qo = a.qk_buf, *ko = a.qk_buf + rows * a.nqk * HD;
        VX_LAUNCH(ctx, dn_qk_norm_kernel, dim3((unsigned)rows, (unsigned)a.nqk), dim3(HD), a, qo, ko);
        a.q = qo;
        a.k = ko;
        a.q_tok = a.k_tok = (size_t)a.nqk * HD;
        a.flags |= VX_DN_QK_READY;
    }
    // (With the output gate, one workgroup per head keeps the norm in the
    // kernel; splitting would need the dn_out_gate launch, which costs more
    // than the split gains.)
    int CS = 1;
    if (!a.fused_conv && !gate)
        while (heads * CS < 512 && CS < 8) CS *= 2;
#if defined(VX_DN_CS)
    if (CS > 1 || VX_DN_CS == 1) CS = VX_DN_CS;   // build-time override for tuning sweeps
#endif
    const dim3 grid((unsigned)(heads * CS));
    switch (CS) {
        case 1:
            if (heads >= 1024)
                VX_LAUNCH_NAMED(ctx, "dn_decode_kernel", (dn_decode_kernel<1, 1>), grid, dim3(HD), a);
            else if (heads >= 256)
                VX_LAUNCH_NAMED(ctx, "dn_decode_kernel", (dn_decode_kernel<2, 1>), grid, dim3(HD * 2), a);
            else
                VX_LAUNCH_NAMED(ctx, "dn_decode_kernel", (dn_decode_kernel<4, 1>), grid, dim3(HD * 4), a);
            break;
#ifndef VX_DN_RS
#define VX_DN_RS 2   // lanes per column = CS * VX_DN_RS
#endif
        case 2:
            VX_LAUNCH_NAMED(ctx, "dn_decode_kernel", (dn_decode_kernel<2 * VX_DN_RS, 2>), grid, dim3(HD * VX_DN_RS), a);
            break;
        case 4:
            VX_LAUNCH_NAMED(ctx, "dn_decode_kernel", (dn_decode_kernel<4 * VX_DN_RS, 4>), grid, dim3(HD * VX_DN_RS), a);
            break;
        default:
            VX_LAUNCH_NAMED(ctx, "dn_decode_kernel", (dn_decode_kernel<8 * VX_DN_RS, 8>), grid, dim3(HD * VX_DN_RS), a);
            break;
    }
    DnArgs f = a;
    if (CS > 1 && gate) VX_LAUNCH(ctx, dn_out_gate, dim3((unsigned)heads), dim3(HD), f);
    return 0;
}

extern "C" int vx27_hip_dn_decode(vx27_hip_ctx *ctx, const vx27_dn_desc *d) {
    if (vx_ctx_enter(ctx)) return -1;
    VX_REQUIRE(d != nullptr, "vx27_hip_dn_decode: null descriptor");
    VX_REQUIRE(d->hd == HD, "vx27_hip_dn_decode: hd must be 128 (got %d)", d->hd);
    VX_REQUIRE(d->B >= 1 && d->nqk >= 1 && d->nv >= 1 && d->steps >= 1,
               "vx27_hip_dn_decode: B, nqk, nv, steps must be >= 1");
    VX_REQUIRE(d->nv % d->nqk == 0, "vx27_hip_dn_decode: nv must be a multiple of nqk (nqk=%d nv=%d)",
               d->nqk, d->nv);
    VX_REQUIRE((d->flags & ~15u) == 0, "vx27_hip_dn_decode: unknown flags %#x", d->flags);
    VX_REQUIRE(d->S && d->out && d->a && d->b && d->A_log && d->dt_bias,
               "vx27_hip_dn_decode: S, out, a, b, A_log, dt_bias are required");
    const bool conv = (d->flags & VX27_DN_CONV) != 0;
    if (conv) {
        VX_REQUIRE(d->x && d->conv_state && d->conv_w, "vx27_hip_dn_decode: conv needs x, conv_state, conv_w");
        VX_REQUIRE(d->conv_w_dtype == VX27_F32 || d->conv_w_dtype == VX27_BF16,
                   "vx27_hip_dn_decode: conv_w_dtype must be VX27_F32 or VX27_BF16");
        VX_REQUIRE(((uintptr_t)d->conv_w & 15) == 0, "vx27_hip_dn_decode: conv_w must be 16-byte aligned");
    } else {
        VX_REQUIRE(d->q && d->k && d->v, "vx27_hip_dn_decode: q, k, v are required without conv");
    }
    if (d->flags & (VX27_DN_PRE_RMS | VX27_DN_OUT_GATE))
        VX_REQUIRE(d->norm_w != nullptr, "vx27_hip_dn_decode: norm_w required by PRE_RMS/OUT_GATE");
    if (d->flags & VX27_DN_OUT_GATE) VX_REQUIRE(d->z != nullptr, "vx27_hip_dn_decode: z required by OUT_GATE");

    const int qd = d->nqk * HD, vd = d->nv * HD, C = 2 * qd + vd;
    DnArgs a = {};
    a.B = d->B; a.nqk = d->nqk; a.nv = d->nv; a.steps = d->steps; a.flags = d->flags;
    a.S = d->S; a.conv_state = d->conv_state; a.conv_w = d->conv_w;
    a.conv_bf16 = d->conv_w_dtype == VX27_BF16;
    a.norm_w = d->norm_w; a.z = d->z; a.out = d->out;
    const bool sep_conv = conv && d->nv != d->nqk;
    if (!conv) {
        a.q = d->q; a.k = d->k; a.v = d->v;
        a.q_tok = (size_t)qd; a.k_tok = (size_t)qd; a.v_tok = (size_t)vd;
    } else if (!sep_conv) {
        a.fused_conv = 1;
        a.x = d->x;
    }
    // scratch: gates [steps][B][nv] double2, pre-norm outputs [B][nv][128],
    // then (unfused conv) activations
    const size_t n_gate = (size_t)d->steps * d->B * d->nv;
    const size_t gate_bytes = (n_gate * sizeof(double2) + 255) & ~(size_t)255;
    const size_t opre_bytes = ((size_t)d->B * vd * sizeof(float) + 255) & ~(size_t)255;
    const size_t act_bytes = ((sep_conv ? (size_t)d->steps * d->B * C : 0) * sizeof(float) + 255) & ~(size_t)255;
    const size_t qk_bytes = d->steps > 1 ? vx_dn_qk_bytes(d->steps, d->B, d->nqk) : 0;
    void *scr;
    if (vx_ctx_scratch(ctx, gate_bytes + opre_bytes + act_bytes + qk_bytes, &scr)) return -1;
    if (qk_bytes) a.qk_buf = (float *)((char *)scr + gate_bytes + opre_bytes + act_bytes);
    double2 *gates = (double2 *)scr;
    a.o_pre = (float *)((char *)scr + gate_bytes);
    a.ga = d->a; a.gb = d->b; a.A_log = d->A_log; a.dt_bias = d->dt_bias;
    if (!vx_dn_single_step(a)) {
        VX_LAUNCH(ctx, dn_gate_kernel, dim3((unsigned)((n_gate + 255) / 256)), dim3(256), (int)n_gate, d->nv, d->a,
                  d->b, d->A_log, d->dt_bias, gates);
        a.gates = gates;
    }
    if (sep_conv) {
        // shared q/k channels: convolve all channels first
        float *act = (float *)((char *)scr + gate_bytes + opre_bytes);
        ConvArgs ca = {d->B, C, d->steps, a.conv_bf16, d->conv_state, d->conv_w, d->x, act, d->B, 1, nullptr};
        const size_t nthr = (size_t)d->B * C;
        VX_LAUNCH(ctx, dn_conv_kernel, dim3((unsigned)((nthr + 255) / 256)), dim3(256), ca);
        a.q = act; a.k = act + qd; a.v = act + 2 * qd;
        a.q_tok = a.k_tok = a.v_tok = (size_t)C;
    }
    a.z_tok = (size_t)vd;
    a.out_tok = (size_t)vd;
    return vx_dn_recurrence(ctx, a);
}

int vx_dn_gates(vx27_hip_ctx *ctx, size_t n, int nv, const float *ga, const float *gb, const float *A_log,
                const float *dt_bias, double2 *gates) {
    VX_LAUNCH(ctx, dn_gate_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), (int)n, nv, ga, gb, A_log, dt_bias,
              gates);
    return 0;
}

int vx_dn_conv(vx27_hip_ctx *ctx, const ConvArgs &ca) {
    const size_t nthr = (size_t)ca.B * ca.C;
    VX_LAUNCH(ctx, dn_conv_kernel, dim3((unsigned)((nthr + 255) / 256)), dim3(256), ca);
    return 0;
}
