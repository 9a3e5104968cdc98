"""Helpers shared by the GPU parity tests: oracle runs over the same inputs."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np

from oracle import oracle as O


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def oracle_dn(d, flags, B, nqk, nv, steps, hd=128, threads=None):
    """Run the oracle's DeltaNet decode (orc_dn_run) on dict d of a workload;
    returns (out [steps][B][nv][hd], S, conv_state)."""
    S = np.ascontiguousarray(d["S0"], np.float32).copy()
    C_ = 2 * nqk * hd + nv * hd
    conv = np.ascontiguousarray(d.get("conv0", np.zeros((B, C_, 3), np.float32)), np.float32).copy()
    out = np.empty((steps, B, nv, hd), np.float32)
    keep = {}

    def p(name):
        if name not in d or d[name] is None:
            return None
        keep[name] = np.ascontiguousarray(d[name], np.float32)
        return keep[name].ctypes.data

    r = O.DnRunArgs(B, nqk, nv, hd, steps, flags, threads or O.default_threads(),
                    S.ctypes.data, conv.ctypes.data, p("conv_w"), p("x"), p("q"), p("k"), p("v"),
                    p("a"), p("b"), p("A_log"), p("dt_bias"), p("norm_w"), p("z"), out.ctypes.data)
    secs = O.lib().orc_dn_run(C.byref(r))
    return out, S, conv, secs


def maxabs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def bitexact_frac(a, b):
    return float(np.mean(np.asarray(a) == np.asarray(b)))


def oracle_gqa_decode(d, Lcap, threads=None, no_gate=False, rope_dim=64):
    """Oracle for one gated-GQA decode step of every sequence of workload d
    (gqa_decode): bf16 cache [B][Lcap][n_kv][hd] holding the prefix, append at
    pos, attend 0..pos (double dot), gate.  Returns (out [B][n_q][hd],
    appended k row, v row) per sequence."""
    qg = np.ascontiguousarray(d["qg"], np.float32)
    B, n_q, two_hd = qg.shape
    hd = two_hd // 2
    n_kv = d["k_new"].shape[1]
    outs = np.empty((B, n_q, hd), np.float32)
    kr = np.empty((B, n_kv, hd), np.uint16)
    vr = np.empty((B, n_kv, hd), np.uint16)
    qn = np.ascontiguousarray(d["q_norm_w"], np.float32)
    kn = np.ascontiguousarray(d["k_norm_w"], np.float32)
    for b in range(B):
        pos = int(d["pos"][b])
        kc = np.zeros((Lcap, n_kv, hd), np.uint16)
        vc = np.zeros((Lcap, n_kv, hd), np.uint16)
        nk = d["K"].shape[1]
        kc[:nk] = d["K"][b]
        vc[:nk] = d["V"][b]
        cs, sn = O.rope_cos_sin(pos, max(rope_dim, 2))
        cfg = O.GqaCfg(n_q, n_kv, hd, rope_dim, 1, qn.ctypes.data, kn.ctypes.data, kc.ctypes.data,
                       vc.ctypes.data, n_kv * hd, hd, n_kv * hd, hd, int(no_gate))
        out = np.empty((n_q, hd), np.float32)
        k1 = np.ascontiguousarray(d["k_new"][b], np.float32)
        v1 = np.ascontiguousarray(d["v_new"][b], np.float32)
        qb = np.ascontiguousarray(qg[b])
        O.lib().orc_gqa_token(C.byref(cfg), qb.reshape(-1), 2 * hd, qb.ctypes.data + hd * 4, 2 * hd,
                              k1.reshape(-1), v1.reshape(-1), pos, cs, sn, out.reshape(-1))
        outs[b] = out
        kr[b] = kc[pos]
        vr[b] = vc[pos]
    return outs, kr, vr


def oracle_matvec_batch(W_bf16, x, threads=None):
    """y[b] = W x[b] with the reference's F32 matvec (double serial sums) on
    bf16 weights widened exactly; x [B][K] -> y [B][N]."""
    W_bf16 = np.ascontiguousarray(W_bf16, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    B, K = x.shape
    N = W_bf16.shape[0]
    y = np.empty((B, N), np.float32)
    O.lib().orc_matvec_batch(W_bf16.ctypes.data, 1, x, y, N, K, B, threads or O.default_threads())
    return y


def oracle_dn_layer(w, x, S, conv, nqk, nv, hd=128):
    """The DeltaNet mixer of one layer (projections, all glue stages,
    out_proj) for one token of each sequence; S [B][nv][hd][hd] and conv
    [B][C][3] are updated in place.  w: w_in, w_out (bf16 bits), conv_w
    (float), A_log, dt_bias, norm_w."""
    B = x.shape[0]
    qd, vd = nqk * hd, nv * hd
    C_ = 2 * qd + vd
    y = oracle_matvec_batch(w["w_in"], x)
    keep = {k: np.ascontiguousarray(w[k], np.float32) for k in ("A_log", "dt_bias", "norm_w", "conv_w")}
    cfg = O.DnCfg(nqk, nv, hd, O.DN_CONV | O.DN_PRE_RMS | O.DN_PRE_L2 | O.DN_OUT_GATE,
                  keep["A_log"].ctypes.data, keep["dt_bias"].ctypes.data, keep["norm_w"].ctypes.data,
                  keep["conv_w"].ctypes.data)
    o = np.empty((B, vd), np.float32)
    for b in range(B):
        qkv = np.ascontiguousarray(y[b, :C_])
        z = np.ascontiguousarray(y[b, C_:C_ + vd])
        a = np.ascontiguousarray(y[b, C_ + vd:C_ + vd + nv])
        bb = np.ascontiguousarray(y[b, C_ + vd + nv:])
        Sb = np.ascontiguousarray(S[b]); cb = np.ascontiguousarray(conv[b])
        O.lib().orc_dn_token(C.byref(cfg), qkv, a, bb, z.ctypes.data, Sb.reshape(-1), cb.ctypes.data, o[b])
        S[b] = Sb; conv[b] = cb
    return oracle_matvec_batch(w["w_out"], o)


def oracle_gqa_layer(w, x, kc, vc, pos, n_q=24, n_kv=4, hd=256):
    """The gated-GQA mixer of one layer for one token of each sequence; kc,
    vc bf16 caches [B][Lcap][n_kv][hd] updated at pos[b]."""
    B = x.shape[0]
    y = oracle_matvec_batch(w["w_qkv"], x)
    Nq = n_q * 2 * hd
    qn = np.ascontiguousarray(w["q_norm_w"], np.float32)
    kn = np.ascontiguousarray(w["k_norm_w"], np.float32)
    att = np.empty((B, n_q * hd), np.float32)
    for b in range(B):
        p = int(pos[b])
        qg = np.ascontiguousarray(y[b, :Nq])
        k1 = np.ascontiguousarray(y[b, Nq:Nq + n_kv * hd])
        v1 = np.ascontiguousarray(y[b, Nq + n_kv * hd:])
        kb = np.ascontiguousarray(kc[b]); vb = np.ascontiguousarray(vc[b])
        cs, sn = O.rope_cos_sin(p)
        cfg = O.GqaCfg(n_q, n_kv, hd, 64, 1, qn.ctypes.data, kn.ctypes.data, kb.ctypes.data, vb.ctypes.data,
                       n_kv * hd, hd, n_kv * hd, hd)
        O.lib().orc_gqa_token(C.byref(cfg), qg, 2 * hd, qg.ctypes.data + hd * 4, 2 * hd, k1, v1, p, cs, sn,
                              att[b])
        kc[b] = kb; vc[b] = vb
    return oracle_matvec_batch(w["w_o"], att)
