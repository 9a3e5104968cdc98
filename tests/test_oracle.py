"""The oracle pinned: against golden vectors minted from the compiled reference,
against the reference's own known-answer checks, and against independent
float64 / closed-form restatements of the mathematics.  CPU only.
"""
import ctypes as C
import math

import numpy as np
import pytest

from conftest import golden
import inputs as I


def f32(a):
    return np.ascontiguousarray(a, np.float32)


# ------------------------------------------------------------------ gates
def test_gate_golden(O):
    g = golden("gate_params")
    for (a, al, b, dt), be, gg in zip(g["inp"], g["beta"], g["g"]):
        beta, glog = O.gate_params(a, al, b, dt)
        assert beta == be and glog == gg


def _sp(x):
    return x if x > 20.0 else (math.exp(x) if x < -20.0 else math.log(1.0 + math.exp(x)))


def test_gate_known_answers(O):
    # tests/test_deltanet_exact.c:43-58: bit-identical to a double restatement,
    # beta in (0,1), g <= 0; dt_bias enters g only.
    cases = [(0.1, 0.5, -0.3, 1.0), (3.0, -1.2, 2.0, 1.0), (-25.0, 0.0, 0.0, 1.0),
             (25.0, 2.0, -2.0, 1.0), (0.0, -5.0, 5.0, -3.0), (-30.0, 1.0, 30.0, 30.0)]
    for a, al, b, dt in cases:
        beta, glog = O.gate_params(a, al, b, dt)
        assert beta == 1.0 / (1.0 + math.exp(-b))
        assert glog == -math.exp(al) * _sp(a + dt)
        assert 0.0 < beta < 1.0 and glog <= 0.0
    # dt_bias must not enter beta
    assert O.gate_params(0.0, 0.0, 0.7, 5.0)[0] == O.gate_params(0.0, 0.0, 0.7, -5.0)[0]


# ---------------------------------------------------------------- l2norm
def test_l2norm_golden(O):
    g = golden("l2norm")
    for i in range(int(g["n"])):
        y = O.l2norm(g[f"x{i}"])
        assert np.array_equal(y, g[f"y{i}"])


def test_l2norm_closed_form(O):
    # eps inside the sqrt and no /n: ||y||^2 = S/(S+1e-6) for S = sum x^2
    x = f32([3.0, 4.0])
    y = O.l2norm(x)
    np.testing.assert_allclose(y, x / np.sqrt(25.0 + 1e-6), rtol=1e-7)
    assert np.all(O.l2norm(np.zeros(8, np.float32)) == 0)


# ------------------------------------------------------------ step_exact
def test_step_golden(O):
    g = golden("step_exact")
    S = g["S0"].copy()
    T, NH, hd = g["q"].shape
    for t in range(T):
        for h in range(NH):
            Sh = np.ascontiguousarray(S[h])
            o = O.step_exact(Sh, g["q"][t, h], g["k"][t, h], g["v"][t, h], g["beta"][t, h],
                             g["g"][t, h])
            S[h] = Sh
            assert np.array_equal(o, g["o"][t, h]), (t, h)
    assert np.array_equal(S, g["S"])


def dbl_step(S, q, k, v, beta, glog):
    """Independent float64 delta rule (the double oracle of
    tests/test_deltanet_exact.c:18-30)."""
    hd = q.size
    q = q.astype(np.float64); k = k.astype(np.float64); v = v.astype(np.float64)
    qn = q / math.sqrt(float(q @ q) + 1e-6) / math.sqrt(hd)
    kn = k / math.sqrt(float(k @ k) + 1e-6)
    S *= math.exp(glog)
    kv = S.T @ kn
    S += np.outer(kn, (v - kv) * beta)
    return S.T @ qn


def test_step_vs_double_oracle(O):
    # 40 trials x (1 + 5) chained steps, reference tolerance out<1e-4, S<1e-3
    r = I.rng("dbl_oracle")
    hd = 128
    md_o = md_s = 0.0
    for trial in range(40):
        Sf = I.uniform(r, (hd, hd), -0.5, 0.5)
        Sd = Sf.astype(np.float64)
        for t in range(6):
            q = I.uniform(r, hd, -1, 1); k = I.uniform(r, hd, -1, 1); v = 2 * I.uniform(r, hd, -1, 1)
            beta = 0.05 + 0.9 * r.uniform(); glog = -8.0 * r.uniform()
            of = O.step_exact(Sf, q, k, v, beta, glog)
            od = dbl_step(Sd, q, k, v, beta, glog)
            md_o = max(md_o, float(np.abs(of - od).max()))
            md_s = max(md_s, float(np.abs(Sf - Sd).max()))
    assert md_o < 1e-6 and md_s < 1e-6, (md_o, md_s)


def test_step_deterministic_and_decay_only(O):
    hd = 128
    i = np.arange(hd, dtype=np.float32)
    q = f32(i * 0.01 - 0.5); k = f32((i % 7) * 0.03); v = f32((i % 5) * 0.07)
    S1 = np.zeros((hd, hd), np.float32); S2 = np.zeros((hd, hd), np.float32)
    assert np.array_equal(O.step_exact(S1, q, k, v, 0.7, -0.5), O.step_exact(S2, q, k, v, 0.7, -0.5))
    # beta = 0 leaves only the decay: S' = (float)(S*exp(g)); o = S'^T qn
    S = I.normal(I.rng("decay_only"), (hd, hd))
    S0 = S.copy()
    O.step_exact(S, q, k, v, 0.0, -0.25)
    assert np.array_equal(S, (S0.astype(np.float64) * math.exp(-0.25)).astype(np.float32))


# ----------------------------------------------------------------- conv1d
def test_conv_golden(O):
    g = golden("conv1d")
    T, C_ = g["x"].shape
    st = np.zeros((C_, 3), np.float32)
    L = O.lib()
    for t in range(T):
        y = np.empty(C_, np.float32)
        L.orc_conv1d_step(st.reshape(-1), f32(g["x"][t]), f32(g["w"]).reshape(-1), y, C_, 1)
        assert np.array_equal(y, g["y"][t]), t
    assert np.array_equal(st, g["state"])
    st2 = g["st2_0"].copy(); y2 = np.empty(C_, np.float32)
    L.orc_conv1d_step(st2.reshape(-1), f32(g["x"][0]), f32(g["w"]).reshape(-1), y2, C_, 0)
    assert np.array_equal(y2, g["y2"]) and np.array_equal(st2, g["st2"])


def test_conv_vs_naive(O):
    # tests/test_deltanet_exact.c:109-138: carryover == zero-left-padded full
    # convolution with tap 0 the oldest sample, then SiLU; C=32, T=8, <1e-5.
    r = I.rng("conv_naive")
    C_, T, K = 32, 8, 4
    w = 0.3 * I.uniform(r, (C_, K), -1, 1); xs = I.uniform(r, (T, C_), -1, 1)
    st = np.zeros((C_, 3), np.float32)
    for t in range(T):
        y = np.empty(C_, np.float32)
        O.lib().orc_conv1d_step(st.reshape(-1), xs[t], w.reshape(-1), y, C_, 1)
        acc = np.zeros(C_)
        for j in range(K):
            tt = t - (K - 1) + j
            if tt >= 0:
                acc += w[:, j].astype(np.float64) * xs[tt]
        want = acc / (1.0 + np.exp(-acc))
        assert np.abs(y - want).max() < 1e-5


# ----------------------------------------------- simplified update/retrieve
def test_simple_update_golden(O):
    g = golden("simple_update")
    S = g["S0"].copy()
    O.lib().orc_update_simple(S.reshape(-1), g["k"], g["v"], 0.9, 128)
    o = np.empty(128, np.float32)
    O.lib().orc_retrieve_simple(S.reshape(-1), g["q"], o, 128)
    assert np.array_equal(S, g["S_ref"]) and np.array_equal(o, g["o_ref"])
    # tests/test_deltanet.c:41-61: tiled == ref within 1e-5, AVX2 within 1e-4
    assert np.abs(g["S_tiled"] - g["S_ref"]).max() < 1e-5
    assert np.abs(g["S_avx2"] - g["S_ref"]).max() < 1e-4
    assert np.abs(g["o_avx2"] - g["o_ref"]).max() < 1e-4


def test_avx2_primitives_golden(O):
    """The restated AVX2 update/retrieve (the CPU-AVX2 baseline's
    primitives) are bit-exact to the compiled reference's
    vx27_deltanet_update_avx2 / retrieve_avx2 outputs."""
    g = golden("simple_update")
    S = g["S0"].copy()
    O.lib().orc_update_avx2_pub(S.reshape(-1), g["k"], g["v"], 0.9, 128)
    o = np.empty(128, np.float32)
    O.lib().orc_retrieve_avx2_pub(S.reshape(-1), g["q"], o, 128)
    assert np.array_equal(S, g["S_avx2"]) and np.array_equal(o, g["o_avx2"])


def test_avx2_run_is_the_primitive_chain(O):
    """orc_dn_run_avx2 (2 heads x 5 steps, 2 threads) equals the chain
    retrieve(S,k) -> d = beta (v - decay kv) -> update(S,k,d,decay) ->
    retrieve(S,q) of the pinned primitives; with the compiled reference's
    own primitives (where oracle/_ref is built) the run is the same bit for
    bit."""
    r = np.random.default_rng(5)
    H, T, hd = 2, 5, 128
    q = r.standard_normal((T, H, hd), dtype=np.float32)
    k = r.standard_normal((T, H, hd), dtype=np.float32) / np.float32(11.3)
    v = r.standard_normal((T, H, hd), dtype=np.float32)
    beta = r.uniform(0.1, 0.9, (T, H))
    decay = r.uniform(0.5, 1.0, (T, H))
    S0 = r.standard_normal((H, hd, hd), dtype=np.float32) * np.float32(0.02)
    S = S0.copy()
    out = np.empty((T, H, hd), np.float32)
    O.lib().orc_dn_run_avx2(1, H, hd, T, 2, S.reshape(-1), q.reshape(-1), k.reshape(-1), v.reshape(-1),
                            beta.reshape(-1), decay.reshape(-1), out.reshape(-1), None, None)
    Sw = S0.copy()
    for t in range(T):
        for h in range(H):
            kv = np.empty(hd, np.float32)
            O.lib().orc_retrieve_avx2_pub(Sw[h].reshape(-1), k[t, h], kv, hd)
            dec, bt = np.float32(decay[t, h]), np.float32(beta[t, h])
            dd = (bt * (v[t, h] - dec * kv)).astype(np.float32)
            O.lib().orc_update_avx2_pub(Sw[h].reshape(-1), k[t, h], dd, dec, hd)
            o = np.empty(hd, np.float32)
            O.lib().orc_retrieve_avx2_pub(Sw[h].reshape(-1), q[t, h], o, hd)
            assert np.array_equal(o, out[t, h]), (t, h)
    assert np.array_equal(Sw, S)
    upd, ret = O.ref_avx2_fns()
    if upd is not None:
        S2 = S0.copy()
        out2 = np.empty_like(out)
        O.lib().orc_dn_run_avx2(1, H, hd, T, 2, S2.reshape(-1), q.reshape(-1), k.reshape(-1), v.reshape(-1),
                                beta.reshape(-1), decay.reshape(-1), out2.reshape(-1), upd, ret)
        assert np.array_equal(out2, out) and np.array_equal(S2, S)


# ------------------------------------------------------------- GQA pieces
def test_rmsnorm_golden(O):
    g = golden("gqa")
    y = np.empty(2, np.float32)
    O.lib().orc_rmsnorm_w(f32([3, 4]), f32([1, 1]), y, 2, 0.0)
    assert np.array_equal(y, g["rms34"])
    assert abs(y[0] - 0.8485) < 1e-3 and abs(y[1] - 1.1314) < 1e-3   # tests/test_gqa.c:19-21
    for n, eps in ((256, 1e-6), (5120, 1e-6), (128, 1e-5)):
        yy = np.empty(n, np.float32)
        O.lib().orc_rmsnorm_w(g[f"rx{n}"], g[f"rw{n}"], yy, n, eps)
        assert np.array_equal(yy, g[f"ry{n}"])
    assert [O.lib().orc_kv_for_q(h) for h in range(24)] == list(g["kv_map"])


def test_attn_1q_golden(O):
    g = golden("gqa")
    for n_pos in (1, 2, 64, 160):
        o = np.empty(24 * 256, np.float32)
        O.lib().orc_attn_1q(g[f"aq{n_pos}"], g[f"ak{n_pos}"], g[f"av{n_pos}"], n_pos, o)
        assert np.array_equal(o, g[f"ao{n_pos}"]), n_pos


def test_attn_1q_known_answers(O):
    # tests/test_gqa.c:23-52
    i = np.arange(24 * 256)
    q = f32((i % 7) * 0.01)
    j = np.arange(4 * 256)
    kc = f32((j % 5) * 0.02); vc = f32((j % 11) * 0.03 + (j // 256))
    out = np.empty(24 * 256, np.float32)
    O.lib().orc_attn_1q(q, kc, vc, 1, out)
    for h in range(24):
        kvh = h // 6
        assert np.abs(out[h * 256:(h + 1) * 256] - vc[kvh * 256:(kvh + 1) * 256]).max() < 1e-4
    kc2 = np.concatenate([kc, kc]); vc2 = np.concatenate([vc, vc + 2.0])
    O.lib().orc_attn_1q(q, kc2, vc2, 2, out)
    for h in range(24):
        kvh = h // 6
        want = (vc[kvh * 256:(kvh + 1) * 256] + vc2[1024 + kvh * 256:1024 + (kvh + 1) * 256]) * 0.5
        assert np.abs(out[h * 256:(h + 1) * 256] - want).max() < 1e-3


def test_attend_bf16_closed_forms(O):
    # one key -> its value; identical keys -> mean of values; both dot forms
    r = I.rng("attend_cf")
    hd, nq, nkv = 256, 24, 4
    q = I.normal(r, (nq, hd))
    k1 = O.to_bf16(I.normal(r, (1, nkv, hd))); v1 = O.to_bf16(I.normal(r, (1, nkv, hd)))
    for dd in (0, 1):
        out = O.attend(q, k1, v1, 1, (nkv * hd, hd), (nkv * hd, hd), nkv, dot_double=dd, kv_bf16=1)
        vv = O.from_bf16(v1)[0]
        for h in range(nq):
            assert np.array_equal(out[h], vv[h // 6])
    kk = np.repeat(k1, 5, axis=0); vv = O.to_bf16(I.normal(r, (5, nkv, hd)))
    out = O.attend(q, kk, vv, 5, (nkv * hd, hd), (nkv * hd, hd), nkv, dot_double=1, kv_bf16=1)
    mean = O.from_bf16(vv).astype(np.float64).mean(0)
    for h in range(nq):
        assert np.abs(out[h] - mean[h // 6]).max() < 1e-5


# ------------------------------------------------------------------ RoPE
def test_rope_golden(O):
    g = golden("rope")
    for i, p in enumerate(g["pos"]):
        c, s = O.rope_cos_sin(int(p))
        assert np.array_equal(c, g["cos"][i]) and np.array_equal(s, g["sin"][i]), int(p)
    c, s = O.rope_cos_sin(32, yarn=4.0)
    assert np.array_equal(c, g["yarn_cos"]) and np.array_equal(s, g["yarn_sin"])
    mc = np.empty(32, np.float32); ms = np.empty(32, np.float32)
    O.lib().orc_mrope_cos_sin_text(8192, mc, ms)
    assert np.array_equal(mc, g["mrope_cos"]) and np.array_equal(ms, g["mrope_sin"])
    v = g["vin"].copy()
    O.lib().orc_rope_apply(v.reshape(-1), 24, 256, 64, g["cos"][8], g["sin"][8])
    assert np.array_equal(v, g["vout"])


def test_rope_invariants(O):
    # tests/test_rope.c:11-42
    c, s = O.rope_cos_sin(0)
    assert np.all(np.abs(c - 1) <= 1e-6) and np.all(np.abs(s) <= 1e-6)
    c1, s1 = O.rope_cos_sin(8); c2, s2 = O.rope_cos_sin(32, yarn=4.0)
    assert max(np.abs(c1 - c2).max(), np.abs(s1 - s2).max()) < 1e-5
    i = np.arange(256)
    v = f32((i % 13) * 0.05 - 0.3); w = v.copy()
    c, s = O.rope_cos_sin(7)
    O.lib().orc_rope_apply(v, 1, 256, 64, c, s)
    assert np.array_equal(v[64:], w[64:])
    n0 = float((w[:64].astype(np.float64) ** 2).sum()); n1 = float((v[:64].astype(np.float64) ** 2).sum())
    assert abs(n0 - n1) / (n0 + 1e-9) < 1e-5
    # angle of pair i is pos * theta^(-2i/64): float64 closed form at small pos
    c, s = O.rope_cos_sin(5)
    ang = 5.0 * 1e7 ** (-2.0 * np.arange(32) / 64.0)
    assert np.abs(c - np.cos(ang)).max() < 1e-6 and np.abs(s - np.sin(ang)).max() < 1e-6


# ------------------------------------------------------- vx27_qlayer glue
def _dn_layer_w(O, d):
    return O.DnLayerW(*[O.ptr(d[n]) for n in ("ln_w", "w_qkv", "w_z", "w_a", "w_b", "conv_w",
                                              "A_log", "dt_bias", "norm_w", "w_out")])


@pytest.mark.slow
def test_qlayer_dn_golden(O):
    g = golden("qlayer_dn")
    d = I.qlayer_dn_inputs()
    assert I.digest(*[d[k] for k in sorted(d)]) == str(g["digest"]), "input regeneration drifted"
    w = _dn_layer_w(O, d)
    S = d["S0"].copy(); conv = d["conv0"].copy()
    for tok in range(2):
        out = np.empty(I.H, np.float32)
        O.lib().orc_dn_layer_token(C.byref(w), f32(d["x"][tok]), S.reshape(-1), conv.reshape(-1), out)
        assert np.array_equal(out, g["out"][tok]), tok
    assert np.array_equal(S[:, :2, :], g["S_slice"])
    assert S.astype(np.float64).sum() == g["S_sum"]
    assert (S.astype(np.float64) ** 2).sum() == g["S_sq"]
    assert np.array_equal(conv, g["conv"])


@pytest.mark.slow
def test_qlayer_gqa_golden(O):
    g = golden("qlayer_gqa")
    n_pos = int(g["n_pos"])
    d = I.qlayer_gqa_inputs(n_pos=n_pos)
    assert I.digest(*[d[k] for k in sorted(d)]) == str(g["digest"]), "input regeneration drifted"
    w = O.GqaLayerW(*[O.ptr(d[n]) for n in ("ln_w", "w_q", "w_k", "w_v", "q_norm_w", "k_norm_w", "w_o")])
    kc, vc = d["kc"].copy(), d["vc"].copy()
    out = np.empty(I.H, np.float32)
    O.lib().orc_gqa_layer_token(C.byref(w), d["x"], n_pos, kc.reshape(-1), vc.reshape(-1), out)
    assert np.array_equal(out, g["out"])
    assert np.array_equal(kc[n_pos], g["k_row"]) and np.array_equal(vc[n_pos], g["v_row"])


# ------------------------------------------- live cross-check (this host)
@pytest.mark.skipif("__import__('oracle.oracle', fromlist=['x']).ref() is None",
                    reason="compiled reference not built here")
def test_live_vs_reference(O):
    R = O.ref()
    r = I.rng("live")
    hd = 128
    for trial in range(8):
        S1 = I.normal(r, (hd, hd), 0.1); S2 = S1.copy()
        q, k, v = I.normal(r, hd), I.normal(r, hd), I.normal(r, hd)
        beta, glog = r.uniform(0, 1), -r.uniform(0, 5)
        o1 = O.step_exact(S1, q, k, v, beta, glog)
        o2 = np.empty(hd, np.float32)
        R.vx27_deltanet_step_exact(S2.reshape(-1), q, k, v, beta, glog, o2, hd)
        assert np.array_equal(o1, o2) and np.array_equal(S1, S2)
    for p in list(range(0, 300000, 9973)) + [131072 + i for i in range(32)]:
        c1, s1 = O.rope_cos_sin(p)
        c2 = np.empty(32, np.float32); s2 = np.empty(32, np.float32)
        R.vx27_rope_cos_sin(p, c2, s2, 64, 1e7, 1.0)
        assert np.array_equal(c1, c2) and np.array_equal(s1, s2), p


# ------------------------------ compositions used as multi-token oracles
def test_dn_run_equals_chained_steps(O):
    """orc_dn_run (the batched / multi-token driver, also the DeltaNet prefill
    oracle) equals chained orc_step_exact + orc_gate_params calls bit for bit,
    including the QK-head sharing vh*nqk/nv (vx27_qfwd.c:136-137)."""
    r = I.rng("dn_run_chain")
    B, nqk, nv, hd, T = 2, 2, 4, 128, 5
    q, k = I.normal(r, (T, B, nqk, hd)), I.normal(r, (T, B, nqk, hd))
    v = I.normal(r, (T, B, nv, hd))
    a, b = I.normal(r, (T, B, nv)), I.normal(r, (T, B, nv))
    A_log, dt = f32(r.uniform(-2, 1, nv)), I.normal(r, nv, 0.1)
    S0 = I.normal(r, (B, nv, hd, hd), 0.05)
    S = S0.copy()
    out = np.empty((T, B, nv, hd), np.float32)
    args = O.DnRunArgs(B, nqk, nv, hd, T, 0, 3, S.ctypes.data, None, None, None, q.ctypes.data,
                       k.ctypes.data, v.ctypes.data, a.ctypes.data, b.ctypes.data, A_log.ctypes.data,
                       dt.ctypes.data, None, None, out.ctypes.data)
    O.lib().orc_dn_run(C.byref(args))
    Sr = S0.copy()
    for t in range(T):
        for bb in range(B):
            for vh in range(nv):
                g = vh * nqk // nv
                beta, glog = O.gate_params(a[t, bb, vh], A_log[vh], b[t, bb, vh], dt[vh])
                o = O.step_exact(Sr[bb, vh], q[t, bb, g], k[t, bb, g], v[t, bb, vh], beta, glog)
                assert np.array_equal(o, out[t, bb, vh]), (t, bb, vh)
    assert np.array_equal(S, Sr)


def test_gqa_prefill_equals_token_chain(O):
    """orc_gqa_prefill (the GQA prefill oracle, parallel over tokens and heads)
    equals orc_gqa_token applied token by token (pinned to vx27_qlayer)
    bit for bit, with an earlier context in the cache."""
    r = I.rng("gqa_prefill_chain")
    n_q, n_kv, hd, T, pos0, L = 24, 4, 256, 4, 3, 8
    q, gate = I.normal(r, (1, T, n_q, hd)), I.normal(r, (1, T, n_q, hd))
    k, v = I.normal(r, (1, T, n_kv, hd)), I.normal(r, (1, T, n_kv, hd))
    qw, kw = I.normal(r, hd, 0.1), I.normal(r, hd, 0.1)
    kc0 = np.zeros((1, L, n_kv, hd), np.float32); vc0 = np.zeros_like(kc0)
    kc0[0, :pos0], vc0[0, :pos0] = I.normal(r, (pos0, n_kv, hd)), I.normal(r, (pos0, n_kv, hd))
    kc, vc = kc0.copy(), vc0.copy()
    out = np.empty((1, T, n_q, hd), np.float32)
    a = O.GqaPrefillArgs(1, T, n_q, n_kv, hd, 64, pos0, L, 3, 1e7, 1.0, q.ctypes.data, gate.ctypes.data,
                         k.ctypes.data, v.ctypes.data, qw.ctypes.data, kw.ctypes.data, kc.ctypes.data,
                         vc.ctypes.data, out.ctypes.data)
    O.lib().orc_gqa_prefill(C.byref(a))
    kr, vr = kc0.copy(), vc0.copy()
    cfg = O.GqaCfg(n_q, n_kv, hd, 64, 0, qw.ctypes.data, kw.ctypes.data, kr.ctypes.data, vr.ctypes.data,
                   n_kv * hd, hd, n_kv * hd, hd)
    for t in range(T):
        c, s = O.rope_cos_sin(pos0 + t)
        o = np.empty((n_q, hd), np.float32)
        gt = f32(gate[0, t])
        O.lib().orc_gqa_token(C.byref(cfg), f32(q[0, t]), hd, gt.ctypes.data, hd, f32(k[0, t]), f32(v[0, t]),
                              pos0 + t, c, s, o)
        assert np.array_equal(o, out[0, t]), t
    assert np.array_equal(kc, kr) and np.array_equal(vc, vr)


def test_gqa_no_gate_pinned(O):
    """The no-gate branch (vx27_mtp.c:258 with use_gate = 0) equals the gated
    path (pinned to vx27_qlayer) with gate logits of 100, whose sigmoid is
    1.0f exactly, bit for bit: for one token and for the prefill."""
    r = I.rng("gqa_no_gate")
    n_q, n_kv, hd, T, pos0, L = 24, 4, 256, 3, 2, 8
    q = I.normal(r, (1, T, n_q, hd))
    k, v = I.normal(r, (1, T, n_kv, hd)), I.normal(r, (1, T, n_kv, hd))
    qw, kw = I.normal(r, hd, 0.1), I.normal(r, hd, 0.1)
    big = np.full((1, T, n_q, hd), 100.0, np.float32)
    assert np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-100.0))) == np.float32(1.0)
    kc0 = np.zeros((1, L, n_kv, hd), np.float32)
    kc0[0, :pos0] = I.normal(r, (pos0, n_kv, hd))
    outs = []
    for no_gate in (0, 1):
        kc, vc = kc0.copy(), kc0.copy()
        out = np.empty((1, T, n_q, hd), np.float32)
        a = O.GqaPrefillArgs(1, T, n_q, n_kv, hd, 64, pos0, L, 3, 1e7, 1.0, q.ctypes.data, big.ctypes.data,
                             k.ctypes.data, v.ctypes.data, qw.ctypes.data, kw.ctypes.data, kc.ctypes.data,
                             vc.ctypes.data, out.ctypes.data, no_gate)
        O.lib().orc_gqa_prefill(C.byref(a))
        outs.append(out)
    assert np.array_equal(outs[0], outs[1])
    tok = []
    for no_gate in (0, 1):
        kr, vr = kc0.copy(), kc0.copy()
        cfg = O.GqaCfg(n_q, n_kv, hd, 64, 0, qw.ctypes.data, kw.ctypes.data, kr.ctypes.data, vr.ctypes.data,
                       n_kv * hd, hd, n_kv * hd, hd, no_gate)
        c, s_ = O.rope_cos_sin(pos0)
        o = np.empty((n_q, hd), np.float32)
        gt = f32(big[0, 0])
        O.lib().orc_gqa_token(C.byref(cfg), f32(q[0, 0]), hd, gt.ctypes.data, hd, f32(k[0, 0]), f32(v[0, 0]),
                              pos0, c, s_, o)
        tok.append(o)
    assert np.array_equal(tok[0], tok[1])
    assert np.array_equal(tok[1], outs[1][0, 0])
