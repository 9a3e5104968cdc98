"""GPU parity of the decode mixers through the C ABI against the oracle.

Tolerances (fixed by the parity contract of this path):
  fp32 recurrence (DeltaNet outputs and state)   max |gpu - oracle| <= 1e-5
  bf16 attention outputs                         |gpu - oracle| <= 2e-2 + 1e-2 |oracle|
                                                 and max |d| <= 2% of max |oracle|
"""
import numpy as np
import pytest

from gpu_common import bitexact_frac, maxabs, oracle_dn, oracle_gqa_decode, say

pytestmark = pytest.mark.gpu

DN_TOL = 1e-5
ATOL, RTOL, SCALE = 2e-2, 1e-2, 0.02


@pytest.fixture(scope="module")
def ctx():
    from vx27_amd import lib as L
    c = L.Ctx(0)
    yield c
    c.close()


def _dn_layer(ctx, d, B, nqk, nv, conv=False, norm_w=None):
    from vx27_amd import lib as L, mixers as M
    kw = {}
    if conv:
        kw = dict(conv_w=d["conv_w_bf16"], conv_w_dtype=L.BF16, conv0=d["conv0"])
    return M.DeltaNetLayer(ctx, B, nqk, nv, d["A_log"], d["dt_bias"], norm_w=norm_w, S0=d["S0"], **kw)


# ------------------------------------------------------------ DeltaNet
def test_dn_recurrent_full_2000_steps(ctx):
    """16 heads x 2000 steps of step_exact from zero state, one call."""
    from vx27_amd import workloads as W
    d = W.dn_recurrent(B=1, H=16, steps=2000)
    say("dn_recurrent: B=1 H=16 steps=2000")
    lay = _dn_layer(ctx, d, 1, 16, 16)
    out = lay.decode(2000, 0, d["a"], d["b"], q=d["q"], k=d["k"], v=d["v"])
    ref, S, _, _ = oracle_dn(d, 0, 1, 16, 16, 2000)
    e_o, e_s = maxabs(out, ref), maxabs(lay.state(), S)
    say(f"  max|d out|={e_o:.3e} max|d S|={e_s:.3e} bit-exact out={bitexact_frac(out, ref):.4f}")
    assert e_o <= DN_TOL and e_s <= DN_TOL


def test_dn_chunk_invariance(ctx):
    """Splitting the steps over several calls gives the same bits as one call."""
    from vx27_amd import workloads as W
    d = W.dn_recurrent(B=2, H=16, steps=40, S0_std=0.05)
    one = _dn_layer(ctx, d, 2, 16, 16)
    o1 = one.decode(40, 0, d["a"], d["b"], q=d["q"], k=d["k"], v=d["v"])
    many = _dn_layer(ctx, d, 2, 16, 16)
    outs, t = [], 0
    for n in (1, 7, 3, 29):
        sl = slice(t, t + n)
        outs.append(many.decode(n, 0, d["a"][sl], d["b"][sl], q=d["q"][sl], k=d["k"][sl], v=d["v"][sl]))
        t += n
    assert np.array_equal(np.concatenate(outs), o1)
    assert np.array_equal(many.state(), one.state())


def test_dn_conv_batched_full(ctx):
    """Batch 64 x 16 heads x 256 steps with the fused conv (bf16 weights),
    l2norm q,k and q/sqrt(128) before the exact step; state ~N(0,0.02)."""
    from vx27_amd import lib as L, workloads as W
    d = W.dn_conv(B=64, H=16, steps=256)
    flags = L.DN_CONV | L.DN_PRE_L2
    say("dn_conv: B=64 H=16 steps=256 conv+l2")
    lay = _dn_layer(ctx, d, 64, 16, 16, conv=True)
    out = lay.decode(256, flags, d["a"], d["b"], x=d["x"])
    ref, S, conv, _ = oracle_dn(d, flags, 64, 16, 16, 256)
    e_o, e_s = maxabs(out, ref), maxabs(lay.state(), S)
    say(f"  max|d out|={e_o:.3e} max|d S|={e_s:.3e} max|d conv|={maxabs(lay.conv(), conv):.3e}")
    assert e_o <= DN_TOL and e_s <= DN_TOL
    assert np.array_equal(lay.conv(), conv)


@pytest.mark.parametrize("B,flags,conv", [(1, 0, False), (2, 0, False), (4, 4, False), (8, 2 | 4, False),
                                           (1, 1 | 4, True), (4, 1 | 4, True), (8, 1 | 4, True)])
def test_dn_single_step_calls(ctx, B, flags, conv):
    """One step per call with few heads (B x 16).  Without the conv this is
    the column-split step kernel (8, 4 or 2 workgroups per head for 16, 64
    and 128 heads), with it the one-block-per-head kernel.  24 calls in a
    row against the oracle: outputs and state within 1e-5, conv state
    bit-exact; and the same calls again from the same start give the same
    bits."""
    from vx27_amd import workloads as W
    H, steps = 16, 24
    if conv:
        d = W.dn_conv(B=B, H=H, steps=steps, config=11)
    else:
        d = W.dn_recurrent(B=B, H=H, steps=steps, S0_std=0.05, config=11)
    nw = None
    if flags & 2:   # rmsn(1+w) pre-norm
        nw = d["norm_w"] = W.normal(W.rng(11, "split_norm_w"), 128, 0.1, 1.0)
    say(f"dn single-step calls: B={B} flags={flags} conv={conv}")

    def run():
        lay = _dn_layer(ctx, d, B, H, H, conv=conv, norm_w=nw)
        outs = []
        for t in range(steps):
            sl = slice(t, t + 1)
            if conv:
                outs.append(lay.decode(1, flags, d["a"][sl], d["b"][sl], x=d["x"][sl]))
            else:
                outs.append(lay.decode(1, flags, d["a"][sl], d["b"][sl], q=d["q"][sl], k=d["k"][sl], v=d["v"][sl]))
        return np.concatenate(outs), lay.state(), (lay.conv() if conv else None)
    out, S, cv = run()
    ref, Sr, cr, _ = oracle_dn(d, flags, B, H, H, steps)
    e_o, e_s = maxabs(out, ref), maxabs(S, Sr)
    say(f"  max|d out|={e_o:.3e} max|d S|={e_s:.3e} bit-exact out={bitexact_frac(out, ref):.4f}")
    assert e_o <= DN_TOL and e_s <= DN_TOL
    if conv:
        assert np.array_equal(cv, cr)
    out2, S2, cv2 = run()
    assert np.array_equal(out2, out) and np.array_equal(S2, S)
    if conv:
        assert np.array_equal(cv2, cv)


@pytest.mark.parametrize("nv", [16, 32, 48])
def test_dn_qlayer_glue(ctx, nv):
    """All stages of the vx27_qlayer DeltaNet branch: conv, rmsn(1+w), l2norm,
    exact step, gated rmsn_std * silu(z); nv > nqk shares q/k across heads."""
    from vx27_amd import lib as L, workloads as W
    B, nqk, steps = 3, 16, 5
    d = W.dn_conv(B=B, H=nqk, steps=steps, nv=nv, config=5)
    r = W.rng(5, f"glue{nv}")
    d["norm_w"] = W.normal(r, 128, 0.1, 1.0)
    d["z"] = W.normal(r, (steps, B, nv, 128))
    d["conv0"] = W.normal(r, d["conv0"].shape, 0.5)
    flags = L.DN_CONV | L.DN_PRE_RMS | L.DN_PRE_L2 | L.DN_OUT_GATE
    lay = _dn_layer(ctx, d, B, nqk, nv, conv=True, norm_w=d["norm_w"])
    out = lay.decode(steps, flags, d["a"], d["b"], x=d["x"], z=d["z"])
    ref, S, conv, _ = oracle_dn(d, flags, B, nqk, nv, steps)
    e_o, e_s = maxabs(out, ref), maxabs(lay.state(), S)
    say(f"  glue nv={nv}: max|d out|={e_o:.3e} max|d S|={e_s:.3e}")
    assert e_o <= DN_TOL and e_s <= DN_TOL
    assert np.array_equal(lay.conv(), conv)


# ----------------------------------------------------------------- GQA
def _gqa_layer(ctx, d, B, Lcap):
    from vx27_amd import mixers as M
    lay = M.GatedGQALayer(ctx, B, Lcap, d["q_norm_w"], d["k_norm_w"])
    nk = d["K"].shape[1]
    from vx27_amd import workloads as W
    for b in range(B):
        if nk:
            lay.write_kv(b, 0, W.bf16_to_f32(d["K"][b]), W.bf16_to_f32(d["V"][b]))
    return lay


def _check_gqa(out, ref, tag):
    """The attention bar, plus max|d| <= 2% of max|ref|: outputs at 8K keys
    are ~0.05, where the absolute 2e-2 alone would pass a dropped tile."""
    err = np.abs(out.astype(np.float64) - ref)
    lim = ATOL + RTOL * np.abs(ref)
    big = float(np.abs(ref).max())
    say(f"  {tag}: max|d|={err.max():.3e} max|ref|={big:.3e} (worst/limit {float((err / lim).max()):.3f}, "
        f"d/scale {err.max() / (SCALE * big):.3f})")
    assert np.all(np.isfinite(out))
    assert np.all(err <= lim)
    assert err.max() <= SCALE * big


@pytest.mark.parametrize("B", [1, 32])
def test_gqa_decode_8k(ctx, B):
    """24Q/4KV hd 256, bf16 cache of 8192 positions, new token at 8192."""
    from vx27_amd import workloads as W
    d = W.gqa_decode(B=B, L=8192)
    Lcap = 8256
    say(f"gqa_decode: B={B} L=8192")
    lay = _gqa_layer(ctx, d, B, Lcap)
    out = lay.decode(d["pos"], d["qg"], d["k_new"], d["v_new"])
    ref, kr, vr = oracle_gqa_decode(d, Lcap)
    _check_gqa(out, ref, f"B={B}")
    for b in range(B):
        k, v = lay.read_kv(b, int(d["pos"][b]), 1)
        assert np.array_equal(W.bf16_bits(v[0]), vr[b])
        kd = np.abs(k[0] - W.bf16_to_f32(kr[b]))
        assert np.all(kd <= np.abs(W.bf16_to_f32(kr[b])) * 2 ** -7 + 1e-30)


def test_gqa_decode_no_gate(ctx):
    """VX27_GQA_NO_GATE: the attention without the output gate, as the MTP
    drafter's decoder layer runs with use_gate = 0 (vx27_mtp.c:219-258)."""
    from vx27_amd import lib as L, workloads as W
    d = W.gqa_decode(B=2, L=300, config=23)
    Lcap = 320
    lay = _gqa_layer(ctx, d, 2, Lcap)
    lay.flags |= L.GQA_NO_GATE
    out = lay.decode(d["pos"], d["qg"], d["k_new"], d["v_new"])
    ref, _, _ = oracle_gqa_decode(d, Lcap, no_gate=True)
    _check_gqa(out, ref, "no gate")
    gated, _, _ = oracle_gqa_decode(d, Lcap)
    assert np.abs(ref - gated).max() > 0.1   # the flag changes the answer


def test_gqa_edges_and_splits(ctx):
    """Ragged positions across tile edges (0, 1, 31, 32, 33, 63, 64, 100), and
    the same answer for every split count."""
    from vx27_amd import workloads as W
    pos = np.array([0, 1, 31, 32, 33, 63, 64, 100], np.int32)
    B = len(pos)
    d = W.gqa_decode(B=B, L=101, config=22)
    d["pos"] = pos
    Lcap = 128
    lay = _gqa_layer(ctx, d, B, Lcap)
    ref, _, _ = oracle_gqa_decode(d, Lcap)
    outs = []
    for ns in (1, 2, 3, 0):
        lay2 = _gqa_layer(ctx, d, B, Lcap)
        outs.append(lay2.decode(pos, d["qg"], d["k_new"], d["v_new"], n_split=ns))
        _check_gqa(outs[-1], ref, f"n_split={ns}")
    # pos 0 attends only the new key: out = v_new (bf16) * sigmoid(gate)
    g = d["qg"][0, :, 256:].astype(np.float64)
    vb = W.bf16_to_f32(W.bf16_bits(d["v_new"][0])).astype(np.float64)
    want = np.stack([vb[h // 6] for h in range(24)]) / (1 + np.exp(-g))
    assert np.abs(outs[-1][0] - want).max() < 1e-5


@pytest.mark.parametrize("rope_dim", [0, 32, 128, 256])
def test_gqa_decode_rope_dims(ctx, rope_dim):
    """Other rotary widths (0: no rotation; 256: every dim rotated), ragged
    positions; the appended k, v rows are checked too."""
    from vx27_amd import mixers as M, workloads as W
    d = W.gqa_decode(B=3, L=700, config=25)
    d["pos"] = np.array([700, 31, 415], np.int32)
    Lcap = 768
    say(f"gqa_decode: rope_dim={rope_dim} B=3 pos={d['pos'].tolist()}")
    lay = M.GatedGQALayer(ctx, 3, Lcap, d["q_norm_w"], d["k_norm_w"], rope_dim=rope_dim)
    for b in range(3):
        lay.write_kv(b, 0, W.bf16_to_f32(d["K"][b]), W.bf16_to_f32(d["V"][b]))
    out = lay.decode(d["pos"], d["qg"], d["k_new"], d["v_new"])
    ref, kr, vr = oracle_gqa_decode(d, Lcap, rope_dim=rope_dim)
    _check_gqa(out, ref, f"rope_dim={rope_dim}")
    for b in range(3):
        k, v = lay.read_kv(b, int(d["pos"][b]), 1)
        assert np.array_equal(W.bf16_bits(v[0]), vr[b])
        kd = np.abs(k[0] - W.bf16_to_f32(kr[b]))
        assert np.all(kd <= np.abs(W.bf16_to_f32(kr[b])) * 2 ** -7 + 1e-30)
    if rope_dim:   # the width changes the answer
        other, _, _ = oracle_gqa_decode(d, Lcap, rope_dim=rope_dim // 2)
        assert np.abs(other - ref).max() > 1e-3


def test_gqa_decode_norm_w(ctx):
    """VX27_GQA_NORM_W on the decode (q/k norm as x*s*w, vx27_gqa.c:10-15).
    Oracle: the (1+w) form with w - 1, exact for w in [0.5, 2] (Sterbenz)."""
    from vx27_amd import lib as L, workloads as W
    d = W.gqa_decode(B=3, L=500, config=24)
    d["pos"] = np.array([500, 77, 300], np.int32)
    r = W.rng(24, "norm_w")
    w_q = np.clip(W.normal(r, 256, 0.1, 1.0), 0.5, 2.0).astype(np.float32)
    w_k = np.clip(W.normal(r, 256, 0.1, 1.0), 0.5, 2.0).astype(np.float32)
    Lcap = 512
    dev = dict(d, q_norm_w=w_q, k_norm_w=w_k)
    lay = _gqa_layer(ctx, dev, 3, Lcap)
    lay.flags |= L.GQA_NORM_W
    out = lay.decode(d["pos"], d["qg"], d["k_new"], d["v_new"])
    orc = dict(d, q_norm_w=(w_q - np.float32(1)).astype(np.float32),
               k_norm_w=(w_k - np.float32(1)).astype(np.float32))
    assert np.array_equal(orc["q_norm_w"] + np.float32(1), w_q)
    ref, _, _ = oracle_gqa_decode(orc, Lcap)
    _check_gqa(out, ref, "norm_w")
    alt, _, _ = oracle_gqa_decode(dev, Lcap)
    assert np.abs(alt - ref).max() > 1e-3   # the flag changes the answer
