"""GPU parity of the prefill mixers through the C ABI against the oracle.

DeltaNet prefill (vx27_hip_dn_prefill) is the chunked form of the exact delta
rule with bf16 MFMA products; its oracle is the reference's own sequential
step_exact (vx27_deltanet.c:71-102) applied token by token to the same bf16
inputs widened to fp32 (orc_dn_run).  The chunked products are bf16, so the
outputs are held to the bf16 bar (|gpu - oracle| <= 2e-2 + 1e-2 |oracle|), not
to the fp32 recurrence's 1e-5; the final-state error is reported and held to
the same bf16 bar.  The elementwise bar is loose next to the outputs'
magnitude (|o| < 0.1 here), so the error is also held to 2% of max|oracle|,
which a dropped or mis-decayed term of the chunked form exceeds.
"""
import ctypes as C

import numpy as np
import pytest

from gpu_common import maxabs, oracle_dn, say

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2
SCALE_TOL = 2e-2


@pytest.fixture(scope="module")
def ctx():
    from vx27_amd import lib as L
    c = L.Ctx(0)
    yield c
    c.close()


def run_dn_prefill(ctx, d, S=None, t0=0, t1=None, flags=0):
    """Prefill tokens t0..t1-1 of workload d on the device; returns (out, S)."""
    from vx27_amd import lib as L
    B, T, nqk, hd = d["q"].shape
    nv = d["v"].shape[2]
    t1 = T if t1 is None else t1
    sl = slice(t0, t1)
    bufs = {k: ctx.put(np.ascontiguousarray(d[k][:, sl])) for k in ("q", "k", "v", "a", "b")}
    bufs["A_log"], bufs["dt_bias"] = ctx.put(d["A_log"]), ctx.put(d["dt_bias"])
    Sd = ctx.put(np.ascontiguousarray(d["S0"] if S is None else S, np.float32))
    n = t1 - t0
    ob = ctx.buf(B * n * nv * hd * 4)
    desc = L.DnPrefillDesc(B, n, nqk, nv, hd, flags, Sd.ptr, bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr,
                           bufs["a"].ptr, bufs["b"].ptr, bufs["A_log"].ptr, bufs["dt_bias"].ptr, ob.ptr)
    L.check(L.lib().vx27_hip_dn_prefill(ctx.h, C.byref(desc)), "dn_prefill")
    out = ob.download((B, n, nv, hd), np.float32)
    Sn = Sd.download(d["S0"].shape, np.float32)
    for bb in list(bufs.values()) + [Sd, ob]:
        bb.free()
    return out, Sn


def oracle_dn_prefill(d):
    """Sequential step_exact over the bf16 inputs widened to fp32."""
    from vx27_amd import workloads as W
    B, T, nqk, hd = d["q"].shape
    nv = d["v"].shape[2]
    seq = {k: np.ascontiguousarray(np.swapaxes(W.bf16_to_f32(d[k]), 0, 1)) for k in ("q", "k", "v")}
    seq.update({k: np.ascontiguousarray(np.swapaxes(d[k], 0, 1)) for k in ("a", "b")})
    seq.update(A_log=d["A_log"], dt_bias=d["dt_bias"], S0=d["S0"])
    out, S, _, secs = oracle_dn(seq, 0, B, nqk, nv, T)
    return np.swapaxes(out, 0, 1), S, secs


def check_bf16(got, ref, tag):
    err = np.abs(got.astype(np.float64) - ref)
    lim = ATOL + RTOL * np.abs(ref)
    worst = float((err / lim).max())
    say(f"  {tag}: max|d|={err.max():.3e} (max|ref|={np.abs(ref).max():.3f}, worst/limit {worst:.3f})")
    assert np.all(err <= lim), tag
    assert err.max() <= SCALE_TOL * np.abs(ref).max(), tag


X3_REL = 1e-4   # split-precision bar: max|d| <= 1e-4 of max|ref| (bf16 products reach ~4e-3)


@pytest.mark.parametrize("bf16", [False, True])
def test_dn_prefill_4096(ctx, bf16):
    """One 4096-token prompt, 16 heads, zero state (the prefill workload):
    the default split-precision products within 1e-4 of max|ref| (outputs
    and final state), the bf16 form (VX27_DN_BF16) on the bf16 bar."""
    from vx27_amd import lib as L, workloads as W
    d = W.dn_prefill(B=1, T=4096)
    say(f"dn_prefill: B=1 T=4096 nqk=nv=16 {'bf16' if bf16 else 'split'}")
    out, S = run_dn_prefill(ctx, d, flags=L.DN_BF16 if bf16 else 0)
    ref, Sr, secs = oracle_dn_prefill(d)
    say(f"  oracle {secs:.2f}s")
    check_bf16(out, ref, "out")
    say(f"  final state max|d|={maxabs(S, Sr):.3e} (max|S|={np.abs(Sr).max():.3f})")
    check_bf16(S, Sr, "state")
    if not bf16:
        assert maxabs(out, ref) <= X3_REL * np.abs(ref).max()
        assert maxabs(S, Sr) <= X3_REL * np.abs(Sr).max()
        # the fp32 recurrence's absolute bar on the outputs of this workload
        assert maxabs(out, ref) <= 1e-5


@pytest.mark.parametrize("B,T,nqk,nv,S0", [(2, 200, 4, 8, 0.02), (1, 193, 4, 12, 0.02), (3, 64, 2, 2, 0.0),
                                           (1, 5, 16, 48, 0.02)])
def test_dn_prefill_shapes(ctx, B, T, nqk, nv, S0):
    """Ragged T (partial last chunk), several sequences, nv = 3 nqk (QK head
    sharing), a nonzero initial state, and head counts off the XCD grouping."""
    from vx27_amd import workloads as W
    d = W.dn_prefill(B=B, T=T, nqk=nqk, nv=nv, S0_std=S0)
    say(f"dn_prefill: B={B} T={T} nqk={nqk} nv={nv} S0_std={S0}")
    out, S = run_dn_prefill(ctx, d)
    ref, Sr, _ = oracle_dn_prefill(d)
    check_bf16(out, ref, "out")
    check_bf16(S, Sr, "state")
    assert maxabs(out, ref) <= X3_REL * np.abs(ref).max() and maxabs(S, Sr) <= X3_REL * np.abs(Sr).max()
    ob, Sb = run_dn_prefill(ctx, d, flags=32)   # VX27_DN_BF16
    check_bf16(ob, ref, "out (bf16 products)")
    check_bf16(Sb, Sr, "state (bf16 products)")


def test_dn_prefill_split_prompt(ctx):
    """A prompt prefilled in two calls at a chunk boundary (state carried in
    global memory) equals the one-call result bit for bit."""
    from vx27_amd import workloads as W
    d = W.dn_prefill(B=2, T=384, nqk=4, nv=8, S0_std=0.02, config=41)
    out, S = run_dn_prefill(ctx, d)
    o1, S1 = run_dn_prefill(ctx, d, t0=0, t1=128)
    o2, S2 = run_dn_prefill(ctx, d, S=S1, t0=128, t1=384)
    assert np.array_equal(np.concatenate([o1, o2], axis=1), out)
    assert np.array_equal(S2, S)


# ------------------------------------------------------------------ GQA
def run_gqa_prefill(ctx, d, L, prior=None, interleave=False, flags=0, rope_dim=64, stale=0xFF):
    """Prefill the workload's T tokens at positions pos0.. into a fresh cache of
    capacity L (rows < pos0 from `prior` = (k, v) fp32 [B][pos0][n_kv][256],
    every other row filled with the byte `stale`); returns out [B][T][n_q][256]."""
    from vx27_amd import lib as L_
    lib = L_.lib()
    B, T, n_q, hd = d["q"].shape
    n_kv = d["k"].shape[2]
    pos0 = d["pos0"]
    kc = ctx.buf(B * n_kv * L * hd * 2)
    vc = ctx.buf(B * n_kv * L * hd * 2)
    lib.vx27_hip_memset(ctx.h, kc.ptr, stale, kc.nbytes)       # 0xFF: stale rows hold NaN bit patterns
    lib.vx27_hip_memset(ctx.h, vc.ptr, stale, vc.nbytes)
    keep = []
    if prior is not None:
        for b in range(B):
            kb, vb = ctx.put(np.ascontiguousarray(prior[0][b])), ctx.put(np.ascontiguousarray(prior[1][b]))
            L_.check(lib.vx27_hip_kv_write(ctx.h, kc.ptr, vc.ptr, B, n_kv, hd, L, b, 0, pos0, kb.ptr, vb.ptr),
                     "kv_write")
            keep += [kb, vb]
    if interleave:
        qg = np.empty((B, T, n_q, 2, hd), np.uint16)
        qg[:, :, :, 0], qg[:, :, :, 1] = d["q"], d["gate"]
        qb = ctx.put(qg)
        qp, gp, ts, hs = qb.ptr, qb.ptr + hd * 2, n_q * 2 * hd, 2 * hd
    else:
        qb, gb = ctx.put(d["q"]), ctx.put(d["gate"])
        keep.append(gb)
        qp, gp, ts, hs = qb.ptr, gb.ptr, 0, 0
    kn, vn = ctx.put(d["k"]), ctx.put(d["v"])
    qw, kw = ctx.put(d["q_norm_w"]), ctx.put(d["k_norm_w"])
    ob = ctx.buf(B * T * n_q * hd * 4)
    desc = L_.GqaPrefillDesc(B, T, n_q, n_kv, hd, rope_dim, 1e7, 1.0, L, pos0, flags, qp, ts, hs, gp, ts, hs,
                             kn.ptr, vn.ptr, qw.ptr, kw.ptr, kc.ptr, vc.ptr, ob.ptr)
    L_.check(lib.vx27_hip_gqa_prefill(ctx.h, C.byref(desc)), "gqa_prefill")
    out = ob.download((B, T, n_q, hd), np.float32)
    for bb in keep + [qb, kn, vn, qw, kw, ob, kc, vc]:
        bb.free()
    return out


def oracle_gqa_prefill(d, L, prior=None, no_gate=False, rope_dim=64):
    from oracle import oracle as O
    from vx27_amd import workloads as W
    B, T, n_q, hd = d["q"].shape
    n_kv = d["k"].shape[2]
    f = {k: np.ascontiguousarray(W.bf16_to_f32(d[k])) for k in ("q", "gate", "k", "v")}
    qw, kw = np.ascontiguousarray(d["q_norm_w"]), np.ascontiguousarray(d["k_norm_w"])
    kc = np.zeros((B, L, n_kv, hd), np.float32)
    vc = np.zeros((B, L, n_kv, hd), np.float32)
    if prior is not None:
        kc[:, :d["pos0"]], vc[:, :d["pos0"]] = prior
    out = np.empty((B, T, n_q, hd), np.float32)
    a = O.GqaPrefillArgs(B, T, n_q, n_kv, hd, rope_dim, d["pos0"], L, O.default_threads(), 1e7, 1.0,
                         f["q"].ctypes.data, f["gate"].ctypes.data, f["k"].ctypes.data, f["v"].ctypes.data,
                         qw.ctypes.data, kw.ctypes.data, kc.ctypes.data, vc.ctypes.data, out.ctypes.data,
                         int(no_gate))
    secs = O.lib().orc_gqa_prefill(C.byref(a))
    return out, secs


def test_gqa_prefill_4096(ctx):
    """One 4096-token prompt, 24Q/4KV hd 256 (the prefill workload)."""
    from vx27_amd import workloads as W
    d = W.gqa_prefill(B=1, T=4096)
    say("gqa_prefill: B=1 T=4096")
    out = run_gqa_prefill(ctx, d, 4096)
    ref, secs = oracle_gqa_prefill(d, 4096)
    say(f"  oracle {secs:.2f}s")
    check_bf16(out, ref, "out")


@pytest.mark.parametrize("B,T,pos0,L,inter", [(2, 200, 100, 320, False), (1, 130, 0, 192, True),
                                              (3, 1, 63, 64, False), (1, 300, 37, 384, True)])
def test_gqa_prefill_shapes(ctx, B, T, pos0, L, inter):
    """Ragged T, an earlier context in the cache (pos0 > 0, unaligned), one
    token, the interleaved q_proj layout, and stale NaN rows past the end."""
    from vx27_amd import workloads as W
    d = W.gqa_prefill(B=B, T=T, pos0=pos0, config=51)
    say(f"gqa_prefill: B={B} T={T} pos0={pos0} L={L} interleaved={inter}")
    prior = None
    if pos0:
        r = W.rng(52, "gqa_prefill_prior")
        prior = tuple(W.bf16_to_f32(W.bf16_bits(W.normal(r, (B, pos0, 4, 256)))) for _ in range(2))
    out = run_gqa_prefill(ctx, d, L, prior, inter)
    ref, _ = oracle_gqa_prefill(d, L, prior)
    check_bf16(out, ref, "out")


@pytest.mark.parametrize("B,T,pos0,L", [(1, 1300, 0, 1408), (2, 200, 100, 320), (1, 40, 0, 64), (1, 97, 20, 128)])
def test_gqa_prefill_stale_rows_inert(ctx, B, T, pos0, L):
    """Cache rows past pos0 + T take no part in any output bit: the same
    prefill over caches whose stale rows hold zeros, huge finite values
    (bf16 0x7F7F) and NaNs gives identical outputs.  The shapes leave the
    last query block partly (or, for whole waves, entirely) past T, the rows
    whose positions run into the stale keys."""
    from vx27_amd import workloads as W
    d = W.gqa_prefill(B=B, T=T, pos0=pos0, config=55)
    say(f"gqa_prefill stale rows: B={B} T={T} pos0={pos0} L={L}")
    prior = None
    if pos0:
        r = W.rng(56, "gqa_prefill_prior")
        prior = tuple(W.bf16_to_f32(W.bf16_bits(W.normal(r, (B, pos0, 4, 256)))) for _ in range(2))
    outs = [run_gqa_prefill(ctx, d, L, prior, stale=f) for f in (0x00, 0x7F, 0xFF)]
    assert np.isfinite(outs[0]).all()
    for o, f in zip(outs[1:], ("0x7F", "0xFF")):
        assert np.array_equal(o, outs[0]), f"stale rows filled with {f} change the output"


@pytest.mark.parametrize("rope_dim", [0, 128])
def test_gqa_prefill_rope_dims(ctx, rope_dim):
    """rope_dim 0 (no rotation) and 128 (RoPE pairs 64 dims apart) over an
    unaligned earlier context."""
    from vx27_amd import workloads as W
    B, T, pos0, L = 2, 150, 21, 192
    d = W.gqa_prefill(B=B, T=T, pos0=pos0, config=61)
    r = W.rng(62, "gqa_prefill_prior")
    prior = tuple(W.bf16_to_f32(W.bf16_bits(W.normal(r, (B, pos0, 4, 256)))) for _ in range(2))
    say(f"gqa_prefill: B={B} T={T} pos0={pos0} rope_dim={rope_dim}")
    out = run_gqa_prefill(ctx, d, L, prior, rope_dim=rope_dim)
    ref, _ = oracle_gqa_prefill(d, L, prior, rope_dim=rope_dim)
    check_bf16(out, ref, "out")


def test_gqa_prefill_no_gate(ctx):
    """VX27_GQA_NO_GATE on the prefill (the MTP drafter's batch verify with
    use_gate = 0, vx27_mtp.c:258): ragged T, an earlier context."""
    from vx27_amd import lib as L_, workloads as W
    B, T, pos0, L = 1, 250, 40, 320
    d = W.gqa_prefill(B=B, T=T, pos0=pos0, config=58)
    r = W.rng(59, "gqa_prefill_prior")
    prior = tuple(W.bf16_to_f32(W.bf16_bits(W.normal(r, (B, pos0, 4, 256)))) for _ in range(2))
    say(f"gqa_prefill: B={B} T={T} pos0={pos0}, no gate")
    out = run_gqa_prefill(ctx, d, L, prior, flags=L_.GQA_NO_GATE)
    ref, _ = oracle_gqa_prefill(d, L, prior, no_gate=True)
    check_bf16(out, ref, "out")


def test_gqa_prefill_wide_scores(ctx):
    """Scores hundreds of log2 units apart, exact in bf16: raw q and k rows
    one-hot (+-1) in an unrotated dim 64..127 whose norm weight has 1+w = 4,
    so after rmsn every score is 0 or +-(64*64/16)*log2(e), and equal scores
    stay equal after rounding.  A query whose matching key first appears
    after its first key tile overflows fp32 against that tile's max: the
    attention kernel's overflow check must catch it and redo the query with
    the rescaling (online) softmax.  Ragged T, stale NaN rows past the end."""
    from vx27_amd import workloads as W
    B, T, L, n_q, n_kv = 1, 300, 320, 24, 4
    d = W.gqa_prefill(B=B, T=T, config=55)
    r = W.rng(56, "gqa_wide")
    def one_hot(shape):
        x = np.zeros(shape + (256,), np.float32)
        dim = r.integers(64, 128, size=shape)
        sgn = np.where(r.random(shape) < 0.5, -1.0, 1.0)
        np.put_along_axis(x, dim[..., None], sgn[..., None], axis=-1)
        return W.bf16_bits(x)
    d["q"], d["k"] = one_hot((B, T, n_q)), one_hot((B, T, n_kv))
    w = np.zeros(256, np.float32)
    w[64:128] = 3.0
    d["q_norm_w"], d["k_norm_w"] = w.copy(), w.copy()
    say("gqa_prefill: B=1 T=300 L=320, one-hot q/k with scores 0 or +-369 (log2 units)")
    out = run_gqa_prefill(ctx, d, L)
    ref, _ = oracle_gqa_prefill(d, L)
    check_bf16(out, ref, "out")


def test_gqa_prefill_graph():
    """gqa_prefill captured in a HIP graph on a fresh context, for a shape not
    seen outside the capture (1300 tokens: more (query tile, head) items than
    CUs): the attention kernel then runs as one workgroup per item instead of
    from a per-CU schedule (which is built and uploaded outside captures
    only).  Every replay, with eager work between replays, must equal the
    eager (scheduled) call bit for bit."""
    from vx27_amd import lib as L_, workloads as W
    lib = L_.lib()
    c = L_.Ctx(0)
    try:
        def make(T, Lc):
            d = W.gqa_prefill(B=1, T=T, config=57)
            kc, vc = c.buf(4 * Lc * 256 * 2), c.buf(4 * Lc * 256 * 2)
            bufs = {k: c.put(d[k]) for k in ("q", "gate", "k", "v", "q_norm_w", "k_norm_w")}
            ob = c.buf(T * 24 * 256 * 4)
            desc = L_.GqaPrefillDesc(1, T, 24, 4, 256, 64, 1e7, 1.0, Lc, 0, 0, bufs["q"].ptr, 0, 0,
                                     bufs["gate"].ptr, 0, 0, bufs["k"].ptr, bufs["v"].ptr, bufs["q_norm_w"].ptr,
                                     bufs["k_norm_w"].ptr, kc.ptr, vc.ptr, ob.ptr)
            return d, desc, ob, list(bufs.values()) + [kc, vc, ob]
        _, big, _, keep_big = make(300, 320)       # sizes the scratch (and caches its own schedule)
        L_.check(lib.vx27_hip_gqa_prefill(c.h, C.byref(big)), "gqa_prefill")
        c.sync()
        d, desc, ob, keep = make(1300, 1344)
        c.graph_begin()
        L_.check(lib.vx27_hip_gqa_prefill(c.h, C.byref(desc)), "gqa_prefill (capture)")
        g = c.graph_end()
        assert c.mem_info()["schedules"] == 0    # nothing was built inside the capture
        try:
            replays = []
            for _ in range(3):
                c.graph_launch(g)
                c.sync()
                replays.append(ob.download((1, 1300, 24, 256), np.float32))
                L_.check(lib.vx27_hip_gqa_prefill(c.h, C.byref(big)), "gqa_prefill")   # eager work between
                c.sync()
        finally:
            lib.vx27_hip_graph_destroy(g)
        L_.check(lib.vx27_hip_gqa_prefill(c.h, C.byref(desc)), "gqa_prefill")       # eager, scheduled
        c.sync()
        assert c.mem_info()["schedules"] == 1
        eager = ob.download((1, 1300, 24, 256), np.float32)
        for i, r in enumerate(replays):
            assert np.array_equal(r, eager), f"graph replay {i} differs from the eager call"
        ref, _ = oracle_gqa_prefill(d, 1344)
        check_bf16(eager, ref, "out")
        for bb in keep + keep_big:
            bb.free()
    finally:
        c.close()


def test_prefill_deterministic(ctx):
    """Both prefills are deterministic: the same call twice gives identical
    bits (the kernels use fixed reduction orders; a missed wait on an
    asynchronous tile load would show up here as run-to-run differences)."""
    from vx27_amd import workloads as W
    d = W.gqa_prefill(B=1, T=2048, config=53)
    a = run_gqa_prefill(ctx, d, 2048)
    b = run_gqa_prefill(ctx, d, 2048)
    assert np.array_equal(a, b), "gqa prefill differs between identical calls"
    e = W.dn_prefill(B=1, T=2048, config=54)
    o1, S1 = run_dn_prefill(ctx, e)
    o2, S2 = run_dn_prefill(ctx, e)
    assert np.array_equal(o1, o2) and np.array_equal(S1, S2), "dn prefill differs between identical calls"


def test_gqa_prefill_norm_w(ctx):
    """VX27_GQA_NORM_W: q/k norm as x*s*w (vx27_gqa.c:10-15's form).  The
    oracle runs the (1+w) form with w - 1: for w in [0.5, 2] the difference
    is exact (Sterbenz) and (w - 1) + 1 == w, so both forms multiply by the
    same float."""
    from vx27_amd import lib as L_, workloads as W
    B, T, pos0, L = 1, 300, 0, 320
    d = W.gqa_prefill(B=B, T=T, pos0=pos0, config=60)
    r = W.rng(60, "norm_w")
    w_q = np.clip(W.normal(r, 256, 0.1, 1.0), 0.5, 2.0).astype(np.float32)
    w_k = np.clip(W.normal(r, 256, 0.1, 1.0), 0.5, 2.0).astype(np.float32)
    dev = dict(d, q_norm_w=w_q, k_norm_w=w_k)
    orc = dict(d, q_norm_w=(w_q - np.float32(1)).astype(np.float32), k_norm_w=(w_k - np.float32(1)).astype(np.float32))
    assert np.array_equal(orc["q_norm_w"] + np.float32(1), w_q)
    out = run_gqa_prefill(ctx, dev, L, None, flags=L_.GQA_NORM_W)
    ref, _ = oracle_gqa_prefill(orc, L)
    check_bf16(out, ref, "norm_w prefill")
    # the flag changes the answer (the (1+w) form with the same w differs)
    alt, _ = oracle_gqa_prefill(dev, L)
    assert np.abs(alt - ref).max() > 1e-2
