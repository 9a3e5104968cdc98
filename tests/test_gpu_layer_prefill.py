"""GPU parity of the layer-level batched steps (the device form of
vx27_qlayer_batch's mixer branches, vx27_qfwd.c:249-376, as
vx27_engine_batch_step runs them per layer, vx27_run.c:187-238): T tokens of
each sequence through projections, mixer core and output projection.

DeltaNet: with checkpoints (the exact recurrence) bit for bit equal to T
calls of vx27_hip_dn_layer_decode, states and checkpoints included, and
within 1e-5 of the oracle's layer glue applied token by token; the chunked
default (split-precision products) on the oracle's outputs within 1e-3 of
max|ref| and the bf16 bar.  GQA: the attention bar and 2% of max|ref| against
the oracle's per-token layer (q/k/v enter the prefill attention as bf16).
From 256 tokens on, the projections run in the long-prompt GEMM: 4096-token
prompts of both layers, checked on a 256-token prefix, and two-sequence
calls of 280 and 300 rows (ragged tiles, a token tile shared by both
sequences), checked whole."""
import ctypes as C

import numpy as np
import pytest

from gpu_common import maxabs, oracle_dn_layer, oracle_gqa_layer, say
from test_gpu_layers import H, dn_layer_inputs, gqa_layer_inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from vx27_amd import lib as L
    c = L.Ctx(0)
    yield c
    c.close()


def dn_device(ctx, w):
    dev = {k: ctx.put(w[k]) for k in ("conv_w_bf16", "A_log", "dt_bias", "norm_w")}
    dev["w_in"], dev["w_out"] = ctx.put_tiled(w["w_in"]), ctx.put_tiled(w["w_out"])
    return dev


def run_dn_layer_prefill(ctx, dev, x, S, conv, flags=0, ckpt=False, nqk=16, nv=48):
    from vx27_amd import lib as L
    B, T, _ = x.shape
    C_ = conv.shape[1]
    Sd, cd, xb = ctx.put(S), ctx.put(conv), ctx.put(x)
    ob = ctx.buf(B * T * H * 4)
    d = L.DnLayerPrefillDesc(B, T, nqk, nv, 128, H, flags, xb.ptr, dev["w_in"].ptr, dev["w_out"].ptr,
                             dev["conv_w_bf16"].ptr, L.BF16, dev["A_log"].ptr, dev["dt_bias"].ptr, dev["norm_w"].ptr,
                             Sd.ptr, cd.ptr, ob.ptr)
    sk = ck = None
    if ckpt:
        sk, ck = ctx.buf(B * T * nv * 128 * 128 * 4), ctx.buf(B * T * C_ * 3 * 4)
        d.S_ckpt, d.conv_ckpt = sk.ptr, ck.ptr
    L.check(L.lib().vx27_hip_dn_layer_prefill(ctx.h, C.byref(d)), "dn_layer_prefill")
    res = {"out": ob.download((B, T, H), np.float32), "S": Sd.download(S.shape, np.float32),
           "conv": cd.download(conv.shape, np.float32)}
    if ckpt:
        res["S_ckpt"] = sk.download((B, T, nv, 128, 128), np.float32)
        res["conv_ckpt"] = ck.download((B, T, C_, 3), np.float32)
    for b in (Sd, cd, xb, ob) + ((sk, ck) if ckpt else ()):
        b.free()
    return res


def test_dn_layer_prefill_verify_window(ctx):
    """B = 2 sequences x T = 8 tokens with checkpoints (the MTP verify batch)."""
    from vx27_amd import lib as L, workloads as W
    B, T, nqk, nv = 2, 8, 16, 48
    r = W.rng(12, "dn_layer_prefill")
    w, S, conv = dn_layer_inputs(r, B, nqk, nv)
    x = W.normal(r, (B, T, H))
    dev = dn_device(ctx, w)
    g = run_dn_layer_prefill(ctx, dev, x, S, conv, ckpt=True)
    # T single-token layer calls on the same start state
    Sd, cd = ctx.put(S), ctx.put(conv)
    xb, ob = ctx.buf(B * H * 4), ctx.buf(B * H * 4)
    d = L.DnLayerDesc(B, nqk, nv, 128, H, xb.ptr, None, dev["w_in"].ptr, dev["w_out"].ptr, dev["conv_w_bf16"].ptr,
                      L.BF16, dev["A_log"].ptr, dev["dt_bias"].ptr, dev["norm_w"].ptr, Sd.ptr, cd.ptr, ob.ptr)
    for t in range(T):
        xb.upload(np.ascontiguousarray(x[:, t]))
        L.check(L.lib().vx27_hip_dn_layer_decode(ctx.h, C.byref(d)), "dn_layer")
        assert np.array_equal(ob.download((B, H), np.float32), g["out"][:, t]), f"out token {t}"
        assert np.array_equal(Sd.download(S.shape, np.float32), g["S_ckpt"][:, t]), f"S checkpoint {t}"
        assert np.array_equal(cd.download(conv.shape, np.float32), g["conv_ckpt"][:, t]), f"conv checkpoint {t}"
    say("  verify window: bit-exact to 8 single-token layer calls (outputs, states, checkpoints)")
    Sr, cr = S.copy(), conv.copy()
    worst = 0.0
    for t in range(T):
        ref = oracle_dn_layer(w, np.ascontiguousarray(x[:, t]), Sr, cr, nqk, nv)
        worst = max(worst, maxabs(g["out"][:, t], ref))
    say(f"  vs oracle: max|d out|={worst:.3e} max|d S|={maxabs(g['S'], Sr):.3e}")
    assert worst <= 1e-5 and maxabs(g["S"], Sr) <= 1e-5


@pytest.mark.parametrize("B,T", [(1, 130), (2, 150)])
def test_dn_layer_prefill_chunked(ctx, B, T):
    """The chunked default on a 130-token prompt of one sequence (three
    chunks, the last one ragged, so the state crosses chunk boundaries), and
    on 2 x 150 tokens: 300 rows take the long-prompt GEMM, with the second
    sequence's tokens inside the first token tile, and the gated norm writes
    out_proj's packed tokens, its last block of 16 ragged."""
    from vx27_amd import workloads as W
    nqk, nv = 16, 48
    r = W.rng(13, f"dn_layer_prefill_chunked{B}x{T}")
    w, S, conv = dn_layer_inputs(r, B, nqk, nv)
    x = W.normal(r, (B, T, H))
    dev = dn_device(ctx, w)
    g = run_dn_layer_prefill(ctx, dev, x, S, conv)
    Sr, cr = S.copy(), conv.copy()
    ref = np.stack([oracle_dn_layer(w, np.ascontiguousarray(x[:, t]), Sr, cr, nqk, nv) for t in range(T)], axis=1)
    err = np.abs(g["out"].astype(np.float64) - ref)
    big = np.abs(ref).max()
    say(f"  chunked: max|d out|={err.max():.3e} (max|ref|={big:.3f}) max|d S|={maxabs(g['S'], Sr):.3e}")
    # split-precision products: within 1e-4 of max|ref| (single bf16 products reach ~4e-3)
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)) and err.max() <= 1e-4 * big
    assert maxabs(g["S"], Sr) <= 1e-4 * np.abs(Sr).max()
    # the conv state holds projection outputs of the last tokens: below 256
    # rows the GEMV's exact activations (fp32 MFMA sums vs the oracle's double
    # sums: 1e-5); from 256 rows the GEMM's two-part activations, within its
    # bound of 2^-15 sum_k |W||x| per output (as in test_gpu_gemm)
    if B * T < 256:
        assert maxabs(g["conv"], cr) <= 1e-5
    else:
        Wc = np.abs(W.bf16_to_f32(w["w_in"][:conv.shape[1]]).astype(np.float64))
        mag = np.stack([np.abs(x[:, T - 3 + j]).astype(np.float64) @ Wc.T for j in range(3)], axis=-1)
        bound = 2.0 ** -15 * mag.max(axis=-1, keepdims=True)
        say(f"  conv state: max|d|={maxabs(g['conv'], cr):.3e}, max of |d| / bound "
            f"{float(np.max(np.abs(g['conv'].astype(np.float64) - cr) / bound)):.3f}")
        assert np.all(np.abs(g["conv"].astype(np.float64) - cr) <= bound)


@pytest.mark.parametrize("B,T,Lcap,pos0", [(2, 8, 320, 300), (2, 140, 192, 10)])
def test_gqa_layer_prefill(ctx, B, T, Lcap, pos0):
    """B = 2 sequences x T = 8 tokens at positions 300.. of a 320-row cache,
    and x 140 tokens at positions 10.. (280 rows: the long-prompt GEMM, the
    second sequence's tokens inside the first token tile)."""
    from vx27_amd import lib as L, mixers as M, workloads as W
    r = W.rng(14, "gqa_layer_prefill" if T == 8 else f"gqa_layer_prefill{B}x{T}")
    w, kc, vc = gqa_layer_inputs(r, B, Lcap, pos0)
    x = W.normal(r, (B, T, H))
    lay = M.GatedGQALayer(ctx, B, Lcap, w["q_norm_w"], w["k_norm_w"])
    for b in range(B):
        lay.write_kv(b, 0, W.bf16_to_f32(kc[b, :pos0]), W.bf16_to_f32(vc[b, :pos0]))
    wq, wo = ctx.put_tiled(w["w_qkv"]), ctx.put_tiled(w["w_o"])
    xb, ob = ctx.put(x), ctx.buf(B * T * H * 4)
    d = L.GqaLayerPrefillDesc(B, T, 24, 4, 256, H, 64, 1e7, 1.0, Lcap, pos0, 0, xb.ptr, wq.ptr, wo.ptr,
                              lay.q_norm_w.ptr, lay.k_norm_w.ptr, lay.k_cache.ptr, lay.v_cache.ptr, ob.ptr)
    L.check(L.lib().vx27_hip_gqa_layer_prefill(ctx.h, C.byref(d)), "gqa_layer_prefill")
    out = ob.download((B, T, H), np.float32)
    ref = np.stack([oracle_gqa_layer(w, np.ascontiguousarray(x[:, t]), kc, vc, np.full(B, pos0 + t, np.int32))
                    for t in range(T)], axis=1)
    err = np.abs(out.astype(np.float64) - ref)
    big = np.abs(ref).max()
    say(f"  gqa layer prefill: max|d|={err.max():.3e} (max|ref|={big:.3f})")
    assert np.all(np.isfinite(out))
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)) and err.max() <= 0.02 * big


def test_dn_layer_prefill_long_prompt(ctx):
    """A 4096-token prompt through the DeltaNet layer (nqk 16, nv 48, hidden
    5120): the projections run in the long-prompt GEMM (x as two bf16 parts)
    and the core in the chunked form.  Its first 256 outputs depend on the
    first 256 tokens only, so they are checked against the oracle's per-token
    layer on that prefix, to the chunked form's bar (1e-4 of max|ref|)."""
    import time
    from vx27_amd import workloads as W
    B, T, P, nqk, nv = 1, 4096, 256, 16, 48
    r = W.rng(15, "dn_layer_prefill_long")
    w, S, conv = dn_layer_inputs(r, B, nqk, nv)
    x = W.normal(r, (B, T, H))
    dev = dn_device(ctx, w)
    g = run_dn_layer_prefill(ctx, dev, x, S, conv)
    assert np.all(np.isfinite(g["out"])) and np.all(np.isfinite(g["S"]))
    t0 = time.perf_counter()
    Sr, cr = S.copy(), conv.copy()
    ref = np.stack([oracle_dn_layer(w, np.ascontiguousarray(x[:, t]), Sr, cr, nqk, nv) for t in range(P)], axis=1)
    err = np.abs(g["out"][:, :P].astype(np.float64) - ref)
    big = np.abs(ref).max()
    say(f"  4096-token layer, first {P} tokens: max|d out|={err.max():.3e} (max|ref|={big:.3f}); "
        f"oracle {time.perf_counter() - t0:.1f}s")
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)) and err.max() <= 1e-4 * big


def test_gqa_layer_prefill_long_prompt(ctx):
    """A 4096-token prompt through the gated GQA layer from position 0: the
    projections run in the long-prompt GEMM; the first 256 outputs against the
    oracle's per-token layer (the attention bar)."""
    from vx27_amd import lib as L, mixers as M, workloads as W
    B, T, P, Lcap = 1, 4096, 256, 4096
    r = W.rng(16, "gqa_layer_prefill_long")
    w, kc, vc = gqa_layer_inputs(r, B, Lcap, 0)
    x = W.normal(r, (B, T, H))
    lay = M.GatedGQALayer(ctx, B, Lcap, w["q_norm_w"], w["k_norm_w"])
    wq, wo = ctx.put_tiled(w["w_qkv"]), ctx.put_tiled(w["w_o"])
    xb, ob = ctx.put(x), ctx.buf(B * T * H * 4)
    d = L.GqaLayerPrefillDesc(B, T, 24, 4, 256, H, 64, 1e7, 1.0, Lcap, 0, 0, xb.ptr, wq.ptr, wo.ptr,
                              lay.q_norm_w.ptr, lay.k_norm_w.ptr, lay.k_cache.ptr, lay.v_cache.ptr, ob.ptr)
    L.check(L.lib().vx27_hip_gqa_layer_prefill(ctx.h, C.byref(d)), "gqa_layer_prefill")
    out = ob.download((B, T, H), np.float32)
    assert np.all(np.isfinite(out))
    ref = np.stack([oracle_gqa_layer(w, np.ascontiguousarray(x[:, t]), kc, vc, np.full(B, t, np.int32))
                    for t in range(P)], axis=1)
    err = np.abs(out[:, :P].astype(np.float64) - ref)
    big = np.abs(ref).max()
    say(f"  4096-token gqa layer, first {P} tokens: max|d|={err.max():.3e} (max|ref|={big:.3f})")
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)) and err.max() <= 0.02 * big
