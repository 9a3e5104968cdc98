"""Captured HIP graphs and the context's scratch memory.

A captured graph keeps the raw addresses of the context scratch and of the
prefill schedules it was captured with.  The context must not free them
while the graph can still be replayed, even when a later eager call grows
the scratch or prefills a prompt of a new shape.  Regression test: eager(A),
capture(A), eager calls that grow the scratch and add a schedule, new
allocations that could take the freed memory, replay(A) == eager(A) bit for
bit; then a capture of a call whose scratch is not sized yet fails cleanly.
"""
import ctypes as C

import numpy as np
import pytest

from gpu_common import say

pytestmark = pytest.mark.gpu


def test_graph_survives_scratch_growth():
    from vx27_amd import lib as L, mixers as M, workloads as W
    lib = L.lib()
    with L.Ctx(0) as ctx:
        # A: a gated GQA decode step of 2 sequences (scratch: q, split partials)
        d = W.gqa_decode(B=2, L=300, config=41)
        Lcap = 320
        lay = M.GatedGQALayer(ctx, 2, Lcap, d["q_norm_w"], d["k_norm_w"])
        for b in range(2):
            lay.write_kv(b, 0, W.bf16_to_f32(d["K"][b]), W.bf16_to_f32(d["V"][b]))
        hd, n_q = 256, 24
        qb, kb, vb = ctx.put(d["qg"]), ctx.put(d["k_new"]), ctx.put(d["v_new"])
        pb, ob = ctx.put(d["pos"]), ctx.buf(2 * n_q * hd * 4)
        desc = lay.desc(pb.ptr, qb.ptr, (n_q * 2 * hd, 2 * hd), qb.ptr + hd * 4, (n_q * 2 * hd, 2 * hd),
                        kb.ptr, vb.ptr, ob.ptr)

        def run_a():
            L.check(lib.vx27_hip_gqa_decode(ctx.h, C.byref(desc)), "gqa_decode")

        run_a()
        eager = ob.download((2, n_q, hd), np.float32)
        ctx.graph_begin()
        run_a()
        g = ctx.graph_end()
        say("  captured A")
        # B: a 2048-token DeltaNet prefill (tens of MB of chunk records: the
        # scratch grows) and a GQA prefill of a shape not seen (a new schedule)
        dp = W.dn_prefill(B=1, T=2048, config=42)
        bufs = {k: ctx.put(dp[k]) for k in ("q", "k", "v", "a", "b", "A_log", "dt_bias", "S0")}
        po = ctx.buf(2048 * 16 * 128 * 4)
        pd = L.DnPrefillDesc(1, 2048, 16, 16, 128, 0, bufs["S0"].ptr, bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr,
                             bufs["a"].ptr, bufs["b"].ptr, bufs["A_log"].ptr, bufs["dt_bias"].ptr, po.ptr)
        L.check(lib.vx27_hip_dn_prefill(ctx.h, C.byref(pd)), "dn_prefill")
        # (1300 tokens: 11 query tiles x 24 heads, more items than CUs, so a schedule is built)
        gp = W.gqa_prefill(B=1, T=1300, config=43)
        gb = {k: ctx.put(gp[k]) for k in ("q", "gate", "k", "v", "q_norm_w", "k_norm_w")}
        kc, vc, go = ctx.buf(4 * 1344 * 256 * 2), ctx.buf(4 * 1344 * 256 * 2), ctx.buf(1300 * 24 * 256 * 4)
        gd = L.GqaPrefillDesc(1, 1300, 24, 4, 256, 64, 1e7, 1.0, 1344, 0, 0, gb["q"].ptr, 0, 0, gb["gate"].ptr, 0,
                              0, gb["k"].ptr, gb["v"].ptr, gb["q_norm_w"].ptr, gb["k_norm_w"].ptr, kc.ptr, vc.ptr,
                              go.ptr)
        L.check(lib.vx27_hip_gqa_prefill(ctx.h, C.byref(gd)), "gqa_prefill")
        ctx.sync()
        say("  eager B calls done (scratch grown, new schedule)")
        # new allocations that would take freed memory, filled with garbage
        junk = [ctx.buf(1 << 20) for _ in range(8)]
        for j, bj in enumerate(junk):
            ctx.fill_normal(bj, (1 << 20) // 4, 900 + j, 1e30)
        ob.zero()
        try:
            for rep in range(3):
                ctx.graph_launch(g)
                ctx.sync()
                got = ob.download((2, n_q, hd), np.float32)
                say(f"  replay {rep}: equal to eager = {np.array_equal(got, eager)}")
                assert np.array_equal(got, eager), rep
                run_a()                       # eager A between replays, same answer
                ctx.sync()
                assert np.array_equal(ob.download((2, n_q, hd), np.float32), eager)
        finally:
            L.check(lib.vx27_hip_graph_destroy(g), "graph_destroy")
        # after the last graph is gone the retired memory is released; calls still work
        L.check(lib.vx27_hip_dn_prefill(ctx.h, C.byref(pd)), "dn_prefill")
        run_a()
        ctx.sync()
        assert np.array_equal(ob.download((2, n_q, hd), np.float32), eager)


def test_capture_needing_scratch_fails_cleanly():
    """Inside a capture, a call whose scratch is not yet sized returns -1
    with a message (no allocation in the capture); the capture still ends."""
    from vx27_amd import lib as L, workloads as W
    lib = L.lib()
    with L.Ctx(0) as ctx:
        dp = W.dn_prefill(B=1, T=512, config=44)
        bufs = {k: ctx.put(dp[k]) for k in ("q", "k", "v", "a", "b", "A_log", "dt_bias", "S0")}
        po = ctx.buf(512 * 16 * 128 * 4)
        pd = L.DnPrefillDesc(1, 512, 16, 16, 128, 0, bufs["S0"].ptr, bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr,
                             bufs["a"].ptr, bufs["b"].ptr, bufs["A_log"].ptr, bufs["dt_bias"].ptr, po.ptr)
        pos = ctx.put(np.zeros(4, np.int32))
        ctx.graph_begin()
        L.check(lib.vx27_hip_advance_pos(ctx.h, pos.ptr, 4), "advance_pos")   # one node in the graph
        rc = lib.vx27_hip_dn_prefill(ctx.h, C.byref(pd))
        msg = lib.vx27_hip_last_error().decode()
        g = ctx.graph_end()
        L.check(lib.vx27_hip_graph_destroy(g), "graph_destroy")
        say(f"  rc={rc}: {msg}")
        assert rc == -1 and "before capturing" in msg
        # the same call outside a capture sizes the scratch and runs
        L.check(lib.vx27_hip_dn_prefill(ctx.h, C.byref(pd)), "dn_prefill")
        ctx.sync()


def test_sync_reports_position_outside_cache():
    """A decode position past the cache is clamped on the device (no access
    leaves the cache) and reported by the next vx27_hip_sync."""
    from vx27_amd import lib as L, mixers as M, workloads as W
    lib = L.lib()
    with L.Ctx(0) as ctx:
        d = W.gqa_decode(B=1, L=60, config=45)
        lay = M.GatedGQALayer(ctx, 1, 64, d["q_norm_w"], d["k_norm_w"])
        lay.decode(np.array([63], np.int32), d["qg"], d["k_new"], d["v_new"])
        ctx.sync()                                    # in range: no report
        lay.decode(np.array([64], np.int32), d["qg"], d["k_new"], d["v_new"])
        with pytest.raises(L.HipError, match="outside its KV cache"):
            ctx.sync()
        # the flag is cleared by the report
        L.check(lib.vx27_hip_sync(ctx.h), "sync")


def test_dn_prefill_graph_replay():
    """A chunked DeltaNet prefill (glue-free, 2048 tokens) captured as a
    graph: every replay, with eager work and synchronisations between
    replays, equals the eager call bit for bit (output and final state)."""
    from vx27_amd import lib as L, workloads as W
    lib = L.lib()
    with L.Ctx(0) as ctx:
        T = 2048
        dp = W.dn_prefill(B=1, T=T, S0_std=0.02, config=44)
        bufs = {k: ctx.put(dp[k]) for k in ("q", "k", "v", "a", "b", "A_log", "dt_bias")}
        S0 = ctx.put(np.ascontiguousarray(dp["S0"], np.float32))
        Sd = ctx.buf(S0.nbytes)
        po = ctx.buf(T * 16 * 128 * 4)
        pd = L.DnPrefillDesc(1, T, 16, 16, 128, 0, Sd.ptr, bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr,
                             bufs["a"].ptr, bufs["b"].ptr, bufs["A_log"].ptr, bufs["dt_bias"].ptr, po.ptr)

        def reset():
            L.check(lib.vx27_hip_d2d(ctx.h, Sd.ptr, S0.ptr, S0.nbytes), "d2d")

        def run():
            L.check(lib.vx27_hip_dn_prefill(ctx.h, C.byref(pd)), "dn_prefill")

        reset(); run(); ctx.sync()
        o_e, S_e = po.download((T, 16, 128), np.float32), Sd.download(dp["S0"].shape, np.float32)
        reset()
        ctx.graph_begin()
        run()
        g = ctx.graph_end()
        try:
            for rep in range(3):
                po.zero()
                reset()
                ctx.graph_launch(g)
                ctx.sync()
                o_g, S_g = po.download((T, 16, 128), np.float32), Sd.download(dp["S0"].shape, np.float32)
                say(f"  replay {rep}: output equal {np.array_equal(o_g, o_e)}, state equal {np.array_equal(S_g, S_e)}")
                assert np.array_equal(o_g, o_e) and np.array_equal(S_g, S_e), rep
                reset(); run(); ctx.sync()     # eager between replays, same answer
                assert np.array_equal(po.download((T, 16, 128), np.float32), o_e)
        finally:
            L.check(lib.vx27_hip_graph_destroy(g), "graph_destroy")


def _gqa_prefill_setup(ctx, T, Lc, config):
    from vx27_amd import lib as L, workloads as W
    d = W.gqa_prefill(B=1, T=T, config=config)
    bufs = {k: ctx.put(d[k]) for k in ("q", "gate", "k", "v", "q_norm_w", "k_norm_w")}
    kc, vc, ob = ctx.buf(4 * Lc * 256 * 2), ctx.buf(4 * Lc * 256 * 2), ctx.buf(T * 24 * 256 * 4)
    desc = L.GqaPrefillDesc(1, T, 24, 4, 256, 64, 1e7, 1.0, Lc, 0, 0, bufs["q"].ptr, 0, 0, bufs["gate"].ptr, 0, 0,
                            bufs["k"].ptr, bufs["v"].ptr, bufs["q_norm_w"].ptr, bufs["k_norm_w"].ptr, kc.ptr, vc.ptr,
                            ob.ptr)
    return desc, ob


def test_schedule_cache_bounded_with_live_graph():
    """Prefills at many distinct start positions while a captured graph is
    alive (a serving loop that keeps a decode graph): the schedule cache
    flushes at 64 shapes and frees the schedules no capture launched, so the
    context keeps only the one schedule the graph uses; that one is released
    when the graph is destroyed.  A short window (one query tile per head)
    builds no schedule at all."""
    from vx27_amd import lib as L
    lib = L.lib()
    with L.Ctx(0) as ctx:
        T, Lc = 1300, 1408
        desc, ob = _gqa_prefill_setup(ctx, T, Lc, 61)
        L.check(lib.vx27_hip_gqa_prefill(ctx.h, C.byref(desc)), "gqa_prefill")   # sizes scratch, caches pos0 = 0
        ctx.sync()
        eager = ob.download((1, T, 24, 256), np.float32)
        ctx.graph_begin()
        L.check(lib.vx27_hip_gqa_prefill(ctx.h, C.byref(desc)), "gqa_prefill (capture)")
        g = ctx.graph_end()
        info0 = ctx.mem_info()
        say(f"  after capture: {info0}")
        try:
            for p0 in range(1, 100):
                desc.pos0 = p0
                L.check(lib.vx27_hip_gqa_prefill(ctx.h, C.byref(desc)), "gqa_prefill")
            ctx.sync()
            info = ctx.mem_info()
            say(f"  after 99 more start positions: {info}")
            assert info["schedules"] <= 64
            assert info["retired"] <= info0["retired"] + 1     # only the captured schedule is kept
            desc.pos0 = 0
            ob.zero()
            ctx.graph_launch(g)
            ctx.sync()
            assert np.array_equal(ob.download((1, T, 24, 256), np.float32), eager)
        finally:
            L.check(lib.vx27_hip_graph_destroy(g), "graph_destroy")
        assert ctx.mem_info()["retired"] == 0 and ctx.mem_info()["live_graphs"] == 0
        # a verify window of 8 tokens at a moving position caches nothing
        n0 = ctx.mem_info()["schedules"]
        small, _ = _gqa_prefill_setup(ctx, 8, 256, 62)
        for p0 in range(0, 80, 8):
            small.pos0 = p0
            L.check(lib.vx27_hip_gqa_prefill(ctx.h, C.byref(small)), "gqa_prefill (window)")
        ctx.sync()
        assert ctx.mem_info()["schedules"] == n0


def test_memset_kernel_and_capture():
    """vx27_hip_memset fills any byte range (unaligned head and tail) by a
    kernel, so it may be captured: a captured fill replays correctly with
    other writes between the replays."""
    from vx27_amd import lib as L
    lib = L.lib()
    with L.Ctx(0) as ctx:
        n = 10007
        buf = ctx.buf(n)
        for off, cnt, byte in ((0, n, 0xAB), (3, 5000, 0x00), (17, 1, 0x7F), (5, 16, 0x11), (1, 40, 0xFE)):
            L.check(lib.vx27_hip_memset(ctx.h, buf.ptr, 0x5A, n), "memset")
            L.check(lib.vx27_hip_memset(ctx.h, buf.ptr + off, byte, cnt), "memset")
            ctx.sync()
            got = buf.download((n,), np.uint8)
            want = np.full(n, 0x5A, np.uint8)
            want[off:off + cnt] = byte
            assert np.array_equal(got, want), (off, cnt, byte)
        ctx.graph_begin()
        L.check(lib.vx27_hip_memset(ctx.h, buf.ptr + 9, 0x33, 9000), "memset (capture)")
        g = ctx.graph_end()
        try:
            for rep in range(3):
                L.check(lib.vx27_hip_memset(ctx.h, buf.ptr, 0xC3, n), "memset")
                ctx.sync()
                ctx.graph_launch(g)
                ctx.sync()
                want = np.full(n, 0xC3, np.uint8)
                want[9:9009] = 0x33
                assert np.array_equal(buf.download((n,), np.uint8), want), rep
        finally:
            L.check(lib.vx27_hip_graph_destroy(g), "graph_destroy")


def test_dn_conv_step_graph_replay():
    """One fused-conv decode step at batch 1 (16 heads, the conv state
    advanced in place by the step kernel) captured as a graph.  Replayed
    once per token with the token's inputs copied into the captured
    buffers, eager calls and synchronisations between replays: every
    output, the state and the conv state equal eager calls bit for bit."""
    from vx27_amd import lib as L, mixers as M, workloads as W
    lib = L.lib()
    with L.Ctx(0) as ctx:
        B, H, steps = 1, 16, 6
        d = W.dn_conv(B=B, H=H, steps=steps, config=12)
        flags = L.DN_CONV | L.DN_PRE_L2
        lay = M.DeltaNetLayer(ctx, B, H, H, d["A_log"], d["dt_bias"], conv_w=d["conv_w_bf16"],
                              conv_w_dtype=L.BF16, S0=d["S0"], conv0=d["conv0"])
        S0 = ctx.put(np.ascontiguousarray(d["S0"], np.float32))
        c0 = ctx.put(np.ascontiguousarray(d["conv0"], np.float32))
        xs, as_, bs = (ctx.put(np.ascontiguousarray(d[k], np.float32)) for k in ("x", "a", "b"))
        xb, ab, bb = ctx.buf(xs.nbytes // steps), ctx.buf(as_.nbytes // steps), ctx.buf(bs.nbytes // steps)
        ob = ctx.buf(B * H * 128 * 4)
        desc = lay.desc(1, flags, ob.ptr, ab.ptr, bb.ptr, x=xb.ptr)

        def reset():
            L.check(lib.vx27_hip_d2d(ctx.h, lay.S.ptr, S0.ptr, S0.nbytes), "d2d")
            L.check(lib.vx27_hip_d2d(ctx.h, lay.conv_state.ptr, c0.ptr, c0.nbytes), "d2d")

        def feed(t):
            for src, dst in ((xs, xb), (as_, ab), (bs, bb)):
                L.check(lib.vx27_hip_d2d(ctx.h, dst.ptr, src.ptr + t * dst.nbytes, dst.nbytes), "d2d")

        def eager_all():
            outs = []
            for t in range(steps):
                feed(t)
                L.check(lib.vx27_hip_dn_decode(ctx.h, C.byref(desc)), "dn_decode")
                outs.append(ob.download((B, H, 128), np.float32))
            return outs, lay.state(), lay.conv()

        reset()
        o_e, S_e, c_e = eager_all()
        reset()
        feed(0)
        ctx.graph_begin()
        L.check(lib.vx27_hip_dn_decode(ctx.h, C.byref(desc)), "dn_decode (capture)")
        g = ctx.graph_end()
        try:
            reset()
            for t in range(steps):
                feed(t)
                ctx.graph_launch(g)
                ctx.sync()
                o_g = ob.download((B, H, 128), np.float32)
                say(f"  replay {t}: output equal {np.array_equal(o_g, o_e[t])}")
                assert np.array_equal(o_g, o_e[t]), t
            S_g, c_g = lay.state(), lay.conv()
            assert np.array_equal(S_g, S_e) and np.array_equal(c_g, c_e)
            reset()
            o_2, S_2, c_2 = eager_all()       # eager again after the replays, same bits
            assert all(np.array_equal(a, b) for a, b in zip(o_2, o_e))
            assert np.array_equal(S_2, S_e) and np.array_equal(c_2, c_e)
        finally:
            L.check(lib.vx27_hip_graph_destroy(g), "graph_destroy")
