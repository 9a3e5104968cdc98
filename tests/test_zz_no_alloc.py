"""vx27_hip_gqa_decode_noalloc: the GQA decode step on the library's static
per-device scratch (no allocation in the call), against vx27_hip_gqa_decode
on the same inputs, through the C ABI: two calls in a row, the second with
a smaller input (the static scratch keeps the first call's contents), bit
for bit, since both run the same kernels on the same scratch layout.  Also:
a call needing more than the static scratch fails with a message."""
import ctypes as C

import numpy as np
import pytest

from gpu_common import oracle_gqa_decode, say

pytestmark = pytest.mark.gpu


def _setup(ctx, B, nk, Lcap, config):
    from vx27_amd import mixers as M, workloads as W
    d = W.gqa_decode(B=B, L=nk, config=config)
    lay = M.GatedGQALayer(ctx, B, Lcap, d["q_norm_w"], d["k_norm_w"])
    for b in range(B):
        lay.write_kv(b, 0, W.bf16_to_f32(d["K"][b]), W.bf16_to_f32(d["V"][b]))
    hd, n_q = 256, 24
    bufs = [ctx.put(d["qg"]), ctx.put(d["k_new"]), ctx.put(d["v_new"]), ctx.put(d["pos"])]
    qb, kb, vb, pb = bufs
    ob = ctx.buf(B * n_q * hd * 4)
    desc = lay.desc(pb.ptr, qb.ptr, (n_q * 2 * hd, 2 * hd), qb.ptr + hd * 4, (n_q * 2 * hd, 2 * hd),
                    kb.ptr, vb.ptr, ob.ptr)
    return d, lay, desc, ob


def test_noalloc_matches_gqa_decode():
    from vx27_amd import lib as L
    lib = L.lib()
    with L.Ctx(0) as ctx:
        for B, nk, Lcap, cfg in ((4, 8192, 8256, 71), (2, 1000, 1024, 72)):
            say(f"noalloc: B={B} keys={nk + 1}")
            d, lay, desc, ob = _setup(ctx, B, nk, Lcap, cfg)
            # reference entry point first (writes the new k,v rows, then attends)
            L.check(lib.vx27_hip_gqa_decode(ctx.h, C.byref(desc)), "gqa_decode")
            ref = ob.download((B, 24, 256), np.float32)
            ob.zero()
            L.check(lib.vx27_hip_gqa_decode_noalloc(ctx.h, C.byref(desc)), "gqa_decode_noalloc")
            ctx.sync()
            got = ob.download((B, 24, 256), np.float32)
            same = np.array_equal(got, ref)
            say(f"  equal to vx27_hip_gqa_decode: {same}")
            assert same
            orc, _, _ = oracle_gqa_decode(d, Lcap)
            err = np.abs(got.astype(np.float64) - orc)
            assert np.all(err <= 2e-2 + 1e-2 * np.abs(orc)) and err.max() <= 0.02 * np.abs(orc).max()
        # beyond the static scratch: 2 sequences x 4096 splits x 24 query heads of
        # partials (258 floats each) need about 50 MB, over the 16 MiB array
        desc.B = 2
        desc.n_split = 4096
        rc = lib.vx27_hip_gqa_decode_noalloc(ctx.h, C.byref(desc))
        msg = lib.vx27_hip_last_error().decode()
        say(f"  oversize: rc={rc} {msg}")
        assert rc == -1 and "static buffer" in msg


def test_noalloc_captured_on_fresh_context():
    """The no-allocation entry point captured into a graph as the first call
    on a fresh context (no earlier call sized anything): two replays, with
    eager work between them, equal the eager vx27_hip_gqa_decode bit for bit."""
    from vx27_amd import lib as L
    lib = L.lib()
    with L.Ctx(0) as ctx:
        B, nk, Lcap = 2, 3000, 3072
        say(f"noalloc capture on a fresh context: B={B} keys={nk + 1}")
        d, lay, desc, ob = _setup(ctx, B, nk, Lcap, 73)
        ctx.graph_begin()
        L.check(lib.vx27_hip_gqa_decode_noalloc(ctx.h, C.byref(desc)), "gqa_decode_noalloc (capture)")
        g = ctx.graph_end()
        try:
            replays = []
            for _ in range(2):
                ob.zero()
                ctx.sync()
                ctx.graph_launch(g)
                ctx.sync()
                replays.append(ob.download((B, 24, 256), np.float32))
                L.check(lib.vx27_hip_gqa_decode_noalloc(ctx.h, C.byref(desc)), "gqa_decode_noalloc")   # eager between
                ctx.sync()
        finally:
            L.check(lib.vx27_hip_graph_destroy(g), "graph_destroy")
        ob.zero()
        L.check(lib.vx27_hip_gqa_decode(ctx.h, C.byref(desc)), "gqa_decode")
        ctx.sync()
        ref = ob.download((B, 24, 256), np.float32)
        for i, r in enumerate(replays):
            say(f"  replay {i}: equal to vx27_hip_gqa_decode {np.array_equal(r, ref)}")
            assert np.array_equal(r, ref), i
