"""Token-mixer benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c5|dn_conv]
                    [--context L] [--no-extra] [--no-cpu]

Prints ONE JSON line.  A "step" is one decode step of the workload (one token
for every sequence of the batch), inputs already resident in HBM.  `value` is
mixer microseconds per token (whole job), lower is better.  The line also
carries:
  roofline      the dominant kernel's algorithmic bytes per launch divided by
                its average duration, measured with HIP events on the
                library's stream during one profiled step, against 8 TB/s;
                `traffic` is the HBM bytes per launch that rocprofv3's
                FETCH_SIZE and WRITE_SIZE counters read for that kernel at the
                default workload (scaled by a copy-kernel calibration);
                `measured_read_GBs` / `measured_copy_GBs` are what a plain
                streaming read and a plain copy kernel reach over 4 GiB on
                the same GPU (vx27_hip_bw_probe), and `frac_of_measured_read`
                is the kernel's rate against the read
  cpu_baseline  the oracle (CPU restatement of the reference path) timed on
                this host on a bounded sample of the same workload
  extra         the other decode configurations, measured the same way

Workloads (synthetic, seeded, random-init):
  c5        (default) one decode step of all 64 token mixers of the model:
            48 Gated DeltaNet mixers (16 QK / 48 V heads, 128x128 fp32 state
            per V head, conv, gates, gated norm) and 16 gated GQA mixers
            (24 Q / 4 KV heads of 256, QK RMSNorm, partial RoPE, sigmoid gate)
            with their input and output projections (bf16 weights, hidden
            5120), batch 4 at context 131072 (bf16 KV cache); the 64 layers
            are replayed as one HIP graph
  dn_conv   batched Gated DeltaNet decode with the fused causal conv:
            64 sequences x 16 heads x 128x128 fp32 state, 6144 conv channels
            (bf16 weights), l2norm q/k, exact delta rule; 256 steps
Extras (without --no-extra), each with its algorithmic bytes (or flops)
and roofline fraction, and the oracle timed on this host where noted:
  c1_dn_recurrent   DeltaNet recurrence, 1 sequence x 16 heads, 2000 steps:
                    one multi-step call (state resident) and per-step calls
                    (state streamed, 2,130,048 B/step); CPU-exact and
                    CPU-AVX2 (the compiled reference's AVX2 primitives when
                    oracle/_ref is built), 16 threads and 1 thread
  c2_gqa8k_B{1,4,32}  gated GQA decode at 8192 cached positions
                    (33,640,448 B per sequence); CPU at B=1 and 32
  c3_dn_conv_B{1,4,16,64}  batched DeltaNet decode with the fused conv;
                    CPU at B=64 (16 threads and 1 thread)
  layer_decode_B{16,64}  one DeltaNet and one gated-GQA mixer layer with
                    their projections (GQA at 4096 cached positions), per
                    layer and per projection kernel against 8 TB/s
  c4a/c4b           the two prefills of a 4096-token prompt (chunked
                    DeltaNet, 16 heads; causal gated GQA, 24Q/4KV hd 256)
                    against the bf16 MFMA peak
  host              nproc, usable CPUs, CPU model, threads of the CPU legs
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12           # bytes/s, MI355X
# rocprofv3 --pmc summary of this script's default workload (FETCH_SIZE and
# WRITE_SIZE per dispatch, scaled by a copy-kernel calibration); its line
# "gqa_split (the dominant kernel): traffic = T B per launch" gives the
# roofline's `traffic`
PMC_SUMMARY = os.path.join(ROOT, "profiles", "c5_decode_step_pmc.txt")


def measured_traffic(kernel="gqa_split"):
    """HBM bytes per launch of `kernel` from the committed PMC summary, or None."""
    import re
    try:
        txt = open(PMC_SUMMARY).read()
    except OSError:
        return None
    m = re.search(re.escape(kernel) + r" \(the dominant kernel\): traffic = ([0-9.eE+]+) B per launch", txt)
    return float(m.group(1)) if m else None
METRIC = "mixer µs/token decode (B=1..64) + % HBM roofline; prefill tok/s + MFMA util"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------- full 64-mixer decode step
def bench_c5(ctx, steps, warmup, B=4, Lctx=131072, cpu=True):
    from vx27_amd import lib as L
    from vx27_amd.stack import MixerStack
    t0 = time.perf_counter()
    st = MixerStack(ctx, B=B, Lctx=Lctx, extra_pos=steps + warmup + 8)
    log(f"  c5: setup {time.perf_counter() - t0:.1f}s, weights {st.w_bytes / 1e9:.2f} GB, "
        f"KV cap {st.Lcap}")
    xs = ctx.buf((steps + warmup + 2) * B * st.H * 4)
    ctx.fill_normal(xs, (steps + warmup + 2) * B * st.H, 77, 1.0)
    lib = L.lib()

    def load_x(t):
        L.check(lib.vx27_hip_d2d(ctx.h, st.x.ptr, xs.ptr + t * B * st.H * 4, B * st.H * 4), "d2d")

    # eager step (sizes the scratch), then the per-kernel profile of one eager step
    load_x(0)
    st.step()
    ctx.sync()
    ctx.prof_enable(True)
    load_x(1)
    st.step()
    ctx.sync()
    prof = {}
    for k in ("gqa_split", "gqa_prep", "gqa_combine", "gemv_dn_in", "gemv_wk_store", "dn_step_kernel",
              "dn_decode_kernel", "pack_x"):
        n, ms = ctx.prof_read(k)
        prof[k] = (n, ms)
    ctx.prof_enable(False)
    # capture one step into a graph
    ctx.graph_begin()
    st.step()
    g = ctx.graph_end()
    for t in range(warmup):
        load_x(2 + t)
        ctx.graph_launch(g)
    ctx.sync()
    t0 = time.perf_counter()
    for t in range(steps):
        load_x(2 + warmup + t)
        ctx.graph_launch(g)
    ctx.sync()
    wall = time.perf_counter() - t0
    lib.vx27_hip_graph_destroy(g)
    pos_mid = Lctx + 2 + warmup + steps // 2
    alg = st.alg_bytes(pos_mid)
    n_split, ms_split = prof["gqa_split"]
    split_bytes = B * 4 * (Lctx + 2) * 256 * 2 * 2          # one layer's KV at the profiled step
    res = {
        "workload": f"64 mixers (48 DeltaNet nv=48 + 16 gated GQA) decode step, B={B}, context {Lctx}",
        "ms_per_step": wall / steps * 1e3, "us_per_token": wall / steps / B * 1e6,
        "alg_bytes_per_step": alg, "step_GBs": alg / (wall / steps) / 1e9,
        "kernel": "gqa_split", "kernel_us": ms_split / n_split * 1e3,
        "kernel_alg_bytes": split_bytes, "kernel_GBs": split_bytes / (ms_split / n_split / 1e3) / 1e9,
        "profile_ms_per_step": {k: round(v[1], 4) for k, v in prof.items()},
        "profile_launches": {k: v[0] for k, v in prof.items()},
    }
    if cpu:
        res["cpu"] = cpu_c5(B)
    return res


def cpu_c5(B, ctx_sample=8192):
    """Oracle on a bounded sample: one DeltaNet mixer (projections, glue,
    out_proj) and one gated-GQA mixer with its attention at `ctx_sample`
    keys, B sequences; the step time is extrapolated as 48 DeltaNet mixers +
    16 GQA mixers with attention scaled linearly to 131073 keys."""
    from oracle import oracle as O
    from gpu_common import oracle_dn_layer, oracle_matvec_batch
    from vx27_amd import workloads as W
    r = W.rng(5, "cpu_c5")
    th = O.default_threads()
    H, nqk, nv, hd = 5120, 16, 48, 128
    qd, vd = nqk * hd, nv * hd
    C_ = 2 * qd + vd
    w = {"w_in": W.bf16_bits(W.normal(r, (C_ + vd + 2 * nv, H), 0.02)),
         "w_out": W.bf16_bits(W.normal(r, (H, vd), 0.02)),
         "conv_w": W.normal(r, (C_, 4), 0.2), "A_log": r.uniform(-2, 1, nv).astype(np.float32),
         "dt_bias": W.normal(r, nv, 0.1), "norm_w": W.normal(r, hd, 0.1, 1.0)}
    S = W.normal(r, (B, nv, hd, hd), 0.02)
    conv = np.zeros((B, C_, 3), np.float32)
    x = W.normal(r, (B, H))
    t0 = time.perf_counter()
    oracle_dn_layer(w, x, S, conv, nqk, nv)
    t_dn = time.perf_counter() - t0
    wq = W.bf16_bits(W.normal(r, (24 * 512 + 2048, H), 0.02))
    wo = W.bf16_bits(W.normal(r, (H, 24 * 256), 0.02))
    t0 = time.perf_counter()
    oracle_matvec_batch(wq, x); oracle_matvec_batch(wo, np.zeros((B, 24 * 256), np.float32))
    t_gproj = time.perf_counter() - t0
    kv = W.bf16_bits(W.normal(r, (B, ctx_sample, 4, 256)))
    q = W.normal(r, (B, 24, 256))
    nk = np.full(B, ctx_sample, np.int32)
    out = np.empty((B, 24, 256), np.float32)
    a = O.AttendBatchArgs(B, 24, 4, 256, th, 1, 1, nk.ctypes.data, q.ctypes.data, kv.ctypes.data,
                          kv.ctypes.data, ctx_sample * 1024, 1024, 256, 1024, 256, out.ctypes.data)
    t_att = O.lib().orc_attend_batch(C.byref(a))
    t_step = 48 * t_dn + 16 * (t_gproj + t_att * 131073 / ctx_sample)
    return {"value": t_step / B * 1e6, "unit": "us/token", "cores": th, "kind": "port",
            "sample": (f"oracle: 1 DeltaNet mixer ({t_dn*1e3:.0f} ms) + 1 GQA projection pair "
                       f"({t_gproj*1e3:.0f} ms) + GQA attention at {ctx_sample} keys "
                       f"({t_att*1e3:.0f} ms), B={B}, {th} threads; step = 48 DN + 16 GQA with "
                       f"attention scaled x{131073/ctx_sample:.1f} to 131073 keys")}


# --------------------------------------------------------------- DeltaNet
def dn_conv_alg_bytes(B, H=16, hd=128):
    """Algorithmic bytes of one batched DeltaNet + conv decode step: state
    r+w, conv state r+w, x, o, conv weights (bf16) and gate inputs."""
    C_ = 3 * H * hd
    return (2 * B * H * hd * hd * 4 + 2 * B * C_ * 3 * 4 + B * C_ * 4 + B * H * hd * 4 + C_ * 4 * 2
            + B * H * 2 * 4)


def bench_dn_conv(ctx, steps, warmup, B=64, H=16, cpu=True):
    """Batched DeltaNet decode with the fused conv, one step per call (one
    launch: conv, gates, norms, exact step)."""
    from vx27_amd import lib as L, mixers as M, workloads as W
    hd, C_ = 128, 3 * 16 * 128
    total = steps + warmup
    d = W.dn_conv(B=B, H=H, steps=total)
    lay = M.DeltaNetLayer(ctx, B, H, H, d["A_log"], d["dt_bias"], conv_w=d["conv_w_bf16"],
                          conv_w_dtype=L.BF16, S0=d["S0"], conv0=d["conv0"])
    x = ctx.put(d["x"])
    a = ctx.put(d["a"])
    b = ctx.put(d["b"])
    out = ctx.buf(total * B * H * hd * 4)
    flags = L.DN_CONV | L.DN_PRE_L2
    descs = []
    for t in range(total):
        descs.append(lay.desc(1, flags, out.ptr + t * B * H * hd * 4, a.ptr + t * B * H * 4,
                              b.ptr + t * B * H * 4, x=x.ptr + t * B * C_ * 4))
    fn = L.lib().vx27_hip_dn_decode
    for t in range(warmup):
        L.check(fn(ctx.h, C.byref(descs[t])), "dn_decode")
    ctx.sync()
    # wall clock of the timed steps without the profiler; then the same steps
    # again (states continue) with per-kernel events
    t0 = time.perf_counter()
    for t in range(warmup, total):
        L.check(fn(ctx.h, C.byref(descs[t])), "dn_decode")
    ctx.sync()
    wall = time.perf_counter() - t0
    ctx.prof_enable(True)
    for t in range(warmup, total):
        L.check(fn(ctx.h, C.byref(descs[t])), "dn_decode")
    ctx.sync()
    # one step per call: the single-step kernel (conv and gates fused), column-split for few heads
    for kname in ("dn_step_kernel", "dn_step_split", "dn_decode_kernel"):
        n, ms = ctx.prof_read(kname)
        if n:
            break
    ctx.prof_enable(False)
    alg = dn_conv_alg_bytes(B, H, hd)
    avg_s = ms / n / 1e3
    step_s = wall / steps
    res = {
        "workload": f"dn_conv B={B} heads={H} hd=128 conv=6144ch bf16w, {steps} steps",
        "us_per_step": step_s * 1e6, "us_per_token": step_s / B * 1e6,
        "kernel": kname, "kernel_us": avg_s * 1e6,
        "alg_bytes_per_step": alg, "achieved_GBs": alg / avg_s / 1e9,
        "hbm_frac_kernel": alg / avg_s / HBM_PEAK, "hbm_frac_step": alg / step_s / HBM_PEAK,
    }
    if cpu:
        res["cpu"] = cpu_dn_conv(d, B, H)
    for bb in (x, a, b, out, lay.S, lay.conv_state):
        bb.free()
    return res


def cpu_dn_conv(d, B, H, steps=96, steps_1t=8):
    """Oracle (CPU restatement, CPU-exact semantics) on the first `steps`
    steps of the same workload, all B x H units in parallel; and on the
    first `steps_1t` steps on one thread."""
    from oracle import oracle as O
    from gpu_common import oracle_dn
    from vx27_amd import lib as L
    th = O.default_threads()
    res = {}
    for nth, ns in ((th, steps), (1, steps_1t)):
        sub = dict(d)
        for k in ("x", "a", "b"):
            sub[k] = np.ascontiguousarray(d[k][:ns])
        _, _, _, secs = oracle_dn(sub, L.DN_CONV | L.DN_PRE_L2, B, H, H, ns, threads=nth)
        res[nth] = secs / (ns * B) * 1e6
    return {"value": res[th], "unit": "us/token", "cores": th, "kind": "port",
            "value_1thread": res[1],
            "sample": f"oracle step_exact path (conv, l2 pre-norm), {B} seq x {H} heads: the first {steps} "
                      f"steps on {th} threads, the first {steps_1t} on 1 thread"}


C1_BYTES_PER_STEP = 2130048   # S r+w 2,097,152 + q,k,v 24,576 + a,b 128 + o 8,192 (16 heads)


def bench_dn_recurrent(ctx, steps=2000, cpu=True):
    """16 heads x 2000 steps, one sequence: one multi-step launch (state
    resident in registers: µs/step only) and per-step launches (the state
    streamed from HBM and back every step: %HBM against 2,130,048 B/step)."""
    from vx27_amd import lib as L, mixers as M, workloads as W
    H, hd = 16, 128
    d = W.dn_recurrent(B=1, H=H, steps=steps)
    lay = M.DeltaNetLayer(ctx, 1, H, H, d["A_log"], d["dt_bias"], S0=d["S0"])
    bufs = {k: ctx.put(d[k]) for k in ("q", "k", "v", "a", "b")}
    out = ctx.buf(steps * H * hd * 4)
    fn = L.lib().vx27_hip_dn_decode
    one = lay.desc(steps, 0, out.ptr, bufs["a"].ptr, bufs["b"].ptr, q=bufs["q"].ptr, k=bufs["k"].ptr,
                   v=bufs["v"].ptr)
    L.check(fn(ctx.h, C.byref(one)), "dn_decode")
    ctx.sync()
    t0 = time.perf_counter()
    L.check(fn(ctx.h, C.byref(one)), "dn_decode")
    ctx.sync()
    multi = time.perf_counter() - t0
    per = []
    for t in range(steps):
        per.append(lay.desc(1, 0, out.ptr + t * H * hd * 4, bufs["a"].ptr + t * H * 4,
                            bufs["b"].ptr + t * H * 4, q=bufs["q"].ptr + t * H * hd * 4,
                            k=bufs["k"].ptr + t * H * hd * 4, v=bufs["v"].ptr + t * H * hd * 4))
    for t in range(8):
        L.check(fn(ctx.h, C.byref(per[t])), "dn_decode")
    ctx.sync()
    t0 = time.perf_counter()
    for t in range(steps):
        L.check(fn(ctx.h, C.byref(per[t])), "dn_decode")
    ctx.sync()
    single = time.perf_counter() - t0
    ctx.prof_enable(True)
    for t in range(200):
        L.check(fn(ctx.h, C.byref(per[t])), "dn_decode")
    ctx.sync()
    kern = {k: ctx.prof_read(k) for k in ("dn_step_kernel", "dn_step_split", "dn_decode_kernel", "dn_gate_kernel")}
    ctx.prof_enable(False)
    # the same per-step calls captured as one graph of 200 launches: the
    # device-side time per step without the host's per-call cost
    ctx.graph_begin()
    for t in range(200):
        L.check(fn(ctx.h, C.byref(per[t])), "dn_decode")
    g = ctx.graph_end()
    ctx.graph_launch(g)
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(5):
        ctx.graph_launch(g)
    ctx.sync()
    graph_step = (time.perf_counter() - t0) / (5 * 200)
    L.check(L.lib().vx27_hip_graph_destroy(g), "graph_destroy")
    # the floor of a one-step call: the same 200 launches of the smallest
    # kernel of the library (a one-workgroup 64-byte fill), eager and graphed
    tiny = ctx.buf(64)
    fill = L.lib().vx27_hip_memset
    for _ in range(20):
        L.check(fill(ctx.h, tiny.ptr, 0, 64), "memset")
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(200):
        L.check(fill(ctx.h, tiny.ptr, 0, 64), "memset")
    ctx.sync()
    floor_eager = (time.perf_counter() - t0) / 200
    ctx.graph_begin()
    for _ in range(200):
        L.check(fill(ctx.h, tiny.ptr, 0, 64), "memset")
    g = ctx.graph_end()
    ctx.graph_launch(g)
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(5):
        ctx.graph_launch(g)
    ctx.sync()
    floor_graph = (time.perf_counter() - t0) / (5 * 200)
    L.check(L.lib().vx27_hip_graph_destroy(g), "graph_destroy")
    tiny.free()
    k_us = sum(ms for _, ms in kern.values()) / 200 * 1e3
    res = {"workload": f"dn_recurrent B=1 heads=16 {steps} steps",
           "us_per_step_resident": multi / steps * 1e6,
           "us_per_step_streamed": single / steps * 1e6,
           "us_per_step_streamed_graph": graph_step * 1e6,
           "launch_floor_us": {"eager": floor_eager * 1e6, "graph": floor_graph * 1e6,
                               "kernel": "vx_fill_kernel, 1 workgroup, 64 bytes"},
           "kernel_us_streamed": k_us,
           "kernels_streamed": {k: v[0] / 200 for k, v in kern.items() if v[0]},
           "alg_bytes_per_step_streamed": C1_BYTES_PER_STEP,
           "hbm_frac_streamed_kernel": C1_BYTES_PER_STEP / (k_us / 1e6) / HBM_PEAK,
           "hbm_frac_streamed_step": C1_BYTES_PER_STEP / (single / steps) / HBM_PEAK}
    if cpu:
        res.update(cpu_dn_recurrent(d, steps))
    for bb in list(bufs.values()) + [out, lay.S]:
        bb.free()
    return res


def cpu_dn_recurrent(d, steps, steps_1t=250):
    """C1 on the host: CPU-exact (the oracle's step_exact, 16 heads in
    parallel) and CPU-AVX2 (the reference's AVX2 update/retrieve composed
    into the gated delta rule: the compiled reference's own functions when
    oracle/_ref is built, else their pinned restatement), each on 16 threads
    over the 2000 steps and on 1 thread over the first 250."""
    from oracle import oracle as O
    from gpu_common import oracle_dn
    H, hd = 16, 128
    th = min(H, O.default_threads())
    exact = {}
    for nth, ns in ((th, steps), (1, steps_1t)):
        sub = dict(d)
        for k in ("q", "k", "v", "a", "b"):
            sub[k] = np.ascontiguousarray(d[k][:ns])
        _, _, _, secs = oracle_dn(sub, 0, 1, H, H, ns, threads=nth)
        exact[nth] = secs / ns * 1e6
    # the AVX2 composition takes normalised q (with the 1/sqrt(hd) scale) and k,
    # beta and the decay exp(g) per (step, head) (vx27_deltanet.c:58-69)
    q = np.ascontiguousarray(np.stack([O.l2norm(r) for r in d["q"].reshape(-1, hd)]).reshape(d["q"].shape)
                             * np.float32(1.0 / np.sqrt(np.float32(hd))), np.float32)
    k = np.ascontiguousarray(np.stack([O.l2norm(r) for r in d["k"].reshape(-1, hd)]).reshape(d["k"].shape))
    a = d["a"].astype(np.float64)
    b = d["b"].astype(np.float64)
    x = a + d["dt_bias"].astype(np.float64)
    sp = np.where(x > 20, x, np.where(x < -20, np.exp(x), np.log1p(np.exp(np.minimum(x, 20)))))
    decay = np.ascontiguousarray(np.exp(-np.exp(d["A_log"].astype(np.float64)) * sp))
    beta = np.ascontiguousarray(1.0 / (1.0 + np.exp(-b)))
    v = np.ascontiguousarray(d["v"])
    upd, ret = O.ref_avx2_fns()
    kind = "reference" if upd is not None else "port"
    avx = {}
    for nth, ns in ((th, steps), (1, steps_1t)):
        S = np.zeros((H, hd, hd), np.float32)
        out = np.empty((ns, H, hd), np.float32)
        secs = O.lib().orc_dn_run_avx2(1, H, hd, ns, nth, S.reshape(-1), q[:ns].reshape(-1), k[:ns].reshape(-1),
                                       v[:ns].reshape(-1), beta[:ns].reshape(-1), decay[:ns].reshape(-1),
                                       out.reshape(-1), upd, ret)
        avx[nth] = secs / ns * 1e6
    return {"cpu_exact": {"value": exact[th], "unit": "us/step", "cores": th, "kind": "port",
                          "value_1thread": exact[1],
                          "sample": f"oracle step_exact, 16 heads x {steps} steps on {th} threads; "
                                    f"first {steps_1t} steps on 1 thread"},
            "cpu_avx2": {"value": avx[th], "unit": "us/step", "cores": th, "kind": kind,
                         "value_1thread": avx[1],
                         "sample": ("compiled reference vx27_deltanet_update_avx2/retrieve_avx2"
                                    if kind == "reference" else "restated AVX2 update/retrieve")
                                   + f" composed into the gated delta rule, 16 heads x {steps} steps on {th} "
                                   f"threads; first {steps_1t} steps on 1 thread"}}


# -------------------------------------------------------------------- GQA
GQA_SEQ_EXTRA_BYTES = 24 * 256 * 4 * 3 + 2 * 4 * 256 * 4   # q, gate, out fp32 + k_new, v_new


def gqa_alg_bytes(B, n_keys):
    """K and V (bf16) of every attended position plus the per-sequence q,
    gate, out and new k,v rows: 33,640,448 B per sequence at 8193 keys."""
    return B * (4 * n_keys * 256 * 2 * 2 + GQA_SEQ_EXTRA_BYTES)


def bench_gqa(ctx, B, Lctx=8192, iters=20, cpu=False):
    from vx27_amd import lib as L, mixers as M, workloads as W
    d = W.gqa_decode(B=B, L=Lctx)
    Lcap = (Lctx + 1 + 63) // 64 * 64
    lay = M.GatedGQALayer(ctx, B, Lcap, d["q_norm_w"], d["k_norm_w"])
    for b in range(B):
        lay.write_kv(b, 0, W.bf16_to_f32(d["K"][b]), W.bf16_to_f32(d["V"][b]))
    hd, n_q = 256, 24
    qb = ctx.put(d["qg"]); kb = ctx.put(d["k_new"]); vb = ctx.put(d["v_new"])
    pb = ctx.put(d["pos"]); ob = ctx.buf(B * n_q * hd * 4)
    desc = lay.desc(pb.ptr, qb.ptr, (n_q * 2 * hd, 2 * hd), qb.ptr + hd * 4, (n_q * 2 * hd, 2 * hd),
                    kb.ptr, vb.ptr, ob.ptr)
    fn = L.lib().vx27_hip_gqa_decode
    for _ in range(3):
        L.check(fn(ctx.h, C.byref(desc)), "gqa_decode")
    ctx.sync()
    # wall clock without the profiler, then a profiled pass for the kernel time
    t0 = time.perf_counter()
    for _ in range(iters):
        L.check(fn(ctx.h, C.byref(desc)), "gqa_decode")
    ctx.sync()
    wall = (time.perf_counter() - t0) / iters
    ctx.prof_enable(True)
    for _ in range(iters):
        L.check(fn(ctx.h, C.byref(desc)), "gqa_decode")
    ctx.sync()
    kern = {k: ctx.prof_read(k) for k in ("gqa_prep", "gqa_split", "gqa_combine")}
    ctx.prof_enable(False)
    nk = Lctx + 1
    kv = B * 4 * nk * hd * 2 * 2          # K and V bf16 of every attended position
    alg = gqa_alg_bytes(B, nk)
    split_s = kern["gqa_split"][1] / kern["gqa_split"][0] / 1e3
    kern_s = sum(ms for _, ms in kern.values()) / iters / 1e3
    res = {"workload": f"gqa_decode B={B} L={Lctx}", "us_per_step": wall * 1e6,
           "us_per_token": wall / B * 1e6,
           "kernels_us": {k: v[1] / v[0] * 1e3 for k, v in kern.items() if v[0]},
           "kernel": "gqa_split", "kernel_us": split_s * 1e6,
           "alg_bytes_per_step": alg, "kernel_alg_bytes": kv, "achieved_GBs": kv / split_s / 1e9,
           "hbm_frac_kernel": kv / split_s / HBM_PEAK, "hbm_frac_kernels": alg / kern_s / HBM_PEAK,
           "hbm_frac_step": alg / wall / HBM_PEAK}
    if cpu:
        res["cpu"] = cpu_gqa(d, B, nk)
    for bb in (qb, kb, vb, pb, ob, lay.k_cache, lay.v_cache):
        bb.free()
    return res


def cpu_gqa(d, B, nk):
    """The oracle's attention (the vx27_qlayer loop: double dot, float
    softmax and P.V) over the same bf16 cache, B x 24 (sequence, head)
    units in parallel, median of 3 runs (the raw q rows stand in for the
    normed ones: the time does not depend on the values)."""
    from oracle import oracle as O
    th = O.default_threads()
    kv_k = np.ascontiguousarray(d["K"])     # [B][L][4][256] bf16 (the new row is not appended here)
    kv_v = np.ascontiguousarray(d["V"])
    L_ = kv_k.shape[1]
    q = np.ascontiguousarray(d["qg"][:, :, :256])
    n_keys = np.full(B, min(nk, L_), np.int32)
    out = np.empty((B, 24, 256), np.float32)
    a = O.AttendBatchArgs(B, 24, 4, 256, th, 1, 1, n_keys.ctypes.data, q.ctypes.data, kv_k.ctypes.data,
                          kv_v.ctypes.data, L_ * 1024, 1024, 256, 1024, 256, out.ctypes.data)
    O.lib().orc_attend_batch(C.byref(a))
    t = sorted(O.lib().orc_attend_batch(C.byref(a)) for _ in range(3))[1]
    return {"value": t / B * 1e6, "unit": "us/token", "cores": th, "kind": "port",
            "sample": f"oracle attention over {int(n_keys[0])} bf16 keys, B={B} x 24 heads on {th} threads, "
                      "median of 3"}


# ------------------------------------------------------- whole mixer layers
def bench_layer_decode(ctx, B, Lctx=4096, iters=10):
    """One decode token of B sequences through a Gated DeltaNet mixer layer
    (16 QK / 48 V heads of 128, hidden 5120) and a gated-GQA mixer layer
    (24 Q / 4 KV heads of 256, Lctx cached positions), bf16 weights, each
    with its input and output projection (one pass over each weight matrix
    for up to 65 sequences).  The stack holds 9 DeltaNet and 3 GQA layers
    and each timing runs all layers of one kind in turn (HIP graph, 'iters'
    replays), so that every layer streams its weights from HBM as in a full
    decode step (one layer's weights alone would stay in the 256 MiB
    last-level cache between replays).  Per-kernel times from a profiled
    eager pass.  Algorithmic bytes: weights, DeltaNet state and conv state
    r+w (or the K/V rows attended and written), x and out."""
    from vx27_amd import lib as L
    from vx27_amd.stack import GQ, HD, H, MixerStack
    st = MixerStack(ctx, B=B, Lctx=Lctx, extra_pos=8, n_layers=12)
    lib = L.lib()
    ctx.fill_normal(st.x, B * H, 91, 1.0)
    L.check(lib.vx27_hip_pack_x(ctx.h, st.x.ptr, B, H, st.xp.ptr), "pack_x")
    nv = st.nv
    vd, C_ = nv * HD, st.C
    res = {"workload": f"DeltaNet and gated-GQA mixer layer decode, B={B}, GQA context {Lctx}"}
    for kind in ("dn", "gqa"):
        lays = [lay for lay in st.layers if lay["kind"] == kind]
        fn = lib.vx27_hip_dn_layer_decode if kind == "dn" else lib.vx27_hip_gqa_layer_decode

        def call():
            for lay in lays:
                L.check(fn(ctx.h, C.byref(lay["desc"])), kind)
        call()
        ctx.sync()
        ctx.graph_begin()
        call()
        g = ctx.graph_end()
        ctx.graph_launch(g)
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(iters):
            ctx.graph_launch(g)
        ctx.sync()
        wall = (time.perf_counter() - t0) / iters / len(lays)
        lib.vx27_hip_graph_destroy(g)
        kernels = (("gemv_dn_in", "gemv_wk_store", "dn_step_kernel", "dn_step_split", "dn_decode_kernel")
                   if kind == "dn" else ("gemv_wk_store", "gqa_prep", "gqa_split", "gqa_combine"))
        _, per = _time_calls(ctx, call, kernels, iters)
        per = {k: v / len(lays) for k, v in per.items()}
        io = 2 * B * H * 4
        if kind == "dn":
            w_in, w_out = (C_ + vd + 2 * nv) * H * 2, H * vd * 2
            alg = w_in + w_out + 2 * B * nv * HD * HD * 4 + 2 * B * C_ * 3 * 4 + C_ * 4 * 2 + io
            proj = {"gemv_dn_in": (w_in, per["gemv_dn_in"]), "gemv_wk_store": (w_out, per["gemv_wk_store"])}
        else:
            w_qkv, w_o = (24 * 2 * GQ + 2 * 4 * GQ) * H * 2, H * 24 * GQ * 2
            alg = w_qkv + w_o + B * 4 * (Lctx + 1) * GQ * 2 * 2 + B * 4 * GQ * 2 * 2 + io
            proj = {"gemv_wk_store": (w_qkv + w_o, per["gemv_wk_store"])}
        res[kind] = {
            "layers_timed": len(lays),
            "us_per_layer": round(wall * 1e6, 2), "us_per_token": round(wall / B * 1e6, 3),
            "alg_bytes": alg, "hbm_frac": round(alg / wall / HBM_PEAK, 4),
            "kernels_us": {k: round(v, 2) for k, v in per.items() if v > 0},
            "projection_hbm_frac": {k: round(b / (us / 1e6) / HBM_PEAK, 4) for k, (b, us) in proj.items() if us > 0},
        }
    return res


# ---------------------------------------------------------------- prefill
MFMA_BF16_PEAK = 2.5e15     # flop/s, MI355X dense bf16


def _time_calls(ctx, fn, kernels, iters):
    """Run fn() iters times with the profiler on; wall time per call and the
    summed kernel time per call (HIP events on the library stream)."""
    ctx.sync()
    ctx.prof_enable(True)
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    ctx.sync()
    wall = (time.perf_counter() - t0) / iters
    per = {k: ctx.prof_read(k)[1] / iters * 1e3 for k in kernels}
    ctx.prof_enable(False)
    return wall * 1e6, per


DNP_KERNELS = ("dnp_glue_in", "dnp_conv_state", "dnp_prept", "dnp_scant", "dnp_prep3", "dnp_scan3", "dnp_prep", "dnp_scan",
               "dnp_out_gate_packed",
               "dnp_out_gate")


def dn_prefill_flops(T, H, hd=128, C_=64):
    """Algorithmic flops of the chunked form: H (T/C) (10 C^2 d + 6 C d^2 + 2 C^3 / 3)."""
    return H * (T // C_) * (10 * C_ * C_ * hd + 6 * C_ * hd * hd + 2 * C_ ** 3 / 3)


def bench_dn_prefill(ctx, T=4096, iters=20, cpu=True):
    """Chunked Gated DeltaNet prefill: one T-token prompt, 16 heads of 128,
    bf16 q/k/v in: the default split-precision products, and the bf16 form
    (VX27_DN_BF16) beside it."""
    from vx27_amd import lib as L, workloads as W
    d = W.dn_prefill(B=1, T=T)
    H, hd = 16, 128
    bufs = {k: ctx.put(d[k]) for k in ("q", "k", "v", "a", "b", "A_log", "dt_bias", "S0")}
    ob = ctx.buf(T * H * hd * 4)
    flops = dn_prefill_flops(T, H)
    nbytes = T * H * hd * 2 * 3 + T * H * 8 + T * H * hd * 4 + 2 * H * hd * hd * 4
    res = {"workload": f"dn_prefill B=1 T={T} heads=16 chunk=64 (split-precision products)",
           "alg_flops": flops, "alg_bytes": nbytes}
    for tag, flags in (("", 0), ("bf16_", L.DN_BF16)):
        desc = L.DnPrefillDesc(1, T, H, H, hd, flags, bufs["S0"].ptr, bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr,
                               bufs["a"].ptr, bufs["b"].ptr, bufs["A_log"].ptr, bufs["dt_bias"].ptr, ob.ptr)

        def run():
            L.check(L.lib().vx27_hip_dn_prefill(ctx.h, C.byref(desc)), "dn_prefill")
        for _ in range(3):
            run()
        wall_us, per = _time_calls(ctx, run, DNP_KERNELS, iters)
        per = {k: v for k, v in per.items() if v > 0}
        k_us = sum(per.values())
        res.update({tag + "us_per_call": wall_us, tag + "kernel_us": k_us, tag + "kernels_us": per,
                    tag + "tokens_per_s": T / (k_us / 1e6), tag + "mfma_frac": flops / (k_us / 1e6) / MFMA_BF16_PEAK,
                    tag + "hbm_frac": nbytes / (k_us / 1e6) / HBM_PEAK})
    if cpu:
        from gpu_common import oracle_dn
        seq = {k: np.ascontiguousarray(np.swapaxes(W.bf16_to_f32(d[k]), 0, 1)) for k in ("q", "k", "v")}
        seq.update({k: np.ascontiguousarray(np.swapaxes(d[k], 0, 1)) for k in ("a", "b")})
        seq.update(A_log=d["A_log"], dt_bias=d["dt_bias"], S0=d["S0"])
        from oracle import oracle as O
        _, _, _, secs = oracle_dn(seq, 0, 1, H, H, T)
        res["cpu"] = {"value": T / secs, "unit": "tokens/s", "cores": min(H, O.default_threads()),
                      "kind": "port", "sample": f"oracle sequential step_exact, {T} tokens x 16 heads"}
    for b in bufs.values():
        b.free()
    ob.free()
    return res


def bench_dn_prefill_glue(ctx, T=4096, iters=10):
    """The DeltaNet branch of vx27_qlayer_batch for one T-token prompt at
    the real layer's shape (16 QK / 48 V heads): conv over 10240 channels,
    rmsn(1+w) + l2 pre-norms, the chunked core (split precision), gated
    output norm."""
    from vx27_amd import lib as L, workloads as W
    nqk, nv, hd = 16, 48, 128
    d = W.dn_prefill_glue(B=1, T=T, nqk=nqk, nv=nv)
    bufs = {k: ctx.put(d[k]) for k in ("x", "a", "b", "A_log", "dt_bias", "S0", "conv0", "conv_w_bf16", "norm_w",
                                       "z")}
    ob = ctx.buf(T * nv * hd * 4)
    desc = L.DnPrefillDesc()
    desc.B, desc.T, desc.nqk, desc.nv, desc.hd, desc.flags = 1, T, nqk, nv, hd, 15
    desc.S, desc.out, desc.a, desc.b = bufs["S0"].ptr, ob.ptr, bufs["a"].ptr, bufs["b"].ptr
    desc.A_log, desc.dt_bias, desc.x, desc.conv_state = bufs["A_log"].ptr, bufs["dt_bias"].ptr, bufs["x"].ptr, \
        bufs["conv0"].ptr
    desc.conv_w, desc.conv_w_dtype, desc.norm_w, desc.z = bufs["conv_w_bf16"].ptr, L.BF16, bufs["norm_w"].ptr, \
        bufs["z"].ptr

    def run():
        L.check(L.lib().vx27_hip_dn_prefill(ctx.h, C.byref(desc)), "dn_prefill")
    for _ in range(2):
        run()
    wall_us, per = _time_calls(ctx, run, DNP_KERNELS, iters)
    per = {k: v for k, v in per.items() if v > 0}
    k_us = sum(per.values())
    flops = dn_prefill_flops(T, nv)
    res = {"workload": f"dn_prefill with conv, pre-norms, gated norm: B=1 T={T} nqk=16 nv=48",
           "us_per_call": wall_us, "kernel_us": k_us, "kernels_us": per, "tokens_per_s": T / (k_us / 1e6),
           "alg_flops": flops, "mfma_frac": flops / (k_us / 1e6) / MFMA_BF16_PEAK}
    for b in list(bufs.values()) + [ob]:
        b.free()
    return res


def bench_layer_prefill(ctx, T=4096, iters=5):
    """Both mixer layers on one T-token prompt with their projections
    (vx27_hip_dn_layer_prefill, vx27_hip_gqa_layer_prefill at the real layer
    shapes, hidden 5120): from 256 tokens on the projections run in the
    long-prompt GEMM (weights read once per 256 tokens, x as two bf16 parts).
    Synthetic weights filled on the device straight into the tiled layout."""
    from vx27_amd import lib as L, workloads as W
    H, nqk, nv, hd = 5120, 16, 48, 128
    qd, vd = nqk * hd, nv * hd
    C_ = 2 * qd + vd
    Nin = C_ + vd + 2 * nv
    Nqkv, Ka = 24 * 2 * 256 + 2 * 4 * 256, 24 * 256
    x = ctx.buf(T * H * 4)
    ctx.fill_normal(x, T * H, 31)
    out = ctx.buf(T * H * 4)
    res = {}
    # DeltaNet layer
    d = W.dn_prefill_glue(B=1, T=1, nqk=nqk, nv=nv)
    w_in, w_out = ctx.buf(Nin * H * 2), ctx.buf(H * vd * 2)
    ctx.fill_normal(w_in, Nin * H, 32, 0.02, bf16=True)
    ctx.fill_normal(w_out, H * vd, 33, 0.02, bf16=True)
    bufs = {k: ctx.put(d[k]) for k in ("A_log", "dt_bias", "S0", "conv0", "conv_w_bf16", "norm_w")}
    desc = L.DnLayerPrefillDesc(1, T, nqk, nv, hd, H, 0, x.ptr, w_in.ptr, w_out.ptr, bufs["conv_w_bf16"].ptr,
                                L.BF16, bufs["A_log"].ptr, bufs["dt_bias"].ptr, bufs["norm_w"].ptr,
                                bufs["S0"].ptr, bufs["conv0"].ptr, out.ptr)

    def run_dn():
        L.check(L.lib().vx27_hip_dn_layer_prefill(ctx.h, C.byref(desc)), "dn_layer_prefill")
    run_dn()
    kern = ("gemm_pack", "gemm_wx", "gemm_reduce", "pack_x", "gemv_wk_store") + DNP_KERNELS
    wall_us, per = _time_calls(ctx, run_dn, kern, iters)
    per = {k: round(v, 1) for k, v in per.items() if v > 0}
    proj_flops = 2.0 * T * (Nin * H + H * vd)
    res["dn"] = {"workload": f"DeltaNet layer prefill B=1 T={T} nqk=16 nv=48 hidden=5120 (projections + "
                             f"chunked core)", "us_per_call": wall_us, "kernel_us": sum(per.values()),
                 "kernels_us": per, "tokens_per_s": T / (sum(per.values()) / 1e6),
                 "projection_tflops": proj_flops / ((per.get("gemm_pack", 0) + per.get("gemm_wx", 0) + per.get("gemm_reduce", 0)) * 1e-6) / 1e12
                 if per.get("gemm_wx") else None}
    for b in list(bufs.values()) + [w_in, w_out]:
        b.free()
    # gated GQA layer, positions 0 .. T-1 of a T-row cache
    w_qkv, w_o = ctx.buf(Nqkv * H * 2), ctx.buf(H * Ka * 2)
    ctx.fill_normal(w_qkv, Nqkv * H, 34, 0.02, bf16=True)
    ctx.fill_normal(w_o, H * Ka, 35, 0.02, bf16=True)
    qn, kn = ctx.put(W.normal(W.rng(36, "lp_qn"), 256, 0.1)), ctx.put(W.normal(W.rng(37, "lp_kn"), 256, 0.1))
    kc, vc = ctx.buf(T * 4 * 256 * 2), ctx.buf(T * 4 * 256 * 2)
    g = L.GqaLayerPrefillDesc(1, T, 24, 4, 256, H, 64, 1e7, 1.0, T, 0, 0, x.ptr, w_qkv.ptr, w_o.ptr, qn.ptr, kn.ptr,
                              kc.ptr, vc.ptr, out.ptr)

    def run_gqa():
        L.check(L.lib().vx27_hip_gqa_layer_prefill(ctx.h, C.byref(g)), "gqa_layer_prefill")
    run_gqa()
    kern = ("gemm_pack", "gemm_wx", "gemm_reduce", "pack_x", "gemv_wk_store", "qkv_to_bf16", "gqp_kv", "gqp_attn")
    wall_us, per = _time_calls(ctx, run_gqa, kern, iters)
    per = {k: round(v, 1) for k, v in per.items() if v > 0}
    proj_flops = 2.0 * T * (Nqkv * H + H * Ka)
    res["gqa"] = {"workload": f"gated GQA layer prefill B=1 T={T} 24Q/4KV hd 256 hidden=5120 (projections + "
                              f"causal attention)", "us_per_call": wall_us, "kernel_us": sum(per.values()),
                  "kernels_us": per, "tokens_per_s": T / (sum(per.values()) / 1e6),
                  "projection_tflops": proj_flops / ((per.get("gemm_pack", 0) + per.get("gemm_wx", 0) + per.get("gemm_reduce", 0)) * 1e-6) / 1e12
                  if per.get("gemm_wx") else None}
    for b in (w_qkv, w_o, qn, kn, kc, vc, x, out):
        b.free()
    return res


def bench_gqa_prefill(ctx, T=4096, iters=10, cpu=True):
    """Causal gated GQA prefill: one T-token prompt, 24Q/4KV hd 256."""
    from vx27_amd import lib as L, workloads as W
    d = W.gqa_prefill(B=1, T=T)
    n_q, n_kv, hd = 24, 4, 256
    Lc = (T + 63) // 64 * 64
    kc, vc = ctx.buf(n_kv * Lc * hd * 2), ctx.buf(n_kv * Lc * hd * 2)
    bufs = {k: ctx.put(d[k]) for k in ("q", "gate", "k", "v", "q_norm_w", "k_norm_w")}
    ob = ctx.buf(T * n_q * hd * 4)
    desc = L.GqaPrefillDesc(1, T, n_q, n_kv, hd, 64, 1e7, 1.0, Lc, 0, 0, bufs["q"].ptr, 0, 0,
                            bufs["gate"].ptr, 0, 0, bufs["k"].ptr, bufs["v"].ptr, bufs["q_norm_w"].ptr,
                            bufs["k_norm_w"].ptr, kc.ptr, vc.ptr, ob.ptr)

    def run():
        L.check(L.lib().vx27_hip_gqa_prefill(ctx.h, C.byref(desc)), "gqa_prefill")
    for _ in range(3):
        run()
    wall_us, per = _time_calls(ctx, run, ("gqp_kv", "gqp_attn"), iters)
    k_us = sum(per.values())
    flops = 2 * hd * n_q * T * (T + 1)
    res = {"workload": f"gqa_prefill B=1 T={T} 24Q/4KV hd256 causal", "us_per_call": wall_us,
           "kernel_us": k_us, "kernels_us": per, "tokens_per_s": T / (k_us / 1e6),
           "alg_flops": flops, "mfma_frac": flops / (k_us / 1e6) / MFMA_BF16_PEAK,
           "attn_mfma_frac": flops / (per["gqp_attn"] / 1e6) / MFMA_BF16_PEAK}
    if cpu:
        # oracle on the first 1024 query rows (causal work 1/16 of the prompt's), scaled
        from oracle import oracle as O
        Ts = 1024
        f = {k: np.ascontiguousarray(W.bf16_to_f32(d[k][:, :Ts])) for k in ("q", "gate", "k", "v")}
        kco = np.zeros((1, Ts, n_kv, hd), np.float32); vco = np.zeros_like(kco)
        out = np.empty((1, Ts, n_q, hd), np.float32)
        qw, kw = np.ascontiguousarray(d["q_norm_w"]), np.ascontiguousarray(d["k_norm_w"])
        a = O.GqaPrefillArgs(1, Ts, n_q, n_kv, hd, 64, 0, Ts, O.default_threads(), 1e7, 1.0,
                             f["q"].ctypes.data, f["gate"].ctypes.data, f["k"].ctypes.data, f["v"].ctypes.data,
                             qw.ctypes.data, kw.ctypes.data, kco.ctypes.data, vco.ctypes.data, out.ctypes.data)
        secs = O.lib().orc_gqa_prefill(C.byref(a)) * (T * (T + 1)) / (Ts * (Ts + 1))
        res["cpu"] = {"value": T / secs, "unit": "tokens/s", "cores": O.default_threads(), "kind": "port",
                      "sample": f"oracle prefill of the first {Ts} tokens, time scaled by the causal "
                                f"work ratio {T * (T + 1) / (Ts * (Ts + 1)):.1f}"}
    for b in list(bufs.values()) + [kc, vc, ob]:
        b.free()
    return res


# ------------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--workload", default="c5", choices=["c5", "dn_conv"])
    ap.add_argument("--context", type=int, default=131072)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c4", "layers"],
                    help="run one extra configuration alone and print its figures (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (asked for {args.gpus}); the mixers shard per "
              "(sequence, head) with no exchange, so N GPUs run N independent shards", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from vx27_amd import lib as L
    ctx = L.Ctx(0)
    log(f"bench: {L.lib().vx27_hip_version().decode()} workload={args.workload}")
    if args.only:
        cpu = not args.no_cpu
        runs = {"c1": lambda: {"c1_dn_recurrent": bench_dn_recurrent(ctx, cpu=cpu)},
                "c2": lambda: {f"c2_gqa8k_B{B}": bench_gqa(ctx, B, cpu=cpu) for B in (1, 4, 32)},
                "c3": lambda: {f"c3_dn_conv_B{B}": bench_dn_conv(ctx, 256, 8, B=B, cpu=cpu and B == 64)
                               for B in (1, 4, 16, 64)},
                "layers": lambda: dict({f"layer_decode_B{B}": bench_layer_decode(ctx, B) for B in (4, 16, 64)},
                                       layer_prefill_T4096=bench_layer_prefill(ctx)),
                "c4": lambda: {"c4a_dn_prefill_T4096": bench_dn_prefill(ctx, cpu=cpu),
                               "c4a_dn_prefill_layer_T4096": bench_dn_prefill_glue(ctx),
                               "c4b_gqa_prefill_T4096": bench_gqa_prefill(ctx, cpu=cpu)}}
        print(json.dumps({"only": args.only, "extra": runs[args.only]()}), flush=True)
        ctx.close()
        return
    extra = {}
    if args.workload == "c5":
        res = bench_c5(ctx, args.steps, args.warmup, Lctx=args.context, cpu=not args.no_cpu)
        log(f"  c5: {res['ms_per_step']:.3f} ms/step, {res['us_per_token']:.1f} us/token, "
            f"{res['step_GBs']:.0f} GB/s algorithmic; gqa_split {res['kernel_us']:.1f} us "
            f"({res['kernel_GBs']:.0f} GB/s)")
        value, unit = res["us_per_token"], "us/token"
        ms_step = res["ms_per_step"]
        config = {"workload": res["workload"], "batch": 4, "context": args.context, "layers": 64,
                  "deltanet_layers": 48, "gqa_layers": 16, "deltanet_v_heads": 48, "weights": "bf16",
                  "kv_cache": "bf16", "state": "fp32"}
        kbytes, kus = res["kernel_alg_bytes"], res["kernel_us"]
        traffic = measured_traffic() if args.context == 131072 else None
        step_frac = res["step_GBs"] * 1e9 / HBM_PEAK
        extra["c5_step"] = {k: v for k, v in res.items() if k != "cpu"}
        extra["c5_step"]["step_roofline_frac"] = round(step_frac, 4)
        dtype = "bf16 weights/KV, fp32 state (fp64 recurrence accumulation)"
    else:
        res = bench_dn_conv(ctx, args.steps, args.warmup, cpu=not args.no_cpu)
        extra["c3_dn_conv_B64"] = {k: v for k, v in res.items() if k != "cpu"}
        value, unit = res["us_per_token"], "us/token"
        ms_step = res["us_per_step"] / 1e3
        config = {"workload": res["workload"], "batch": 64, "heads": 16, "head_dim": 128}
        kbytes, kus = res["alg_bytes"], res["kernel_us"]
        traffic = None
        dtype = "fp32 (fp64 accumulation)"
    if not args.no_extra:
        cpu = not args.no_cpu
        for B in (1, 4, 16, 64):
            if args.workload == "dn_conv" and B == 64:
                continue
            r = bench_dn_conv(ctx, 256, 8, B=B, cpu=cpu and B == 64)
            extra[f"c3_dn_conv_B{B}"] = r
            log(f"  dn_conv B={B}: {r['us_per_token']:.3f} us/token, kernel {r['kernel_us']:.1f} us, "
                f"{r['achieved_GBs']:.0f} GB/s ({100 * r['hbm_frac_kernel']:.1f}% HBM)")
        for B in (1, 4, 32):
            r = bench_gqa(ctx, B, cpu=cpu and B in (1, 32))
            extra[f"c2_gqa8k_B{B}"] = r
            log(f"  gqa B={B}: {r['us_per_step']:.1f} us/step, split kernel {r['kernel_us']:.1f} us, "
                f"{r['achieved_GBs']:.0f} GB/s ({100 * r['hbm_frac_kernel']:.1f}% HBM), "
                f"step {100 * r['hbm_frac_step']:.1f}% HBM")
        for B in (16, 64):
            r = bench_layer_decode(ctx, B)
            extra[f"layer_decode_B{B}"] = r
            for kind in ("dn", "gqa"):
                q = r[kind]
                log(f"  {kind} layer decode B={B}: {q['us_per_layer']:.1f} us/layer, "
                    f"{100 * q['hbm_frac']:.1f}% HBM; projections {q['projection_hbm_frac']}")
        r = bench_dn_prefill(ctx, cpu=cpu)
        extra["c4a_dn_prefill_T4096"] = r
        log(f"  dn_prefill: {r['kernel_us']:.1f} us ({r['tokens_per_s']:.3g} tok/s), "
            f"MFMA {100 * r['mfma_frac']:.1f}%, HBM {100 * r['hbm_frac']:.1f}%  {r['kernels_us']}; bf16 products "
            f"{r['bf16_kernel_us']:.1f} us")
        r = bench_dn_prefill_glue(ctx)
        extra["c4a_dn_prefill_layer_T4096"] = r
        log(f"  dn_prefill layer (nv=48, glue): {r['kernel_us']:.1f} us, MFMA {100 * r['mfma_frac']:.1f}%  "
            f"{r['kernels_us']}")
        r = bench_gqa_prefill(ctx, cpu=cpu)
        extra["c4b_gqa_prefill_T4096"] = r
        log(f"  gqa_prefill: {r['kernel_us']:.1f} us ({r['tokens_per_s']:.3g} tok/s), "
            f"MFMA {100 * r['mfma_frac']:.1f}% (attention kernel {100 * r['attn_mfma_frac']:.1f}%)  "
            f"{r['kernels_us']}")
        r = bench_layer_prefill(ctx)
        extra["layer_prefill_T4096"] = r
        for kind in ("dn", "gqa"):
            q = r[kind]
            log(f"  {kind} layer prefill T=4096 with projections: {q['kernel_us']:.0f} us "
                f"({q['tokens_per_s']:.3g} tok/s), projections {q['projection_tflops']:.0f} TFLOP/s  {q['kernels_us']}")
        r = bench_dn_recurrent(ctx, cpu=cpu)
        extra["c1_dn_recurrent"] = r
        log(f"  dn_recurrent: {r['us_per_step_resident']:.2f} us/step (state resident, one call), "
            f"{r['us_per_step_streamed']:.2f} us/step (per-step calls; kernel {r['kernel_us_streamed']:.2f} us, "
            f"{100 * r['hbm_frac_streamed_kernel']:.1f}% HBM; a one-workgroup fill launch takes "
            f"{r['launch_floor_us']['eager']:.2f} us eager, {r['launch_floor_us']['graph']:.2f} graphed)")
        if cpu:
            log(f"  dn_recurrent cpu: exact {r['cpu_exact']['value']:.1f} us/step, avx2 "
                f"{r['cpu_avx2']['value']:.1f} us/step ({r['cpu_avx2']['kind']})")
    if not args.no_cpu:
        from oracle import oracle as O
        extra["host"] = dict(O.host_info(), cpu_baseline_threads=O.default_threads())
    ach = kbytes / (kus / 1e6)
    rbw, cbw = C.c_double(), C.c_double()
    L.check(L.lib().vx27_hip_bw_probe(ctx.h, 4 << 30, 5, C.byref(rbw), C.byref(cbw)), "bw_probe")
    log(f"  bandwidth probe (4 GiB): read {rbw.value:.0f} GB/s, copy {cbw.value:.0f} GB/s")
    line = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": unit,
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": dtype, "data": "synthetic (seeded random inputs and random-init weights)",
        "config": config,
        "roofline": {"bound": "hbm", "achieved": round(ach / 1e9, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK, 4), "traffic": traffic,
                     "kernel": res["kernel"], "kernel_us": round(kus, 2),
                     "alg_bytes_per_launch": kbytes,
                     "measured_read_GBs": round(rbw.value, 1), "measured_copy_GBs": round(cbw.value, 1),
                     "frac_of_measured_read": round(ach / (rbw.value * 1e9), 4) if rbw.value > 0 else None},
        "cpu_baseline": res.get("cpu"),
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
