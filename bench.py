"""Token-mixer benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line.  A "step" is one decode step of the workload (one token
for every sequence of the batch), inputs already resident in HBM.  `value` is
mixer microseconds per token (whole job), lower is better.  The line also
carries:
  roofline      the dominant kernel's algorithmic bytes per launch divided by
                its average duration, measured with HIP events on the
                library's stream over the timed region, against 8 TB/s
  cpu_baseline  the oracle (CPU restatement of the reference path) timed on
                this host on a bounded sample of the same workload
  extra         the other decode configurations, measured the same way

Workloads (synthetic, seeded, random-init):
  dn_conv   batched Gated DeltaNet decode with the fused causal conv:
            64 sequences x 16 heads x 128x128 fp32 state, 6144 conv channels
            (bf16 weights), l2norm q/k, exact delta rule; 256 steps
  gqa8k     gated GQA decode, 24Q/4KV hd 256, bf16 KV cache of 8192
            positions, batch 1 and 32
  dn_recur  DeltaNet recurrence alone, 1 sequence x 16 heads, 2000 steps
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
METRIC = "mixer µs/token decode (B=1..64) + % HBM roofline; prefill tok/s + MFMA util"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --------------------------------------------------------------- DeltaNet
def bench_dn_conv(ctx, steps, warmup, B=64, H=16, cpu=True):
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
    ctx.prof_enable(True)
    t0 = time.perf_counter()
    for t in range(warmup, total):
        L.check(fn(ctx.h, C.byref(descs[t])), "dn_decode")
    ctx.sync()
    wall = time.perf_counter() - t0
    n, ms = ctx.prof_read("dn_decode_kernel")
    ng, msg = ctx.prof_read("dn_gate_kernel")
    ctx.prof_enable(False)
    # algorithmic bytes of the decode kernel per launch (one step of B sequences)
    alg = (2 * B * H * hd * hd * 4        # S read + write
           + 2 * B * C_ * 3 * 4           # conv state read + write
           + B * C_ * 4                   # x
           + B * H * hd * 4               # out
           + C_ * 4 * 2)                  # conv weights (bf16)
    avg_s = ms / n / 1e3
    res = {
        "workload": f"dn_conv B={B} heads={H} hd=128 conv=6144ch bf16w, {steps} steps",
        "us_per_step": wall / steps * 1e6,
        "us_per_token": wall / steps / B * 1e6,
        "kernel": "dn_decode_kernel", "kernel_us": avg_s * 1e6,
        "gate_kernel_us": msg / max(ng, 1) * 1e3,
        "alg_bytes": alg, "achieved_GBs": alg / avg_s / 1e9,
    }
    if cpu:
        res["cpu"] = cpu_dn_conv(d, B, H)
    return res


def cpu_dn_conv(d, B, H, steps=96):
    """Oracle (CPU restatement, CPU-exact semantics) on the first `steps`
    steps of the same workload, all B x H units in parallel."""
    from oracle import oracle as O
    from gpu_common import oracle_dn  # noqa: F401  (same driver as the tests)
    sub = dict(d)
    for k in ("x", "a", "b"):
        sub[k] = np.ascontiguousarray(d[k][:steps])
    from vx27_amd import lib as L
    th = O.default_threads()
    _, _, _, secs = oracle_dn(sub, L.DN_CONV | L.DN_PRE_L2, B, H, H, steps, threads=th)
    return {"value": secs / (steps * B) * 1e6, "unit": "us/token", "cores": th, "kind": "port",
            "sample": f"oracle step_exact path, {B} seq x {H} heads x {steps} of the steps, {th} threads"}


def bench_dn_recurrent(ctx, steps=2000):
    """16 heads x 2000 steps, one sequence: per-step launches and one
    multi-step launch (state resident in registers)."""
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
    ctx.sync()
    t0 = time.perf_counter()
    for t in range(steps):
        L.check(fn(ctx.h, C.byref(per[t])), "dn_decode")
    ctx.sync()
    single = time.perf_counter() - t0
    return {"workload": f"dn_recurrent B=1 heads=16 {steps} steps",
            "us_per_step_multistep_call": multi / steps * 1e6,
            "us_per_step_per_step_calls": single / steps * 1e6}


# -------------------------------------------------------------------- GQA
def bench_gqa(ctx, B, Lctx=8192, iters=20):
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
    ctx.prof_enable(True)
    t0 = time.perf_counter()
    for _ in range(iters):
        L.check(fn(ctx.h, C.byref(desc)), "gqa_decode")
    ctx.sync()
    wall = (time.perf_counter() - t0) / iters
    n, ms = ctx.prof_read("gqa_split")
    ctx.prof_enable(False)
    nk = Lctx + 1
    alg = B * 4 * nk * hd * 2 * 2          # K and V bf16 of every attended position
    avg_s = ms / n / 1e3
    return {"workload": f"gqa_decode B={B} L={Lctx}", "us_per_step": wall * 1e6,
            "us_per_token": wall / B * 1e6, "kernel": "gqa_split", "kernel_us": avg_s * 1e6,
            "alg_bytes": alg, "achieved_GBs": alg / avg_s / 1e9}


# ------------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="dn_conv")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the mixers "
              "shard per (sequence, head) with no exchange -- see DESIGN.md", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from vx27_amd import lib as L
    ctx = L.Ctx(0)
    log(f"bench: {L.lib().vx27_hip_version().decode()} workload={args.workload}")
    if args.workload != "dn_conv":
        sys.exit(f"unknown workload {args.workload}")
    main_res = bench_dn_conv(ctx, args.steps, args.warmup, cpu=not args.no_cpu)
    log(f"  dn_conv: {main_res['us_per_token']:.3f} us/token, kernel {main_res['kernel_us']:.1f} us, "
        f"{main_res['achieved_GBs']:.0f} GB/s")
    extra = {}
    if not args.no_extra:
        for B in (1, 32):
            r = bench_gqa(ctx, B)
            extra[f"gqa8k_B{B}"] = r
            log(f"  gqa B={B}: {r['us_per_step']:.1f} us/step, split kernel {r['kernel_us']:.1f} us, "
                f"{r['achieved_GBs']:.0f} GB/s")
        r = bench_dn_recurrent(ctx)
        extra["dn_recurrent"] = r
        log(f"  dn_recurrent: {r['us_per_step_multistep_call']:.2f} us/step (one call), "
            f"{r['us_per_step_per_step_calls']:.2f} us/step (per-step calls)")
    ach = main_res["achieved_GBs"] * 1e9
    line = {
        "metric": METRIC,
        "value": round(main_res["us_per_token"], 4),
        "unit": "us/token",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(main_res["us_per_step"] / 1e3, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (fp64 accumulation)", "data": "synthetic",
        "config": {"workload": main_res["workload"], "batch": 64, "heads": 16, "head_dim": 128},
        "roofline": {"bound": "hbm", "achieved": round(ach / 1e9, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK, 4), "traffic": None,
                     "kernel": main_res["kernel"], "kernel_us": round(main_res["kernel_us"], 2),
                     "alg_bytes_per_launch": main_res["alg_bytes"]},
        "cpu_baseline": main_res.get("cpu"),
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
