"""The 64 token mixers of one decode step, on device (host harness).

MixerStack holds 48 Gated DeltaNet mixers and 16 gated GQA mixers (every
4th layer is attention, vx27_config.h:10-12) for B sequences at a given
context: random-init bf16 weights (std 0.02, generated on the device by the
seeded counter generator and tiled once), fp32 DeltaNet state and conv
state, and a bf16 KV cache per attention layer, prefilled with N(0,1)
values.  step() runs one decode token of every sequence through all 64
mixers (each reads the same input x, as a mixer benchmark does; the FFN and
residual stream between layers are outside the mixer path) and advances the
positions.  The layer calls are those of vx27_qlayer's two mixer branches
(src/vx27_qfwd.c:92-215) through vx27_hip_dn_layer_decode and
vx27_hip_gqa_layer_decode.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import lib as L
from . import workloads as W

H = 5120          # hidden size
GQ = 256          # GQA head dim
HD = 128          # DeltaNet head dim


class MixerStack:
    def __init__(self, ctx, B=4, Lctx=131072, extra_pos=64, n_layers=64, nqk=16, nv=48, pos=None):
        """pos: optional initial positions [B] (default Lctx for every
        sequence); the cache holds rows up to Lctx + extra_pos."""
        self.ctx, self.B, self.Lctx, self.nv, self.nqk = ctx, B, Lctx, nv, nqk
        self.H = H
        qd, vd = nqk * HD, nv * HD
        self.C = C_ = 2 * qd + vd
        p0 = np.full(B, Lctx, np.int32) if pos is None else np.ascontiguousarray(pos, np.int32)
        self.Lcap = (max(Lctx, int(p0.max())) + extra_pos + 63) // 64 * 64
        r = W.rng(5, "mixer_stack")
        s = 5000
        fill = ctx.fill_normal
        self.x = ctx.buf(B * H * 4)
        self.xp = ctx.buf(L.lib().vx27_hip_pack_bytes(H, B))
        self.out = ctx.buf(n_layers * B * H * 4)
        self.pos = ctx.put(p0)
        self.layers = []
        self.kv_bytes = self.w_bytes = self.s_bytes = 0
        self._tmp_elems = (C_ + vd + 2 * nv) * H
        tmp = ctx.buf(self._tmp_elems * 2)      # row-major staging for weight tiling
        lib = L.lib()

        def weight(N, K, seed):
            """bf16 ~N(0, 0.02) [N][K] generated row-major, stored tiled."""
            fill(tmp, N * K, seed, 0.02, bf16=True)
            wt = ctx.buf(N * K * 2)
            L.check(lib.vx27_hip_pack_weights_bf16(ctx.h, tmp.ptr, N, K, wt.ptr), "pack_weights")
            return wt
        for li in range(n_layers):
            full = (li + 1) % 4 == 0
            s += 10
            lay = {"kind": "gqa" if full else "dn", "seed": s}
            if full:
                Nq = 24 * 2 * GQ + 2 * 4 * GQ
                lay["w_qkv_shape"], lay["w_o_shape"] = (Nq, H), (H, 24 * GQ)
                wq = weight(Nq, H, s + 1)
                wo = weight(H, 24 * GQ, s + 2)
                lay["q_norm_w"], lay["k_norm_w"] = W.normal(r, GQ, 0.1), W.normal(r, GQ, 0.1)
                qn, kn = ctx.put(lay["q_norm_w"]), ctx.put(lay["k_norm_w"])
                n = B * 4 * self.Lcap * GQ
                kc = ctx.buf(n * 2); fill(kc, n, s + 3, 1.0, bf16=True)
                vc = ctx.buf(n * 2); fill(vc, n, s + 4, 1.0, bf16=True)
                lay["k_cache"], lay["v_cache"] = kc, vc
                lay["desc"] = L.GqaLayerDesc(B, 24, 4, GQ, H, 64, 1e7, 1.0, self.Lcap, self.x.ptr, self.xp.ptr,
                                             wq.ptr, wo.ptr, qn.ptr, kn.ptr, self.pos.ptr, kc.ptr, vc.ptr,
                                             self.out.ptr + li * B * H * 4, 0)
                self.w_bytes += wq.nbytes + wo.nbytes
            else:
                Ni = C_ + vd + 2 * nv
                lay["w_in_shape"], lay["w_out_shape"] = (Ni, H), (H, vd)
                wi = weight(Ni, H, s + 1)
                wo = weight(H, vd, s + 2)
                cw = ctx.buf(C_ * 4 * 2); fill(cw, C_ * 4, s + 3, 0.2, bf16=True)
                lay["A_log"] = r.uniform(-2, 1, nv).astype(np.float32)
                lay["dt_bias"] = W.normal(r, nv, 0.1)
                lay["norm_w"] = W.normal(r, HD, 0.1, 1.0)
                A_log, dtb, nw = ctx.put(lay["A_log"]), ctx.put(lay["dt_bias"]), ctx.put(lay["norm_w"])
                S = ctx.buf(B * nv * HD * HD * 4); fill(S, B * nv * HD * HD, s + 4, 0.02)
                cs = ctx.buf(B * C_ * 3 * 4); fill(cs, B * C_ * 3, s + 5, 0.5)
                lay["S"], lay["conv_state"], lay["conv_w"] = S, cs, cw
                lay["desc"] = L.DnLayerDesc(B, nqk, nv, HD, H, self.x.ptr, self.xp.ptr, wi.ptr, wo.ptr, cw.ptr,
                                            L.BF16, A_log.ptr, dtb.ptr, nw.ptr, S.ptr, cs.ptr,
                                            self.out.ptr + li * B * H * 4)
                self.w_bytes += wi.nbytes + wo.nbytes
                self.s_bytes += 2 * S.nbytes + 2 * cs.nbytes
            self.layers.append(lay)
        ctx.sync()
        tmp.free()

    def step(self):
        lib = L.lib()
        L.check(lib.vx27_hip_pack_x(self.ctx.h, self.x.ptr, self.B, self.H, self.xp.ptr), "pack_x")
        for lay in self.layers:
            fn = lib.vx27_hip_gqa_layer_decode if lay["kind"] == "gqa" else lib.vx27_hip_dn_layer_decode
            L.check(fn(self.ctx.h, C.byref(lay["desc"])), lay["kind"])
        L.check(lib.vx27_hip_advance_pos(self.ctx.h, self.pos.ptr, self.B), "advance_pos")

    def alg_bytes(self, pos):
        """Algorithmic HBM bytes of one step at key count pos+1: KV of every
        attended position, all weights, DeltaNet state and conv state r+w."""
        kv = 16 * self.B * 4 * (pos + 1) * GQ * 2 * 2
        return kv + self.w_bytes + self.s_bytes

    # ---------------------------------------------------- host copies (checks)
    def outputs(self):
        """[n_layers][B][H] outputs of the last step."""
        return self.out.download((len(self.layers), self.B, H), np.float32)

    def weights_rowmajor(self, li):
        """The row-major bf16 weights of layer li (regenerated from their seeds)."""
        lay = self.layers[li]
        names = ("w_qkv", "w_o") if lay["kind"] == "gqa" else ("w_in", "w_out")
        tmp = self.ctx.buf(self._tmp_elems * 2)
        out = {}
        for j, nm in enumerate(names):
            N, K = lay[nm + "_shape"]
            self.ctx.fill_normal(tmp, N * K, lay["seed"] + 1 + j, 0.02, bf16=True)
            out[nm] = tmp.download((N, K), np.uint16)
        tmp.free()
        return out
