"""Host-side mirror of the reference's mixer interface over the C ABI.

Two levels, both calling libvx27_hip (no host compute):
  * the reference's own per-head functions (deltanet_step_exact, conv1d_step,
    rmsnorm, attn_1q, rope_*), host arrays in / out, exactly the reference's
    arguments (src/vx27_deltanet.h:10-59, src/vx27_gqa.h:8-13,
    src/vx27_rope.h:11-17);
  * device-resident layer objects (DeltaNetLayer, GatedGQALayer) holding the
    state / KV cache of B sequences and running the batched decode kernels,
    the form vx27_qlayer's mixer sections (src/vx27_qfwd.c:92-215) take here.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import lib as L
from .lib import check, hptr


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


# ----------------------------------------------- the reference's own calls
def deltanet_step_exact(S, q, k, v, beta, g_log):
    """vx27_deltanet_step_exact: S (float32 [hd][hd]) updated in place; returns o."""
    assert S.dtype == np.float32 and S.flags["C_CONTIGUOUS"]
    q, k, v = _f32(q), _f32(k), _f32(v)
    o = np.empty(q.size, np.float32)
    L.lib().vx27_deltanet_step_exact(hptr(S), hptr(q), hptr(k), hptr(v), float(beta), float(g_log),
                                     hptr(o), q.size)
    return o


def deltanet_gate_params(a, A_log, b, dt_bias):
    be, g = C.c_double(), C.c_double()
    L.lib().vx27_deltanet_gate_params(float(a), float(A_log), float(b), float(dt_bias),
                                      C.byref(be), C.byref(g))
    return be.value, g.value


def deltanet_l2norm(x):
    x = _f32(x)
    y = np.empty_like(x)
    L.lib().vx27_deltanet_l2norm(hptr(x), hptr(y), x.size)
    return y


def conv1d_step(state, x, w, apply_silu=True):
    """vx27_conv1d_step: state float32 [C][3] updated in place; returns y."""
    assert state.dtype == np.float32 and state.flags["C_CONTIGUOUS"]
    x, w = _f32(x), _f32(w)
    y = np.empty(x.size, np.float32)
    L.lib().vx27_conv1d_step(hptr(state), hptr(x), hptr(w), hptr(y), x.size, int(bool(apply_silu)))
    return y


def rmsnorm(x, w, eps):
    x, w = _f32(x), _f32(w)
    y = np.empty_like(x)
    L.lib().vx27_rmsnorm(hptr(x), hptr(w), hptr(y), x.size, float(eps))
    return y


def attn_1q(q, kcache, vcache, n_pos):
    q, kc, vc = _f32(q), _f32(kcache), _f32(vcache)
    out = np.empty(24 * 256, np.float32)
    L.lib().vx27_attn_1q(hptr(q), hptr(kc), hptr(vc), int(n_pos), hptr(out))
    return out


def rope_cos_sin(pos, rope_dim=64, theta=1e7, yarn=1.0):
    c = np.empty(rope_dim // 2, np.float32)
    s = np.empty(rope_dim // 2, np.float32)
    L.lib().vx27_rope_cos_sin(int(pos), hptr(c), hptr(s), rope_dim, float(theta), float(yarn))
    return c, s


def rope_apply(v, n_heads, head_dim, rope_dim, cosv, sinv):
    """vx27_rope_apply in place on float32 v."""
    assert v.dtype == np.float32 and v.flags["C_CONTIGUOUS"]
    cosv, sinv = _f32(cosv), _f32(sinv)
    L.lib().vx27_rope_apply(hptr(v), n_heads, head_dim, rope_dim, hptr(cosv), hptr(sinv))


# ------------------------------------------------- device-resident layers
class DeltaNetLayer:
    """One Gated DeltaNet layer's mixer core for B sequences, state on device.

    S [B][nv][128][128] fp32 (row = key dim), conv state [B][C][3] fp32.
    decode() runs `steps` tokens per sequence through vx27_hip_dn_decode.
    """

    def __init__(self, ctx, B, nqk, nv, A_log, dt_bias, norm_w=None, conv_w=None,
                 conv_w_dtype=L.F32, S0=None, conv0=None, hd=128):
        self.ctx, self.B, self.nqk, self.nv, self.hd = ctx, B, nqk, nv, hd
        self.C = 2 * nqk * hd + nv * hd
        nS = B * nv * hd * hd
        self.S = ctx.buf(nS * 4)
        if S0 is None:
            self.S.zero()
        else:
            self.S.upload(_f32(S0).reshape(-1))
        self.conv_state = ctx.buf(B * self.C * 3 * 4)
        if conv0 is None:
            self.conv_state.zero()
        else:
            self.conv_state.upload(_f32(conv0).reshape(-1))
        self.A_log = ctx.put(_f32(A_log))
        self.dt_bias = ctx.put(_f32(dt_bias))
        self.norm_w = ctx.put(_f32(norm_w)) if norm_w is not None else None
        self.conv_w_dtype = conv_w_dtype
        if conv_w is not None:
            cw = np.ascontiguousarray(conv_w, np.uint16 if conv_w_dtype == L.BF16 else np.float32)
            self.conv_w = ctx.put(cw)
        else:
            self.conv_w = None

    def desc(self, steps, flags, out, a, b, x=None, q=None, k=None, v=None, z=None):
        """Descriptor over device pointers (ints)."""
        d = L.DnDesc()
        d.B, d.nqk, d.nv, d.hd, d.steps, d.flags = self.B, self.nqk, self.nv, self.hd, steps, flags
        d.S = self.S.ptr
        d.conv_state = self.conv_state.ptr
        d.conv_w = self.conv_w.ptr if self.conv_w else None
        d.conv_w_dtype = self.conv_w_dtype
        d.x, d.q, d.k, d.v, d.a, d.b, d.z, d.out = x, q, k, v, a, b, z, out
        d.A_log, d.dt_bias = self.A_log.ptr, self.dt_bias.ptr
        d.norm_w = self.norm_w.ptr if self.norm_w else None
        return d

    def decode(self, steps, flags, a, b, x=None, q=None, k=None, v=None, z=None):
        """Host arrays in, host output [steps][B][nv][hd] back."""
        ctx = self.ctx
        bufs = {n: ctx.put(_f32(arr)) for n, arr in
                (("a", a), ("b", b), ("x", x), ("q", q), ("k", k), ("v", v), ("z", z))
                if arr is not None}
        out = ctx.buf(steps * self.B * self.nv * self.hd * 4)
        p = {n: bb.ptr for n, bb in bufs.items()}
        d = self.desc(steps, flags, out.ptr, p["a"], p["b"], p.get("x"), p.get("q"), p.get("k"),
                      p.get("v"), p.get("z"))
        check(L.lib().vx27_hip_dn_decode(ctx.h, C.byref(d)), "dn_decode")
        res = out.download((steps, self.B, self.nv, self.hd), np.float32)
        for bb in list(bufs.values()) + [out]:
            bb.free()
        return res

    def state(self):
        return self.S.download((self.B, self.nv, self.hd, self.hd), np.float32)

    def conv(self):
        return self.conv_state.download((self.B, self.C, 3), np.float32)


class GatedGQALayer:
    """One gated GQA layer's mixer core for B sequences over a bf16 KV cache
    of capacity L positions (format of vx27_hip.h)."""

    def __init__(self, ctx, B, Lcap, q_norm_w, k_norm_w, n_q=24, n_kv=4, hd=256, rope_dim=64,
                 theta=1e7, yarn=1.0, flags=0):
        assert Lcap % 64 == 0
        self.ctx, self.B, self.L, self.n_q, self.n_kv, self.hd = ctx, B, Lcap, n_q, n_kv, hd
        self.rope_dim, self.theta, self.yarn, self.flags = rope_dim, theta, yarn, flags
        n = B * n_kv * Lcap * hd
        self.k_cache = ctx.buf(n * 2).zero()
        self.v_cache = ctx.buf(n * 2).zero()
        self.q_norm_w = ctx.put(_f32(q_norm_w))
        self.k_norm_w = ctx.put(_f32(k_norm_w))

    def write_kv(self, b, p0, k_rows, v_rows):
        """Rows [n][n_kv][hd] (fp32, rounded to bf16) at positions p0.. of sequence b."""
        k_rows, v_rows = _f32(k_rows), _f32(v_rows)
        n = k_rows.shape[0]
        kb, vb = self.ctx.put(k_rows), self.ctx.put(v_rows)
        check(L.lib().vx27_hip_kv_write(self.ctx.h, self.k_cache.ptr, self.v_cache.ptr, self.B,
                                        self.n_kv, self.hd, self.L, b, p0, n, kb.ptr, vb.ptr),
              "kv_write")
        self.ctx.sync()
        kb.free(); vb.free()

    def read_kv(self, b, p0, n):
        kb = self.ctx.buf(max(n, 1) * self.n_kv * self.hd * 4)
        vb = self.ctx.buf(max(n, 1) * self.n_kv * self.hd * 4)
        check(L.lib().vx27_hip_kv_read(self.ctx.h, self.k_cache.ptr, self.v_cache.ptr, self.B,
                                       self.n_kv, self.hd, self.L, b, p0, n, kb.ptr, vb.ptr),
              "kv_read")
        k = kb.download((n, self.n_kv, self.hd), np.float32)
        v = vb.download((n, self.n_kv, self.hd), np.float32)
        kb.free(); vb.free()
        return k, v

    def desc(self, pos, q, q_strides, gate, g_strides, k_new, v_new, out, n_split=0):
        d = L.GqaDesc()
        d.B, d.n_q, d.n_kv, d.hd = self.B, self.n_q, self.n_kv, self.hd
        d.rope_dim, d.rope_theta, d.rope_yarn, d.L, d.flags = (self.rope_dim, self.theta,
                                                              self.yarn, self.L, self.flags)
        d.pos, d.q, d.gate, d.k_new, d.v_new, d.out = pos, q, gate, k_new, v_new, out
        d.q_seq_stride, d.q_head_stride = q_strides
        d.gate_seq_stride, d.gate_head_stride = g_strides
        d.q_norm_w, d.k_norm_w = self.q_norm_w.ptr, self.k_norm_w.ptr
        d.k_cache, d.v_cache = self.k_cache.ptr, self.v_cache.ptr
        d.n_split = n_split
        return d

    def decode(self, pos, qg, k_new, v_new, n_split=0):
        """qg [B][n_q][2*hd] interleaved q|gate (vx27_qfwd.c:160-167); k_new, v_new
        [B][n_kv][hd]; pos [B].  Returns out [B][n_q][hd]."""
        ctx = self.ctx
        hd = self.hd
        qb = ctx.put(_f32(qg))
        kb, vb = ctx.put(_f32(k_new)), ctx.put(_f32(v_new))
        pb = ctx.put(np.ascontiguousarray(pos, np.int32))
        ob = ctx.buf(self.B * self.n_q * hd * 4)
        d = self.desc(pb.ptr, qb.ptr, (self.n_q * 2 * hd, 2 * hd), qb.ptr + hd * 4,
                      (self.n_q * 2 * hd, 2 * hd), kb.ptr, vb.ptr, ob.ptr, n_split)
        check(L.lib().vx27_hip_gqa_decode(ctx.h, C.byref(d)), "gqa_decode")
        out = ob.download((self.B, self.n_q, hd), np.float32)
        for bb in (qb, kb, vb, pb, ob):
            bb.free()
        return out
