"""ctypes binding of libvx27_hip.so (the C ABI in include/vx27_hip.h).

The library is loaded from this package directory; if it is missing the
import fails loudly -- there is no host fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libvx27_hip.so")

VP = C.c_void_p
F32, BF16 = 0, 1
DN_CONV, DN_PRE_RMS, DN_PRE_L2, DN_OUT_GATE, DN_EXACT, DN_BF16 = 1, 2, 4, 8, 16, 32
GQA_NORM_W = 1
GQA_NO_GATE = 2
ERR_ABORT, ERR_POISON = 0, 1


class DnDesc(C.Structure):
    _fields_ = [("B", C.c_int), ("nqk", C.c_int), ("nv", C.c_int), ("hd", C.c_int),
                ("steps", C.c_int), ("flags", C.c_uint),
                ("S", VP), ("conv_state", VP), ("conv_w", VP), ("conv_w_dtype", C.c_int),
                ("x", VP), ("q", VP), ("k", VP), ("v", VP), ("a", VP), ("b", VP),
                ("A_log", VP), ("dt_bias", VP), ("norm_w", VP), ("z", VP), ("out", VP)]


class DnPrefillDesc(C.Structure):
    _fields_ = [("B", C.c_int), ("T", C.c_int), ("nqk", C.c_int), ("nv", C.c_int), ("hd", C.c_int),
                ("flags", C.c_uint), ("S", VP), ("q", VP), ("k", VP), ("v", VP), ("a", VP), ("b", VP),
                ("A_log", VP), ("dt_bias", VP), ("out", VP),
                ("x", VP), ("conv_state", VP), ("conv_w", VP), ("conv_w_dtype", C.c_int),
                ("norm_w", VP), ("z", VP), ("S_ckpt", VP), ("conv_ckpt", VP)]


class GqaPrefillDesc(C.Structure):
    _fields_ = [("B", C.c_int), ("T", C.c_int), ("n_q", C.c_int), ("n_kv", C.c_int), ("hd", C.c_int),
                ("rope_dim", C.c_int), ("rope_theta", C.c_float), ("rope_yarn", C.c_float),
                ("L", C.c_int), ("pos0", C.c_int), ("flags", C.c_uint),
                ("q", VP), ("q_tok_stride", C.c_size_t), ("q_head_stride", C.c_size_t),
                ("gate", VP), ("gate_tok_stride", C.c_size_t), ("gate_head_stride", C.c_size_t),
                ("k_new", VP), ("v_new", VP), ("q_norm_w", VP), ("k_norm_w", VP),
                ("k_cache", VP), ("v_cache", VP), ("out", VP)]


class GqaDesc(C.Structure):
    _fields_ = [("B", C.c_int), ("n_q", C.c_int), ("n_kv", C.c_int), ("hd", C.c_int),
                ("rope_dim", C.c_int), ("rope_theta", C.c_float), ("rope_yarn", C.c_float),
                ("L", C.c_int), ("flags", C.c_uint), ("pos", VP),
                ("q", VP), ("q_seq_stride", C.c_size_t), ("q_head_stride", C.c_size_t),
                ("gate", VP), ("gate_seq_stride", C.c_size_t), ("gate_head_stride", C.c_size_t),
                ("k_new", VP), ("v_new", VP), ("q_norm_w", VP), ("k_norm_w", VP),
                ("k_cache", VP), ("v_cache", VP), ("out", VP), ("n_split", C.c_int),
                ("kv_seq_stride", C.c_size_t)]


class DnLayerDesc(C.Structure):
    _fields_ = [("B", C.c_int), ("nqk", C.c_int), ("nv", C.c_int), ("hd", C.c_int), ("hidden", C.c_int),
                ("x", VP), ("x_packed", VP), ("w_in", VP), ("w_out", VP), ("conv_w", VP),
                ("conv_w_dtype", C.c_int), ("A_log", VP), ("dt_bias", VP), ("norm_w", VP),
                ("S", VP), ("conv_state", VP), ("out", VP)]


class GqaLayerDesc(C.Structure):
    _fields_ = [("B", C.c_int), ("n_q", C.c_int), ("n_kv", C.c_int), ("hd", C.c_int), ("hidden", C.c_int),
                ("rope_dim", C.c_int), ("rope_theta", C.c_float), ("rope_yarn", C.c_float), ("L", C.c_int),
                ("x", VP), ("x_packed", VP), ("w_qkv", VP), ("w_o", VP), ("q_norm_w", VP), ("k_norm_w", VP),
                ("pos", VP), ("k_cache", VP), ("v_cache", VP), ("out", VP), ("n_split", C.c_int)]


class DnLayerPrefillDesc(C.Structure):
    _fields_ = [("B", C.c_int), ("T", C.c_int), ("nqk", C.c_int), ("nv", C.c_int), ("hd", C.c_int),
                ("hidden", C.c_int), ("flags", C.c_uint), ("x", VP), ("w_in", VP), ("w_out", VP), ("conv_w", VP),
                ("conv_w_dtype", C.c_int), ("A_log", VP), ("dt_bias", VP), ("norm_w", VP), ("S", VP),
                ("conv_state", VP), ("out", VP), ("S_ckpt", VP), ("conv_ckpt", VP)]


class GqaLayerPrefillDesc(C.Structure):
    _fields_ = [("B", C.c_int), ("T", C.c_int), ("n_q", C.c_int), ("n_kv", C.c_int), ("hd", C.c_int),
                ("hidden", C.c_int), ("rope_dim", C.c_int), ("rope_theta", C.c_float), ("rope_yarn", C.c_float),
                ("L", C.c_int), ("pos0", C.c_int), ("flags", C.c_uint), ("x", VP), ("w_qkv", VP), ("w_o", VP),
                ("q_norm_w", VP), ("k_norm_w", VP), ("k_cache", VP), ("v_cache", VP), ("out", VP)]


_SIGS = {
    "vx27_hip_open": (C.c_int, [C.POINTER(VP), C.c_int, C.c_char_p, C.c_size_t]),
    "vx27_hip_close": (None, [VP]),
    "vx27_hip_sync": (C.c_int, [VP]),
    "vx27_hip_set_stream": (C.c_int, [VP, VP]),
    "vx27_hip_get_stream": (VP, [VP]),
    "vx27_hip_last_error": (C.c_char_p, []),
    "vx27_hip_device_count": (C.c_int, []),
    "vx27_hip_version": (C.c_char_p, []),
    "vx27_hip_default_ctx": (VP, []),
    "vx27_hip_enable": (C.c_int, []),
    "vx27_hip_disable": (None, []),
    "vx27_hip_enabled": (C.c_int, []),
    "vx27_hip_prof_enable": (C.c_int, [VP, C.c_int]),
    "vx27_hip_prof_read": (C.c_int, [VP, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_double)]),
    "vx27_hip_set_error_mode": (None, [C.c_int]),
    "vx27_hip_get_error_mode": (C.c_int, []),
    "vx27_hip_alloc": (C.c_int, [VP, C.POINTER(VP), C.c_size_t]),
    "vx27_hip_free": (C.c_int, [VP, VP]),
    "vx27_hip_h2d": (C.c_int, [VP, VP, VP, C.c_size_t]),
    "vx27_hip_d2h": (C.c_int, [VP, VP, VP, C.c_size_t]),
    "vx27_hip_d2d": (C.c_int, [VP, VP, VP, C.c_size_t]),
    "vx27_hip_memset": (C.c_int, [VP, VP, C.c_int, C.c_size_t]),
    "vx27_hip_mem_info": (C.c_int, [VP, C.POINTER(C.c_size_t), C.POINTER(C.c_int), C.POINTER(C.c_int),
                                    C.POINTER(C.c_int)]),
    "vx27_hip_bw_probe": (C.c_int, [VP, C.c_size_t, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "vx27_hip_dn_decode": (C.c_int, [VP, C.POINTER(DnDesc)]),
    "vx27_hip_dn_prefill": (C.c_int, [VP, C.POINTER(DnPrefillDesc)]),
    "vx27_hip_dn_commit": (C.c_int, [VP] + [C.c_int] * 5 + [VP] * 5),
    "vx27_hip_gqa_prefill": (C.c_int, [VP, C.POINTER(GqaPrefillDesc)]),
    "vx27_hip_gqa_decode": (C.c_int, [VP, C.POINTER(GqaDesc)]),
    "vx27_hip_gqa_decode_noalloc": (C.c_int, [VP, C.POINTER(GqaDesc)]),
    "vx27_hip_kv_write": (C.c_int, [VP, VP, VP] + [C.c_int] * 7 + [VP, VP]),
    "vx27_hip_kv_read": (C.c_int, [VP, VP, VP] + [C.c_int] * 7 + [VP, VP]),
    "vx27_hip_rope_table": (C.c_int, [VP, VP, C.c_int, C.c_int, C.c_float, C.c_float, VP, VP]),
    "vx27_hip_gemv_bf16": (C.c_int, [VP, VP, C.c_int, C.c_int, VP, C.c_size_t, C.c_int, VP, C.c_size_t]),
    "vx27_hip_dn_layer_decode": (C.c_int, [VP, C.POINTER(DnLayerDesc)]),
    "vx27_hip_gqa_layer_decode": (C.c_int, [VP, C.POINTER(GqaLayerDesc)]),
    "vx27_hip_dn_layer_prefill": (C.c_int, [VP, C.POINTER(DnLayerPrefillDesc)]),
    "vx27_hip_gqa_layer_prefill": (C.c_int, [VP, C.POINTER(GqaLayerPrefillDesc)]),
    "vx27_hip_pack_bytes": (C.c_size_t, [C.c_int, C.c_int]),
    "vx27_hip_pack_weights_bf16": (C.c_int, [VP, VP, C.c_int, C.c_int, VP]),
    "vx27_hip_gemm_bf16": (C.c_int, [VP, VP, C.c_int, C.c_int, VP, C.c_size_t, C.c_int, VP, C.c_size_t]),
    "vx27_hip_pack_x": (C.c_int, [VP, VP, C.c_int, C.c_int, VP]),
    "vx27_hip_advance_pos": (C.c_int, [VP, VP, C.c_int]),
    "vx27_hip_graph_begin": (C.c_int, [VP]),
    "vx27_hip_graph_end": (C.c_int, [VP, C.POINTER(VP)]),
    "vx27_hip_graph_launch": (C.c_int, [VP, VP]),
    "vx27_hip_graph_destroy": (C.c_int, [VP]),
    "vx27_hip_fill_normal_f32": (C.c_int, [VP, VP, C.c_size_t, C.c_uint64, C.c_float, C.c_float]),
    "vx27_hip_fill_normal_bf16": (C.c_int, [VP, VP, C.c_size_t, C.c_uint64, C.c_float, C.c_float]),
    "vx27_hip_step_exact": (C.c_int, [VP, VP, VP, VP, VP, C.c_double, C.c_double, VP, C.c_int]),
    "vx27_hip_update_simple": (C.c_int, [VP, VP, VP, VP, C.c_float, C.c_int, C.c_int]),
    "vx27_hip_retrieve_simple": (C.c_int, [VP, VP, VP, VP, C.c_int, C.c_int]),
    "vx27_hip_l2norm": (C.c_int, [VP, VP, VP, C.c_int]),
    "vx27_hip_rmsnorm": (C.c_int, [VP, VP, VP, VP, C.c_int, C.c_float]),
    "vx27_hip_conv1d_step": (C.c_int, [VP, VP, VP, VP, VP, C.c_int, C.c_int]),
    "vx27_hip_rope_apply": (C.c_int, [VP, VP, C.c_int, C.c_int, C.c_int, VP, VP]),
    "vx27_hip_attn_1q": (C.c_int, [VP, VP, VP, VP, C.c_int, VP]),
    "vx27_hip_staging": (C.c_int, [VP, C.c_size_t, C.POINTER(VP)]),
    # the reference's own API (host pointers), exported by the same library
    "vx27_deltanet_state_per_layer": (C.c_int, []),
    "vx27_deltanet_state_total": (C.c_int, []),
    "vx27_deltanet_state_mb": (C.c_double, [C.c_int]),
    "vx27_deltanet_update_ref": (None, [VP, VP, VP, C.c_float, C.c_int]),
    "vx27_deltanet_retrieve_ref": (None, [VP, VP, VP, C.c_int]),
    "vx27_deltanet_update_tiled": (None, [VP, VP, VP, C.c_float, C.c_int]),
    "vx27_deltanet_retrieve_tiled": (None, [VP, VP, VP, C.c_int]),
    "vx27_deltanet_update_avx2": (None, [VP, VP, VP, C.c_float, C.c_int]),
    "vx27_deltanet_retrieve_avx2": (None, [VP, VP, VP, C.c_int]),
    "vx27_deltanet_l2norm": (None, [VP, VP, C.c_int]),
    "vx27_deltanet_step_exact": (None, [VP, VP, VP, VP, C.c_double, C.c_double, VP, C.c_int]),
    "vx27_deltanet_gate_params": (None, [C.c_double] * 4 + [C.POINTER(C.c_double)] * 2),
    "vx27_conv1d_step": (None, [VP, VP, VP, VP, C.c_int, C.c_int]),
    "vx27_gqa_kv_for_q": (C.c_int, [C.c_int]),
    "vx27_rmsnorm": (None, [VP, VP, VP, C.c_int, C.c_float]),
    "vx27_attn_1q": (None, [VP, VP, VP, C.c_int, VP]),
    "vx27_rope_cos_sin": (None, [C.c_int, VP, VP, C.c_int, C.c_float, C.c_float]),
    "vx27_rope_apply": (None, [VP, C.c_int, C.c_int, C.c_int, VP, VP]),
    "vx27_mrope_cos_sin_text": (None, [C.c_int, VP, VP]),
}

_lib = None


def lib():
    """The loaded library; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m vx27_amd.build` "
                          "(there is no host fallback)")
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def exported_symbols():
    return list(_SIGS)


class HipError(RuntimeError):
    pass


def check(rc, what=""):
    if rc != 0:
        msg = lib().vx27_hip_last_error().decode(errors="replace")
        raise HipError(f"{what}: {msg}" if what else msg)


def hptr(a):
    """Host address of a C-contiguous numpy array."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class DevBuf:
    """A device allocation owned by a context."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = VP()
        check(lib().vx27_hip_alloc(ctx.h, C.byref(p), self.nbytes), "alloc")
        self.ptr = p.value

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes, (arr.nbytes, self.nbytes)
        check(lib().vx27_hip_h2d(self.ctx.h, self.ptr, arr.ctypes.data, arr.nbytes), "h2d")
        return self

    def download(self, shape, dtype):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().vx27_hip_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def zero(self):
        check(lib().vx27_hip_memset(self.ctx.h, self.ptr, 0, self.nbytes), "memset")
        return self

    def free(self):
        if self.ptr:
            lib().vx27_hip_free(self.ctx.h, self.ptr)
            self.ptr = None


class Ctx:
    """A vx27_hip context (device + stream)."""

    def __init__(self, device=0):
        h = VP()
        err = C.create_string_buffer(512)
        if lib().vx27_hip_open(C.byref(h), device, err, 512) != 0:
            raise HipError(err.value.decode(errors="replace"))
        self.h = h.value
        self._bufs = []

    def buf(self, nbytes):
        b = DevBuf(self, nbytes)
        self._bufs.append(b)
        return b

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        return self.buf(max(arr.nbytes, 1)).upload(arr)

    def sync(self):
        check(lib().vx27_hip_sync(self.h), "sync")

    def mem_info(self):
        """dict(scratch_bytes, retired, schedules, live_graphs) of the context."""
        sb, r, sc, lg = C.c_size_t(), C.c_int(), C.c_int(), C.c_int()
        check(lib().vx27_hip_mem_info(self.h, C.byref(sb), C.byref(r), C.byref(sc), C.byref(lg)), "mem_info")
        return {"scratch_bytes": sb.value, "retired": r.value, "schedules": sc.value, "live_graphs": lg.value}

    def prof_enable(self, on=True):
        check(lib().vx27_hip_prof_enable(self.h, int(on)), "prof_enable")

    def prof_read(self, kernel):
        """(launch count, summed ms) of the recorded launches of `kernel`."""
        n, ms = C.c_int(), C.c_double()
        check(lib().vx27_hip_prof_read(self.h, kernel.encode(), C.byref(n), C.byref(ms)), "prof_read")
        return n.value, ms.value

    def fill_normal(self, buf, n, seed, std=1.0, mean=0.0, bf16=False):
        fn = lib().vx27_hip_fill_normal_bf16 if bf16 else lib().vx27_hip_fill_normal_f32
        check(fn(self.h, buf.ptr if isinstance(buf, DevBuf) else buf, int(n), int(seed), float(mean),
                 float(std)), "fill_normal")

    def put_tiled(self, W_bf16):
        """Upload row-major bf16 weights [N][K] and return them in the MFMA
        tile layout the layer entry points read."""
        W_bf16 = np.ascontiguousarray(W_bf16, np.uint16)
        N, K = W_bf16.shape
        src = DevBuf(self, W_bf16.nbytes).upload(W_bf16)
        dst = self.buf(W_bf16.nbytes)
        check(lib().vx27_hip_pack_weights_bf16(self.h, src.ptr, N, K, dst.ptr), "pack_weights")
        self.sync()
        src.free()
        return dst

    def graph_begin(self):
        check(lib().vx27_hip_graph_begin(self.h), "graph_begin")

    def graph_end(self):
        g = VP()
        check(lib().vx27_hip_graph_end(self.h, C.byref(g)), "graph_end")
        return g.value

    def graph_launch(self, g):
        check(lib().vx27_hip_graph_launch(self.h, g), "graph_launch")

    def close(self):
        for b in self._bufs:
            b.free()
        self._bufs = []
        if self.h:
            lib().vx27_hip_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
