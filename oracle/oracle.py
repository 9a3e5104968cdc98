"""Python binding of the oracle (CPU restatement of the reference mixer math).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker and by bench.py's cpu_baseline leg.  The product package (vx27_amd)
never imports it.

Two libraries are bound here:
  liboracle.so          the restatement (oracle/vx27_oracle.c, orc_cpu.c)
  _ref/libvx27ref.so    the reference's own hot-path C compiled unmodified by
                        oracle/Makefile (present only where it was built).
"""
from __future__ import annotations

import ctypes as C
import os
import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libvx27ref.so")

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
F64P = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
VP = C.c_void_p
DN_CONV, DN_PRE_RMS, DN_PRE_L2, DN_OUT_GATE = 1, 2, 4, 8


def ptr(a):
    """Raw address of a C-contiguous numpy array (or None)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data


class DnCfg(C.Structure):
    _fields_ = [("nqk", C.c_int), ("nv", C.c_int), ("hd", C.c_int), ("flags", C.c_int),
                ("A_log", VP), ("dt_bias", VP), ("norm_w", VP), ("conv_w", VP)]


class GqaCfg(C.Structure):
    _fields_ = [("n_q", C.c_int), ("n_kv", C.c_int), ("hd", C.c_int), ("rope_dim", C.c_int),
                ("kv_bf16", C.c_int), ("q_norm_w", VP), ("k_norm_w", VP),
                ("k_cache", VP), ("v_cache", VP),
                ("k_pos_stride", C.c_size_t), ("k_head_stride", C.c_size_t),
                ("v_pos_stride", C.c_size_t), ("v_head_stride", C.c_size_t), ("no_gate", C.c_int)]


class AttendArgs(C.Structure):
    _fields_ = [("n_q", C.c_int), ("n_kv", C.c_int), ("hd", C.c_int), ("n_keys", C.c_int),
                ("dot_double", C.c_int), ("kv_bf16", C.c_int), ("q", VP), ("k", VP), ("v", VP),
                ("k_pos_stride", C.c_size_t), ("k_head_stride", C.c_size_t),
                ("v_pos_stride", C.c_size_t), ("v_head_stride", C.c_size_t), ("out", VP)]


class AttendBatchArgs(C.Structure):
    _fields_ = [("B", C.c_int), ("n_q", C.c_int), ("n_kv", C.c_int), ("hd", C.c_int),
                ("threads", C.c_int), ("kv_bf16", C.c_int), ("dot_double", C.c_int),
                ("n_keys", VP), ("q", VP), ("k", VP), ("v", VP),
                ("seq_stride", C.c_size_t), ("k_pos_stride", C.c_size_t),
                ("k_head_stride", C.c_size_t), ("v_pos_stride", C.c_size_t),
                ("v_head_stride", C.c_size_t), ("out", VP)]


class DnRunArgs(C.Structure):
    _fields_ = [("B", C.c_int), ("nqk", C.c_int), ("nv", C.c_int), ("hd", C.c_int),
                ("steps", C.c_int), ("flags", C.c_int), ("threads", C.c_int),
                ("S", VP), ("conv_state", VP), ("conv_w", VP), ("x", VP),
                ("q", VP), ("k", VP), ("v", VP), ("a", VP), ("b", VP),
                ("A_log", VP), ("dt_bias", VP), ("norm_w", VP), ("z", VP), ("out", VP)]


class GqaPrefillArgs(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("B", "T", "n_q", "n_kv", "hd", "rope_dim", "pos0", "L", "threads")] + \
               [("rope_theta", C.c_float), ("rope_yarn", C.c_float)] + \
               [(n, VP) for n in ("q", "gate", "k", "v", "q_norm_w", "k_norm_w", "k_cache", "v_cache", "out")] + \
               [("no_gate", C.c_int)]


class DnLayerW(C.Structure):
    _fields_ = [(n, VP) for n in ("ln_w", "w_qkv", "w_z", "w_a", "w_b", "conv_w",
                                   "A_log", "dt_bias", "norm_w", "w_out")]


class GqaLayerW(C.Structure):
    _fields_ = [(n, VP) for n in ("ln_w", "w_q", "w_k", "w_v", "q_norm_w", "k_norm_w", "w_o")]


_lib = None


def lib():
    """The restatement library, with argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
    L = C.CDLL(LIB_PATH)
    sig = {
        "orc_f32_to_bf16_n": (None, [F32P, U16P, C.c_size_t]),
        "orc_bf16_to_f32_n": (None, [U16P, F32P, C.c_size_t]),
        "orc_state_per_layer": (C.c_int, []),
        "orc_state_total": (C.c_int, []),
        "orc_state_mb": (C.c_double, [C.c_int]),
        "orc_update_simple": (None, [F32P, F32P, F32P, C.c_float, C.c_int]),
        "orc_retrieve_simple": (None, [F32P, F32P, F32P, C.c_int]),
        "orc_l2norm": (None, [F32P, F32P, C.c_int]),
        "orc_gate_params": (None, [C.c_double] * 4 + [C.POINTER(C.c_double)] * 2),
        "orc_step_exact": (None, [F32P, F32P, F32P, F32P, C.c_double, C.c_double, F32P, C.c_int]),
        "orc_conv1d_step": (None, [F32P, F32P, F32P, F32P, C.c_int, C.c_int]),
        "orc_kv_for_q": (C.c_int, [C.c_int]),
        "orc_rmsnorm_w": (None, [F32P, F32P, F32P, C.c_int, C.c_float]),
        "orc_rmsn_1pw": (None, [F32P, VP, F32P, C.c_int]),
        "orc_rmsn_std": (None, [F32P, VP, F32P, C.c_int]),
        "orc_silu": (C.c_float, [C.c_float]),
        "orc_attn_1q": (None, [F32P, F32P, F32P, C.c_int, F32P]),
        "orc_attend": (None, [C.POINTER(AttendArgs)]),
        "orc_rope_cos_sin": (None, [C.c_int, F32P, F32P, C.c_int, C.c_float, C.c_float]),
        "orc_rope_apply": (None, [F32P, C.c_int, C.c_int, C.c_int, F32P, F32P]),
        "orc_mrope_cos_sin_text": (None, [C.c_int, F32P, F32P]),
        "orc_matvec": (None, [VP, C.c_int, F32P, F32P, C.c_int, C.c_int]),
        "orc_dn_token": (None, [C.POINTER(DnCfg), F32P, F32P, F32P, VP, F32P, VP, F32P]),
        "orc_gqa_token": (None, [C.POINTER(GqaCfg), F32P, C.c_size_t, VP, C.c_size_t,
                                 F32P, F32P, C.c_int, F32P, F32P, F32P]),
        "orc_dn_layer_token": (None, [C.POINTER(DnLayerW), F32P, F32P, F32P, F32P]),
        "orc_gqa_layer_token": (None, [C.POINTER(GqaLayerW), F32P, C.c_int, F32P, F32P, F32P]),
        "orc_dn_run": (C.c_double, [C.POINTER(DnRunArgs)]),
        "orc_dn_run_avx2": (C.c_double, [C.c_int] * 5 + [F32P, F32P, F32P, F32P, F64P, F64P, F32P, VP, VP]),
        "orc_update_avx2_pub": (None, [F32P, F32P, F32P, C.c_float, C.c_int]),
        "orc_retrieve_avx2_pub": (None, [F32P, F32P, F32P, C.c_int]),
        "orc_attend_batch": (C.c_double, [C.POINTER(AttendBatchArgs)]),
        "orc_gqa_prefill": (C.c_double, [C.POINTER(GqaPrefillArgs)]),
        "orc_matvec_batch": (C.c_double, [VP, C.c_int, F32P, F32P, C.c_int, C.c_int, C.c_int, C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


_ref = None


def ref():
    """The compiled reference (oracle/_ref/libvx27ref.so) or None if not built."""
    global _ref
    if _ref is not None:
        return _ref
    if not os.path.exists(REF_PATH):
        return None
    R = C.CDLL(REF_PATH, mode=os.RTLD_LAZY | os.RTLD_LOCAL)
    sig = {
        "vx27_deltanet_state_per_layer": (C.c_int, []),
        "vx27_deltanet_state_total": (C.c_int, []),
        "vx27_deltanet_state_mb": (C.c_double, [C.c_int]),
        "vx27_deltanet_update_ref": (None, [F32P, F32P, F32P, C.c_float, C.c_int]),
        "vx27_deltanet_retrieve_ref": (None, [F32P, F32P, F32P, C.c_int]),
        "vx27_deltanet_update_tiled": (None, [F32P, F32P, F32P, C.c_float, C.c_int]),
        "vx27_deltanet_retrieve_tiled": (None, [F32P, F32P, F32P, C.c_int]),
        "vx27_deltanet_update_avx2": (None, [F32P, F32P, F32P, C.c_float, C.c_int]),
        "vx27_deltanet_retrieve_avx2": (None, [F32P, F32P, F32P, C.c_int]),
        "vx27_deltanet_l2norm": (None, [F32P, F32P, C.c_int]),
        "vx27_deltanet_step_exact": (None, [F32P, F32P, F32P, F32P, C.c_double, C.c_double, F32P, C.c_int]),
        "vx27_deltanet_gate_params": (None, [C.c_double] * 4 + [C.POINTER(C.c_double)] * 2),
        "vx27_conv1d_step": (None, [F32P, F32P, F32P, F32P, C.c_int, C.c_int]),
        "vx27_gqa_kv_for_q": (C.c_int, [C.c_int]),
        "vx27_rmsnorm": (None, [F32P, F32P, F32P, C.c_int, C.c_float]),
        "vx27_attn_1q": (None, [F32P, F32P, F32P, C.c_int, F32P]),
        "vx27_rope_cos_sin": (None, [C.c_int, F32P, F32P, C.c_int, C.c_float, C.c_float]),
        "vx27_rope_apply": (None, [F32P, C.c_int, C.c_int, C.c_int, F32P, F32P]),
        "vx27_mrope_cos_sin_text": (None, [C.c_int, F32P, F32P]),
        "vx27_qlayer": (None, [VP, C.c_int, C.c_int, F32P, F32P, C.c_int, I32P,
                               VP, VP, VP, VP, VP, VP]),
    }
    for name, (res, args) in sig.items():
        f = getattr(R, name)
        f.restype = res
        f.argtypes = args
    _ref = R
    return R


# ----------------------------------------------------------------- helpers
def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def to_bf16(x):
    x = f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def from_bf16(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_f32_n(h.reshape(-1), out.reshape(-1), h.size)
    return out


def round_bf16(x):
    return from_bf16(to_bf16(x))


def gate_params(a, A_log, b, dt_bias):
    be, g = C.c_double(), C.c_double()
    lib().orc_gate_params(float(a), float(A_log), float(b), float(dt_bias), C.byref(be), C.byref(g))
    return be.value, g.value


def step_exact(S, q, k, v, beta, g_log):
    """One step_exact on S (mutated in place); returns o."""
    o = np.empty(q.shape[-1], np.float32)
    lib().orc_step_exact(S.reshape(-1), f32(q), f32(k), f32(v), float(beta), float(g_log), o,
                         q.shape[-1])
    return o


def l2norm(x):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_l2norm(x, y, x.size)
    return y


def rope_cos_sin(pos, rope_dim=64, theta=1e7, yarn=1.0):
    c = np.empty(rope_dim // 2, np.float32)
    s = np.empty(rope_dim // 2, np.float32)
    lib().orc_rope_cos_sin(int(pos), c, s, rope_dim, float(theta), float(yarn))
    return c, s


def rope_table(positions, rope_dim=64, theta=1e7, yarn=1.0):
    """[n][rope_dim/2] cos and sin tables for the given positions."""
    positions = list(positions)
    cs = np.empty((len(positions), rope_dim // 2), np.float32)
    sn = np.empty_like(cs)
    for i, p in enumerate(positions):
        cs[i], sn[i] = rope_cos_sin(p, rope_dim, theta, yarn)
    return cs, sn


def attend(q, k, v, n_keys, k_strides, v_strides, n_kv, dot_double=1, kv_bf16=0):
    """orc_attend over one sequence; q [n_q][hd]; returns out [n_q][hd]."""
    q = f32(q)
    n_q, hd = q.shape
    out = np.empty((n_q, hd), np.float32)
    a = AttendArgs(n_q, n_kv, hd, int(n_keys), int(dot_double), int(kv_bf16), ptr(q), ptr(k), ptr(v),
                   k_strides[0], k_strides[1], v_strides[0], v_strides[1], ptr(out))
    lib().orc_attend(C.byref(a))
    return out


def default_threads():
    """Threads for the CPU baseline: the CPUs this process may run on, at
    most 16 (the host CPU share of one GPU on the GPU machines, whatever
    nproc reports there)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def host_info():
    """nproc, usable CPUs, and the CPU model name of this host."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"nproc": os.cpu_count(), "usable_cpus": usable, "cpu_model": model}


def ref_avx2_fns():
    """(update, retrieve) function pointers of the compiled reference's
    vx27_deltanet_update_avx2 / retrieve_avx2, or (None, None) if
    oracle/_ref was not built."""
    R = ref()
    if R is None:
        return None, None
    return (C.cast(R.vx27_deltanet_update_avx2, VP).value, C.cast(R.vx27_deltanet_retrieve_avx2, VP).value)
