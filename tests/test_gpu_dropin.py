"""The reference's own API (host pointers) served by the GPU, against the
golden vectors minted from the reference.  Exact where the kernel walks the
reference's order with IEEE operations; 1e-5 where a device libm function
(expf in SiLU, exp in the attention softmax) may differ in the last bit."""
import numpy as np
import pytest

from conftest import golden
from gpu_common import bitexact_frac, maxabs, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    from vx27_amd import lib, mixers
    lib.lib()
    return mixers


def test_dropin_step_exact(M):
    g = golden("step_exact")
    S = g["S0"].copy()
    T, NH, hd = g["q"].shape
    worst = 0.0
    for t in range(T):
        for h in range(NH):
            Sh = np.ascontiguousarray(S[h])
            o = M.deltanet_step_exact(Sh, g["q"][t, h], g["k"][t, h], g["v"][t, h], g["beta"][t, h],
                                      g["g"][t, h])
            S[h] = Sh
            worst = max(worst, maxabs(o, g["o"][t, h]))
    say(f"  step_exact chain: max|d o|={worst:.3e} max|d S|={maxabs(S, g['S']):.3e} "
        f"bit-exact S={bitexact_frac(S, g['S']):.4f}")
    assert worst <= 1e-5 and maxabs(S, g["S"]) <= 1e-5


def test_dropin_l2norm_and_gates(M):
    g = golden("l2norm")
    for i in range(int(g["n"])):
        assert np.array_equal(M.deltanet_l2norm(g[f"x{i}"]), g[f"y{i}"])
    gp = golden("gate_params")
    for (a, al, b, dt), be, gg in zip(gp["inp"], gp["beta"], gp["g"]):
        assert M.deltanet_gate_params(a, al, b, dt) == (be, gg)


def test_dropin_conv1d(M):
    g = golden("conv1d")
    T, C_ = g["x"].shape
    st = np.zeros((C_, 3), np.float32)
    worst = 0.0
    for t in range(T):
        y = M.conv1d_step(st, g["x"][t], g["w"], True)
        worst = max(worst, maxabs(y, g["y"][t]))
    assert np.array_equal(st, g["state"])
    st2 = g["st2_0"].copy()
    y2 = M.conv1d_step(st2, g["x"][0], g["w"], False)
    assert np.array_equal(y2, g["y2"]) and np.array_equal(st2, g["st2"])
    say(f"  conv1d: max|d y|={worst:.3e}")
    assert worst <= 1e-5


def test_dropin_simple_update(M):
    from vx27_amd import lib as L
    g = dict(golden("simple_update"))   # keep the arrays alive across the calls
    k, v, q = g["k"], g["v"], g["q"]
    lib = L.lib()
    for var, upd, ret in (("ref", "update_ref", "retrieve_ref"), ("avx2", "update_avx2", "retrieve_avx2")):
        S = g["S0"].copy()
        getattr(lib, "vx27_deltanet_" + upd)(S.ctypes.data, k.ctypes.data, v.ctypes.data, 0.9, 128)
        o = np.empty(128, np.float32)
        getattr(lib, "vx27_deltanet_" + ret)(S.ctypes.data, q.ctypes.data, o.ctypes.data, 128)
        say(f"  {var}: S bit-exact {bitexact_frac(S, g[f'S_{var}']):.4f} max|d|={maxabs(S, g[f'S_{var}']):.3e}; "
            f"o bit-exact {bitexact_frac(o, g[f'o_{var}']):.4f} max|d|={maxabs(o, g[f'o_{var}']):.3e}")
        assert np.array_equal(S, g[f"S_{var}"]), var + " S"
        assert np.array_equal(o, g[f"o_{var}"]), var + " o"
    S = g["S0"].copy()
    lib.vx27_deltanet_update_tiled(S.ctypes.data, k.ctypes.data, v.ctypes.data, 0.9, 128)
    o = np.empty(128, np.float32)
    lib.vx27_deltanet_retrieve_tiled(S.ctypes.data, q.ctypes.data, o.ctypes.data, 128)
    assert np.array_equal(S, g["S_tiled"]) and np.array_equal(o, g["o_tiled"])


def test_dropin_rmsnorm_attn_rope(M):
    g = golden("gqa")
    assert np.array_equal(M.rmsnorm([3.0, 4.0], [1.0, 1.0], 0.0), g["rms34"])
    for n, eps in ((256, 1e-6), (5120, 1e-6), (128, 1e-5)):
        assert np.array_equal(M.rmsnorm(g[f"rx{n}"], g[f"rw{n}"], eps), g[f"ry{n}"])
    for n_pos in (1, 2, 64, 160):
        o = M.attn_1q(g[f"aq{n_pos}"], g[f"ak{n_pos}"], g[f"av{n_pos}"], n_pos)
        e = maxabs(o, g[f"ao{n_pos}"])
        say(f"  attn_1q n_pos={n_pos}: max|d|={e:.3e} bit-exact={bitexact_frac(o, g[f'ao{n_pos}']):.4f}")
        assert e <= 1e-5
    r = golden("rope")
    for i, p in enumerate(r["pos"]):
        c, s = M.rope_cos_sin(int(p))
        assert np.array_equal(c, r["cos"][i]) and np.array_equal(s, r["sin"][i])
    v = r["vin"].copy()
    M.rope_apply(v, 24, 256, 64, r["cos"][8], r["sin"][8])
    assert np.array_equal(v, r["vout"])


def test_dropin_attn_1q_long(M):
    """vx27_attn_1q past the reference's 1024-position cap (n_pos 3000)
    against the oracle's restatement without the cap (float dots, as
    vx27_gqa.c:30-31)."""
    from oracle import oracle as O
    from vx27_amd import workloads as W
    r = W.rng(61, "attn_1q_long")
    n_pos = 3000
    q = W.normal(r, 24 * 256)
    kc = W.normal(r, n_pos * 4 * 256)
    vc = W.normal(r, n_pos * 4 * 256)
    o = M.attn_1q(q, kc, vc, n_pos)
    ref = np.empty(24 * 256, np.float32)
    O.lib().orc_attn_1q(q, kc, vc, n_pos, ref)
    e = maxabs(o, ref)
    say(f"  attn_1q n_pos={n_pos}: max|d|={e:.3e} (max|ref|={np.abs(ref).max():.3f})")
    assert e <= 1e-5


def test_dropin_poison_mode(M):
    """Error path without a host fallback: an unsupported size poisons the
    outputs with NaN in poison mode."""
    from vx27_amd import lib as L
    lib = L.lib()
    lib.vx27_hip_set_error_mode(L.ERR_POISON)
    try:
        S = np.zeros((300, 300), np.float32)
        q = np.ones(300, np.float32)
        o = np.zeros(300, np.float32)
        lib.vx27_deltanet_step_exact(S.ctypes.data, q.ctypes.data, q.ctypes.data, q.ctypes.data,
                                     0.5, -0.1, o.ctypes.data, 300)
        assert np.all(np.isnan(o))
    finally:
        lib.vx27_hip_set_error_mode(L.ERR_ABORT)


def test_route_switch(M):
    """vx27_hip_enable/disable mirror vx27_gpu_reg_on/off (vx27_gpu_reg.h:10-11):
    off by default, on once the default context is open."""
    from vx27_amd import lib as L
    lib = L.lib()
    assert lib.vx27_hip_enabled() == 0
    assert lib.vx27_hip_enable() == 0
    assert lib.vx27_hip_enabled() == 1
    lib.vx27_hip_disable()
    assert lib.vx27_hip_enabled() == 0
