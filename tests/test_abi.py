"""The C-ABI library loads and exports every function include/*.h declares;
argument validation and error reporting work without a GPU (no compute)."""
import ctypes as C
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(vx27_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_the_reference_api():
    names = set(declared_functions())
    # the reference API of src/vx27_deltanet.h:10-59, vx27_gqa.h:8-13, vx27_rope.h:11-17
    ref = {"vx27_deltanet_state_per_layer", "vx27_deltanet_state_total", "vx27_deltanet_state_mb",
           "vx27_deltanet_update_ref", "vx27_deltanet_retrieve_ref", "vx27_deltanet_update_tiled",
           "vx27_deltanet_retrieve_tiled", "vx27_deltanet_update_avx2", "vx27_deltanet_retrieve_avx2",
           "vx27_deltanet_l2norm", "vx27_deltanet_step_exact", "vx27_deltanet_gate_params",
           "vx27_conv1d_step", "vx27_gqa_kv_for_q", "vx27_rmsnorm", "vx27_attn_1q",
           "vx27_rope_cos_sin", "vx27_rope_apply", "vx27_mrope_cos_sin_text"}
    assert ref <= names, sorted(ref - names)


def test_library_exports_every_declared_symbol():
    from vx27_amd import lib as L
    so = L.lib()
    missing = [n for n in declared_functions() if not hasattr(so, n)]
    assert not missing, missing
    # and the Python binding declares a signature for every one of them
    assert set(declared_functions()) <= set(L.exported_symbols())


def test_scalar_dropins_match_reference_golden():
    """Host-side scalar helpers of the drop-in layer (no GPU): state sizing,
    KV-head map, gate parameters, RoPE tables."""
    import numpy as np
    from conftest import golden
    from vx27_amd import mixers as M, lib as L
    so = L.lib()
    assert so.vx27_deltanet_state_per_layer() == 16 * 128 * 128        # tests/test_deltanet.c:24
    assert so.vx27_deltanet_state_total() == 262144 * 48               # :25
    assert 24.0 < so.vx27_deltanet_state_mb(2) < 26.0                  # :27
    assert [so.vx27_gqa_kv_for_q(h) for h in (0, 5, 6, 11, 12, 23)] == [0, 0, 1, 1, 2, 3]
    gp = golden("gate_params")
    for (a, al, b, dt), be, gg in zip(gp["inp"], gp["beta"], gp["g"]):
        assert M.deltanet_gate_params(a, al, b, dt) == (be, gg)
    r = golden("rope")
    for i, p in enumerate(r["pos"]):
        c, s = M.rope_cos_sin(int(p))
        assert np.array_equal(c, r["cos"][i]) and np.array_equal(s, r["sin"][i])
    # the product's vx27_mrope_cos_sin_text (vx27_rope.c:31-33) and the YaRN factor
    c = np.empty(32, np.float32); s = np.empty(32, np.float32)
    so.vx27_mrope_cos_sin_text(8192, c.ctypes.data, s.ctypes.data)
    assert np.array_equal(c, r["mrope_cos"]) and np.array_equal(s, r["mrope_sin"])
    c, s = M.rope_cos_sin(32, yarn=4.0)
    assert np.array_equal(c, r["yarn_cos"]) and np.array_equal(s, r["yarn_sin"])


def test_entry_points_validate_without_device():
    from vx27_amd import lib as L
    so = L.lib()
    d = L.DnDesc()
    assert so.vx27_hip_dn_decode(None, C.byref(d)) == -1
    assert b"null context" in so.vx27_hip_last_error()
    g = L.GqaDesc()
    assert so.vx27_hip_gqa_decode(None, C.byref(g)) == -1
    h = C.c_void_p()
    err = C.create_string_buffer(256)
    if so.vx27_hip_device_count() == 0:
        assert so.vx27_hip_open(C.byref(h), 0, err, 256) == -1
        assert b"no HIP device" in err.value or b"device" in err.value
        # the route switch stays off when no context can open
        assert so.vx27_hip_enable() == -1
    assert so.vx27_hip_enabled() == 0


def test_product_never_imports_the_oracle():
    """The product package and C sources do not reference oracle/."""
    for path in glob.glob(os.path.join(ROOT, "vx27_amd", "**", "*.*"), recursive=True):
        if path.endswith((".py", ".hip", ".c", ".h")):
            text = open(path).read()
            assert "from oracle" not in text and "import oracle" not in text and "liboracle" not in text, path
