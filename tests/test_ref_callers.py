"""The reference's own callers of the drop-in boundary link against
libvx27_hip.so.

oracle/Makefile's `callers` target compiles vx27_block.c, vx27_forward64.c,
vx27_qfwd.c and vx27_mtp.c from the reference's sources, unmodified, to
objects.  Every symbol of the three hot-path headers (vx27_deltanet.h,
vx27_gqa.h, vx27_rope.h) that those objects import must be a defined,
exported function of libvx27_hip.so, and so must every function those
headers declare (the callers of vx27_block_forward / vx27_forward64 reach
the rest through vx27_block.o).  Runs where the reference sources are
present (the build container); no GPU needed."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/src"
HOT = re.compile(r"^vx27_(deltanet_\w+|gqa_kv_for_q|rmsnorm|attn_1q|conv1d_step|rope_\w+|mrope_\w+)$")
CALLERS = ("vx27_block", "vx27_forward64", "vx27_qfwd", "vx27_mtp")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="reference sources not present")


def _nm(path, *flags):
    r = subprocess.run(["nm", *flags, path], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return r.stdout.splitlines()


def _exports():
    from vx27_amd import lib as L
    L.lib()
    so = os.path.join(ROOT, "vx27_amd", "libvx27_hip.so")
    return {ln.split()[-1] for ln in _nm(so, "-D", "--defined-only") if ln.split()[-2] in ("T", "W")}


@pytest.fixture(scope="module")
def caller_objects():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "callers"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    objs = {c: os.path.join(ROOT, "oracle", "_ref", "callers", c + ".o") for c in CALLERS}
    for o in objs.values():
        assert os.path.exists(o), o
    return objs


def test_caller_imports_resolve(caller_objects):
    exports = _exports()
    seen = set()
    for name, obj in caller_objects.items():
        imports = {ln.split()[-1] for ln in _nm(obj, "-u")}
        hot = sorted(s for s in imports if HOT.match(s))
        print(f"{name}.o imports {hot}")
        missing = [s for s in hot if s not in exports]
        assert not missing, f"{name}.o imports {missing}, not exported by libvx27_hip.so"
        seen |= set(hot)
    # the callers reach step_exact, conv, gates, l2norm, rmsnorm, rope and the AVX2 rule
    assert {"vx27_deltanet_step_exact", "vx27_conv1d_step", "vx27_deltanet_gate_params", "vx27_rmsnorm",
            "vx27_rope_cos_sin", "vx27_rope_apply", "vx27_deltanet_update_avx2"} <= seen


def test_header_functions_exported():
    """Every function declared in include/vx27_{deltanet,gqa,rope}.h (the
    reference's headers, signature for signature) is exported."""
    exports = _exports()
    decl = re.compile(r"^\s*(?:int|void|double)\s+\**(vx27_\w+)\s*\(", re.M)
    names = set()
    for h in ("vx27_deltanet.h", "vx27_gqa.h", "vx27_rope.h"):
        names |= set(decl.findall(open(os.path.join(ROOT, "include", h)).read()))
    assert len(names) >= 18, names
    assert names <= exports, sorted(names - exports)
