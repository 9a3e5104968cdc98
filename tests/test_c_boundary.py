"""The C boundary seen from C: a C11 caller (tests/c/caller.c) compiled
unchanged against include/*.h and linked to libvx27_hip.so.  Its printed
sizeof/offsetof of every descriptor field must equal the ctypes mirrors in
vx27_amd/lib.py that the GPU tests use, so a layout drift between a C struct
and its mirror fails here rather than as wrong numbers.  No GPU needed."""
import ctypes as C
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

STRUCTS = {   # C typedef -> ctypes mirror
    "vx27_dn_desc": "DnDesc",
    "vx27_dn_prefill_desc": "DnPrefillDesc",
    "vx27_gqa_desc": "GqaDesc",
    "vx27_gqa_prefill_desc": "GqaPrefillDesc",
    "vx27_dn_layer_desc": "DnLayerDesc",
    "vx27_gqa_layer_desc": "GqaLayerDesc",
    "vx27_dn_layer_prefill_desc": "DnLayerPrefillDesc",
    "vx27_gqa_layer_prefill_desc": "GqaLayerPrefillDesc",
}


@pytest.fixture(scope="module")
def caller(tmp_path_factory):
    from vx27_amd import lib as L
    L.lib()   # built
    d = tmp_path_factory.mktemp("cb")
    lines = ["static void print_layout(void) {"]
    for cname, pyname in STRUCTS.items():
        cls = getattr(L, pyname)
        lines.append(f'    printf("size {pyname} %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'    printf("off {pyname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("}")
    (d / "layout.inc").write_text("\n".join(lines) + "\n")
    exe = d / "caller"
    lib_dir = os.path.join(ROOT, "vx27_amd")
    cmd = ["gcc", "-std=c11", "-Wall", "-Werror", "-pedantic", f"-I{ROOT}/include", f"-I{d}",
           os.path.join(ROOT, "tests", "c", "caller.c"), "-o", str(exe), f"-L{lib_dir}", "-l:libvx27_hip.so",
           f"-Wl,-rpath,{lib_dir}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    return out.stdout


def test_descriptor_layouts_match_ctypes(caller):
    from vx27_amd import lib as L
    got = {}
    for line in caller.splitlines():
        k, _, v = line.partition(" ")
        if k in ("size", "off"):
            name, val = v.rsplit(" ", 1)
            got[(k, name)] = int(val)
    n = 0
    for pyname in STRUCTS.values():
        cls = getattr(L, pyname)
        assert got[("size", pyname)] == C.sizeof(cls), pyname
        for fname, _ in cls._fields_:
            assert got[("off", f"{pyname}.{fname}")] == getattr(cls, fname).offset, (pyname, fname)
            n += 1
    assert n > 100


def test_c_caller_links_and_runs_host_functions(caller):
    import numpy as np
    from conftest import golden
    kv = dict(line.split(" ", 1) for line in caller.splitlines())
    assert kv["fns"].split()[1:] == ["null", "0"]
    assert int(kv["state_per_layer"]) == 16 * 128 * 128
    assert int(kv["state_total"]) == 16 * 128 * 128 * 48
    assert int(kv["kv_for_q_23"]) == 3
    r = golden("rope")
    i = list(r["pos"]).index(131072)
    assert np.float32(float(kv["rope_c0_131072"])) == r["cos"][i, 0]
    assert kv["version"].startswith("vx27_hip")
