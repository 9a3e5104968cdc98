"""The HBM bandwidth probe (vx27_hip_bw_probe), the measured ceiling the
benchmark reports beside the 8 TB/s spec: it runs, gives rates inside the
physically possible range, and rejects bad arguments."""
import ctypes as C

import pytest

from gpu_common import say

pytestmark = pytest.mark.gpu


def test_bw_probe():
    from vx27_amd import lib as L
    lib = L.lib()
    with L.Ctx(0) as ctx:
        r, c = C.c_double(), C.c_double()
        L.check(lib.vx27_hip_bw_probe(ctx.h, 1 << 30, 3, C.byref(r), C.byref(c)), "bw_probe")
        say(f"  1 GiB: read {r.value:.0f} GB/s, copy {c.value:.0f} GB/s")
        assert 500.0 < r.value < 10000.0 and 500.0 < c.value < 10000.0
        assert lib.vx27_hip_bw_probe(ctx.h, 1 << 10, 3, C.byref(r), C.byref(c)) == -1
        assert lib.vx27_hip_bw_probe(ctx.h, 1 << 30, 0, C.byref(r), C.byref(c)) == -1
        assert lib.vx27_hip_bw_probe(ctx.h, 1 << 30, 3, None, C.byref(c)) == -1
