"""Build libvx27_hip.so in-tree: HIP kernels for gfx950 plus the C drop-ins.

    python -m vx27_amd.build          (or vx27_amd.build.build())

hipcc compiles every csrc/*.hip for --offload-arch=gfx950 with:
  -ffp-contract=off                   no implicit FMA contraction: the DeltaNet
                                      kernels reproduce the reference's
                                      separate multiply/add roundings
  -target-feature -packed-fp32-ops    no packed FP32 instructions
and, for the DeltaNet prefill kernels (FILE_FLAGS), -amdgpu-mfma-vgpr-form:
their accumulators stay in arch VGPRs, where the state updates touch them
with VALU ops, instead of being copied in and out of AGPRs.  (The attention
kernel's O accumulators are only ever touched by MFMAs in its loop, so they
live in AGPRs.)
gcc compiles the C drop-in layer (-std=c11) against include/vx27_hip.h.
Objects go to vx27_amd/_build/, the library to vx27_amd/libvx27_hip.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INC = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libvx27_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
HIP_FLAGS = ["-O3", f"--offload-arch={ARCH}", "-fPIC", "-std=c++17", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-result", f"-I{INC}", f"-I{CSRC}"]
FILE_FLAGS = {
    "vx_dn_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}
CC = os.environ.get("CC", "gcc")
C_FLAGS = ["-std=c11", "-O2", "-fPIC", "-ffp-contract=off", "-Wall", f"-I{INC}"]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = True, jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hips = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    cs = sorted(glob.glob(os.path.join(CSRC, "*.c")))
    jobs_list = []
    for src in hips:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        jobs_list.append([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj])
    for src in cs:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        jobs_list.append([CC, *C_FLAGS, "-c", src, "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for out in ex.map(_run, jobs_list):
            if verbose and out.strip():
                print(out)
    objs = [j[-1] for j in jobs_list]
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
