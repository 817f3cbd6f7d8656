"""Build libmind_det_hip.so in-tree with hipcc for gfx950.

Every .hip file under csrc/ is compiled to an object with hipcc (device code
for gfx950 only), the host-only .cpp files with the same compiler driver, and
everything is linked into ``mind_amd/lib/libmind_det_hip.so``.  Objects go to
``mind_amd/_build/`` (not committed).  ``shim/gemmq_kn.c`` becomes
``mind_amd/lib/libmind_det_gemmq_kn.so``: the Q16 benches' ``gemmq`` (B
un-transposed), forwarding into the main library.

Run ``python -m mind_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libmind_det_hip.so")
SHIM_LIB = os.path.join(LIBDIR, "libmind_det_gemmq_kn.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: never let the compiler form packed fp32 VALU ops (the
# kernels are integer-only; the flag keeps any incidental float code scalar).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-pthread"]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if src.endswith(".hip"):
        cmd = [HIPCC, *DEVICE_FLAGS, "-c", src, "-o", obj]
    else:
        cmd = ["g++", *HOST_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    # the bench form of `gemmq` (B un-transposed), a separate small library
    # that forwards into libmind_det_hip.so
    tmp = SHIM_LIB + ".tmp"
    cmd = ["gcc", "-O2", "-Wall", "-Werror", "-shared", "-fPIC", os.path.join(HERE, "shim", "gemmq_kn.c"),
           "-L", LIBDIR, "-lmind_det_hip", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"shim link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, SHIM_LIB)
    if verbose:
        print(f"built {LIB} and {SHIM_LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
