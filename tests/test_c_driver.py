"""A C caller of the library (tests/c_driver/det_driver.c), shaped like the
reference's cross-node gate driver (tests/cross_substrate_identity/
xnode_driver.c:123-156): it is compiled with gcc -Wall -Wextra -Werror
against include/mind_det.h, dlopens libmind_det_hip.so and the bench-form
gemmq library, dlsyms the harness symbols through i64-ABI typedefs and
prints one SHA-256 per committed workload.

CPU tier: the driver (and so the header, as C) compiles warning-free, and its
own SHA-256 and LCG agree with Python's.  GPU tier: every hash it prints is
the reference's committed one.
"""
import hashlib
import os
import subprocess

import numpy as np
import pytest

import mind_amd
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "c_driver", "det_driver.c")
SHIM = os.path.join(os.path.dirname(mind_amd.LIB_PATH), "libmind_det_gemmq_kn.so")


def _compile(tmp_path):
    exe = str(tmp_path / "det_driver")
    r = subprocess.run(["gcc", "-Wall", "-Wextra", "-Werror", "-std=c11", "-O1", "-I", os.path.join(ROOT, "include"),
                        SRC, "-ldl", "-o", exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return exe


def _sha(v):
    return hashlib.sha256(np.asarray(v).astype("<i4").tobytes()).hexdigest()


def test_c_driver_compiles_against_the_header_and_self_checks(tmp_path):
    exe = _compile(tmp_path)
    out = subprocess.run([exe, "--selftest"], capture_output=True, text=True, timeout=60, check=True).stdout
    got = dict(line.split() for line in out.strip().splitlines())
    a, b = O.gen_q16(0xDEADBEEF, 64 * 64, 64 * 64)
    assert got["lcg-q16-8192"] == _sha(np.concatenate([a, b]))
    assert got["ramp-1000"] == _sha(np.arange(1000) - 500)
    assert got["empty"] == hashlib.sha256(b"").hexdigest()


def test_bench_gemmq_library_exports_gemmq_over_the_main_library():
    """libmind_det_gemmq_kn.so exports gemmq and resolves the fused Q16
    intrinsic from libmind_det_hip.so (no kernel is launched here)."""
    assert os.path.exists(SHIM)
    nm = subprocess.run(["nm", "-D", SHIM], capture_output=True, text=True, check=True).stdout
    assert any(line.split()[-2:] == ["T", "gemmq"] for line in nm.splitlines() if len(line.split()) >= 2)
    assert any(line.split()[-2:] == ["U", "__mind_blas_matmul_mm_q16_v"] for line in nm.splitlines())
    ldd = subprocess.run(["ldd", SHIM], capture_output=True, text=True, check=True).stdout
    assert os.path.realpath(mind_amd.LIB_PATH) in {os.path.realpath(p) for p in ldd.split() if p.startswith("/")}


@pytest.mark.gpu
def test_c_driver_reproduces_the_golden_hashes(tmp_path, canaries):
    exe = _compile(tmp_path)
    print(f"[c-driver] {exe} {mind_amd.LIB_PATH} {SHIM}", flush=True)
    r = subprocess.run([exe, mind_amd.LIB_PATH, SHIM], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    w = canaries["workloads"]
    lines = [line.split() for line in r.stdout.strip().splitlines()]
    seen = set()
    for wid, symbol, h in lines:
        assert h == w[wid]["avx2"], (wid, symbol)
        seen.add(symbol)
    assert seen == {"gemmi8", "gemmi8mt", "__mind_blas_matmul_mm_i8_v", "det_matmul_i8", "gemmq", "gemmqmm",
                    "gemmq(kn)", "mmq", "gemvq", "mmi16", "dotq", "dotl1q", "doti16"}
