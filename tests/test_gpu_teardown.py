"""Teardown at unload (the reference joins its thread pool in a destructor at
dlclose, runtime-support/mind_intrinsics.c:2066-2080).

A fresh child process loads libmind_det_hip.so, makes a host-pointer call
that grows the library's staging buffer (and its stream / event), releases
the library's state with det_shutdown() and unloads it, 20 times, reading the
device's free memory (hipMemGetInfo, through the HIP runtime directly) with
the library loaded after the call and again after det_shutdown + dlclose.
The library must be gone from the process after every dlclose, each round
must give the 128+ MiB staging buffer back, and the level must stay flat from
round to round: without the teardown each round would leave its staging
buffer behind.  (The first kernel launch in a process costs the HIP runtime a
one-time ~150 MiB of its own, which the first round's figure includes.  The
runtime can hand back the memory of a buffer last written by a DMA copy a few
milliseconds after hipFree returns, so the reading after dlclose waits until
free memory has stopped changing, for at most a second: a buffer that is never
given back still fails.)
"""
import os
import subprocess
import sys

import pytest

import mind_amd

CHILD = r"""
import ctypes, _ctypes, sys
import numpy as np
lib_path = sys.argv[1]
hip = ctypes.CDLL("libamdhip64.so.7")
free_b, total_b = ctypes.c_size_t(), ctypes.c_size_t()
assert hip.hipSetDevice(0) == 0
def free_mem():
    assert hip.hipMemGetInfo(ctypes.byref(free_b), ctypes.byref(total_b)) == 0
    return free_b.value
def settled_free_mem():
    import time
    last, same, t0 = free_mem(), 0, time.monotonic()
    while same < 5 and time.monotonic() - t0 < 1.0:
        time.sleep(0.001)
        now = free_mem()
        same = same + 1 if now == last else 0
        last = now
    return last
base = free_mem()
M, K = 2048, 16384                      # W = 128 MiB of Q16
rng = np.random.default_rng(7)
W = rng.integers(-(1 << 16), 1 << 16, size=(M, K), dtype=np.int32)
x = rng.integers(-(1 << 16), 1 << 16, size=K, dtype=np.int32)
first = None
for it in range(20):
    L = ctypes.CDLL(lib_path)
    f = L.det_gemv_q16
    f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 2
    f.restype = ctypes.c_int64
    y = np.empty(M, np.int32)
    assert f(W.ctypes.data, x.ctypes.data, y.ctypes.data, M, K) == 0
    if first is None:
        first = y.copy()
    assert (y == first).all()
    held = free_mem()
    L.det_shutdown.restype = ctypes.c_int64
    assert L.det_shutdown() == 0
    handle = L._handle
    del f, L
    _ctypes.dlclose(handle)
    loaded = os.path.realpath(lib_path) in open("/proc/self/maps").read()
    after = settled_free_mem()
    print(f"round {it}: loaded {(base - held) >> 20} MiB below baseline, after dlclose {(base - after) >> 20} MiB, "
          f"still mapped {loaded}", flush=True)
    assert not loaded, "dlclose did not unload the library"
""".replace("import ctypes, _ctypes, sys", "import ctypes, _ctypes, os, sys")


@pytest.mark.gpu
def test_unload_releases_device_memory():
    print("[teardown] 20x load / det_gemv_q16 2048x16384 / det_shutdown / dlclose in a child", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD, mind_amd.LIB_PATH], capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0
    held, after = [], []
    for line in r.stdout.splitlines():
        if line.startswith("round "):
            held.append(int(line.split("loaded ")[1].split(" MiB")[0]))
            after.append(int(line.split("after dlclose ")[1].split(" MiB")[0]))
    assert len(after) == 20
    # each det_shutdown + dlclose returns the 128 MiB staging buffer (and more)
    assert all(h - a >= 128 for h, a in zip(held, after)), list(zip(held, after))
    # and nothing accumulates: a leaked staging buffer would add 128 MiB a round
    assert max(after) - min(after) < 32, after
    assert max(after) < 256, after


@pytest.mark.gpu
def test_det_shutdown_then_reuse():
    """det_shutdown releases the state; the next call recreates it."""
    import numpy as np

    import oracle as O

    L = mind_amd.lib()
    a, b = O.gen_i8(0x7E57, 96 * 80, 80 * 112)
    want = O.gemm_i8(a, b, 96, 80, 112)
    for _ in range(3):
        np.testing.assert_array_equal(mind_amd.det_matmul_i8(a.reshape(96, 80), b.reshape(80, 112)), want)
        assert L.det_shutdown() == 0
        assert L.det_shutdown() == 0    # idempotent
