"""det_matmul_scratch_dev (the entry point that allocates nothing) against
det_matmul_ws_dev (the existing workspace entry point) through the C ABI:
bit-identical outputs on two calls in a row, the second smaller, for the
int16 and Q16 limb GEMMs (which use the scratch; the Q16 shapes here are too
large for the direct kernel, which needs none) and int8 (which uses it only
to repack operands into padded panels); a limb-GEMM shape beyond the fixed
scratch is rejected before any launch.  The property the entry
point exists for is checked directly: after one warm-up call per op, further
calls leave the device's free memory unchanged, and one call per op captured
into a HIP graph (capture fails on hipMalloc or any synchronising call)
replays three times, with eager work and synchronisations between replays,
each time equal to the eager result."""
import ctypes

import numpy as np
import pytest

import mind_amd as M
import oracle as O

pytestmark = pytest.mark.gpu


def _bind():
    L = M.lib()
    f = L.det_matmul_scratch_dev
    f.argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                  ctypes.c_int64, ctypes.c_void_p]
    f.restype = ctypes.c_int64
    return L, f


def _inputs(op, m, k, n, seed):
    if op == M.DET_OP_I8:
        a, b = O.gen_i8(seed, m * k, k * n)
        return a, b, O.gemm_i8(a, b, m, k, n)
    if op == M.DET_OP_I16:
        a, b = O.gen_i16(seed, m * k, k * n)
        return a, b, O.gemm_i16(a, b, m, k, n)
    a, b = O.gen_q16_sat(seed, m * k, k * n, 13)
    return a, b, O.gemm_q16(a, b, m, k, n)


def _run_both(L, f, op, m, k, n, seed, s):
    a, b, want = _inputs(op, m, k, n, seed)
    print(f"[no-alloc] op={op} {m}x{k}x{n} seed={seed:#x}", flush=True)
    da, db = M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b)
    c_ws, c_sc = M.DeviceBuffer(max(m * n * 4, 4)), M.DeviceBuffer(max(m * n * 4, 4))
    ws_bytes = L.det_workspace_bytes(op, m, k, n)
    ws = M.DeviceBuffer(max(ws_bytes, 256))
    c_ws.fill(0xA5)
    c_sc.fill(0x5A)
    M.check(L.det_matmul_ws_dev(op, da.ptr, db.ptr, c_ws.ptr, m, k, n, ws.ptr, ws_bytes, s.ptr))
    M.check(f(op, da.ptr, db.ptr, c_sc.ptr, m, k, n, s.ptr))
    s.sync()
    got_ws = c_ws.to_array(np.int32, (m, n))
    got_sc = c_sc.to_array(np.int32, (m, n))
    np.testing.assert_array_equal(got_sc, got_ws)
    np.testing.assert_array_equal(got_sc, want.reshape(m, n))
    for buf in (da, db, c_ws, c_sc, ws):
        buf.free()


@pytest.mark.parametrize("op", [M.DET_OP_Q16, M.DET_OP_I16, M.DET_OP_I8])
def test_scratch_entry_matches_workspace_entry_twice(op):
    L, f = _bind()
    s = M.Stream()
    # the second call is smaller: it reuses the scratch the first one filled
    # (Q16: both split in K, the partial sums in the scratch too)
    first, second = ((200, 4160, 300), (100, 4200, 70)) if op == M.DET_OP_Q16 else ((320, 1088, 272), (70, 200, 52))
    if op == M.DET_OP_Q16:
        assert L.det_workspace_bytes(op, *first) > L.det_workspace_bytes(op, *second) > 0
    _run_both(L, f, op, *first, 0x5C1, s)
    _run_both(L, f, op, *second, 0x5C2, s)
    s.destroy()


def test_scratch_entry_int8_repack_twice():
    # both shapes are off the 16-byte grid (K % 16 != 0) and too large for
    # the direct kernel: their padded panels come from the scratch, the
    # second call's smaller ones over the first's
    L, f = _bind()
    s = M.Stream()
    for shape in ((1000, 1000, 77), (700, 200, 90)):
        assert 0 < L.det_workspace_bytes(M.DET_OP_I8, *shape) <= 32 << 20
    assert L.det_workspace_bytes(M.DET_OP_I8, 1000, 1000, 77) > L.det_workspace_bytes(M.DET_OP_I8, 700, 200, 90)
    _run_both(L, f, M.DET_OP_I8, 1000, 1000, 77, 0x5C5, s)
    _run_both(L, f, M.DET_OP_I8, 700, 200, 90, 0x5C6, s)
    s.destroy()


def test_scratch_entry_q16_1024_cubed_then_smaller():
    L, f = _bind()
    s = M.Stream()
    assert L.det_workspace_bytes(M.DET_OP_Q16, 1024, 1024, 1024) <= 32 << 20
    _run_both(L, f, M.DET_OP_Q16, 1024, 1024, 1024, 0x5C3, s)
    _run_both(L, f, M.DET_OP_Q16, 96, 4160, 64, 0x5C4, s)
    s.destroy()


def test_scratch_entry_rejects_oversized_and_handles_k0():
    L, f = _bind()
    s = M.Stream()
    m, k, n = 4096, 4096, 4096
    assert L.det_workspace_bytes(M.DET_OP_Q16, m, k, n) > 32 << 20
    c = M.DeviceBuffer(16)
    rc = f(M.DET_OP_Q16, c.ptr, c.ptr, c.ptr, m, k, n, s.ptr)   # rejected before any launch
    assert rc == M.DET_ERR_ARG and "scratch" in M.last_error()
    dc = M.DeviceBuffer(8 * 8 * 4)
    dc.fill(0xA5)
    M.check(f(M.DET_OP_Q16, c.ptr, c.ptr, dc.ptr, 8, 0, 8, s.ptr))   # K == 0: zeros
    s.sync()
    assert not dc.to_array(np.int32, (8, 8)).any()
    s.destroy()


def _hip():
    """The HIP runtime the library is linked against (already loaded)."""
    H = ctypes.CDLL("libamdhip64.so")
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    H.hipMemGetInfo.argtypes = [ctypes.POINTER(sz), ctypes.POINTER(sz)]
    H.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    H.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    H.hipGraphInstantiateWithFlags.argtypes = [ctypes.POINTER(vp), vp, ctypes.c_ulonglong]
    H.hipGraphLaunch.argtypes = [vp, vp]
    H.hipGraphExecDestroy.argtypes = [vp]
    H.hipGraphDestroy.argtypes = [vp]
    for fn in ("hipMemGetInfo", "hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiateWithFlags",
               "hipGraphLaunch", "hipGraphExecDestroy", "hipGraphDestroy"):
        getattr(H, fn).restype = ctypes.c_int
    return H


def _free_bytes(H):
    """Free device memory once it has stopped changing (five equal readings
    1 ms apart, at most 1 s): the runtime can hand back the memory of a
    buffer freed earlier in this process a few milliseconds late, which
    must not read as an allocation by the call under test.  A buffer that
    the call allocates and keeps still shows."""
    import time

    def read():
        free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
        assert H.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
        return free.value

    last, same, t0 = read(), 0, time.monotonic()
    while same < 5 and time.monotonic() - t0 < 1.0:
        time.sleep(0.001)
        now = read()
        same = same + 1 if now == last else 0
        last = now
    return last


def test_scratch_entry_allocates_nothing_and_captures_into_a_graph():
    L, f = _bind()
    H = _hip()
    s = M.Stream()
    # one shape per op within the scratch (Q16: one on the limb kernel split
    # in K, one on the direct kernel, which uses no scratch); the int8 one off
    # the 16-byte grid, so its panels come from the scratch
    cases = [(M.DET_OP_Q16, 200, 4160, 300, 0x5D1), (M.DET_OP_Q16, 256, 512, 192, 0x5D4),
             (M.DET_OP_I16, 320, 1088, 272, 0x5D2), (M.DET_OP_I8, 1000, 1000, 77, 0x5D3)]
    bufs = []
    for op, m, k, n, seed in cases:
        a, b, want = _inputs(op, m, k, n, seed)
        print(f"[no-alloc graph] op={op} {m}x{k}x{n} seed={seed:#x}", flush=True)
        bufs.append((op, m, k, n, M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b),
                     M.DeviceBuffer(m * n * 4), M.DeviceBuffer(m * n * 4), want.reshape(m, n)))
    # warm-up: the first call per device looks the scratch up
    for op, m, k, n, da, db, c_eager, c_graph, want in bufs:
        M.check(f(op, da.ptr, db.ptr, c_eager.ptr, m, k, n, s.ptr))
    s.sync()
    free0 = _free_bytes(H)
    for _ in range(3):
        for op, m, k, n, da, db, c_eager, c_graph, want in bufs:
            c_eager.fill(0xA5)
            M.check(f(op, da.ptr, db.ptr, c_eager.ptr, m, k, n, s.ptr))
        s.sync()
        for op, m, k, n, da, db, c_eager, c_graph, want in bufs:
            np.testing.assert_array_equal(c_eager.to_array(np.int32, (m, n)), want)
    assert _free_bytes(H) == free0, "a warmed-up det_matmul_scratch_dev call changed free device memory"

    # capture one call per op on this stream (thread-local mode: a hipMalloc
    # or a synchronising call inside the capture fails it)
    graph, exe = ctypes.c_void_p(0), ctypes.c_void_p(0)
    assert H.hipStreamBeginCapture(s.ptr, 1) == 0
    rcs = [f(op, da.ptr, db.ptr, c_graph.ptr, m, k, n, s.ptr) for op, m, k, n, da, db, c_eager, c_graph, want in bufs]
    assert H.hipStreamEndCapture(s.ptr, ctypes.byref(graph)) == 0
    assert rcs == [0] * len(bufs), (rcs, M.last_error())
    assert H.hipGraphInstantiateWithFlags(ctypes.byref(exe), graph, 0) == 0
    try:
        for replay in range(3):
            for op, m, k, n, da, db, c_eager, c_graph, want in bufs:
                c_graph.fill(0x5A + replay)
            # eager work on the same scratch between replays
            op, m, k, n, da, db, c_eager, c_graph, want = bufs[replay % len(bufs)]
            M.check(f(op, da.ptr, db.ptr, c_eager.ptr, m, k, n, s.ptr))
            s.sync()
            assert H.hipGraphLaunch(exe, s.ptr) == 0
            s.sync()
            for op, m, k, n, da, db, c_eager, c_graph, want in bufs:
                np.testing.assert_array_equal(c_graph.to_array(np.int32, (m, n)), want)
                np.testing.assert_array_equal(c_graph.to_array(np.int32, (m, n)), c_eager.to_array(np.int32, (m, n)))
    finally:
        H.hipGraphExecDestroy(exe)
        H.hipGraphDestroy(graph)
    for op, m, k, n, da, db, c_eager, c_graph, want in bufs:
        for buf in (da, db, c_eager, c_graph):
            buf.free()
    s.destroy()
