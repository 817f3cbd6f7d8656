"""det_matmul_scratch_dev (the entry point that allocates nothing) against
det_matmul_ws_dev (the existing workspace entry point) through the C ABI:
bit-identical outputs on two calls in a row, the second smaller, for the
int16 and Q16 limb GEMMs (which always use the scratch) and int8 (which uses
it only to repack operands off the 16-byte grid); a limb-GEMM shape beyond
the fixed scratch is rejected before any launch."""
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
    _run_both(L, f, op, 320, 1088, 272, 0x5C1, s)
    _run_both(L, f, op, 70, 200, 52, 0x5C2, s)
    s.destroy()


def test_scratch_entry_int8_repack_twice():
    # both shapes are off the 16-byte grid (K % 16 != 0): their padded panels
    # come from the scratch, the second call's smaller ones over the first's
    L, f = _bind()
    s = M.Stream()
    for shape in ((300, 1000, 77), (37, 100, 53)):
        assert 0 < L.det_workspace_bytes(M.DET_OP_I8, *shape) <= 32 << 20
    _run_both(L, f, M.DET_OP_I8, 300, 1000, 77, 0x5C5, s)
    _run_both(L, f, M.DET_OP_I8, 37, 100, 53, 0x5C6, s)
    s.destroy()


def test_scratch_entry_q16_1024_cubed_then_smaller():
    L, f = _bind()
    s = M.Stream()
    assert L.det_workspace_bytes(M.DET_OP_Q16, 1024, 1024, 1024) <= 32 << 20
    _run_both(L, f, M.DET_OP_Q16, 1024, 1024, 1024, 0x5C3, s)
    _run_both(L, f, M.DET_OP_Q16, 96, 4000, 64, 0x5C4, s)
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
