"""mind_amd -- MI355X (gfx950) backend for MIND's deterministic integer and
Q16.16 linear-algebra intrinsics.

The product is ``mind_amd/lib/libmind_det_hip.so`` (C ABI declared in
``include/mind_det.h``).  This module is a thin ctypes mirror of the
reference's intrinsic surface for Python callers and tests: the same names,
argument meaning and return convention as the reference's ``pub fn``
wrappers (``gemmi8(a, b, c, m, k, n) -> i64`` and friends,
benches/det_matmul_i8.rs:120-129, tests/cross_substrate_identity.rs:70-150),
taking numpy arrays instead of raw addresses.

There is no CPU fallback: if the HIP library is not built, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmind_det_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "mind_det.h")

DET_OP_I8, DET_OP_I16, DET_OP_Q16 = 1, 2, 3
DET_DOT_Q16, DET_DOT_L1_Q16, DET_DOT_I16 = 0, 1, 2
DET_F32_DOT, DET_F32_L1, DET_F32_LINF, DET_F32_LINF_V = 0, 1, 2, 3
DET_ERR_ARG, DET_ERR_HIP, DET_ERR_DEVICE = -22, -5, -19

_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_p = ctypes.c_void_p
_lib = None


class DetError(RuntimeError):
    """A negative return code from the C ABI (device failure or bad shape)."""


def header_symbols() -> list[str]:
    """Every function declared in include/mind_det.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*([A-Za-z_][A-Za-z_0-9]*)\s*\(", text, flags=re.M)


def _bind(L):
    sig6 = [_i64] * 6
    sig5 = [_i64] * 5
    for name in ("__mind_blas_matmul_mm_i8_v", "__mind_blas_matmul_mm_i8_mt_v", "__mind_blas_matmul_mm_q16_v",
                 "__mind_blas_matmul_mm_q16_mt_v", "gemmi8", "gemmi8mt", "gemmqmm", "gemmq"):
        f = getattr(L, name); f.argtypes = sig6; f.restype = _i64
    for name in ("__mind_blas_gemv_q16_mt", "__mind_blas_matmul_rmajor_q16_v", "__mind_blas_matmul_rmajor_i16_v",
                 "mmq", "mmi16", "gemvq"):
        f = getattr(L, name); f.argtypes = sig5; f.restype = _i64
    for name in ("__mind_blas_dot_q16", "__mind_blas_dot_q16_v", "dotq", "__mind_blas_dot_l1_q16",
                 "__mind_blas_dot_l1_q16_v", "__mind_blas_dot_i16_v", "dotl1q", "doti16"):
        f = getattr(L, name); f.argtypes = [_i64] * 3; f.restype = _i64
    for name in ("det_dot_q16", "det_dot_l1_q16", "det_dot_i16"):
        f = getattr(L, name); f.argtypes = [_p, _p, _i64]; f.restype = _i64
    L.det_dot_dev.argtypes = [_i64, _p, _p, _i64, _p, _p]; L.det_dot_dev.restype = _i64
    for name in ("__mind_blas_dot_f32", "__mind_blas_dot_f32_v", "dotf32", "__mind_blas_dot_l1_f32",
                 "__mind_blas_dot_l1_f32_v", "__mind_blas_dot_linf_f32", "__mind_blas_dot_linf_f32_v"):
        f = getattr(L, name); f.argtypes = [_i64] * 3; f.restype = _i64
    for name in ("__mind_blas_matmul_rmajor_f32", "__mind_blas_matmul_rmajor_f32_v", "mmf32"):
        f = getattr(L, name); f.argtypes = [_i64] * 5; f.restype = _i64
    L.det_dot_f32.argtypes = [_p, _p, _i64, _p]; L.det_dot_f32.restype = _i64
    L.det_matmul_rmajor_f32.argtypes = [_p, _p, _p, _i64, _i64]; L.det_matmul_rmajor_f32.restype = _i64
    L.fft256.argtypes = [_i64] * 5; L.fft256.restype = _i64
    L.det_fft_q16.argtypes = [_p, _p, _p, _i64, _i64, _i64]; L.det_fft_q16.restype = _i64
    L.det_fft_q16_dev.argtypes = [_p, _p, _p, _i64, _i64, _i64, _p]; L.det_fft_q16_dev.restype = _i64
    L.det_fft_q16_oop_dev.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]
    L.det_fft_q16_oop_dev.restype = _i64
    L.det_fft_workspace_bytes.argtypes = [_i64, _i64]; L.det_fft_workspace_bytes.restype = _i64
    L.det_matmul_rmajor_f32_dev.argtypes = [_p, _p, _p, _i64, _i64, _p]
    L.det_matmul_rmajor_f32_dev.restype = _i64
    L.det_rows_metric_f32.argtypes = [_i64, _p, _p, _p, _i64, _i64]; L.det_rows_metric_f32.restype = _i64
    L.det_rows_metric_f32_dev.argtypes = [_i64, _p, _p, _p, _i64, _i64, _p]
    L.det_rows_metric_f32_dev.restype = _i64
    for name in ("det_matmul_i8", "det_matmul_i16", "det_matmul_q16"):
        f = getattr(L, name); f.argtypes = [_p, _p, _p, _i64, _i64, _i64]; f.restype = _i64
    for name in ("det_gemv_q16", "det_gemv_i16"):
        f = getattr(L, name); f.argtypes = [_p, _p, _p, _i64, _i64]; f.restype = _i64
    L.det_gemv_q16_batched.argtypes = [_p, _p, _p, _i64, _i64, _i64]; L.det_gemv_q16_batched.restype = _i64
    for name in ("det_matmul_i8_dev", "det_matmul_i16_dev", "det_matmul_q16_dev"):
        f = getattr(L, name); f.argtypes = [_p, _p, _p, _i64, _i64, _i64, _p]; f.restype = _i64
    L.det_gemv_q16_dev.argtypes = [_p, _p, _p, _i64, _i64, _i64, _p]; L.det_gemv_q16_dev.restype = _i64
    L.det_gemv_workspace_bytes.argtypes = [_i64] * 3; L.det_gemv_workspace_bytes.restype = _i64
    L.det_gemv_q16_ws_dev.argtypes = [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]
    L.det_gemv_q16_ws_dev.restype = _i64
    L.det_gemv_i16_dev.argtypes = [_p, _p, _p, _i64, _i64, _p]; L.det_gemv_i16_dev.restype = _i64
    L.det_workspace_bytes.argtypes = [_i64] * 4; L.det_workspace_bytes.restype = _i64
    L.det_matmul_ws_dev.argtypes = [_i64, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]
    L.det_matmul_ws_dev.restype = _i64
    L.det_matmul_scratch_dev.argtypes = [_i64, _p, _p, _p, _i64, _i64, _i64, _p]
    L.det_matmul_scratch_dev.restype = _i64
    L.det_last_error.argtypes = []; L.det_last_error.restype = ctypes.c_char_p
    L.det_shutdown.argtypes = []; L.det_shutdown.restype = _i64
    L.det_version.argtypes = []; L.det_version.restype = ctypes.c_char_p
    L.det_device_count.argtypes = []; L.det_device_count.restype = _i64
    L.det_set_device.argtypes = [_i64]; L.det_set_device.restype = _i64
    L.det_device_info.argtypes = [ctypes.POINTER(_i64), ctypes.c_char_p, _i64]; L.det_device_info.restype = _i64
    L.det_malloc.argtypes = [ctypes.POINTER(_p), _i64]; L.det_malloc.restype = _i64
    L.det_free.argtypes = [_p]; L.det_free.restype = _i64
    for name in ("det_memcpy_htod", "det_memcpy_dtoh"):
        f = getattr(L, name); f.argtypes = [_p, _p, _i64]; f.restype = _i64
    L.det_memset_dev.argtypes = [_p, _i64, _i64]; L.det_memset_dev.restype = _i64
    L.det_device_sync.argtypes = []; L.det_device_sync.restype = _i64
    L.det_stream_create.argtypes = [ctypes.POINTER(_p)]; L.det_stream_create.restype = _i64
    for name in ("det_stream_destroy", "det_stream_sync", "det_event_destroy"):
        f = getattr(L, name); f.argtypes = [_p]; f.restype = _i64
    L.det_event_create.argtypes = [ctypes.POINTER(_p)]; L.det_event_create.restype = _i64
    L.det_event_record.argtypes = [_p, _p]; L.det_event_record.restype = _i64
    L.det_event_elapsed_ms.argtypes = [_p, _p, ctypes.POINTER(ctypes.c_float)]; L.det_event_elapsed_ms.restype = _i64
    L.det_probe_mfma_i8.argtypes = [_p, _p, _i64, _i64, _i64, _p]; L.det_probe_mfma_i8.restype = _i64
    L.det_probe_read.argtypes = [_p, _i64, _p, _i64, _p]; L.det_probe_read.restype = _i64
    L.det_copy_dev.argtypes = [_p, _p, _i64, _p]; L.det_copy_dev.restype = _i64
    for name in ("det_gen_i8", "det_gen_i16", "det_gen_f32_unit"):
        f = getattr(L, name); f.argtypes = [_u64, _p, _i64, _p, _i64]; f.restype = None
    for name in ("det_gen_q16", "det_gen_q16_sat"):
        f = getattr(L, name); f.argtypes = [_u64, ctypes.c_int, _p, _i64, _p, _i64]; f.restype = None
    for name in ("det_gen_i8_gauss", "det_gen_i8_sym127"):
        f = getattr(L, name); f.argtypes = [_u64, _p, _i64]; f.restype = None


def lib():
    """Load libmind_det_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m mind_amd.build` "
                               "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        _bind(L)
        _lib = L
    return _lib


def last_error() -> str:
    return lib().det_last_error().decode()


def check(rc: int) -> int:
    if rc < 0:
        raise DetError(f"rc={rc}: {last_error()}")
    return rc


def _addr(a: np.ndarray) -> int:
    return a.ctypes.data if a is not None and a.size else 0


def _req(a, dt):
    a = np.asarray(a)
    if a.dtype != dt or not a.flags.c_contiguous:
        a = np.ascontiguousarray(a, dtype=dt)
    return a


# ---------------------------------------------------------------- intrinsics
# Each mirrors one reference intrinsic: same argument order (a, b, c, m, k,
# n) / (w, x, y, rows, cols), output written in place, returns the rc.

def matmul_mm_i8(a, b, c, m, k, n) -> int:
    """__mind_blas_matmul_mm_i8_v: C[m,n] (int32) = A[m,k] (int8) . B[k,n]."""
    return check(lib().__mind_blas_matmul_mm_i8_v(_addr(a), _addr(b), _addr(c), m, k, n))


def matmul_mm_q16(a, b, c, m, k, n) -> int:
    """__mind_blas_matmul_mm_q16_v: Q16.16, per-term floor shift, wrapped."""
    return check(lib().__mind_blas_matmul_mm_q16_v(_addr(a), _addr(b), _addr(c), m, k, n))


def gemv_q16_mt(w, x, y, m, k) -> int:
    """__mind_blas_gemv_q16_mt: y[m] = W[m,k] . x[k] in Q16.16."""
    return check(lib().__mind_blas_gemv_q16_mt(_addr(w), _addr(x), _addr(y), m, k))


def matmul_rmajor_i16(w, x, y, rows, cols) -> int:
    """__mind_blas_matmul_rmajor_i16_v: y[rows] (int32) = W[rows,cols] . x (int16)."""
    return check(lib().__mind_blas_matmul_rmajor_i16_v(_addr(w), _addr(x), _addr(y), rows, cols))


def dot_q16(a, b) -> int:
    """__mind_blas_dot_q16: (int64)(int32) sum (a*b >> 16)."""
    a = _req(a, np.int32); b = _req(b, np.int32)
    return lib().__mind_blas_dot_q16(_addr(a), _addr(b), len(a))


def dot_l1_q16(a, b) -> int:
    """__mind_blas_dot_l1_q16: (int64)(int32) sum |a - b|."""
    a = _req(a, np.int32); b = _req(b, np.int32)
    return lib().__mind_blas_dot_l1_q16(_addr(a), _addr(b), len(a))


def dot_f32_bits(a, b) -> int:
    """__mind_blas_dot_f32: the strict-FP dot's f32 bits (low 32 bits of the int64)."""
    a = _req(a, np.float32); b = _req(b, np.float32)
    return lib().__mind_blas_dot_f32(_addr(a), _addr(b), len(a))


def matmul_rmajor_f32(W, x):
    """__mind_blas_matmul_rmajor_f32: y[rows] (f32) = strict dots of W's rows with x."""
    W = _req(W, np.float32); x = _req(x, np.float32)
    rows, cols = W.shape
    y = np.zeros(rows, np.float32)
    check(lib().__mind_blas_matmul_rmajor_f32(_addr(W), _addr(x), _addr(y), rows, cols))
    return y


def fft_q16(re, im, tw, logn=None):
    """Batched fft256: re / im are [batch, n] (or [n]) int64 Q16.16, tw the n/2
    (wr, wi) pairs as n int64.  Returns new (re, im) arrays; the inputs are
    not modified."""
    re = np.array(re, np.int64, copy=True, order="C")
    im = np.array(im, np.int64, copy=True, order="C")
    if re.shape != im.shape:
        raise ValueError("re and im shapes differ")
    n = re.shape[-1] if re.ndim else 0
    batch = re.size // n if n else 0
    if logn is None:
        logn = max(n.bit_length() - 1, 0)
    tw = _req(np.asarray(tw, np.int64), np.int64) if n >= 4 else np.zeros(2, np.int64)
    if n >= 4 and tw.size < n:
        raise ValueError("tw needs n int64 (n / 2 pairs)")
    check(lib().det_fft_q16(_addr(re), _addr(im), _addr(tw), logn, n, batch))
    return re, im


def dot_i16(a, b) -> int:
    """__mind_blas_dot_i16_v: (int64)(int32) sum a*b over int16 vectors."""
    a = _req(a, np.int16); b = _req(b, np.int16)
    return lib().__mind_blas_dot_i16_v(_addr(a), _addr(b), len(a))


# ---------------------------------------------------------------- conveniences

def det_matmul_i8(A, B):
    A = _req(A, np.int8); B = _req(B, np.int8)
    m, k = A.shape; n = B.shape[1]
    C = np.empty((m, n), np.int32)
    check(lib().det_matmul_i8(_addr(A), _addr(B), _addr(C), m, k, n))
    return C


def det_matmul_i16(A, B):
    A = _req(A, np.int16); B = _req(B, np.int16)
    m, k = A.shape; n = B.shape[1]
    C = np.empty((m, n), np.int32)
    check(lib().det_matmul_i16(_addr(A), _addr(B), _addr(C), m, k, n))
    return C


def det_matmul_q16(A, B):
    A = _req(A, np.int32); B = _req(B, np.int32)
    m, k = A.shape; n = B.shape[1]
    C = np.empty((m, n), np.int32)
    check(lib().det_matmul_q16(_addr(A), _addr(B), _addr(C), m, k, n))
    return C


def det_gemv_q16(W, X):
    """X is [k] or [nb, k]; returns y [m] or [nb, m]."""
    W = _req(W, np.int32); X = _req(X, np.int32)
    m, k = W.shape
    nb = 1 if X.ndim == 1 else X.shape[0]
    Y = np.empty((nb, m), np.int32)
    check(lib().det_gemv_q16_batched(_addr(W), _addr(X), _addr(Y), m, k, nb))
    return Y[0] if X.ndim == 1 else Y


def det_gemv_i16(W, x):
    W = _req(W, np.int16); x = _req(x, np.int16)
    m, k = W.shape
    y = np.empty(m, np.int32)
    check(lib().det_gemv_i16(_addr(W), _addr(x), _addr(y), m, k))
    return y


# ---------------------------------------------------------------- device memory

class DeviceBuffer:
    """Owned device allocation (hipMalloc through the C ABI)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _p()
        check(lib().det_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        if a.nbytes:
            check(lib().det_memcpy_htod(d.ptr, a.ctypes.data, a.nbytes))
        return d

    def to_array(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        if out.nbytes:
            check(lib().det_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def fill(self, byte: int) -> None:
        check(lib().det_memset_dev(self.ptr, byte, self.nbytes))

    def free(self) -> None:
        if self.ptr:
            lib().det_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = _p()
        check(lib().det_stream_create(ctypes.byref(p)))
        self.ptr = p.value

    def sync(self):
        check(lib().det_stream_sync(self.ptr))

    def destroy(self):
        if self.ptr:
            lib().det_stream_destroy(self.ptr)
            self.ptr = None


class Event:
    def __init__(self):
        p = _p()
        check(lib().det_event_create(ctypes.byref(p)))
        self.ptr = p.value

    def record(self, stream: Stream | None):
        check(lib().det_event_record(self.ptr, stream.ptr if stream else None))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().det_event_elapsed_ms(self.ptr, end.ptr, ctypes.byref(ms)))
        return ms.value

    def destroy(self):
        if self.ptr:
            lib().det_event_destroy(self.ptr)
            self.ptr = None


def device_info() -> dict:
    info = (_i64 * 6)()
    name = ctypes.create_string_buffer(256)
    check(lib().det_device_info(info, name, 256))
    return {"name": name.value.decode(), "cus": info[0], "clock_khz": info[1], "hbm_bytes": info[2],
            "lds_bytes": info[3], "mem_clock_khz": info[4], "bus_width": info[5]}


# ---------------------------------------------------------------- generators
# The reference bench harness's seeded inputs (benches/det_matmul_*.rs).

def gen_i8(seed, na, nb):
    a = np.empty(na, np.int8); b = np.empty(nb, np.int8)
    lib().det_gen_i8(seed, _addr(a), na, _addr(b), nb)
    return a, b


def gen_i16(seed, na, nb):
    a = np.empty(na, np.int16); b = np.empty(nb, np.int16)
    lib().det_gen_i16(seed, _addr(a), na, _addr(b), nb)
    return a, b


def gen_q16(seed, na, nb, shift=12):
    a = np.empty(na, np.int32); b = np.empty(nb, np.int32)
    lib().det_gen_q16(seed, shift, _addr(a), na, _addr(b), nb)
    return a, b


def gen_f32_unit(seed, na, nb):
    a = np.empty(na, np.float32); b = np.empty(nb, np.float32)
    lib().det_gen_f32_unit(seed, _addr(a), na, _addr(b), nb)
    return a, b


def fft_twiddles(n):
    """Q16.16 twiddle table for fft256: tw[2k] = round(cos(-2 pi k / n) 2^16),
    tw[2k+1] = round(sin(-2 pi k / n) 2^16), k < n / 2 (the reference
    harness's table, bench/fft/fft_driver.c:23-31)."""
    k = np.arange(n // 2, dtype=np.float64)
    ang = -2.0 * np.pi * k / n
    def llround(v):   # half away from zero, like C llround
        return (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64)

    tw = np.zeros(max(n, 2), np.int64)
    tw[0:n:2] = llround(np.cos(ang) * 65536.0)
    tw[1:n:2] = llround(np.sin(ang) * 65536.0)
    return tw


def gen_q16_sat(seed, na, nb, shift=13):
    a = np.empty(na, np.int32); b = np.empty(nb, np.int32)
    lib().det_gen_q16_sat(seed, shift, _addr(a), na, _addr(b), nb)
    return a, b


def gen_i8_gauss(seed, n):
    x = np.empty(n, np.int8)
    lib().det_gen_i8_gauss(seed, _addr(x), n)
    return x


def gen_i8_sym127(seed, n):
    w = np.empty(n, np.int8)
    lib().det_gen_i8_sym127(seed, _addr(w), n)
    return w
