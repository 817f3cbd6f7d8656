"""CPU oracle for the deterministic integer / Q16.16 GEMM and GEMV intrinsics.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package: it is the checker,
never the thing measured or shipped.  The product (``mind_amd``) never imports
it and has no CPU fallback.

ctypes bindings over ``oracle/liboracle_det.so`` (built from ``det_oracle.c``
and ``det_cpu_mt.c`` by ``oracle/Makefile``) plus, when present, the reference's
own ``runtime-support/mind_intrinsics.c`` compiled into
``oracle/_ref/libmind_intrinsics_ref.so``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_det.so")
REF_PATH = os.path.join(HERE, "_ref", "libmind_intrinsics_ref.so")
FFT_REF_PATH = os.path.join(HERE, "_ref", "libfft_ref.so")

_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_p = ctypes.c_void_p

_lib = None
_ref = None
_fft_ref = None


def build() -> None:
    """Compile liboracle_det.so (and _ref when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.det_or_lcg_next_u32.argtypes = [ctypes.POINTER(_u64)]
        L.det_or_lcg_next_u32.restype = ctypes.c_uint32
        for name in ("det_or_gen_i8", "det_or_gen_i16", "det_or_gen_f32_unit"):
            getattr(L, name).argtypes = [_u64, _p, _i64, _p, _i64]
            getattr(L, name).restype = None
        L.det_or_dot_f32.argtypes = [_p, _p, _i64]
        L.det_or_dot_f32.restype = ctypes.c_float
        L.det_or_matmul_rmajor_f32.argtypes = [_p, _p, _p, _i64, _i64]
        L.det_or_matmul_rmajor_f32.restype = None
        for name in ("det_or_dot_l1_f32", "det_or_dot_linf_f32", "det_or_dot_linf_f32_v"):
            getattr(L, name).argtypes = [_p, _p, _i64]
            getattr(L, name).restype = ctypes.c_uint32
        L.det_or_rows_metric_f32.argtypes = [ctypes.c_int, _p, _p, _p, _i64, _i64]
        L.det_or_rows_metric_f32.restype = None
        for name in ("det_or_gen_q16", "det_or_gen_q16_sat"):
            getattr(L, name).argtypes = [_u64, ctypes.c_int, _p, _i64, _p, _i64]
            getattr(L, name).restype = None
        for name in ("det_or_gen_i8_gauss", "det_or_gen_i8_sym127"):
            getattr(L, name).argtypes = [_u64, _p, _i64]
            getattr(L, name).restype = None
        for name in ("det_or_gemm_i8", "det_or_gemm_q16", "det_or_gemm_i16"):
            getattr(L, name).argtypes = [_p, _p, _p, _i64, _i64, _i64]
            getattr(L, name).restype = None
        for name in ("det_or_gemm_i8_rows", "det_or_gemm_q16_rows", "det_or_gemm_i16_rows"):
            getattr(L, name).argtypes = [_p, _p, _p, _i64, _i64, _i64, _p, _i64]
            getattr(L, name).restype = None
        L.det_or_gemv_q16.argtypes = [_p, _p, _p, _i64, _i64]
        L.det_or_gemv_q16.restype = None
        L.det_or_gemv_q16_batched.argtypes = [_p, _p, _p, _i64, _i64, _i64]
        L.det_or_gemv_q16_batched.restype = None
        L.det_or_gemv_q16_rows.argtypes = [_p, _p, _p, _i64, _i64, _i64, _p, _i64]
        L.det_or_gemv_q16_rows.restype = None
        L.det_or_gemv_i16.argtypes = [_p, _p, _p, _i64, _i64]
        L.det_or_gemv_i16.restype = None
        for name in ("det_or_dot_q16", "det_or_dot_i16", "det_or_dot_l1_q16"):
            getattr(L, name).argtypes = [_p, _p, _i64]
            getattr(L, name).restype = _i64
        for name in ("det_cpu_gemm_i8", "det_cpu_gemm_q16", "det_cpu_gemm_i16"):
            getattr(L, name).argtypes = [_p, _p, _p, _i64, _i64, _i64]
            getattr(L, name).restype = _i64
        L.det_cpu_gemv_q16.argtypes = [_p, _p, _p, _i64, _i64]
        L.det_cpu_gemv_q16.restype = _i64
        L.det_or_fft_q16.argtypes = [_p, _p, _p, _i64, _i64]
        L.det_or_fft_q16.restype = _i64
        L.det_or_fft_twiddles.argtypes = [_p, _i64]
        L.det_or_fft_twiddles.restype = None
        for name in ("det_or_fft_input_lcg", "det_or_fft_input_harness"):
            getattr(L, name).argtypes = [_u64, _p, _p, _i64]
            getattr(L, name).restype = None
        L.det_or_fnv1a_i64.argtypes = [_p, _i64]
        L.det_or_fnv1a_i64.restype = _u64
        L.det_cpu_set_threads.argtypes = [ctypes.c_long]
        L.det_cpu_set_threads.restype = ctypes.c_long
        L.det_cpu_threads_for.argtypes = [_i64]
        L.det_cpu_threads_for.restype = ctypes.c_long
        _lib = L
    return _lib


def ref_built() -> bool:
    """Whether oracle/_ref holds the reference's runtime-support library
    (checked without loading it, so test collection maps nothing)."""
    return os.path.exists(REF_PATH)


def fft_ref_built() -> bool:
    """Whether oracle/_ref holds the reference's C FFT (not loaded here)."""
    return os.path.exists(FFT_REF_PATH)


def ref_lib():
    """The reference's own runtime-support library, or None if not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        R = ctypes.CDLL(REF_PATH)
        for name in ("__mind_blas_dot_q16", "__mind_blas_dot_l1_q16", "__mind_blas_dot_f32",
                     "__mind_blas_dot_l1_f32", "__mind_blas_dot_linf_f32"):
            getattr(R, name).argtypes = [_i64, _i64, _i64]
            getattr(R, name).restype = _i64
        R.__mind_blas_matmul_rmajor_f32.argtypes = [_i64] * 5
        R.__mind_blas_matmul_rmajor_f32.restype = _i64
        R.__mind_blas_set_use_avx2.argtypes = [ctypes.c_int]
        R.__mind_blas_set_use_avx2.restype = ctypes.c_int
        _ref = R
    return _ref


def fft_ref_lib():
    """The reference's C FFT (bench/fft/fft_ref.c, fft256_c), or None if not built."""
    global _fft_ref
    if _fft_ref is None and os.path.exists(FFT_REF_PATH):
        R = ctypes.CDLL(FFT_REF_PATH)
        R.fft256_c.argtypes = [_i64] * 5
        R.fft256_c.restype = _i64
        _fft_ref = R
    return _fft_ref


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data if a.size else 0


# ------------------------------------------------------------------ generators

def lcg_u32(seed: int, count: int) -> np.ndarray:
    L = lib()
    s = _u64(seed)
    return np.array([L.det_or_lcg_next_u32(ctypes.byref(s)) for _ in range(count)], dtype=np.uint32)


def gen_i8(seed: int, na: int, nb: int):
    a = np.empty(na, np.int8)
    b = np.empty(nb, np.int8)
    lib().det_or_gen_i8(seed, _ptr(a), na, _ptr(b), nb)
    return a, b


def gen_i16(seed: int, na: int, nb: int):
    a = np.empty(na, np.int16)
    b = np.empty(nb, np.int16)
    lib().det_or_gen_i16(seed, _ptr(a), na, _ptr(b), nb)
    return a, b


def gen_q16(seed: int, na: int, nb: int, shift: int = 12):
    a = np.empty(na, np.int32)
    b = np.empty(nb, np.int32)
    lib().det_or_gen_q16(seed, shift, _ptr(a), na, _ptr(b), nb)
    return a, b


def gen_f32_unit(seed: int, na: int, nb: int):
    """Reference f32 samples in [-1, 1) (a then b from one LCG stream)."""
    a = np.empty(na, np.float32)
    b = np.empty(nb, np.float32)
    lib().det_or_gen_f32_unit(seed, _ptr(a), na, _ptr(b), nb)
    return a, b


def gen_q16_sat(seed: int, na: int, nb: int, shift: int = 13):
    a = np.empty(na, np.int32)
    b = np.empty(nb, np.int32)
    lib().det_or_gen_q16_sat(seed, shift, _ptr(a), na, _ptr(b), nb)
    return a, b


def gen_i8_gauss(seed: int, n: int):
    x = np.empty(n, np.int8)
    lib().det_or_gen_i8_gauss(seed, _ptr(x), n)
    return x


def gen_i8_sym127(seed: int, n: int):
    w = np.empty(n, np.int8)
    lib().det_or_gen_i8_sym127(seed, _ptr(w), n)
    return w


# ------------------------------------------------------------------ oracles

def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def gemm_i8(A, B, m, k, n):
    A = _c(A, np.int8); B = _c(B, np.int8)
    C = np.empty(m * n, np.int32)
    lib().det_or_gemm_i8(_ptr(A), _ptr(B), _ptr(C), m, k, n)
    return C.reshape(m, n)


def gemm_q16(A, B, m, k, n):
    A = _c(A, np.int32); B = _c(B, np.int32)
    C = np.empty(m * n, np.int32)
    lib().det_or_gemm_q16(_ptr(A), _ptr(B), _ptr(C), m, k, n)
    return C.reshape(m, n)


def gemm_i16(A, B, m, k, n):
    A = _c(A, np.int16); B = _c(B, np.int16)
    C = np.empty(m * n, np.int32)
    lib().det_or_gemm_i16(_ptr(A), _ptr(B), _ptr(C), m, k, n)
    return C.reshape(m, n)


def _rows_call(fn, A, B, dt, m, k, n, rows):
    A = _c(A, dt); B = _c(B, dt)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    C = np.empty(len(rows) * n, np.int32)
    fn(_ptr(A), _ptr(B), _ptr(C), m, k, n, _ptr(rows), len(rows))
    return C.reshape(len(rows), n)


def gemm_i8_rows(A, B, m, k, n, rows):
    return _rows_call(lib().det_or_gemm_i8_rows, A, B, np.int8, m, k, n, rows)


def gemm_q16_rows(A, B, m, k, n, rows):
    return _rows_call(lib().det_or_gemm_q16_rows, A, B, np.int32, m, k, n, rows)


def gemm_i16_rows(A, B, m, k, n, rows):
    return _rows_call(lib().det_or_gemm_i16_rows, A, B, np.int16, m, k, n, rows)


def gemv_q16(W, x, m, k):
    W = _c(W, np.int32); x = _c(x, np.int32)
    y = np.empty(m, np.int32)
    lib().det_or_gemv_q16(_ptr(W), _ptr(x), _ptr(y), m, k)
    return y


def gemv_q16_batched(W, X, m, k, nb):
    W = _c(W, np.int32); X = _c(X, np.int32)
    Y = np.empty(nb * m, np.int32)
    lib().det_or_gemv_q16_batched(_ptr(W), _ptr(X), _ptr(Y), m, k, nb)
    return Y.reshape(nb, m)


def gemv_q16_rows(W, X, m, k, nb, rows):
    W = _c(W, np.int32); X = _c(X, np.int32)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    Y = np.empty(nb * len(rows), np.int32)
    lib().det_or_gemv_q16_rows(_ptr(W), _ptr(X), _ptr(Y), m, k, nb, _ptr(rows), len(rows))
    return Y.reshape(nb, len(rows))


def gemv_i16(W, x, rows, cols):
    W = _c(W, np.int16); x = _c(x, np.int16)
    y = np.empty(rows, np.int32)
    lib().det_or_gemv_i16(_ptr(W), _ptr(x), _ptr(y), rows, cols)
    return y


def dot_q16(a, b):
    a = _c(a, np.int32); b = _c(b, np.int32)
    return lib().det_or_dot_q16(_ptr(a), _ptr(b), len(a))


def dot_i16(a, b):
    a = _c(a, np.int16); b = _c(b, np.int16)
    return lib().det_or_dot_i16(_ptr(a), _ptr(b), len(a))


def dot_f32_bits(a, b) -> int:
    """Strict-FP f32 dot; the result's bits as the reference packs them
    (f32 bits in the low 32 bits of a non-negative int64)."""
    a = _c(a, np.float32); b = _c(b, np.float32)
    return int(np.float32(lib().det_or_dot_f32(_ptr(a), _ptr(b), len(a))).view(np.uint32))


def matmul_rmajor_f32(W, x, rows, cols):
    W = _c(W, np.float32); x = _c(x, np.float32)
    y = np.empty(rows, np.float32)
    lib().det_or_matmul_rmajor_f32(_ptr(W), _ptr(x), _ptr(y), rows, cols)
    return y


F32_DOT, F32_L1, F32_LINF, F32_LINF_V = 0, 1, 2, 3


def dist_f32_bits(op, a, b) -> int:
    """f32 distance op (F32_L1, F32_LINF, F32_LINF_V) as the reference packs
    it: the f32 bits in the low 32 bits of a non-negative int64."""
    a = _c(a, np.float32); b = _c(b, np.float32)
    if op == F32_DOT:
        return dot_f32_bits(a, b)
    fn = {F32_L1: "det_or_dot_l1_f32", F32_LINF: "det_or_dot_linf_f32", F32_LINF_V: "det_or_dot_linf_f32_v"}[op]
    return int(getattr(lib(), fn)(_ptr(a), _ptr(b), len(a)))


def rows_metric_f32_bits(op, W, x, rows, cols):
    """y[r] = op(W row r, x) as uint32 bits."""
    W = _c(W, np.float32); x = _c(x, np.float32)
    y = np.empty(rows, np.uint32)
    lib().det_or_rows_metric_f32(op, _ptr(W), _ptr(x), _ptr(y), rows, cols)
    return y


def dot_l1_q16(a, b):
    a = _c(a, np.int32); b = _c(b, np.int32)
    return lib().det_or_dot_l1_q16(_ptr(a), _ptr(b), len(a))


# ------------------------------------------------------------------ hashing

def sha256_i32_le(v) -> str:
    """Canonical output hash: each i32 little-endian, then sha256 (lowercase
    hex) -- benches/det_matmul_i8.rs:247-256."""
    import hashlib

    return hashlib.sha256(np.ascontiguousarray(v, dtype="<i4").tobytes()).hexdigest()


def sha256_i64_le(v: int) -> str:
    import hashlib

    return hashlib.sha256(int(v).to_bytes(8, "little", signed=True)).hexdigest()


# ------------------------------------------------------------------ Q16 FFT

def fft_q16(re, im, tw, logn: int):
    """Radix-2 DIT Q16.16 FFT of one transform (copies in, returns (re, im));
    examples/fft_q16.mind semantics, wrapping int64."""
    re = np.array(re, np.int64, copy=True)
    im = np.array(im, np.int64, copy=True)
    tw = np.ascontiguousarray(tw, np.int64)
    rc = lib().det_or_fft_q16(_ptr(re), _ptr(im), _ptr(tw), logn, len(re))
    if rc != 0:
        raise ValueError(f"fft_q16: n={len(re)} is not 2^{logn}")
    return re, im


def fft_twiddles(n: int) -> np.ndarray:
    tw = np.zeros(max(n, 2), np.int64)
    lib().det_or_fft_twiddles(_ptr(tw), n)
    return tw[:n] if n >= 2 else tw


def fft_input_lcg(seed: int, n: int):
    re = np.empty(n, np.int64); im = np.empty(n, np.int64)
    lib().det_or_fft_input_lcg(seed, _ptr(re), _ptr(im), n)
    return re, im


def fft_input_harness(seed: int, n: int):
    re = np.empty(n, np.int64); im = np.empty(n, np.int64)
    lib().det_or_fft_input_harness(seed, _ptr(re), _ptr(im), n)
    return re, im


def fnv1a_i64(a) -> int:
    a = np.ascontiguousarray(a, np.int64)
    return int(lib().det_or_fnv1a_i64(_ptr(a), len(a)))
