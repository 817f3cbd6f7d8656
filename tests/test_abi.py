"""CPU tier: the C-ABI library loads, exports every declared symbol, and its
host-side harness (seeded generators) matches the oracle's.  No kernel is
launched here."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

import mind_amd
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_built_and_loads():
    assert os.path.exists(mind_amd.LIB_PATH)
    assert mind_amd.lib().det_version().decode().startswith("mind-det")


def test_every_header_symbol_is_exported():
    syms = mind_amd.header_symbols()
    # the reference's intrinsic and harness names are all declared
    for name in ("__mind_blas_matmul_mm_i8_v", "__mind_blas_matmul_mm_i8_mt_v", "__mind_blas_matmul_mm_q16_v",
                 "__mind_blas_matmul_mm_q16_mt_v", "__mind_blas_gemv_q16_mt", "__mind_blas_matmul_rmajor_q16_v",
                 "__mind_blas_matmul_rmajor_i16_v", "__mind_blas_dot_q16", "gemmi8", "gemmi8mt", "gemmqmm",
                 "gemmq", "mmq", "mmi16", "gemvq", "dotq", "det_matmul_i8", "det_matmul_i16", "det_matmul_q16",
                 "det_gemv_q16", "det_gemv_q16_batched"):
        assert name in syms, name
    raw = ctypes.CDLL(mind_amd.LIB_PATH)
    missing = [s for s in syms if not hasattr(raw, s)]
    assert not missing, missing


def test_reference_arity_is_kept():
    # reference arity table (src/type_checker/mod.rs:2266-2332): GEMMs 6,
    # GEMV / rmajor 5, dot 3 -- all int64 in and out
    text = open(mind_amd.HEADER).read()
    for name, arity in (("__mind_blas_matmul_mm_i8_v", 6), ("__mind_blas_matmul_mm_q16_v", 6),
                        ("__mind_blas_gemv_q16_mt", 5), ("__mind_blas_matmul_rmajor_i16_v", 5),
                        ("__mind_blas_dot_q16", 3), ("__mind_blas_dot_q16_v", 3), ("__mind_blas_dot_l1_q16", 3),
                        ("__mind_blas_dot_l1_q16_v", 3), ("__mind_blas_dot_i16_v", 3), ("dotl1q", 3), ("doti16", 3)):
        m = re.search(r"int64_t " + re.escape(name) + r"\(([^)]*)\)", text)
        args = [a.strip() for a in m.group(1).split(",")]
        assert len(args) == arity and all(a.startswith("int64_t") for a in args), name


@pytest.mark.parametrize("n", [0, 1, 1000, 70001, 300000])
def test_product_generators_match_oracle(n):
    seed = 0xDEADBEEF ^ n
    for gp, go in ((mind_amd.gen_i8, O.gen_i8), (mind_amd.gen_i16, O.gen_i16)):
        for x, y in zip(gp(seed, n, n + 3), go(seed, n, n + 3)):
            np.testing.assert_array_equal(x, y)
    for shift in (12, 13, 15):
        for x, y in zip(mind_amd.gen_q16(seed, n, 5, shift), O.gen_q16(seed, n, 5, shift)):
            np.testing.assert_array_equal(x, y)
    for x, y in zip(mind_amd.gen_q16_sat(seed, n, n, 13), O.gen_q16_sat(seed, n, n, 13)):
        np.testing.assert_array_equal(x, y)
    np.testing.assert_array_equal(mind_amd.gen_i8_gauss(seed, n), O.gen_i8_gauss(seed, n))
    np.testing.assert_array_equal(mind_amd.gen_i8_sym127(seed, n), O.gen_i8_sym127(seed, n))
    for x, y in zip(mind_amd.gen_f32_unit(seed, n, n + 5), O.gen_f32_unit(seed, n, n + 5)):
        np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))


def test_product_fft_twiddles_match_oracle():
    for logn in range(1, 21):
        n = 1 << logn
        np.testing.assert_array_equal(mind_amd.fft_twiddles(n)[:n], O.fft_twiddles(n)[:n])


def test_product_never_touches_the_oracle():
    """The shipped package and its native sources must not import, link or
    load anything under oracle/ (no CPU fallback path)."""
    files = glob.glob(os.path.join(ROOT, "mind_amd", "**", "*.py"), recursive=True)
    files += glob.glob(os.path.join(ROOT, "mind_amd", "csrc", "*"))
    for f in files:
        text = open(f, errors="ignore").read()
        assert not re.search(r"import oracle|from oracle|det_or_|det_cpu_|liboracle|oracle/", text), f


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(mind_amd, "_lib", None)
    monkeypatch.setattr(mind_amd, "LIB_PATH", "/nonexistent/libmind_det_hip.so")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        mind_amd.lib()


def test_bench_refuses_more_than_one_gpu():
    """bench.py's contract: --gpus N > 1 exits non-zero with a message before any GPU call."""
    import subprocess
    import sys
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr and p.stdout == ""
