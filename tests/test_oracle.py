"""CPU tier: pin the oracle before trusting it.

Each oracle function is checked against something other than itself:
the reference's committed golden hashes (tests/cross_substrate_identity/*),
the digest embedded in bench/matmul_det_bench.mind, the reference's own
__mind_blas_dot_q16 (compiled from its C source into oracle/_ref, and
fixture outputs of it in tests/golden/dot_q16_ref.json), closed forms
computed with exact Python integers, and composition.  A final group plants
plausible mistakes in oracle-shaped code and shows those checks reject them.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def h32(v):
    return O.sha256_i32_le(v)


# ------------------------------------------------------------------ golden

def test_lcg_first_draws_follow_recurrence():
    # s <- s*1664525 + 1013904223 mod 2^64, u32 = s >> 16
    s = 0xDEADBEEF
    want = []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) % (1 << 64)
        want.append((s >> 16) & 0xFFFFFFFF)
    assert list(O.lcg_u32(0xDEADBEEF, 5)) == want


@pytest.mark.parametrize("wid", ["gemm-i8-64x64x64", "gemm-i8-mt-64x64x64", "gemm-i8-vnni-64x64x64"])
def test_gemm_i8_canary(canaries, wid):
    w = canaries["workloads"][wid]
    a, b = O.gen_i8(w["seed"], w["m"] * w["k"], w["k"] * w["n"])
    assert w["avx2"] == w["neon"]
    assert h32(O.gemm_i8(a, b, w["m"], w["k"], w["n"])) == w["avx2"]


@pytest.mark.parametrize("wid", ["gemm-q16-64x64x64", "gemm-q16-fused-64x64x64"])
def test_gemm_q16_canary(canaries, wid):
    w = canaries["workloads"][wid]
    a, b = O.gen_q16(w["seed"], w["m"] * w["k"], w["k"] * w["n"])
    assert h32(O.gemm_q16(a, b, w["m"], w["k"], w["n"])) == w["avx2"]


def test_gemv_q16_canary(canaries):
    w = canaries["workloads"]["gemv-q16-256x256"]
    W, x = O.gen_q16(w["seed"], w["rows"] * w["cols"], w["cols"])
    assert h32(O.gemv_q16(W, x, w["rows"], w["cols"])) == w["avx2"]


def test_gemv_i16_canary(canaries):
    w = canaries["workloads"]["gemv-i16-256x256"]
    W, x = O.gen_i16(w["seed"], w["rows"] * w["cols"], w["cols"])
    assert h32(O.gemv_i16(W, x, w["rows"], w["cols"])) == w["avx2"]


def test_dot_canaries(canaries):
    w = canaries["workloads"]["dot-i16-4096"]
    a, b = O.gen_i16(w["seed"], w["length"], w["length"])
    assert O.sha256_i64_le(O.dot_i16(a, b)) == w["avx2"]
    w = canaries["workloads"]["dot-l2-q16"]
    a, b = O.gen_q16(w["seed"], w["length"], w["length"])
    assert O.sha256_i64_le(O.dot_q16(a, b)) == w["avx2"]
    w = canaries["workloads"]["dot-l1-q16"]
    a, b = O.gen_q16(w["seed"], w["length"], w["length"])
    assert O.sha256_i64_le(O.dot_l1_q16(a, b)) == w["avx2"]


def _f32_special_pair(n, seed):
    """f32 inputs whose products and sums hit denormals, signed zeros and
    magnitudes near overflow (no NaN-producing combinations: NaN payloads are
    not pinned by the reference)."""
    rng = np.random.default_rng(seed)
    vals = np.array([1e-20, -1e-20, 3e-39, -0.0, 0.0, 1.0, -1.0, 1e19, -1e19, 0.5, 1e-30, 2.5e-25], np.float32)
    a = vals[rng.integers(0, len(vals), n)]
    b = vals[rng.integers(0, 6, n)]          # finite, |b| <= 1: no inf - inf
    return a, b


def test_f32_strict_canaries(canaries):
    w = canaries["workloads"]["dot-f32-v-4093"]
    a, b = O.gen_f32_unit(w["seed"], w["length"], w["length"])
    assert O.sha256_i64_le(O.dot_f32_bits(a, b)) == w["avx2"]
    w = canaries["workloads"]["matmul-f32-v-64x64"]
    W, x = O.gen_f32_unit(w["seed"], w["rows"] * w["cols"], w["cols"])
    y = O.matmul_rmajor_f32(W, x, w["rows"], w["cols"])
    assert hashlib.sha256(y.view("<u4").tobytes()).hexdigest() == w["avx2"]


def _dot_f32_variant(a, b, fused=False, pairwise=False):
    """The reference schedule with one planted change: a single-rounding
    multiply-add (emulated exactly in float64: a product of two f32 is exact
    there) or a pairwise lane fold."""
    n8 = len(a) // 8 * 8
    acc = np.zeros(8, np.float32)
    for i in range(0, n8, 8):
        if fused:
            acc = (acc.astype(np.float64) + a[i:i + 8].astype(np.float64) * b[i:i + 8].astype(np.float64)).astype(np.float32)
        else:
            acc = (acc + (a[i:i + 8] * b[i:i + 8])).astype(np.float32)
    if pairwise:
        s = np.float32(np.float32(acc[0] + acc[1]) + np.float32(acc[2] + acc[3])) + \
            np.float32(np.float32(acc[4] + acc[5]) + np.float32(acc[6] + acc[7]))
    else:
        s = acc[0]
        for j in range(1, 8):
            s = np.float32(s + acc[j])
    for i in range(n8, len(a)):
        s = np.float32(np.float64(s) + np.float64(a[i]) * np.float64(b[i])) if fused else np.float32(s + np.float32(a[i] * b[i]))
    return np.float32(s)


def test_f32_strict_schedule_is_load_bearing(canaries):
    # the golden hash of the 64-row matmul (64 independent 64-term dots)
    # rejects an FMA-contracted dot, a pairwise lane fold and a float64
    # accumulation: the schedule, not just the sum, is the contract.  (A
    # single dot can coincide: the 4093-term dot canary rounds to the same
    # float under both the pairwise fold and fusion.)
    w = canaries["workloads"]["matmul-f32-v-64x64"]
    W, x = O.gen_f32_unit(w["seed"], w["rows"] * w["cols"], w["cols"])
    rows, cols = w["rows"], w["cols"]

    def ok(rowdot):
        y = np.array([rowdot(W[r * cols:(r + 1) * cols]) for r in range(rows)], np.float32)
        return hashlib.sha256(y.view("<u4").tobytes()).hexdigest() == w["avx2"]

    assert ok(lambda a: _dot_f32_variant(a, x))                            # the restatement itself
    assert not ok(lambda a: _dot_f32_variant(a, x, fused=True))
    assert not ok(lambda a: _dot_f32_variant(a, x, pairwise=True))
    assert not ok(lambda a: np.float32(np.dot(a.astype(np.float64), x.astype(np.float64))))


@pytest.mark.skipif(O.ref_lib() is None, reason="oracle/_ref not built (reference tree absent)")
def test_f32_strict_matches_reference_live():
    R = O.ref_lib()
    prev = R.__mind_blas_set_use_avx2(0)
    try:
        for avx2 in (0, 1):
            R.__mind_blas_set_use_avx2(avx2)
            for n in list(range(0, 18)) + [4093, 65541]:
                for a, b in (O.gen_f32_unit(0xF32 ^ n, n, n), _f32_special_pair(n, n)):
                    assert O.dot_f32_bits(a, b) == R.__mind_blas_dot_f32(a.ctypes.data, b.ctypes.data, n)
            W, x = O.gen_f32_unit(0xF33, 37 * 131, 131)
            y = np.zeros(37, np.float32)
            assert R.__mind_blas_matmul_rmajor_f32(W.ctypes.data, x.ctypes.data, y.ctypes.data, 37, 131) == 0
            assert np.array_equal(O.matmul_rmajor_f32(W, x, 37, 131).view(np.uint32), y.view(np.uint32))
    finally:
        R.__mind_blas_set_use_avx2(prev)


def test_dot_l1_q16_brute_force_and_extremes():
    # exact Python ints: (int64)(int32) sum |a - b|, including |INT32_MIN - INT32_MAX|
    # = 2^32 - 1 per term (wraps the int32 result) and the empty / length-1 cases
    rng = np.random.default_rng(0x11)
    ext = np.array([2147483647, -2147483648, -2147483647, 0, 1, -1, 65536, -65536], np.int32)
    cases = [(np.zeros(0, np.int32), np.zeros(0, np.int32)),
             (np.array([-2147483648], np.int32), np.array([2147483647], np.int32))]
    for n in (1, 2, 7, 64, 1000):
        cases.append((rng.integers(-2**31, 2**31, n, dtype=np.int64).astype(np.int32),
                      rng.integers(-2**31, 2**31, n, dtype=np.int64).astype(np.int32)))
        cases.append((ext[rng.integers(0, 8, n)], ext[rng.integers(0, 8, n)]))
    for a, b in cases:
        want = _to_i32(sum(abs(int(x) - int(y)) for x, y in zip(a, b)))
        assert O.dot_l1_q16(a, b) == want
        assert O.dot_l1_q16(b, a) == want                    # symmetric
        assert O.dot_l1_q16(a, a) == 0


@pytest.mark.skipif(O.ref_lib() is None, reason="oracle/_ref not built (reference tree absent)")
def test_dot_l1_q16_matches_reference_live():
    """The reference's scalar L1 (mind_intrinsics.c:1551-1562, the contract the
    vector-dialect emitter lowering.rs:6035-6060 matches byte for byte) on every
    input family; its AVX2 Track A path (:1566-1596) agrees wherever |a - b| <
    2^31, but forms a - b in 32 bits (_mm256_sub_epi32 + _mm256_abs_epi32), so on
    full-range inputs it differs from its own scalar definition.  This build
    follows the scalar / vector-dialect semantics."""
    R = O.ref_lib()
    prev = R.__mind_blas_set_use_avx2(0)
    try:
        for fam in ("ref12", "full", "extreme"):
            for n in (1, 9, 4093, 65536):
                a, b = _dot_inputs(fam, 0x1D1 ^ n, n)
                assert O.dot_l1_q16(a, b) == R.__mind_blas_dot_l1_q16(a.ctypes.data, b.ctypes.data, n)
        R.__mind_blas_set_use_avx2(1)
        for n in (1, 9, 4093, 65536):            # Q16 range (>> 12): no 32-bit overflow, paths agree
            a, b = _dot_inputs("ref12", 0x1D2 ^ n, n)
            assert O.dot_l1_q16(a, b) == R.__mind_blas_dot_l1_q16(a.ctypes.data, b.ctypes.data, n)
        a = np.array([2147483647] * 8, np.int32)  # |a - b| = 2^32 - 1 per term: AVX2 path wraps
        b = np.array([-2147483648] * 8, np.int32)
        assert O.dot_l1_q16(a, b) == _to_i32(8 * (2**32 - 1))
        assert R.__mind_blas_dot_l1_q16(a.ctypes.data, b.ctypes.data, 8) != O.dot_l1_q16(a, b)
    finally:
        R.__mind_blas_set_use_avx2(prev)


def test_matmul_det_bench_digest(canaries):
    g = canaries["matmul_det_bench_256"]
    n = g["n"]
    idx = np.arange(n * n)
    A = (((idx + 1) % 7) - 3).astype(np.int8)
    B = (((idx + 2) % 7) - 3).astype(np.int8)
    d = hashlib.sha256(O.gemm_i8(A, B, n, n, n).astype("<i4").tobytes()).digest()
    words = [int.from_bytes(d[i:i + 8], "little", signed=True) for i in range(0, 32, 8)]
    assert words == g["digest_words_le_i64"]


# ------------------------------------------------------------------ reference's own dot_q16

def _dot_inputs(fam, seed, n):
    extreme = np.array([2147483647, -2147483647, -2147483648, 65535, -65536, 1, -1, 0], np.int32)
    if fam == "extreme":
        ia, ib = O.gen_q16(seed, n, n, shift=29)
        return extreme[ia & 7], extreme[ib & 7]
    return O.gen_q16(seed, n, n, shift={"ref12": 12, "q4": 13, "full": 0}[fam])


def test_dot_q16_matches_reference_fixture():
    d = json.load(open(os.path.join(GOLD, "dot_q16_ref.json")))
    assert len(d["cases"]) >= 60
    for c in d["cases"]:
        a, b = _dot_inputs(c["family"], c["seed"], c["len"])
        got = O.dot_q16(a, b)
        assert got == c["scalar"] == c["avx2"], c


@pytest.mark.skipif(O.ref_lib() is None, reason="oracle/_ref not built (reference tree absent)")
def test_gemv_rows_match_reference_dot_live():
    R = O.ref_lib()
    m, k = 96, 1031
    for shift in (0, 12, 15):
        W, x = O.gen_q16(0x5EED ^ shift, m * k, k, shift=shift)
        y = O.gemv_q16(W, x, m, k)
        for i in range(m):
            row = np.ascontiguousarray(W[i * k:(i + 1) * k])
            assert y[i] == np.int32(R.__mind_blas_dot_q16(row.ctypes.data, x.ctypes.data, k))


# ------------------------------------------------------------------ closed forms (exact Python ints)

def _to_i32(v):
    v &= 0xFFFFFFFF
    return v - (1 << 32) if v >= 1 << 31 else v


def _q16_closed_form(A, B, m, k, n):
    """C = ((S - R) mod 2^48) >> 16 with S = sum a*b, R = sum (a*b mod 2^16)."""
    A = [[int(A[i * k + t]) for t in range(k)] for i in range(m)]
    B = [[int(B[t * n + j]) for j in range(n)] for t in range(k)]
    C = np.empty((m, n), np.int32)
    for i in range(m):
        for j in range(n):
            S = sum(A[i][t] * B[t][j] for t in range(k))
            R = sum((A[i][t] * B[t][j]) & 0xFFFF for t in range(k))
            C[i, j] = _to_i32((((S - R) % (1 << 48)) >> 16))
    return C


def _q16_alignbit_form(A, B, m, k, n):
    """C = sum (bits [16,48) of the 64-bit two's complement product) mod 2^32."""
    C = np.empty((m, n), np.int32)
    for i in range(m):
        for j in range(n):
            acc = 0
            for t in range(k):
                p = (int(A[i * k + t]) * int(B[t * n + j])) % (1 << 64)
                acc += (p >> 16) & 0xFFFFFFFF
            C[i, j] = _to_i32(acc)
    return C


@pytest.mark.parametrize("shift", [0, 12, 13])
def test_gemm_q16_closed_forms(shift):
    m, k, n = 5, 37, 6
    A, B = O.gen_q16(0xC105ED ^ shift, m * k, k * n, shift=shift)
    A[:3] = [2147483647, -2147483648, -1]
    got = O.gemm_q16(A, B, m, k, n)
    np.testing.assert_array_equal(got, _q16_closed_form(A, B, m, k, n))
    np.testing.assert_array_equal(got, _q16_alignbit_form(A, B, m, k, n))


def test_gemm_q16_saturated_config_closed_form():
    m, k, n = 4, 300, 3
    A, B = O.gen_q16_sat(0x5A7, m * k, k * n, shift=13)
    assert (np.abs(A) == 2147483647).any()
    np.testing.assert_array_equal(O.gemm_q16(A, B, m, k, n), _q16_closed_form(A, B, m, k, n))


def test_gemm_i8_brute_force_and_wrap():
    m, k, n = 3, 50, 4
    A, B = O.gen_i8(7, m * k, k * n)
    want = np.array([[_to_i32(sum(int(A[i * k + t]) * int(B[t * n + j]) for t in range(k)))
                      for j in range(n)] for i in range(m)], np.int32)
    np.testing.assert_array_equal(O.gemm_i8(A, B, m, k, n), want)
    # wrap: K * 16384 > 2^31 for all -128 operands
    k = 131136
    A = np.full(k, -128, np.int8)
    B = np.full(k, -128, np.int8)
    assert O.gemm_i8(A, B, 1, k, 1)[0, 0] == _to_i32(k * 16384)


def test_gemm_i16_composition_and_brute_force():
    m, k, n = 6, 129, 5
    A, B = O.gen_i16(0x1616, m * k, k * n)
    C = O.gemm_i16(A, B, m, k, n)
    Bm = B.reshape(k, n)
    for i in range(m):
        for j in range(n):
            assert C[i, j] == np.int32(O.dot_i16(A[i * k:(i + 1) * k], np.ascontiguousarray(Bm[:, j])))
            assert C[i, j] == _to_i32(sum(int(A[i * k + t]) * int(Bm[t, j]) for t in range(k)))


def test_rows_variants_match_full():
    m, k, n = 40, 70, 33
    rows = [0, 7, 39, 13]
    A, B = O.gen_i8(1, m * k, k * n)
    np.testing.assert_array_equal(O.gemm_i8_rows(A, B, m, k, n, rows), O.gemm_i8(A, B, m, k, n)[rows])
    A, B = O.gen_q16(2, m * k, k * n)
    np.testing.assert_array_equal(O.gemm_q16_rows(A, B, m, k, n, rows), O.gemm_q16(A, B, m, k, n)[rows])
    A, B = O.gen_i16(3, m * k, k * n)
    np.testing.assert_array_equal(O.gemm_i16_rows(A, B, m, k, n, rows), O.gemm_i16(A, B, m, k, n)[rows])
    W, X = O.gen_q16(4, m * k, 3 * k)
    np.testing.assert_array_equal(O.gemv_q16_rows(W, X, m, k, 3, rows), O.gemv_q16_batched(W, X, m, k, 3)[:, rows])


# ------------------------------------------------------------------ planted mistakes

def test_golden_rejects_plausible_mistakes(canaries):
    """Mistakes a restatement could plausibly make all change the canary
    hashes, so the golden checks above are sharp."""
    w = canaries["workloads"]["gemm-q16-64x64x64"]
    m = k = n = 64
    A, B = O.gen_q16(w["seed"], m * k, k * n)
    A64 = A.reshape(m, k).astype(np.int64)
    B64 = B.reshape(k, n).astype(np.int64)
    # (1) shift once at the end instead of per term
    shift_once = ((A64 @ B64) >> 16).astype(np.int32)
    assert h32(shift_once) != w["avx2"]
    # (2) transposed B operand
    per_term = ((A64[:, :, None] * B64.T[None, :, :]) >> 16).sum(1).astype(np.int32)
    assert h32(per_term) != w["avx2"]
    # (3) 32-bit truncating product (mullo) before the shift
    lo32 = (A64[:, :, None] * B64[None, :, :]).astype(np.int32).astype(np.int64)
    assert h32((lo32 >> 16).sum(1).astype(np.int32)) != w["avx2"]
    # (note: a logical instead of arithmetic shift of the 64-bit product is
    # NOT a mistake here: the two agree on bits [16, 48), all that survives
    # the final truncation to 32 bits.)
    # (4) the correct per-term floor does reproduce it (sanity of the harness)
    good = ((A64[:, :, None] * B64[None, :, :]) >> 16).sum(1).astype(np.int32)
    assert h32(good) == w["avx2"]
    # (5) int8: B drawn before A
    w8 = canaries["workloads"]["gemm-i8-64x64x64"]
    b, a = O.gen_i8(w8["seed"], 64 * 64, 64 * 64)
    assert h32(O.gemm_i8(a, b, 64, 64, 64)) != w8["avx2"]


# ------------------------------------------------------------------ CPU baseline restatement

@pytest.mark.parametrize("threads", [1, 3, 8])
def test_cpu_mt_baseline_matches_oracle(threads):
    L = O.lib()
    L.det_cpu_set_threads(threads)
    try:
        for (m, k, n) in [(1, 1, 1), (13, 77, 19), (70, 600, 150), (130, 1100, 40)]:
            A, B = O.gen_i8(m * 31 + k, m * k, k * n)
            C = np.empty(m * n, np.int32)
            L.det_cpu_gemm_i8(A.ctypes.data, B.ctypes.data, C.ctypes.data, m, k, n)
            np.testing.assert_array_equal(C.reshape(m, n), O.gemm_i8(A, B, m, k, n))
            A, B = O.gen_q16_sat(m + k, m * k, k * n)
            L.det_cpu_gemm_q16(A.ctypes.data, B.ctypes.data, C.ctypes.data, m, k, n)
            np.testing.assert_array_equal(C.reshape(m, n), O.gemm_q16(A, B, m, k, n))
            A, B = O.gen_i16(m ^ k, m * k, k * n)
            L.det_cpu_gemm_i16(A.ctypes.data, B.ctypes.data, C.ctypes.data, m, k, n)
            np.testing.assert_array_equal(C.reshape(m, n), O.gemm_i16(A, B, m, k, n))
            W, x = O.gen_q16(m * k, m * k, k, shift=15)
            y = np.empty(m, np.int32)
            L.det_cpu_gemv_q16(W.ctypes.data, x.ctypes.data, y.ctypes.data, m, k)
            np.testing.assert_array_equal(y, O.gemv_q16(W, x, m, k))
    finally:
        L.det_cpu_set_threads(0)


def test_config_generators_shape():
    x = O.gen_i8_gauss(11, 200000)
    assert x.min() >= -127 and x.max() <= 127
    assert abs(float(x.mean())) < 0.5 and 30.0 < float(x.std()) < 34.0
    w = O.gen_i8_sym127(12, 200000)
    assert w.min() == -127 and w.max() == 127
    a, b = O.gen_q16_sat(13, 100000, 10)
    sat = np.abs(a) == 2147483647
    assert 0.005 < sat.mean() < 0.015
    assert np.abs(a[~sat]).max() <= 4 << 16
