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


@pytest.mark.skipif(not O.ref_built(), reason="oracle/_ref not built (reference tree absent)")
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


def _metric_golden():
    import importlib.util
    spec = importlib.util.spec_from_file_location("mk_f32_metric", os.path.join(GOLD, "make_ref_f32_metric_vectors.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.inputs, json.load(open(os.path.join(GOLD, "dot_f32_metric_ref.json")))["cases"]


def test_f32_metrics_match_reference_vectors():
    """L1 / L-inf restatements against the committed outputs of the
    reference's own __mind_blas_dot_l1_f32 / __mind_blas_dot_linf_f32.  This
    build follows the scalar path (the definition every dispatch shares for
    L1 and every non-x86 build runs for L-inf).  The two paths agree on every
    case except L-inf with a NaN in lane 7 of the last full 8-block: the AVX2
    horizontal fold keeps that NaN (vmaxps returns its second operand when
    either is NaN, and lane 7 reaches the result only as a second operand),
    while the scalar loop skips it."""
    inputs, cases = _metric_golden()
    assert len(cases) == 60
    diverge = []
    with np.errstate(all="ignore"):
        for c in cases:
            a, b = inputs(c["family"], c["seed"], c["len"], c.get("pos"))
            assert c["l1_scalar"] == c["l1_avx2"], c
            if c["linf_scalar"] != c["linf_avx2"]:
                diverge.append((c["len"], c["pos"]))
            assert O.dist_f32_bits(O.F32_L1, a, b) == c["l1_scalar"], c
            assert O.dist_f32_bits(O.F32_LINF, a, b) == c["linf_scalar"], c
    nan_cases = [c for c in cases if c["family"] == "nan"]
    assert len(nan_cases) == 21
    assert diverge == [(c["len"], c["pos"]) for c in nan_cases if c["pos"] == c["len"] // 8 * 8 - 1]
    assert all(c["linf_avx2"] == 0x7fc00000 for c in nan_cases if (c["len"], c["pos"]) in diverge)


@pytest.mark.skipif(not O.ref_built(), reason="oracle/_ref not built (reference tree absent)")
def test_f32_metrics_match_reference_live():
    R = O.ref_lib()
    prev = R.__mind_blas_set_use_avx2(0)
    rng = np.random.default_rng(0x71)
    try:
        for avx2 in (0, 1):
            R.__mind_blas_set_use_avx2(avx2)
            for n in list(range(0, 18)) + [4093, 65541]:
                u = rng.integers(0, 1 << 32, 2 * n, dtype=np.uint64).astype(np.uint32)
                u = np.where((u & 0x7f800000) == 0x7f800000, u & 0xbfffffff, u)   # finite, any exponent
                for a, b in (O.gen_f32_unit(0xF32 ^ n, n, n), _f32_special_pair(n, n),
                             (u[:n].view(np.float32).copy(), u[n:].view(np.float32).copy())):
                    pa, pb = (a.ctypes.data, b.ctypes.data) if n else (0, 0)
                    with np.errstate(all="ignore"):
                        assert O.dist_f32_bits(O.F32_L1, a, b) == R.__mind_blas_dot_l1_f32(pa, pb, n)
                        assert O.dist_f32_bits(O.F32_LINF, a, b) == R.__mind_blas_dot_linf_f32(pa, pb, n)
    finally:
        R.__mind_blas_set_use_avx2(prev)


def test_f32_metric_closed_forms():
    rng = np.random.default_rng(0x72)
    with np.errstate(all="ignore"):
        for n in (1, 7, 8, 9, 64, 1000, 4093):
            a = rng.standard_normal(n).astype(np.float32) * np.float32(1e3)
            b = rng.standard_normal(n).astype(np.float32)
            d = np.abs(a - b)
            # L-inf is a max: exact, whatever the order
            assert O.dist_f32_bits(O.F32_LINF, a, b) == int(d.max().view(np.uint32))
            assert O.dist_f32_bits(O.F32_LINF_V, a, b) == int(d.max().view(np.uint32))
            # a vector against itself
            assert O.dist_f32_bits(O.F32_L1, a, a) == 0 and O.dist_f32_bits(O.F32_LINF, a, a) == 0
            # L1 against zero: the pinned 8-lane fold of |a|, against an
            # independent numpy evaluation of that order
            z = np.zeros(n, np.float32)
            lanes = np.zeros(8, np.float32)
            m = n // 8 * 8
            for i in range(0, m, 8):
                lanes = (lanes + np.abs(a[i:i + 8])).astype(np.float32)
            s = lanes[0]
            for j in range(1, 8):
                s = np.float32(s + lanes[j])
            for i in range(m, n):
                s = np.float32(s + np.abs(a[i]))
            assert O.dist_f32_bits(O.F32_L1, a, z) == int(np.float32(s).view(np.uint32))
            # within rounding of the float64 sum
            assert abs(float(np.float32(s)) - float(np.abs(a.astype(np.float64)).sum())) <= 1e-5 * float(np.abs(a).sum())
        # NaN: Track A skips a NaN difference, the vector twin returns NaN
        a = np.array([1.0, np.nan, -3.0, 2.0], np.float32)
        b = np.array([0.0, 0.0, 0.0, np.inf], np.float32)
        assert O.dist_f32_bits(O.F32_LINF, a, b) == int(np.float32(np.inf).view(np.uint32))
        assert O.dist_f32_bits(O.F32_LINF_V, a, b) == 0x7fc00000
        assert O.dist_f32_bits(O.F32_LINF, a[[0, 2]], b[[0, 2]]) == int(np.float32(3.0).view(np.uint32))
        assert np.isnan(np.uint32(O.dist_f32_bits(O.F32_L1, a, b)).view(np.float32))
        # signed zero: |-0 - 0| is +0 under the sign-bit clear
        assert O.dist_f32_bits(O.F32_L1, np.array([-0.0], np.float32), np.array([0.0], np.float32)) == 0
        # the rows form is the single-vector form per row
        W = rng.standard_normal(5 * 37).astype(np.float32)
        x = rng.standard_normal(37).astype(np.float32)
        for op in (O.F32_DOT, O.F32_L1, O.F32_LINF, O.F32_LINF_V):
            y = O.rows_metric_f32_bits(op, W, x, 5, 37)
            assert [int(v) for v in y] == [O.dist_f32_bits(op, W[r * 37:(r + 1) * 37], x) for r in range(5)]


def test_f32_metric_golden_rejects_a_pairwise_fold():
    """A mistake the golden data catches: folding the 8 L1 lanes pairwise
    instead of left to right changes the bits of some reference case."""
    inputs, cases = _metric_golden()
    changed = 0
    with np.errstate(all="ignore"):
        for c in cases:
            if c["family"] in ("special", "nan") or c["len"] < 16:
                continue
            a, b = inputs(c["family"], c["seed"], c["len"])
            d = np.abs(a - b)
            m = len(d) // 8 * 8
            lanes = np.zeros(8, np.float32)
            for i in range(0, m, 8):
                lanes = (lanes + d[i:i + 8]).astype(np.float32)
            p = ((lanes[0] + lanes[1]) + (lanes[2] + lanes[3])) + ((lanes[4] + lanes[5]) + (lanes[6] + lanes[7]))
            s = np.float32(p)
            for i in range(m, len(d)):
                s = np.float32(s + d[i])
            changed += int(np.float32(s).view(np.uint32)) != c["l1_scalar"]
    assert changed > 0


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


@pytest.mark.skipif(not O.ref_built(), reason="oracle/_ref not built (reference tree absent)")
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


@pytest.mark.skipif(not O.ref_built(), reason="oracle/_ref not built (reference tree absent)")
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
        for (m, k, n) in [(1, 1, 1), (13, 77, 19), (70, 600, 150), (130, 1100, 40), (256, 256, 256), (67, 1030, 129)]:
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


# ------------------------------------------------------------------ Q16 FFT

def _fft_harness_case(canaries):
    c = canaries["fft_q16_256_harness"]
    re, im = O.fft_input_harness(c["seed"], c["n"])
    return c, re, im, O.fft_twiddles(c["n"])


def test_fft_golden_harness_hash(canaries):
    c, re, im, tw = _fft_harness_case(canaries)
    r, i = O.fft_q16(re, im, tw, c["logn"])
    assert format(O.fnv1a_i64(r) ^ O.fnv1a_i64(i), "016x") == c["fnv_xor"]


def _py_fft(re, im, tw, logn, mistake=None):
    """Independent pure-Python restatement (Python ints, wrapped to int64),
    with an optional planted mistake."""
    n = 1 << logn
    m64 = (1 << 64) - 1

    def s64(v):
        v &= m64
        return v - (1 << 64) if v >> 63 else v

    def qmul(a, b):
        return s64(a * b) >> 16

    re, im = [int(v) for v in re], [int(v) for v in im]
    if mistake != "no_bitrev":
        perm = [int(format(i, f"0{logn}b")[::-1], 2) if logn else 0 for i in range(n)]
        re, im = [re[p] for p in perm], [im[p] for p in perm]
    span = 2
    while span <= n:
        h = span // 2
        for base in range(0, n, span):
            for j in range(h):
                a, b = base + j, base + j + h
                if span == 2:
                    tr, ti = re[b], im[b]
                else:
                    k = (j * (n // span) + (1 if mistake == "tw_index" else 0)) % (n // 2)
                    wr, wi = int(tw[2 * k]), int(tw[2 * k + 1])
                    if mistake == "conj":
                        wi = -wi
                    if mistake == "round":
                        tr = s64(wr * re[b] - wi * im[b]) >> 16
                        ti = s64(wr * im[b] + wi * re[b]) >> 16
                    else:
                        tr = s64(qmul(wr, re[b]) - qmul(wi, im[b]))
                        ti = s64(qmul(wr, im[b]) + qmul(wi, re[b]))
                re[a], im[a], re[b], im[b] = (s64(re[a] + tr), s64(im[a] + ti), s64(re[a] - tr), s64(im[a] - ti))
        span *= 2
    return np.array(re, np.int64), np.array(im, np.int64)


def test_fft_python_restatement_and_planted_mistakes(canaries):
    # the hash rejects a missing bit reversal, a shifted twiddle index, the
    # conjugate twiddle and a floor after the sum instead of per product
    c, re, im, tw = _fft_harness_case(canaries)

    def h(v):
        return format(O.fnv1a_i64(v[0]) ^ O.fnv1a_i64(v[1]), "016x")

    assert h(_py_fft(re, im, tw, 8)) == c["fnv_xor"]
    for mistake in ("no_bitrev", "tw_index", "conj", "round"):
        assert h(_py_fft(re, im, tw, 8, mistake)) != c["fnv_xor"], mistake
    rng = np.random.default_rng(5)
    for logn in (0, 1, 2, 3, 5, 7):
        n = 1 << logn
        x = rng.integers(-(1 << 40), 1 << 40, (2, n))
        t = O.fft_twiddles(n) if n >= 2 else np.zeros(2, np.int64)
        got = O.fft_q16(x[0], x[1], t, logn)
        want = _py_fft(x[0], x[1], t, logn)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), logn


@pytest.mark.skipif(not O.fft_ref_built(), reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("logn", list(range(1, 14)))
def test_fft_matches_reference_c_live(logn):
    # bench/fft/fft_ref.c (span-2 stage unpeeled) equals the peeled kernel
    # whenever tw[0] = (65536, 0) and |x| < 2^47; inputs below 2^30 keep
    # every intermediate far from int64 overflow (the C file's products are
    # signed, so overflow would be undefined there)
    R = O.fft_ref_lib()
    n = 1 << logn
    rng = np.random.default_rng(logn)
    tws = [O.fft_twiddles(n)]
    rt = rng.integers(-(1 << 20), 1 << 20, n).astype(np.int64)
    rt[0], rt[1] = 65536, 0
    tws.append(rt)
    for tw in tws:
        for x in (O.fft_input_harness(0x1234567 + logn, n), O.fft_input_lcg(0x12345678 ^ logn, n),
                  tuple(rng.integers(-(1 << 30), 1 << 30, (2, n)))):
            a, b = np.array(x[0], np.int64), np.array(x[1], np.int64)
            got = O.fft_q16(a, b, tw, logn)
            R.fft256_c(a.ctypes.data, b.ctypes.data, tw.ctypes.data, logn, n)
            assert np.array_equal(got[0], a) and np.array_equal(got[1], b)


def test_fft_close_to_the_float_dft():
    # each stage floors every product (error < 1 unit per product) on top of
    # twiddles rounded to 2^-16: the result is within a few units * n of the
    # exact DFT of the input; a wrong index, sign or permutation is off by
    # O(|X|)
    for logn in (2, 4, 8, 10):
        n = 1 << logn
        re, im = O.fft_input_lcg(0xF0F0 + logn, n)
        got = O.fft_q16(re, im, O.fft_twiddles(n), logn)
        X = np.fft.fft(re.astype(np.float64) + 1j * im.astype(np.float64))
        err = np.max(np.abs((got[0] + 1j * got[1]) - X))
        bound = 4.0 * logn * (n + np.max(np.abs(X)) * 2.0 ** -16)
        assert err <= bound, (logn, err, bound)
        assert np.max(np.abs(X)) > 100 * bound


@pytest.mark.skipif(not O.fft_ref_built(), reason="oracle/_ref not built (reference tree absent)")
def test_fft_peeled_stage_differs_from_the_c_file_when_tw0_is_not_one():
    # The kernel this build follows (examples/fft_q16.mind) peels the span-2
    # stage as a plain add / subtract; bench/fft/fft_ref.c multiplies by tw[0].
    # They agree for the standard table (tw[0] = (65536, 0)); with another
    # tw[0] they differ, and this build returns the peeled kernel's values.
    n, logn = 16, 4
    tw = O.fft_twiddles(n)
    tw[0], tw[1] = 32768, 0
    re, im = O.fft_input_lcg(7, n)
    a, b = re.copy(), im.copy()
    O.fft_ref_lib().fft256_c(a.ctypes.data, b.ctypes.data, tw.ctypes.data, logn, n)
    got = O.fft_q16(re, im, tw, logn)
    assert not np.array_equal(got[0], a)
    want = _py_fft(re, im, tw, logn)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_fft_rejects_non_power_of_two():
    with pytest.raises(ValueError):
        O.fft_q16(np.zeros(6, np.int64), np.zeros(6, np.int64), np.zeros(6, np.int64), 2)


def test_fft_int32_growth_bound():
    # The GPU's int32 path relies on: with |w| <= 2^16, |qmul(w, x)| <= |x|;
    # the span-2 stage at most doubles the largest magnitude and each later
    # stage at most triples it, so inputs within (2^31 - 1) // (2 * 3^(logn-1))
    # keep every intermediate in int32.  Checked on edge values and on
    # instrumented transforms of worst-sign inputs at exactly the bound.
    edges = [0, 1, -1, 2, -2, 65535, -65535, 65536, -65536, 3, -3, 12345, -12345]
    for w in edges:
        for x in [0, 1, -1, 7, -7, (1 << 31) - 1, -(1 << 31), 123456789, -123456789]:
            assert abs((w * x) >> 16) <= abs(x), (w, x)
    for logn in (1, 2, 5, 8, 11):
        n = 1 << logn
        bound = (2 ** 31 - 1) // (2 * 3 ** (logn - 1))
        tw = [int(v) for v in O.fft_twiddles(n)] if n >= 2 else [65536, 0]
        rng = np.random.default_rng(logn)
        for trial in range(3):
            re = [bound * int(s) for s in rng.choice([-1, 1], n)]
            im = [bound * int(s) for s in rng.choice([-1, 1], n)]
            perm = [int(format(i, f"0{logn}b")[::-1], 2) for i in range(n)]
            re, im = [re[p] for p in perm], [im[p] for p in perm]
            peak, span, stage = bound, 2, 0
            while span <= n:
                h = span // 2
                for base in range(0, n, span):
                    for j in range(h):
                        a, b = base + j, base + j + h
                        if span == 2:
                            tr, ti = re[b], im[b]
                        else:
                            k = j * (n // span)
                            wr, wi = tw[2 * k], tw[2 * k + 1]
                            tr = ((wr * re[b]) >> 16) - ((wi * im[b]) >> 16)
                            ti = ((wr * im[b]) >> 16) + ((wi * re[b]) >> 16)
                        re[a], im[a], re[b], im[b] = re[a] + tr, im[a] + ti, re[a] - tr, im[a] - ti
                stage += 1
                m = max(max(abs(v) for v in re), max(abs(v) for v in im))
                assert m <= peak * (2 if stage == 1 else 3), (logn, stage)
                peak = m
                assert m <= 2 ** 31 - 1, (logn, stage, m)
                span *= 2
