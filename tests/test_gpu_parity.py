"""GPU tier: the HIP kernels, called through the C ABI, are bit-identical to
the oracle (and to the reference's committed golden hashes).

Sizes: small and ragged shapes against the full oracle; BASELINE-size
configs against oracle rows sampled across the output (plus repeat
stability), so the oracle work stays within seconds.
"""
import ctypes
import json
import os
import sys

import numpy as np
import pytest

import mind_amd as M
import oracle as O

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def note(msg):
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def h32(v):
    return O.sha256_i32_le(v)


def addr(a):
    return a.ctypes.data


def call6(name, a, b, c, m, k, n):
    note(f"{name} m={m} k={k} n={n}")
    rc = getattr(M.lib(), name)(addr(a), addr(b), addr(c), m, k, n)
    assert rc == 0, (rc, M.last_error())


def call5(name, w, x, y, r, c):
    note(f"{name} rows={r} cols={c}")
    rc = getattr(M.lib(), name)(addr(w), addr(x), addr(y), r, c)
    assert rc == 0, (rc, M.last_error())


# ------------------------------------------------------------------ golden canaries through the ABI

@pytest.mark.parametrize("sym", ["gemmi8", "gemmi8mt", "__mind_blas_matmul_mm_i8_v", "__mind_blas_matmul_mm_i8_mt_v"])
def test_canary_gemm_i8(canaries, sym):
    w = canaries["workloads"]["gemm-i8-64x64x64"]
    a, b = O.gen_i8(w["seed"], 64 * 64, 64 * 64)
    c = np.full(64 * 64, 0x5A5A5A5A, np.int32)
    call6(sym, a, b, c, 64, 64, 64)
    assert h32(c) == w["avx2"]


@pytest.mark.parametrize("sym", ["gemmqmm", "__mind_blas_matmul_mm_q16_v", "__mind_blas_matmul_mm_q16_mt_v", "gemmq"])
def test_canary_gemm_q16(canaries, sym):
    w = canaries["workloads"]["gemm-q16-fused-64x64x64"]
    a, b = O.gen_q16(w["seed"], 64 * 64, 64 * 64)
    if sym == "gemmq":   # the gemv-composed form takes B^T [N][K]
        b = np.ascontiguousarray(b.reshape(64, 64).T).ravel()
    c = np.zeros(64 * 64, np.int32)
    call6(sym, a, b, c, 64, 64, 64)
    assert h32(c) == w["avx2"]


@pytest.mark.parametrize("sym", ["mmq", "__mind_blas_matmul_rmajor_q16_v", "gemvq", "__mind_blas_gemv_q16_mt"])
def test_canary_gemv_q16(canaries, sym):
    w = canaries["workloads"]["gemv-q16-256x256"]
    W, x = O.gen_q16(w["seed"], 256 * 256, 256)
    y = np.zeros(256, np.int32)
    call5(sym, W, x, y, 256, 256)
    assert h32(y) == w["avx2"]


@pytest.mark.parametrize("sym", ["mmi16", "__mind_blas_matmul_rmajor_i16_v"])
def test_canary_gemv_i16(canaries, sym):
    w = canaries["workloads"]["gemv-i16-256x256"]
    W, x = O.gen_i16(w["seed"], 256 * 256, 256)
    y = np.zeros(256, np.int32)
    call5(sym, W, x, y, 256, 256)
    assert h32(y) == w["avx2"]


def test_canary_dot_l2_q16(canaries):
    w = canaries["workloads"]["dot-l2-q16"]
    a, b = O.gen_q16(w["seed"], w["length"], w["length"])
    note("dotq len=65536")
    assert O.sha256_i64_le(M.lib().dotq(addr(a), addr(b), len(a))) == w["avx2"]


@pytest.mark.parametrize("sym", ["dotl1q", "__mind_blas_dot_l1_q16_v", "__mind_blas_dot_l1_q16"])
def test_canary_dot_l1_q16(canaries, sym):
    w = canaries["workloads"]["dot-l1-q16"]
    a, b = O.gen_q16(w["seed"], w["length"], w["length"])
    note(f"{sym} len=65536")
    assert O.sha256_i64_le(getattr(M.lib(), sym)(addr(a), addr(b), len(a))) == w["avx2"]


@pytest.mark.parametrize("sym", ["doti16", "__mind_blas_dot_i16_v"])
def test_canary_dot_i16(canaries, sym):
    w = canaries["workloads"]["dot-i16-4096"]
    a, b = O.gen_i16(w["seed"], w["length"], w["length"])
    note(f"{sym} len=4096")
    assert O.sha256_i64_le(getattr(M.lib(), sym)(addr(a), addr(b), len(a))) == w["avx2"]


# 16384 is the longest dot one block covers (a plain store of the sum);
# 16385 takes two blocks and the atomic
DOT_LENS = [0, 1, 3, 4, 5, 7, 8, 9, 17, 4093, 16383, 16384, 16385, 65536, 1 << 20]


@pytest.mark.parametrize("n", DOT_LENS)
@pytest.mark.parametrize("fam", ["q16", "full", "extreme"])
def test_dots_vs_oracle(n, fam):
    rng = np.random.default_rng(n * 7 + len(fam))
    ext = np.array([2147483647, -2147483648, -2147483647, 0, 1, -1, 65535, -65536], np.int32)
    if fam == "q16":
        a, b = O.gen_q16(0xD07 ^ n, n, n)
    elif fam == "full":
        a, b = O.gen_q16(0xD08 ^ n, n, n, shift=0)
    else:
        a, b = ext[rng.integers(0, 8, n)], ext[rng.integers(0, 8, n)]
    note(f"dots {fam} n={n}")
    assert M.dot_q16(a, b) == O.dot_q16(a, b)
    assert M.dot_l1_q16(a, b) == O.dot_l1_q16(a, b)
    a16, b16 = (a >> 16).astype(np.int16), a.astype(np.int16)
    assert M.dot_i16(a16, b16) == O.dot_i16(a16, b16)
    if n >= 2:   # misaligned (element offset 1): the unvectorised path
        assert M.dot_l1_q16(a[1:], b[1:]) == O.dot_l1_q16(a[1:], b[1:])
        assert M.dot_q16(a[1:], b[:-1]) == O.dot_q16(a[1:], b[:-1])
        assert M.dot_i16(a16[1:], b16[1:]) == O.dot_i16(a16[1:], b16[1:])


@pytest.mark.parametrize("n", [100003, 16384, 5])
def test_dot_dev_entry_point(n):
    a, b = O.gen_q16(0xDE7, n, n, shift=0)
    a16, b16 = O.gen_i16(0xDE8, n, n)
    s = M.Stream()
    out = M.DeviceBuffer(4)
    cases = [(M.DET_DOT_Q16, a, b, O.dot_q16(a, b)), (M.DET_DOT_L1_Q16, a, b, O.dot_l1_q16(a, b)),
             (M.DET_DOT_I16, a16, b16, O.dot_i16(a16, b16))]
    for op, x, y, want in cases:
        dx, dy = M.DeviceBuffer.from_array(x), M.DeviceBuffer.from_array(y)
        for _ in range(2):   # the output is overwritten, not accumulated
            out.fill(0x5A)
            note(f"det_dot_dev op={op} n={n}")
            M.check(M.lib().det_dot_dev(op, dx.ptr, dy.ptr, n, out.ptr, s.ptr))
            s.sync()
            assert int(out.to_array(np.int32, (1,))[0]) == want
        dx.free(); dy.free()
    assert M.lib().det_dot_dev(7, out.ptr, out.ptr, 4, out.ptr, s.ptr) == M.DET_ERR_ARG
    assert M.lib().dotl1q(0, 0, 5) == 0 and M.lib().doti16(addr(a16), addr(b16), 0) == 0


def test_canary_matmul_det_bench(canaries):
    g = canaries["matmul_det_bench_256"]
    idx = np.arange(256 * 256)
    A = (((idx + 1) % 7) - 3).astype(np.int8)
    B = (((idx + 2) % 7) - 3).astype(np.int8)
    C = np.zeros(256 * 256, np.int32)
    call6("gemmi8", A, B, C, 256, 256, 256)
    import hashlib
    d = hashlib.sha256(C.astype("<i4").tobytes()).digest()
    assert [int.from_bytes(d[i:i + 8], "little", signed=True) for i in range(0, 32, 8)] == g["digest_words_le_i64"]


def test_dot_q16_reference_vectors():
    d = json.load(open(os.path.join(GOLD, "dot_q16_ref.json")))
    ext = np.array([2147483647, -2147483647, -2147483648, 65535, -65536, 1, -1, 0], np.int32)
    for c in d["cases"]:
        if c["family"] == "extreme":
            ia, ib = O.gen_q16(c["seed"], c["len"], c["len"], shift=29)
            a, b = ext[ia & 7], ext[ib & 7]
        else:
            a, b = O.gen_q16(c["seed"], c["len"], c["len"], shift={"ref12": 12, "q4": 13, "full": 0}[c["family"]])
        note(f"dot_q16 family={c['family']} len={c['len']}")
        assert M.dot_q16(a, b) == c["scalar"], c


# ------------------------------------------------------------------ strict-FP f32 dot / row matmul

def f32_same(got, want):
    """Bit equality, except that a NaN result only has to be a NaN: the
    reference's own NaN bits differ by substrate (x86 creates 0xffc00000,
    AArch64 and gfx950 0x7fc00000), so no bit pattern is pinned for it."""
    got = np.asarray(got, np.float32).reshape(-1)
    want = np.asarray(want, np.float32).reshape(-1)
    gn, wn = np.isnan(got), np.isnan(want)
    return bool(np.array_equal(gn, wn) and np.array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32)))


def bits_to_f32(v):
    assert 0 <= v < (1 << 32), v   # the reference zero-extends the f32 bits
    return np.array([v], np.uint32).view(np.float32)


@pytest.mark.parametrize("sym", ["dotf32", "__mind_blas_dot_f32", "__mind_blas_dot_f32_v"])
def test_canary_dot_f32(canaries, sym):
    w = canaries["workloads"]["dot-f32-v-4093"]
    a, b = O.gen_f32_unit(w["seed"], w["length"], w["length"])
    note(f"{sym} len={w['length']}")
    assert O.sha256_i64_le(getattr(M.lib(), sym)(addr(a), addr(b), len(a))) == w["avx2"]


@pytest.mark.parametrize("sym", ["mmf32", "__mind_blas_matmul_rmajor_f32", "__mind_blas_matmul_rmajor_f32_v"])
def test_canary_matmul_f32(canaries, sym):
    w = canaries["workloads"]["matmul-f32-v-64x64"]
    r, c = w["rows"], w["cols"]
    W, x = O.gen_f32_unit(w["seed"], r * c, c)
    y = np.full(r, np.nan, np.float32)
    call5(sym, W, x, y, r, c)
    import hashlib
    assert hashlib.sha256(y.view("<u4").tobytes()).hexdigest() == w["avx2"]


F32_LENS = list(range(0, 18)) + [63, 64, 65, 4093, 65541, 1 << 20]


def f32_family(fam, seed, n):
    rng = np.random.default_rng(seed)
    if fam == "unit":
        return O.gen_f32_unit(seed, n, n)
    if fam == "wide":   # finite values over the whole exponent range, subnormals included
        u = rng.integers(0, 1 << 32, 2 * n, dtype=np.uint64).astype(np.uint32)
        u = np.where((u & 0x7f800000) == 0x7f800000, u & 0xbfffffff, u)
        f = u.view(np.float32)
        return f[:n].copy(), f[n:].copy()
    # special: signed zeros, subnormals, extremes and infinities (inf * 0 and
    # inf - inf make NaN along the way)
    sp = np.array([0.0, -0.0, 1.0, -1.0, 1e-45, -1e-45, 1.1754942e-38, 3.4028235e38, -3.4028235e38,
                   np.inf, -np.inf, 0.5, 3.0, 1e-20, 1e20, -2.5], np.float32)
    return sp[rng.integers(0, len(sp), n)], sp[rng.integers(0, len(sp), n)]


@pytest.mark.parametrize("n", F32_LENS)
@pytest.mark.parametrize("fam", ["unit", "wide", "special"])
def test_dot_f32_vs_oracle(n, fam):
    a, b = f32_family(fam, 0xF32 ^ (n * 131) ^ len(fam), n)
    note(f"dot_f32 {fam} n={n}")
    assert f32_same(bits_to_f32(M.dot_f32_bits(a, b)), bits_to_f32(O.dot_f32_bits(a, b)))
    out = np.full(1, np.nan, np.float32)
    assert M.lib().det_dot_f32(addr(a), addr(b), n, addr(out)) == 0
    assert f32_same(out, bits_to_f32(O.dot_f32_bits(a, b)))
    if n >= 2:   # element offset 1
        assert f32_same(bits_to_f32(M.dot_f32_bits(a[1:], b[:-1])), bits_to_f32(O.dot_f32_bits(a[1:], b[:-1])))


F32_METRIC_SYMS = [("__mind_blas_dot_l1_f32", O.F32_L1), ("__mind_blas_dot_l1_f32_v", O.F32_L1),
                   ("__mind_blas_dot_linf_f32", O.F32_LINF), ("__mind_blas_dot_linf_f32_v", O.F32_LINF_V)]


def test_f32_metric_reference_vectors():
    """Every symbol on the committed outputs of the reference's own L1 / L-inf
    (tests/golden/dot_f32_metric_ref.json, the scalar dispatch path's
    outputs; the vector twins equal them except L-inf_v on NaN, which
    follows the oracle)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("mk_f32_metric", os.path.join(GOLD, "make_ref_f32_metric_vectors.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    cases = json.load(open(os.path.join(GOLD, "dot_f32_metric_ref.json")))["cases"]
    with np.errstate(all="ignore"):
        for c in cases:
            a, b = mod.inputs(c["family"], c["seed"], c["len"], c.get("pos"))
            n = c["len"]
            for sym, op in F32_METRIC_SYMS:
                note(f"{sym} {c['family']} n={n}")
                got = getattr(M.lib(), sym)(addr(a) if n else 0, addr(b) if n else 0, n)
                want = {O.F32_L1: c["l1_scalar"], O.F32_LINF: c["linf_scalar"]}.get(op)
                if want is None:
                    want = O.dist_f32_bits(op, a, b)
                assert f32_same(bits_to_f32(got), bits_to_f32(want)), (sym, c["family"], n, hex(got), hex(want))
                assert M.lib().det_last_error() in (None, b"")


@pytest.mark.parametrize("n", F32_LENS)
@pytest.mark.parametrize("fam", ["unit", "wide", "special"])
def test_f32_metrics_vs_oracle(n, fam):
    a, b = f32_family(fam, 0xF38 ^ (n * 137) ^ len(fam), n)
    with np.errstate(all="ignore"):
        for sym, op in F32_METRIC_SYMS:
            note(f"{sym} {fam} n={n}")
            got = getattr(M.lib(), sym)(addr(a) if n else 0, addr(b) if n else 0, n)
            assert f32_same(bits_to_f32(got), bits_to_f32(O.dist_f32_bits(op, a, b))), (sym, hex(got))


F32_METRIC_ROWS = [(1, 1), (3, 5), (9, 100), (17, 256), (70, 777), (4099, 1024), (5, 65541), (2, 265)]


@pytest.mark.parametrize("rows,cols", F32_METRIC_ROWS, ids=[f"{r}x{c}" for r, c in F32_METRIC_ROWS])
def test_rows_metric_f32_vs_oracle(rows, cols):
    """One query against many rows, host and device entry points, every
    metric and input family (cols % 4 == 0 takes the LDS DMA kernel)."""
    s = M.Stream()
    for fam in ("unit", "wide", "special"):
        W, _ = f32_family(fam, 0xF39 ^ rows * 7 ^ cols, rows * cols)
        x, _ = f32_family(fam, 0xF3A ^ rows ^ cols * 5, cols)
        dW, dx, dy = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(x), M.DeviceBuffer(4 * rows)
        for op in (O.F32_DOT, O.F32_L1, O.F32_LINF, O.F32_LINF_V):
            with np.errstate(all="ignore"):
                want = O.rows_metric_f32_bits(op, W, x, rows, cols).view(np.float32)
            note(f"det_rows_metric_f32[_dev] op={op} {fam} rows={rows} cols={cols}")
            y = np.full(rows, np.nan, np.float32)
            M.check(M.lib().det_rows_metric_f32(op, addr(W), addr(x), addr(y), rows, cols))
            assert f32_same(y, want), (fam, op)
            dy.fill(0x7F)
            M.check(M.lib().det_rows_metric_f32_dev(op, dW.ptr, dx.ptr, dy.ptr, rows, cols, s.ptr))
            s.sync()
            assert f32_same(dy.to_array(np.float32, (rows,)), want), (fam, op)
        for buf in (dW, dx, dy):
            buf.free()
    s.destroy()


def test_rows_metric_f32_arguments():
    L = M.lib()
    y = np.full(3, np.nan, np.float32)
    assert L.det_rows_metric_f32(4, 0, 0, addr(y), 3, 5) == M.DET_ERR_ARG
    assert L.det_rows_metric_f32(-1, 0, 0, addr(y), 3, 5) == M.DET_ERR_ARG
    assert L.det_rows_metric_f32(O.F32_L1, 0, 0, addr(y), 3, 0) == 0 and not np.any(y.view(np.uint32))
    assert L.det_rows_metric_f32(O.F32_L1, 0, 0, 0, 0, 5) == 0
    assert L.det_rows_metric_f32(O.F32_L1, 0, 0, addr(y), 3, 5) == M.DET_ERR_ARG
    for sym, _ in F32_METRIC_SYMS:
        assert getattr(L, sym)(0, 0, 16) == 0 and getattr(L, sym)(addr(y), addr(y), 0) == 0


# cols % 4 == 0 (16-byte rows) take the LDS DMA kernel: one chunk is 256
# floats, so 4, 8, 100, 252 and 1000 end in a partial chunk, 256 / 2048 are
# whole chunks, 260 / 772 add a tail past whole chunks; row counts that are
# not a multiple of 8 leave dead rows in the last wave.  Other widths take the
# register-ring kernel (its ring holds 32 steps: 33 * 8 + 1 = 265 columns
# cross one lap).
F32_MM = [(1, 1), (1, 9), (3, 5), (7, 8), (33, 17), (64, 64), (31, 1000), (1000, 31), (4097, 33), (5, 65541),
          (2048, 2048), (8, 4), (3, 8), (9, 100), (13, 252), (17, 256), (5, 260), (11, 772), (4099, 1024),
          (2, 265), (70, 777), (1, 1 << 18)]


@pytest.mark.parametrize("rows,cols", F32_MM, ids=[f"{r}x{c}" for r, c in F32_MM])
def test_matmul_f32_vs_oracle(rows, cols):
    for fam in ("unit", "wide", "special"):
        W, _ = f32_family(fam, 0xF33 ^ rows * 7 ^ cols, rows * cols)
        x, _ = f32_family(fam, 0xF34 ^ rows ^ cols * 5, cols)
        note(f"matmul_f32 {fam} rows={rows} cols={cols}")
        y = M.matmul_rmajor_f32(W.reshape(rows, cols), x)
        assert f32_same(y, O.matmul_rmajor_f32(W, x, rows, cols)), fam


def test_matmul_f32_unaligned_operands_take_the_register_kernel():
    # device operands 4 bytes off a 16-byte boundary: the DMA kernel needs
    # 16-byte rows, so the register-ring kernel runs; same bits either way
    rows, cols = 517, 1024
    W, x = O.gen_f32_unit(0xF37, rows * cols + 1, cols + 1)
    want = O.matmul_rmajor_f32(W[1:], x[1:], rows, cols)
    s = M.Stream()
    dW, dx, dy = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(x), M.DeviceBuffer(4 * rows)
    for wo, xo in ((4, 0), (0, 4), (4, 4)):
        Wv = W[wo // 4:wo // 4 + rows * cols]
        xv = x[xo // 4:xo // 4 + cols]
        dy.fill(0x7F)
        note(f"det_matmul_rmajor_f32_dev rows={rows} cols={cols} W+{wo} x+{xo}")
        M.check(M.lib().det_matmul_rmajor_f32_dev(dW.ptr + wo, dx.ptr + xo, dy.ptr, rows, cols, s.ptr))
        s.sync()
        assert f32_same(dy.to_array(np.float32, (rows,)), O.matmul_rmajor_f32(Wv, xv, rows, cols))
    M.check(M.lib().det_matmul_rmajor_f32_dev(dW.ptr + 4, dx.ptr + 4, dy.ptr, rows, cols, s.ptr))
    s.sync()
    assert f32_same(dy.to_array(np.float32, (rows,)), want)
    dW.free(); dx.free(); dy.free()


def test_matmul_f32_dev_entry_point():
    rows, cols = 3001, 777
    W, x = O.gen_f32_unit(0xF35, rows * cols, cols)
    want = O.matmul_rmajor_f32(W, x, rows, cols)
    s = M.Stream()
    dW, dx, dy = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(x), M.DeviceBuffer(4 * rows)
    for _ in range(2):
        dy.fill(0x7F)
        note(f"det_matmul_rmajor_f32_dev rows={rows} cols={cols}")
        M.check(M.lib().det_matmul_rmajor_f32_dev(dW.ptr, dx.ptr, dy.ptr, rows, cols, s.ptr))
        s.sync()
        assert f32_same(dy.to_array(np.float32, (rows,)), want)
    # empty shapes launch nothing and leave y alone
    assert M.lib().det_matmul_rmajor_f32_dev(dW.ptr, dx.ptr, dy.ptr, 0, cols, s.ptr) == 0
    assert M.lib().det_matmul_rmajor_f32_dev(dW.ptr, dx.ptr, dy.ptr, rows, 0, s.ptr) == 0
    s.sync()
    assert f32_same(dy.to_array(np.float32, (rows,)), want)
    assert M.lib().det_matmul_rmajor_f32_dev(dW.ptr, dx.ptr, dy.ptr, -1, cols, s.ptr) == M.DET_ERR_ARG
    assert M.lib().det_matmul_rmajor_f32_dev(0, dx.ptr, dy.ptr, rows, cols, s.ptr) == M.DET_ERR_ARG
    dW.free(); dx.free(); dy.free()


def test_f32_null_and_empty_conventions():
    # mind_intrinsics.c:1418-1427: -1 for a null pointer, 0 (y untouched) for
    # an empty shape; the vector twin returns 0 for both; a dot of length
    # <= 0 or with a null operand is +0.0 (bits 0)
    L = M.lib()
    W, x = O.gen_f32_unit(0xF36, 12, 4)
    y = np.full(3, 7.0, np.float32)
    assert L.__mind_blas_matmul_rmajor_f32(0, addr(x), addr(y), 3, 4) == -1
    assert L.__mind_blas_matmul_rmajor_f32(addr(W), addr(x), 0, 3, 4) == -1
    assert L.__mind_blas_matmul_rmajor_f32_v(0, addr(x), addr(y), 3, 4) == 0
    for sym in ("__mind_blas_matmul_rmajor_f32", "__mind_blas_matmul_rmajor_f32_v", "mmf32"):
        assert getattr(L, sym)(addr(W), addr(x), addr(y), 0, 4) == 0
        assert getattr(L, sym)(addr(W), addr(x), addr(y), 3, -2) == 0
    assert (y == 7.0).all()
    for sym in ("__mind_blas_dot_f32", "__mind_blas_dot_f32_v", "dotf32"):
        assert getattr(L, sym)(addr(W), addr(x), 0) == 0
        assert getattr(L, sym)(0, addr(x), 4) == 0
    out = np.full(1, 7.0, np.float32)
    assert L.det_dot_f32(addr(W), addr(x), 0, addr(out)) == 0 and out[0] == 0.0
    assert L.det_dot_f32(addr(W), addr(x), 4, 0) == M.DET_ERR_ARG
    assert L.det_matmul_rmajor_f32(addr(W), addr(x), addr(y), 3, -1) == M.DET_ERR_ARG


# ------------------------------------------------------------------ Q16 FFT

def test_canary_fft256_harness(canaries):
    c = canaries["fft_q16_256_harness"]
    re, im = O.fft_input_harness(c["seed"], c["n"])
    tw = O.fft_twiddles(c["n"])
    note("fft256 n=256 (harness.c signal)")
    assert M.lib().fft256(addr(re), addr(im), addr(tw), c["logn"], c["n"]) == 0
    assert format(O.fnv1a_i64(re) ^ O.fnv1a_i64(im), "016x") == c["fnv_xor"]


def _fft_oracle_batch(re, im, tw, logn):
    out_r, out_i = np.empty_like(re), np.empty_like(im)
    for f in range(re.shape[0]):
        out_r[f], out_i[f] = O.fft_q16(re[f], im[f], tw, logn)
    return out_r, out_i


# batch <= 512 with 32 <= n <= 2048 takes the few-transform kernel (one
# workgroup per transform), larger batches the batched one: both sides of
# that bound are covered (512 / 513, 1000).
FFT_CASES = [(logn, batch) for logn in range(0, 15) for batch in (1, 3, 37)] + [(8, 1000), (5, 513), (5, 512),
                                                                              (10, 512), (11, 9)]


@pytest.mark.parametrize("logn,batch", FFT_CASES, ids=[f"n{1 << l}_b{b}" for l, b in FFT_CASES])
def test_fft_vs_oracle(logn, batch):
    n = 1 << logn
    rng = np.random.default_rng(logn * 131 + batch)
    tw_std = O.fft_twiddles(n) if n >= 2 else np.zeros(2, np.int64)
    tw_rand = rng.integers(-(1 << 20), 1 << 20, max(n, 2)).astype(np.int64)
    for fam in ("q16", "wide", "full"):
        if fam == "q16":
            x = np.stack([np.concatenate(O.fft_input_lcg(0xF00 + f + logn, n)) for f in range(batch)])
        elif fam == "wide":
            x = rng.integers(-(1 << 40), 1 << 40, (batch, 2 * n))
        else:   # full int64 range: every add, product and shift wraps
            x = rng.integers(np.iinfo(np.int64).min, np.iinfo(np.int64).max, (batch, 2 * n), dtype=np.int64,
                             endpoint=True)
        re, im = np.ascontiguousarray(x[:, :n]), np.ascontiguousarray(x[:, n:])
        for tw in ((tw_std, tw_rand) if fam != "q16" else (tw_std,)):
            note(f"fft {fam} n={n} batch={batch}")
            got = M.fft_q16(re, im, tw, logn)
            want = _fft_oracle_batch(re, im, tw, logn)
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), (fam, logn)


def test_fft_dev_entry_point_and_workspace_path():
    s = M.Stream()
    for logn, batch in ((8, 4099), (12, 3), (13, 2)):
        n = 1 << logn
        x = np.random.default_rng(logn).integers(-(1 << 30), 1 << 30, (2, batch, n))
        re, im = np.ascontiguousarray(x[0]), np.ascontiguousarray(x[1])
        tw = O.fft_twiddles(n)
        sel = sorted({0, batch - 1, batch // 2})
        want = _fft_oracle_batch(re[sel], im[sel], tw, logn)
        dre, dim_, dtw = M.DeviceBuffer.from_array(re), M.DeviceBuffer.from_array(im), M.DeviceBuffer.from_array(tw)
        for rep in range(2):   # in place: the second call transforms the first call's output
            note(f"det_fft_q16_dev n={n} batch={batch} rep={rep}")
            M.check(M.lib().det_fft_q16_dev(dre.ptr, dim_.ptr, dtw.ptr, logn, n, batch, s.ptr))
            s.sync()
            gr = dre.to_array(np.int64, (batch, n))
            gi = dim_.to_array(np.int64, (batch, n))
            assert np.array_equal(gr[sel], want[0]) and np.array_equal(gi[sel], want[1])
            want = _fft_oracle_batch(want[0], want[1], tw, logn)
        want_ws = 0 if logn <= 11 else 16 * batch * n
        assert M.lib().det_fft_workspace_bytes(logn, batch) == want_ws
        dre.free(); dim_.free(); dtw.free()


def test_fft_out_of_place_and_path_choice():
    # det_fft_q16_oop_dev leaves the input alone; a block of transforms takes
    # the int32 path only when every input is within the growth bound, and a
    # batch that mixes small and large transforms, or sits exactly on the
    # bound, gives the oracle's integers either way
    s = M.Stream()
    logn, n, batch = 8, 256, 1000
    bound = (2 ** 31 - 1) // (2 * 3 ** 7)
    rng = np.random.default_rng(88)
    x = rng.integers(-bound, bound + 1, (2, batch, n))
    x[:, ::7] *= 1 << 20          # every 7th transform far outside the bound
    x[0, 3, 5], x[1, 4, 9] = bound, -bound
    x[0, 6, 1] = bound + 1        # just outside
    tw = O.fft_twiddles(n)
    re, im = np.ascontiguousarray(x[0]), np.ascontiguousarray(x[1])
    want = _fft_oracle_batch(re, im, tw, logn)
    sre, sim = M.DeviceBuffer.from_array(re), M.DeviceBuffer.from_array(im)
    dre, dim_, dtw = M.DeviceBuffer(re.nbytes), M.DeviceBuffer(im.nbytes), M.DeviceBuffer.from_array(tw)
    for rep in range(2):
        dre.fill(0x11)
        note(f"det_fft_q16_oop_dev n={n} batch={batch} rep={rep}")
        M.check(M.lib().det_fft_q16_oop_dev(sre.ptr, sim.ptr, dre.ptr, dim_.ptr, dtw.ptr, logn, n, batch, s.ptr))
        s.sync()
        assert np.array_equal(dre.to_array(np.int64, (batch, n)), want[0])
        assert np.array_equal(dim_.to_array(np.int64, (batch, n)), want[1])
        assert np.array_equal(sre.to_array(np.int64, (batch, n)), re)
    # a twiddle table with a component above 2^16 keeps every block on int64
    tw2 = tw.copy(); tw2[201] = 70000
    dtw2 = M.DeviceBuffer.from_array(tw2)
    small = np.ascontiguousarray(x[:, 1:64:7]) // (1 << 20)
    want2 = _fft_oracle_batch(small[0], small[1], tw2, logn)
    s0, s1 = M.DeviceBuffer.from_array(small[0]), M.DeviceBuffer.from_array(small[1])
    note("det_fft_q16_dev with a large twiddle component")
    M.check(M.lib().det_fft_q16_dev(s0.ptr, s1.ptr, dtw2.ptr, logn, n, small.shape[1], s.ptr))
    s.sync()
    assert np.array_equal(s0.to_array(np.int64, small[0].shape), want2[0])
    assert np.array_equal(s1.to_array(np.int64, small[1].shape), want2[1])
    assert M.lib().det_fft_q16_oop_dev(sre.ptr, sim.ptr, sre.ptr + 8, dim_.ptr, dtw.ptr, logn, n, batch,
                                       s.ptr) == M.DET_ERR_ARG
    for b in (sre, sim, dre, dim_, dtw, dtw2, s0, s1):
        b.free()


def test_fft_argument_conventions():
    L = M.lib()
    z = np.zeros(16, np.int64)
    assert L.fft256(addr(z), addr(z), addr(z), 3, 6) == M.DET_ERR_ARG        # n != 2^logn
    assert L.fft256(addr(z), addr(z), addr(z), 31, 1 << 31) == M.DET_ERR_ARG
    assert L.fft256(addr(z), addr(z), addr(z), 4, 0) == 0                     # nothing to do
    assert L.fft256(0, addr(z), addr(z), 4, 16) == M.DET_ERR_ARG
    assert L.det_fft_q16(addr(z), addr(z), addr(z), 4, 16, 0) == 0
    assert L.det_fft_q16(addr(z), addr(z), addr(z), 4, 16, (1 << 27) + 1) == M.DET_ERR_ARG   # > 2^31 points
    one_r, one_i = np.array([12345], np.int64), np.array([-7], np.int64)
    assert L.fft256(addr(one_r), addr(one_i), 0, 0, 1) == 0 and one_r[0] == 12345 and one_i[0] == -7


# ------------------------------------------------------------------ concurrency

# Host-pointer calls whose operand layout (inputs, output, each rounded up to
# 256 bytes) fits in 4 MiB travel through the library's pinned staging buffer
# and two copy kernels; in larger ones each buffer of 1 MiB or more goes
# through the pinned ring and smaller ones by DMA copies of the caller's buffer.
# One call on each side of the limit per family, checked whole, then the small
# one again (the pinned buffer keeps the large call's bytes past its end).
HOST_ROUTES = [("gemmi8", 768, 3 << 20), ("gemmi8", 1024, 6 << 20), ("gemvq", 2048, 2 << 20), ("gemvq", 8192, 8 << 20),
               ("dotq", 1 << 18, 2 << 20), ("dotq", 1 << 20, 8 << 20), ("fft256", 600, 3 << 20), ("fft256", 2000, 8 << 20)]


@pytest.mark.parametrize("sym,size,span", HOST_ROUTES, ids=[f"{s}-{n}" for s, n, _ in HOST_ROUTES])
def test_host_staging_routes(sym, size, span):
    L = M.lib()
    small = {"gemmi8": 64, "gemvq": 64, "dotq": 1000, "fft256": 3}[sym]
    for n in (size, small):
        note(f"host {sym} size={n} (layout ~{span >> 20} MiB when large)")
        if sym == "gemmi8":
            a, b = O.gen_i8(0x4A5 ^ n, n * n, n * n)
            c = np.full(n * n, 0x5A5A5A5A, np.int32)
            assert L.gemmi8(addr(a), addr(b), addr(c), n, n, n) == 0
            rows = _sample_rows(n, 16)
            np.testing.assert_array_equal(c.reshape(n, n)[rows], O.gemm_i8_rows(a, b, n, n, n, rows))
        elif sym == "gemvq":
            k = 256
            W, x = O.gen_q16(0x4A6 ^ n, n * k, k, shift=0)
            y = np.full(n, 0x5A5A5A5A, np.int32)
            assert L.gemvq(addr(W), addr(x), addr(y), n, k) == 0
            np.testing.assert_array_equal(y, O.gemv_q16(W, x, n, k))
        elif sym == "dotq":
            a, b = O.gen_q16(0x4A7 ^ n, n, n, shift=0)
            assert M.dot_q16(a, b) == O.dot_q16(a, b)
        else:
            logn, nfft = 8, 256
            x = np.random.default_rng(n).integers(-(1 << 30), 1 << 30, (2, n, nfft))
            re, im = np.ascontiguousarray(x[0]), np.ascontiguousarray(x[1])
            tw = O.fft_twiddles(nfft)
            got = M.fft_q16(re, im, tw, logn)
            sel = sorted({0, n // 2, n - 1})
            want = _fft_oracle_batch(re[sel], im[sel], tw, logn)
            assert np.array_equal(got[0][sel], want[0]) and np.array_equal(got[1][sel], want[1])


# Buffers of 1 MiB and more travel in pieces through a ring of four pinned
# 16 MiB chunks (the CPU copies a piece while earlier pieces' DMA runs; up to
# four threads share each host copy).  Cases: lengths that end mid-chunk,
# operands at element offsets (not 16-byte aligned), an output of more
# pieces than chunks (chunks refilled while others are in flight), ring and
# direct buffers in one call, and a teardown between calls (ring and copy
# threads rebuilt on the next call).
def test_host_ring_transfers():
    L = M.lib()

    def gemv_case(seed):
        rows, cols = 5003, 1001                      # W: 20.0 MB, 4 pieces
        W, x = O.gen_q16(seed, rows * cols + 1, cols + 1, shift=0)
        W, x = W[1:], x[1:]                          # 4 bytes off 16-byte alignment
        y = np.full(rows, 0x5A5A5A5A, np.int32)
        note(f"ring gemvq {rows}x{cols} seed={seed}")
        assert L.gemvq(addr(W), addr(x), addr(y), rows, cols) == 0
        np.testing.assert_array_equal(y, O.gemv_q16(W, x, rows, cols))

    gemv_case(0x91)
    # C = 67.2 MB: five 16 MiB pieces through four chunks; A and B (262 KB)
    # copied directly in the same call; checked whole (exact in float64)
    m, k, n = 4100, 64, 4100
    a, b = O.gen_i8(0x92, m * k, k * n)
    want = (a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)).astype(np.int32)
    buf = np.full(m * n + 1, 0x5A5A5A5A, np.int32)
    c = buf[1:]                                      # output 4 bytes off alignment
    note(f"ring gemmi8 {m}x{k}x{n} (C through the ring)")
    assert L.gemmi8(addr(a), addr(b), addr(c), m, k, n) == 0
    np.testing.assert_array_equal(c.reshape(m, n), want)
    assert buf[0] == 0x5A5A5A5A
    # both dot operands through the ring, odd length
    ln = 5 * (1 << 20) + 3
    da, db = O.gen_q16(0x93, ln + 1, ln, shift=0)
    note(f"ring dotq len={ln}")
    assert M.dot_q16(da[1:], db) == O.dot_q16(da[1:], db)
    # strict f32 rows: W 24 MB
    rows, cols = 3000, 2001
    Wf, xf = O.gen_f32_unit(0x94, rows * cols, cols)
    note(f"ring mmf32 {rows}x{cols}")
    assert f32_same(M.matmul_rmajor_f32(Wf.reshape(rows, cols), xf), O.matmul_rmajor_f32(Wf, xf, rows, cols))
    # FFT: re and im (4.3 MB each) in and out through the ring
    nb, nfft = 2100, 256
    x = np.random.default_rng(0x95).integers(-(1 << 30), 1 << 30, (2, nb, nfft))
    re, im = np.ascontiguousarray(x[0]), np.ascontiguousarray(x[1])
    tw = O.fft_twiddles(nfft)
    note(f"ring fft256 batch={nb}")
    got = M.fft_q16(re, im, tw, 8)
    sel = [0, 1, nb // 2, nb - 2, nb - 1]
    want_r, want_i = _fft_oracle_batch(re[sel], im[sel], tw, 8)
    assert np.array_equal(got[0][sel], want_r) and np.array_equal(got[1][sel], want_i)
    # teardown, then the ring and the copy threads again
    note("ring after det_shutdown")
    assert L.det_shutdown() == 0
    gemv_case(0x96)


def test_host_abi_concurrent_callers():
    # The host-pointer entry points are called from several threads at once
    # (ctypes releases the GIL): one device mutex serialises them, the
    # library stream and staging are shared, and every result must still be
    # the oracle's.  Q16 GEMM and the FFT also use the workspace arena.
    import threading
    L = M.lib()
    a8, b8 = O.gen_i8(0x7A1, 256 * 320, 320 * 192)
    c8 = O.gemm_i8(a8, b8, 256, 320, 192).ravel()
    aq, bq = O.gen_q16(0x7A2, 128 * 96, 96 * 256)
    cq = O.gemm_q16(aq, bq, 128, 96, 256).ravel()
    W, x = O.gen_q16(0x7A3, 1000 * 513, 513)
    y = O.gemv_q16(W, x, 1000, 513)
    fr, fi = O.fft_input_lcg(0x7A4, 256)
    tw = O.fft_twiddles(256)
    fw = O.fft_q16(fr, fi, tw, 8)
    da, db = O.gen_q16(0x7A5, 100003, 100003)
    dq = O.dot_q16(da, db)
    Wf, xf = O.gen_f32_unit(0x7A6, 300 * 777, 777)
    yf = O.matmul_rmajor_f32(Wf, xf, 300, 777)
    Wr, xr = O.gen_q16(0x7A7, 3000 * 1001, 1001)   # W 12 MB: the pinned ring
    yr = O.gemv_q16(Wr, xr, 3000, 1001)

    def job_i8():
        c = np.empty(256 * 192, np.int32)
        assert L.gemmi8(addr(a8), addr(b8), addr(c), 256, 320, 192) == 0
        return np.array_equal(c, c8)

    def job_q16():
        c = np.empty(128 * 256, np.int32)
        assert L.gemmqmm(addr(aq), addr(bq), addr(c), 128, 96, 256) == 0
        return np.array_equal(c, cq)

    def job_gemv():
        yy = np.empty(1000, np.int32)
        assert L.gemvq(addr(W), addr(x), addr(yy), 1000, 513) == 0
        return np.array_equal(yy, y)

    def job_fft():
        r, i = fr.copy(), fi.copy()
        assert L.fft256(addr(r), addr(i), addr(tw), 8, 256) == 0
        return np.array_equal(r, fw[0]) and np.array_equal(i, fw[1])

    def job_dot():
        return L.dotq(addr(da), addr(db), len(da)) == dq

    def job_f32():
        yy = np.empty(300, np.float32)
        assert L.mmf32(addr(Wf), addr(xf), addr(yy), 300, 777) == 0
        return np.array_equal(yy.view(np.uint32), yf.view(np.uint32))

    def job_ring():
        yy = np.empty(3000, np.int32)
        assert L.gemvq(addr(Wr), addr(xr), addr(yy), 3000, 1001) == 0
        return np.array_equal(yy, yr)

    jobs = [job_i8, job_q16, job_gemv, job_fft, job_dot, job_f32, job_ring]
    results, errors = [], []

    def run(job):
        try:
            for _ in range(5):
                results.append((job.__name__, job()))
        except Exception as e:   # reported below, not lost in the thread
            errors.append((job.__name__, repr(e)))

    note("host ABI: 7 threads x 5 calls")
    threads = [threading.Thread(target=run, args=(j,)) for j in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    assert len(results) == 35 and all(ok for _, ok in results), [r for r in results if not r[1]]


def test_device_arena_shared_by_two_streams():
    # det_matmul_q16_dev on two streams: both use the library's workspace
    # arena, ordered by its event, so interleaved calls of different shapes
    # must each give the oracle's C
    L = M.lib()
    shapes = [(1040, 160, 1024), (1024, 96, 1100)]   # limb kernel: both need the arena
    data = []
    for si, (m, k, n) in enumerate(shapes):
        a, b = O.gen_q16(0x7B0 + si, m * k, k * n, shift=0)
        data.append((m, k, n, M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b), M.DeviceBuffer(m * n * 4),
                     O.gemm_q16(a, b, m, k, n).ravel()))
    streams = [M.Stream(), M.Stream()]
    for rep in range(4):
        for si, (m, k, n, dA, dB, dC, _) in enumerate(data):
            dC.fill(0x33)
            note(f"det_matmul_q16_dev stream {si} rep {rep}")
            M.check(L.det_matmul_q16_dev(dA.ptr, dB.ptr, dC.ptr, m, k, n, streams[si].ptr))
        for si, (m, k, n, dA, dB, dC, want) in enumerate(data):
            streams[si].sync()
            assert np.array_equal(dC.to_array(np.int32, (m * n,)), want), (si, rep)
    for _, _, _, dA, dB, dC, _ in data:
        dA.free(); dB.free(); dC.free()


def test_host_batched_gemv_orders_itself_after_device_arena_users():
    # A device-pointer Q16 GEMM queued on a caller stream holds the workspace
    # arena; a host-pointer batched GEMV called right after it (its MFMA path
    # stages the query planes in the same arena) must wait for it: both
    # results must equal the oracle's
    L = M.lib()
    m, k, n = 1024, 2048, 1024
    a, b = O.gen_q16(0xA7E, m * k, k * n, shift=13)
    rows = _sample_rows(m, 8)
    want_c = O.gemm_q16_rows(a, b, m, k, n, rows)
    gm, gk, nb = 4096, 4096, 8
    W, X = O.gen_q16(0xA7F, gm * gk, nb * gk, shift=15)
    want_y = O.gemv_q16_batched(W, X, gm, gk, nb)
    dA, dB, dC = M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b), M.DeviceBuffer(m * n * 4)
    s = M.Stream()
    for rep in range(3):
        dC.fill(0x33)
        note(f"det_matmul_q16_dev {m}x{k}x{n} then host gemv nb={nb}, rep {rep}")
        M.check(L.det_matmul_q16_dev(dA.ptr, dB.ptr, dC.ptr, m, k, n, s.ptr))
        y = M.det_gemv_q16(W.reshape(gm, gk), X.reshape(nb, gk))
        s.sync()
        np.testing.assert_array_equal(dC.to_array(np.int32, (m, n))[rows], want_c)
        np.testing.assert_array_equal(y, want_y)
    s.destroy()
    dA.free(); dB.free(); dC.free()


# ------------------------------------------------------------------ int8 shapes

# The last three are on the 16-byte grid but off the 128-row kernels with an
# edge grid under one round: repacked into panels (both operands, or B only).
I8_SHAPES = [(1, 1, 1), (1, 64, 1), (3, 5, 7), (16, 16, 16), (17, 33, 65), (64, 64, 64), (255, 257, 129),
             (256, 256, 256), (300, 1000, 77), (513, 96, 260), (100, 4096, 8), (8, 4096, 300), (1000, 17, 999),
             (1008, 1008, 1008), (496, 512, 496), (1024, 1024, 1008)]


def test_gemm_i8_repack_rule_leaves_small_grids_alone():
    """Aligned on-grid int8 shapes take a workspace (padded panels) only when
    M, N >= 256 and padding to multiples of 256 adds at most 1/8 per
    dimension: the reference sweep's small cubes and long skinny shapes need
    none (m, k, n order as det_workspace_bytes takes them)."""
    L = M.lib()
    for m, k, n in [(16, 16, 16), (64, 64, 64), (128, 128, 128), (240, 240, 240), (16, 4194304, 16),
                    (304, 304, 304), (1008, 96, 1008)]:
        assert L.det_workspace_bytes(M.DET_OP_I8, m, k, n) == 0, (m, k, n)
    for m, k, n in [(1008, 1008, 1008), (496, 512, 496), (2000, 2000, 2000)]:
        assert L.det_workspace_bytes(M.DET_OP_I8, m, k, n) > 0, (m, k, n)


# Shapes whose 16x16 output tiles fit one round of the CUs take the direct
# v_dot4 kernel while K <= 512, or K <= 4096 when M, N or K is not a multiple
# of 128 (any alignment, no workspace); just past either bound the MFMA
# kernels take over (256x640x256, 16x4097x16, 272x16x256: 17 x 16 tiles).
I8_DIRECT = [(16, 16, 16), (1, 4096, 1), (16, 4096, 16), (256, 512, 256), (255, 4096, 255), (17, 33, 65),
             (5, 1000, 300), (4096, 7, 16), (1, 100, 4096)]
I8_DIRECT_EDGE = [(256, 640, 256), (16, 4097, 16), (272, 16, 256)]


@pytest.mark.parametrize("m,k,n", I8_DIRECT + I8_DIRECT_EDGE, ids=[f"{m}x{k}x{n}" for m, k, n in I8_DIRECT + I8_DIRECT_EDGE])
def test_gemm_i8_direct_route(m, k, n):
    L = M.lib()
    if (m, k, n) in I8_DIRECT:
        assert L.det_workspace_bytes(M.DET_OP_I8, m, k, n) == 0
    a, b = O.gen_i8(0x1D5 ^ (m * 1000003 + k * 1009 + n), m * k, k * n)
    want = O.gemm_i8(a, b, m, k, n).reshape(m, n)
    note(f"det_matmul_i8 direct-route boundary {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_i8(a.reshape(m, k), b.reshape(k, n)), want)
    # extreme operands: every product is 127 * 127, 127 * -128 or -128 * -128
    a2 = np.where(np.arange(m * k) % 3 == 0, -128, 127).astype(np.int8)
    b2 = np.where(np.arange(k * n) % 5 == 0, 127, -128).astype(np.int8)
    np.testing.assert_array_equal(M.det_matmul_i8(a2.reshape(m, k), b2.reshape(k, n)),
                                  O.gemm_i8(a2, b2, m, k, n).reshape(m, n))


def _tiny_sweep(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        m, n = (int(v) for v in rng.integers(1, 300, 2))
        k = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 4097))]))
        out.append((m, k, n))
    return out


TINY_SWEEP = _tiny_sweep(24, 0x7151)


@pytest.mark.parametrize("m,k,n", TINY_SWEEP, ids=[f"{m}x{k}x{n}" for m, k, n in TINY_SWEEP])
def test_tiny_shapes_every_op(m, k, n):
    """Seeded small shapes (M, N < 300, K up to 4096) through int8, int16 and
    Q16 (row-major and transposed B), whichever kernel each routes to, full
    output against the oracle."""
    seed = 0x7152 ^ (m * 1000003 + k * 1009 + n)
    a, b = O.gen_i8(seed, m * k, k * n)
    note(f"tiny sweep int8 {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_i8(a.reshape(m, k), b.reshape(k, n)),
                                  O.gemm_i8(a, b, m, k, n).reshape(m, n))
    a, b = O.gen_i16(seed, m * k, k * n)
    note(f"tiny sweep int16 {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_i16(a.reshape(m, k), b.reshape(k, n)),
                                  O.gemm_i16(a, b, m, k, n).reshape(m, n))
    a, b = O.gen_q16_sat(seed, m * k, k * n, 13)
    want = O.gemm_q16(a, b, m, k, n)
    note(f"tiny sweep q16 {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_q16(a.reshape(m, k), b.reshape(k, n)), want.reshape(m, n))
    c = np.zeros(m * n, np.int32)
    call6("gemmq", a, np.ascontiguousarray(b.reshape(k, n).T), c, m, k, n)
    np.testing.assert_array_equal(c, want.ravel())


@pytest.mark.parametrize("m,k,n", I8_SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in I8_SHAPES])
def test_gemm_i8_shapes(m, k, n):
    a, b = O.gen_i8(0xDEADBEEF00000000 ^ (m * 1000003 + k * 1009 + n), m * k, k * n)
    note(f"det_matmul_i8 {m}x{k}x{n}")
    got = M.det_matmul_i8(a.reshape(m, k), b.reshape(k, n))
    np.testing.assert_array_equal(got, O.gemm_i8(a, b, m, k, n))


# Shapes that route to the 128 x 256-tile kernel (M % 128, N % 256, K % 128
# all zero, and at most one round of 256 x 256 tiles or K % 256 != 0): one
# and two tiles, K of 1, 2, 3 and 128 steps of 128 (the 3-stage loop's
# remainders), K not a multiple of 256.
# 128-row tiles: 128 x 128 tiles for grids of at most 256 of them (all but the
# last two), 128 x 256 tiles in one round (the last two: 256 tiles each).
# 3, 5 and 9 row tiles (M = 384, 640, 1152) end in a partial group of the
# 4 row tiles that one-round 128 x 128 grids take together.
H128_SHAPES = [(128, 128, 256), (128, 256, 256), (256, 256, 256), (384, 384, 512), (1152, 640, 768),
               (128, 16384, 256), (640, 1280, 1536), (2048, 2048, 2048), (128, 128, 128), (384, 1152, 640),
               (2048, 1024, 4096), (4096, 256, 2048)]


@pytest.mark.parametrize("m,k,n", H128_SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in H128_SHAPES])
def test_gemm_i8_h128_tile_shapes(m, k, n):
    a, b = O.gen_i8(0x128128 ^ (m * 1000003 + k * 1009 + n), m * k, k * n)
    note(f"det_matmul_i8_dev (128x256 tiles) {m}x{k}x{n}")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i8_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n))
    if m * n * k <= 1 << 30:
        np.testing.assert_array_equal(C, O.gemm_i8(a, b, m, k, n).reshape(m, n))
    else:
        rows = np.unique(np.r_[_sample_rows(m, 8), 127, 128, m - 128])
        np.testing.assert_array_equal(C[rows], O.gemm_i8_rows(a, b, m, k, n, rows))
        cols = _sample_rows(n, 4)
        Bc = np.ascontiguousarray(b.reshape(k, n)[:, cols]).ravel()
        np.testing.assert_array_equal(C[:, cols], O.gemm_i8(a, Bc, m, k, len(cols)))


def test_gemm_i8_h128_wraps_mod_2_32():
    m, k, n = 128, 131200, 256                   # 1025 steps of 128; k * 128 * 128 > 2^31
    a = np.full((m, k), -128, np.int8)
    b = np.full((k, n), -128, np.int8)
    a[5, :] = 127
    b[:, 7] = 3
    note(f"det_matmul_i8 wrap (128x256 tiles) {m}x{k}x{n}")
    got = M.det_matmul_i8(a, b)
    rows = np.array([0, 5, 127])
    np.testing.assert_array_equal(got[rows], O.gemm_i8_rows(a.ravel(), b.ravel(), m, k, n, rows))
    assert got[0, 0] == np.int32(np.uint32((k * 16384) % (1 << 32)).astype(np.int32))


def _mt_gemm_i8(a, b, m, k, n):
    """Full int8 product from the multithreaded CPU restatement (equal to the
    scalar oracle at every band count, tests/test_oracle.py)."""
    c = np.empty(m * n, np.int32)
    assert O.lib().det_cpu_gemm_i8(a.ctypes.data, b.ctypes.data, c.ctypes.data, m, k, n) == 0
    return c.reshape(m, n)


# 128 x 256 tiles on persistent workgroups: two rounds whose second tile
# carries the first one's stores (272 tiles), uneven rounds (264 tiles on 136
# workgroups), a K too short to carry them (512: stored at the next tile's
# start) and three rounds (561 tiles)
PERSIST_I8 = [(2048, 768, 4352), (1408, 768, 6144), (2048, 512, 4352), (4224, 768, 4352)]
# off the 16-byte grid, repacked into padded panels, on grids of several
# rounds: persistent 128 x 256 tiles with the masked epilogue (2304 x 4352
# panels: 306 tiles; 4352^2: 578 tiles, whose 289 tiles of 256 x 256 would
# fill two rounds only to 0.56)
PERSIST_I8 += [(2100, 1000, 4100), (4100, 300, 4100)]


@pytest.mark.parametrize("m,k,n", PERSIST_I8, ids=[f"{m}x{k}x{n}" for m, k, n in PERSIST_I8])
def test_gemm_i8_persistent_rounds(m, k, n):
    a, b = O.gen_i8(0x9E25 ^ (m * 1000003 + k * 1009 + n), m * k, k * n)
    note(f"det_matmul_i8_dev (persistent 128x256 tiles) {m}x{k}x{n}")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i8_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n))
    np.testing.assert_array_equal(C, _mt_gemm_i8(a, b, m, k, n))
    rows = np.r_[0, 127, 128, m - 1]
    np.testing.assert_array_equal(C[rows], O.gemm_i8_rows(a, b, m, k, n, rows))


# 256 x 256 tiles (grids that fill whole rounds of them): padded panels with
# the masked epilogue in one round (4096^2 panels) and two rounds (4096 x
# 8192), and an unpadded grid of two rounds
T256_I8 = [(4000, 1000, 4000), (4000, 300, 8100), (4096, 512, 8192)]


@pytest.mark.parametrize("m,k,n", T256_I8, ids=[f"{m}x{k}x{n}" for m, k, n in T256_I8])
def test_gemm_i8_t256_tiles(m, k, n):
    a, b = O.gen_i8(0x7256 ^ (m * 1000003 + k * 1009 + n), m * k, k * n)
    note(f"det_matmul_i8_dev (256x256 tiles) {m}x{k}x{n}")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i8_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n))
    np.testing.assert_array_equal(C, _mt_gemm_i8(a, b, m, k, n))
    rows = np.r_[0, 255, 256, m - 1]
    np.testing.assert_array_equal(C[rows], O.gemm_i8_rows(a, b, m, k, n, rows))


def _sweep_shapes(count, seed):
    """Seeded int8 shapes across the router's cases: multiples of 128 / 256
    (128 x 128, 128 x 256 one- and multi-round, 256 x 256), the 16-byte grid
    off those multiples (edge tiles) and ragged shapes (repack)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        kind = i % 4
        if kind == 0:     # 128-multiples, up to 34 x 34 tiles of 128
            m, n, k = (int(rng.integers(1, 35)) * 128 for _ in range(3))
        elif kind == 1:   # 256-multiples
            m, n, k = (int(rng.integers(1, 19)) * 256 for _ in range(3))
        elif kind == 2:   # on the 16-byte grid
            m = int(rng.integers(1, 3000)); n = int(rng.integers(1, 180)) * 16; k = int(rng.integers(1, 120)) * 16
        else:             # ragged
            m, n, k = (int(rng.integers(1, 3000)) for _ in range(3))
        if m * n * k > 1 << 31:   # keep the CPU check short: shrink K on its grid
            g = (128, 256, 16, 1)[kind]
            k = max(g, (1 << 31) // (m * n) // g * g)
        out.append((m, k, n))
    return out


SWEEP_I8 = _sweep_shapes(48, 0x5EE9)


@pytest.mark.parametrize("m,k,n", SWEEP_I8, ids=[f"{m}x{k}x{n}" for m, k, n in SWEEP_I8])
def test_gemm_i8_routing_sweep(m, k, n):
    """Every kernel the router can pick, full output against the CPU
    restatement, through the device entry point (library arena) and through
    det_matmul_ws_dev with exactly the reported workspace."""
    a, b = O.gen_i8(0x5EE9 ^ (m * 1000003 + k * 1009 + n), m * k, k * n)
    want = _mt_gemm_i8(a, b, m, k, n)
    note(f"det_matmul_i8_dev sweep {m}x{k}x{n}")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i8_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n), reps=1)
    np.testing.assert_array_equal(C, want)
    L = M.lib()
    wsb = L.det_workspace_bytes(M.DET_OP_I8, m, k, n)
    ws = M.DeviceBuffer(max(wsb, 256))
    C2 = _dev_run(lambda pa, pb, pc, s: L.det_matmul_ws_dev(M.DET_OP_I8, pa, pb, pc, m, k, n, ws.ptr, wsb, s),
                  [a, b], (m, n), reps=1)
    ws.free()
    np.testing.assert_array_equal(C2, want)


def _mt_gemm(op, a, b, m, k, n):
    """Full Q16 / int16 product from the multithreaded CPU restatement (equal
    to the scalar oracle at every band count, tests/test_oracle.py)."""
    c = np.empty(m * n, np.int32)
    fn = O.lib().det_cpu_gemm_q16 if op == M.DET_OP_Q16 else O.lib().det_cpu_gemm_i16
    assert fn(a.ctypes.data, b.ctypes.data, c.ctypes.data, m, k, n) == 0
    return c.reshape(m, n)


def _limb_sweep(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        if i % 2 == 0:   # tile multiples (64 for Q16, 128 rows for int16's interleave)
            m, n, k = (int(rng.integers(1, 17)) * 64 for _ in range(3))
        else:
            m, n, k = (int(rng.integers(1, 1100)) for _ in range(3))
        out.append((m, k, n))
    return out


SWEEP_LIMB = [(op, *shape) for op in (M.DET_OP_Q16, M.DET_OP_I16) for shape in _limb_sweep(12, 0x11B + op)]


@pytest.mark.parametrize("op,m,k,n", SWEEP_LIMB, ids=[f"op{op}-{m}x{k}x{n}" for op, m, k, n in SWEEP_LIMB])
def test_gemm_limb_sweep(op, m, k, n):
    """Seeded Q16 (saturating generator; direct or limb kernel by shape) and
    int16 shapes, full output against the CPU restatement, through
    det_matmul_ws_dev with exactly the reported workspace refilled with
    garbage first."""
    if op == M.DET_OP_Q16:
        a, b = O.gen_q16_sat(0x11B ^ (m * 7919 + k * 31 + n), m * k, k * n, 13)
    else:
        a, b = O.gen_i16(0x11B ^ (m * 7919 + k * 31 + n), m * k, k * n)
    want = _mt_gemm(op, a, b, m, k, n)
    L = M.lib()
    wsb = L.det_workspace_bytes(op, m, k, n)
    ws = M.DeviceBuffer(max(wsb, 256))
    ws.fill(0xC3)
    note(f"det_matmul_ws_dev op={op} sweep {m}x{k}x{n}")
    C = _dev_run(lambda pa, pb, pc, s: L.det_matmul_ws_dev(op, pa, pb, pc, m, k, n, ws.ptr, wsb, s), [a, b],
                 (m, n), reps=1)
    ws.free()
    np.testing.assert_array_equal(C, want)


# Operands off the 16-byte grid (K or N not a multiple of 16) or not 16-byte
# aligned: repacked into padded panels in the workspace (arena, caller
# workspace or scratch), or, without a workspace, the byte-load kernel.
RAGGED_I8 = [(1, 17, 1),(37, 100, 53), (300, 1000, 77), (256, 4095, 256), (1000, 1000, 1000), (257, 4100, 1003),
             (64, 64, 64), (256, 256, 256),
             # A on the full-tile grid, B ragged: only B is repacked when A is aligned
             (128, 256, 77), (512, 1024, 1000), (1024, 2048, 1000)]


def _offset_buffer(a, off):
    """A device buffer holding `a` at byte offset `off` (a misaligned operand)."""
    buf = M.DeviceBuffer(a.nbytes + 64)
    M.check(M.lib().det_memcpy_htod(buf.ptr + off, a.ctypes.data, a.nbytes))
    return buf


@pytest.mark.parametrize("m,k,n", RAGGED_I8, ids=[f"{m}x{k}x{n}" for m, k, n in RAGGED_I8])
@pytest.mark.parametrize("offs", [(0, 0), (1, 3), (8, 4)], ids=["aligned", "off1_3", "off8_4"])
def test_gemm_i8_ragged_and_misaligned_device_operands(m, k, n, offs):
    a, b = O.gen_i8(0xA11 ^ (m * 7 + k * 3 + n), m * k, k * n)
    want = O.gemm_i8(a, b, m, k, n).reshape(m, n)
    da, db = _offset_buffer(a, offs[0]), _offset_buffer(b, offs[1])
    pa, pb = da.ptr + offs[0], db.ptr + offs[1]
    dc = M.DeviceBuffer(m * n * 4)
    s = M.Stream()
    L = M.lib()
    # the library arena (sized for these addresses), a caller workspace of the
    # reported size (enough only for aligned operands), and none at all
    ws_bytes = L.det_workspace_bytes(M.DET_OP_I8, m, k, n)
    ws = M.DeviceBuffer(max(ws_bytes, 256))
    for how in ("arena", "ws", "no_ws"):
        dc.fill(0xA5)
        note(f"int8 {m}x{k}x{n} offsets {offs} via {how} (reported ws {ws_bytes})")
        if how == "arena":
            M.check(L.det_matmul_i8_dev(pa, pb, dc.ptr, m, k, n, s.ptr))
        elif how == "ws":
            M.check(L.det_matmul_ws_dev(M.DET_OP_I8, pa, pb, dc.ptr, m, k, n, ws.ptr, ws_bytes, s.ptr))
        else:
            M.check(L.det_matmul_ws_dev(M.DET_OP_I8, pa, pb, dc.ptr, m, k, n, None, 0, s.ptr))
        s.sync()
        np.testing.assert_array_equal(dc.to_array(np.int32, (m, n)), want)
    s.destroy()
    for buf in (da, db, dc, ws):
        buf.free()


def test_gemm_i8_k_zero_and_empty():
    note("det_matmul_i8 k=0")
    np.testing.assert_array_equal(M.det_matmul_i8(np.zeros((5, 0), np.int8), np.zeros((0, 7), np.int8)),
                                  np.zeros((5, 7), np.int32))
    c = np.full(4, 7, np.int32)
    assert M.lib().gemmi8(0, 0, addr(c), 0, 4, 4) == 0 and (c == 7).all()


def test_gemm_i8_wraps_mod_2_32():
    k = 131136                                   # k * 128 * 128 > 2^31
    a = np.full((16, k), -128, np.int8)
    b = np.full((k, 16), -128, np.int8)
    a[1, :] = 127
    note(f"det_matmul_i8 wrap 16x{k}x16")
    got = M.det_matmul_i8(a, b)
    np.testing.assert_array_equal(got, O.gemm_i8(a.ravel(), b.ravel(), 16, k, 16))
    assert got[0, 0] == np.int32(np.uint32((k * 16384) % (1 << 32)).astype(np.int32))


# ------------------------------------------------------------------ Q16 / i16 shapes

Q_SHAPES = [(1, 1, 1), (3, 5, 7), (64, 64, 64), (65, 63, 66), (128, 300, 96), (200, 129, 33), (7, 1000, 130)]


@pytest.mark.parametrize("shift", [12, 13, 0])
@pytest.mark.parametrize("m,k,n", Q_SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in Q_SHAPES])
def test_gemm_q16_shapes(m, k, n, shift):
    a, b = O.gen_q16(0xDEADBEEF00000000 ^ (m * 7919 + k * 31 + n) ^ shift, m * k, k * n, shift=shift)
    note(f"det_matmul_q16 {m}x{k}x{n} shift={shift}")
    got = M.det_matmul_q16(a.reshape(m, k), b.reshape(k, n))
    np.testing.assert_array_equal(got, O.gemm_q16(a, b, m, k, n))


# The direct kernel's edges: one K term, K across its 64-k slices and 256-k
# chunks (63, 64, 65, 255, 256, 257, 1000), the longest K it takes for one
# round of tiles (4096) and four rounds of 16 x 16 tiles (512 x 1024 x 512).
Q_DIRECT = [(16, 1, 16), (17, 63, 15), (33, 64, 31), (40, 65, 48), (5, 255, 300), (256, 256, 256), (99, 257, 161),
            (7, 1000, 130), (16, 4096, 16), (64, 4096, 48), (512, 1024, 512), (1, 3, 16384), (16384, 2, 1)]


@pytest.mark.parametrize("m,k,n", Q_DIRECT, ids=[f"{m}x{k}x{n}" for m, k, n in Q_DIRECT])
def test_gemm_q16_direct_route(m, k, n):
    """Small shapes take the direct per-term kernel (no workspace): full-range
    inputs through det_matmul_q16 and the B-transposed gemmq, saturating
    inputs through the device workspace entry with no workspace at all."""
    L = M.lib()
    assert L.det_workspace_bytes(M.DET_OP_Q16, m, k, n) == 0
    a, b = O.gen_q16(0x5D1 ^ (m * 7919 + k * 31 + n), m * k, k * n, shift=0)
    want = O.gemm_q16(a, b, m, k, n).reshape(m, n)
    note(f"det_matmul_q16 direct {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_q16(a.reshape(m, k), b.reshape(k, n)), want)
    bt = np.ascontiguousarray(b.reshape(k, n).T)
    c = np.zeros(m * n, np.int32)
    call6("gemmq", a, bt, c, m, k, n)
    np.testing.assert_array_equal(c.reshape(m, n), want)
    a, b = O.gen_q16_sat(0x5D2 ^ (m * 7919 + k * 31 + n), m * k, k * n, shift=13)
    want = O.gemm_q16(a, b, m, k, n).reshape(m, n)
    s = M.Stream()
    da, db, dc = M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b), M.DeviceBuffer(m * n * 4)
    dc.fill(0xA5)
    note(f"det_matmul_ws_dev q16 direct {m}x{k}x{n} (no workspace)")
    M.check(L.det_matmul_ws_dev(M.DET_OP_Q16, da.ptr, db.ptr, dc.ptr, m, k, n, None, 0, s.ptr))
    s.sync()
    np.testing.assert_array_equal(dc.to_array(np.int32, (m, n)), want)
    for buf in (da, db, dc):
        buf.free()
    s.destroy()


def test_gemm_q16_saturating_config_and_bt():
    m, k, n = 96, 257, 80
    a, b = O.gen_q16_sat(0x9A7, m * k, k * n, shift=13)
    want = O.gemm_q16(a, b, m, k, n)
    note("det_matmul_q16 sat 96x257x80")
    np.testing.assert_array_equal(M.det_matmul_q16(a.reshape(m, k), b.reshape(k, n)), want)
    bt = np.ascontiguousarray(b.reshape(k, n).T)
    c = np.zeros(m * n, np.int32)
    call6("gemmq", a, bt, c, m, k, n)
    np.testing.assert_array_equal(c.reshape(m, n), want)


def test_gemm_q16_long_k_split_halves():
    # K = 40000: each K half of the 8-wave kernel holds 20000 terms, close to
    # the 32-bit bounds of its shift-0 / shift-1 sets and residue
    m, k, n = 16, 40000, 24
    a, b = O.gen_q16(0xF1A5, m * k, k * n, shift=0)
    note(f"det_matmul_q16 long-k {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_q16(a.reshape(m, k), b.reshape(k, n)), O.gemm_q16(a, b, m, k, n))


def test_gemm_q16_long_k_flush():
    # K > 65536 takes the flushing kernel (exact int64 totals every 16384 K)
    m, k, n = 4, 70000, 5
    a, b = O.gen_q16(0xF1A6, m * k, k * n, shift=0)
    note(f"det_matmul_q16 flush {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_q16(a.reshape(m, k), b.reshape(k, n)), O.gemm_q16(a, b, m, k, n))


@pytest.mark.parametrize("shape", [(200, 1000, 136), (1100, 1000, 1000)], ids=["direct", "limb"])
@pytest.mark.parametrize("gen", ["full", "sat"])
def test_gemm_q16_multi_tile(gen, shape):
    # several tiles, ragged in M and N, K not a multiple of 64 (the first
    # shape on the direct kernel, the second on the limb kernel)
    m, k, n = shape
    if gen == "full":
        a, b = O.gen_q16(0x51DE, m * k, k * n, shift=0)
    else:
        a, b = O.gen_q16_sat(0x51DF, m * k, k * n, shift=13)
    note(f"det_matmul_q16 {gen} {m}x{k}x{n}")
    want = O.gemm_q16(a, b, m, k, n)
    np.testing.assert_array_equal(M.det_matmul_q16(a.reshape(m, k), b.reshape(k, n)), want)
    bt = np.ascontiguousarray(b.reshape(k, n).T)
    c = np.zeros(m * n, np.int32)
    call6("gemmq", a, bt, c, m, k, n)
    np.testing.assert_array_equal(c.reshape(m, n), want)


# Shapes whose 16x16 tiles times K are too much for the direct kernel run
# the limb kernel; its grids of 64 x 64 tiles that fill at most half the CUs
# run split in K (up to 8 partial sums per tile over whole 64-k steps,
# reduced by a second kernel): 7 x 5000 x 130 (3 tiles, K off the 64 grid,
# splits of 9-10 steps), 100 x 4200 x 70 (4 ragged tiles, uneven splits),
# 200 x 4160 x 300 (20 tiles), 1000 x 4100 x 33 (16 tiles, one column), 512 x
# 2048 x 512 (64 tiles, 4 splits of 8 steps); 1000 x 100 x 1000 and 1024 x
# 128 x 1024 fill the chip (no split; the first ragged in M, N and K).
Q_SPLIT = [(7, 5000, 130), (100, 4200, 70), (200, 4160, 300), (1000, 4100, 33), (512, 2048, 512), (1000, 100, 1000),
           (1024, 128, 1024)]


@pytest.mark.parametrize("m,k,n", Q_SPLIT, ids=[f"{m}x{k}x{n}" for m, k, n in Q_SPLIT])
def test_gemm_q16_k_split(m, k, n):
    """The limb route (split in K where the grid is small) against the
    oracle: saturating inputs through the
    device workspace entry (the workspace, partials included, refilled with
    garbage before each call), and full-range inputs through gemmqmm and the
    B-transposed gemmq."""
    L = M.lib()
    a, b = O.gen_q16_sat(0x5A17 ^ (m * 7919 + k * 31 + n), m * k, k * n, shift=13)
    want = O.gemm_q16(a, b, m, k, n).reshape(m, n)
    wsb = L.det_workspace_bytes(M.DET_OP_Q16, m, k, n)
    assert wsb > 0   # the limb route (the direct kernel needs no workspace)
    s = M.Stream()
    da, db, dc = M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b), M.DeviceBuffer(m * n * 4)
    ws = M.DeviceBuffer(wsb)
    for rep in range(2):
        note(f"det_matmul_ws_dev q16 split {m}x{k}x{n} rep={rep}")
        ws.fill(0x6B + rep)
        dc.fill(0xA5)
        M.check(L.det_matmul_ws_dev(M.DET_OP_Q16, da.ptr, db.ptr, dc.ptr, m, k, n, ws.ptr, wsb, s.ptr))
        s.sync()
        np.testing.assert_array_equal(dc.to_array(np.int32, (m, n)), want)
    for buf in (da, db, dc, ws):
        buf.free()
    s.destroy()
    a, b = O.gen_q16(0x5A18 ^ (m * 7919 + k * 31 + n), m * k, k * n, shift=0)
    want = O.gemm_q16(a, b, m, k, n)
    note(f"gemmqmm / gemmq full-range split {m}x{k}x{n}")
    c = np.zeros(m * n, np.int32)
    call6("gemmqmm", a, b, c, m, k, n)
    np.testing.assert_array_equal(c, want.ravel())
    bt = np.ascontiguousarray(b.reshape(k, n).T)
    c = np.zeros(m * n, np.int32)
    call6("gemmq", a, bt, c, m, k, n)
    np.testing.assert_array_equal(c, want.ravel())


# int16 shapes whose 16x16 output tiles fit one round of the CUs take the
# direct v_dot2 kernel while K <= 4096 (no workspace); just past either
# bound (16x4097x16, 272x16x256) the limb-interleaved MFMA GEMM takes over.
I16_DIRECT = [(16, 16, 16), (1, 4096, 1), (16, 4096, 16), (255, 4096, 255), (17, 33, 65), (256, 256, 256),
              (4096, 9, 16), (1, 100, 4096)]
I16_DIRECT_EDGE = [(16, 4097, 16), (272, 16, 256)]


@pytest.mark.parametrize("m,k,n", I16_DIRECT + I16_DIRECT_EDGE,
                         ids=[f"{m}x{k}x{n}" for m, k, n in I16_DIRECT + I16_DIRECT_EDGE])
def test_gemm_i16_direct_route(m, k, n):
    L = M.lib()
    assert (L.det_workspace_bytes(M.DET_OP_I16, m, k, n) == 0) == ((m, k, n) in I16_DIRECT)
    a, b = O.gen_i16(0x1D6 ^ (m * 1000003 + k * 1009 + n), m * k, k * n)
    note(f"det_matmul_i16 direct-route boundary {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_i16(a.reshape(m, k), b.reshape(k, n)),
                                  O.gemm_i16(a, b, m, k, n).reshape(m, n))
    # extreme operands: products of 32767 and -32768, sums that wrap
    a2 = np.where(np.arange(m * k) % 3 == 0, -32768, 32767).astype(np.int16)
    b2 = np.where(np.arange(k * n) % 5 == 0, 32767, -32768).astype(np.int16)
    np.testing.assert_array_equal(M.det_matmul_i16(a2.reshape(m, k), b2.reshape(k, n)),
                                  O.gemm_i16(a2, b2, m, k, n).reshape(m, n))


I16_SHAPES = [(1, 1, 1), (3, 5, 7), (64, 64, 64), (65, 127, 66), (200, 300, 100), (33, 2048, 17),
              (300, 1000, 270), (129, 16, 128)]


@pytest.mark.parametrize("m,k,n", I16_SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in I16_SHAPES])
def test_gemm_i16_shapes(m, k, n):
    a, b = O.gen_i16(0xDEADBEEF00000000 ^ (m * 131 + k * 17 + n), m * k, k * n)
    note(f"det_matmul_i16 {m}x{k}x{n}")
    np.testing.assert_array_equal(M.det_matmul_i16(a.reshape(m, k), b.reshape(k, n)), O.gemm_i16(a, b, m, k, n))


# limb interleaves that fill whole rounds of 256 x 256 tiles (the 16x16x64
# kernel with the int16 epilogue): 2048 x 1024 x 2048 (M2 = N2 = 4096, one
# round) and 4096 x 256 x 1024 (8192 x 2048 interleave, one round)
I16_T256 = [(2048, 1024, 2048), (4096, 256, 1024)]


@pytest.mark.parametrize("m,k,n", I16_T256, ids=[f"{m}x{k}x{n}" for m, k, n in I16_T256])
def test_gemm_i16_t256_tiles(m, k, n):
    a, b = O.gen_i16(0x16256 ^ (m * 131 + k * 17 + n), m * k, k * n)
    note(f"det_matmul_i16 (256x256 tiles) {m}x{k}x{n}")
    got = M.det_matmul_i16(a.reshape(m, k), b.reshape(k, n))
    np.testing.assert_array_equal(got, _mt_gemm(M.DET_OP_I16, a, b, m, k, n))


def test_gemm_i16_extremes():
    m, k, n = 8, 70000, 8
    a = np.full((m, k), -32768, np.int16)
    b = np.full((k, n), -32768, np.int16)
    a[1] = 32767
    b[:, 2] = 32767
    note("det_matmul_i16 extremes 8x70000x8")
    np.testing.assert_array_equal(M.det_matmul_i16(a, b), O.gemm_i16(a.ravel(), b.ravel(), m, k, n))


# ------------------------------------------------------------------ GEMV

GEMV_SHAPES = [(1, 1), (5, 3), (64, 64), (512, 130), (128, 96), (256, 1027), (1000, 4096), (11922, 384)]


@pytest.mark.parametrize("nb", [1, 2, 3, 8, 9])
@pytest.mark.parametrize("m,k", GEMV_SHAPES, ids=[f"{m}x{k}" for m, k in GEMV_SHAPES])
def test_gemv_q16_shapes(m, k, nb):
    W, X = O.gen_q16(0xDEADBEEF00000000 ^ ((m << 20) ^ k) ^ nb, m * k, nb * k)
    note(f"det_gemv_q16_batched {m}x{k} nb={nb}")
    got = M.det_gemv_q16(W.reshape(m, k), X.reshape(nb, k))
    np.testing.assert_array_equal(got, O.gemv_q16_batched(W, X, m, k, nb))


GEMV_FULL = [(64, 512, 2), (300, 1024, 3), (130, 2048, 8), (16, 32768, 8)]


@pytest.mark.parametrize("fam", ["full", "extreme"])
@pytest.mark.parametrize("m,k,nb", GEMV_FULL, ids=[f"{m}x{k}b{nb}" for m, k, nb in GEMV_FULL])
def test_gemv_q16_batched_full_range(m, k, nb, fam):
    """The batched (MFMA) path on full-range int32 W and x: every limb of W and
    every digit of x in use (x near 2^31 - 1 needs the fifth digit), up to the
    kernel's largest K."""
    rng = np.random.default_rng(m * 31 + k + nb + len(fam))
    ext = np.array([2147483647, -2147483648, -2147483647, 2139062144, 2139062143, 0, 1, -1, 65535, -65536,
                    -8421505, 8421504], np.int32)
    if fam == "full":
        W, X = O.gen_q16(0xF011 ^ (m * k + nb), m * k, nb * k, shift=0)
    else:
        W, X = ext[rng.integers(0, len(ext), m * k)], ext[rng.integers(0, len(ext), nb * k)]
    note(f"det_gemv_q16_batched {fam} {m}x{k} nb={nb}")
    got = M.det_gemv_q16(W.reshape(m, k), X.reshape(nb, k))
    np.testing.assert_array_equal(got, O.gemv_q16_batched(W, X, m, k, nb))


GEMV_WS = [(64, 512, 8), (1000, 1024, 13), (16, 32768, 2), (300, 512, 1), (130, 1000, 8)]


@pytest.mark.parametrize("m,k,nb", GEMV_WS, ids=[f"{m}x{k}b{nb}" for m, k, nb in GEMV_WS])
def test_gemv_q16_ws_dev(m, k, nb):
    """det_gemv_q16_ws_dev: the caller's workspace (garbage-filled, exactly
    det_gemv_workspace_bytes), a workspace one byte short and none at all
    (both take the one-vector kernel) give the oracle's output, twice in a
    row on poisoned outputs; 130 x 1000 (K % 512 != 0) needs no workspace."""
    L = M.lib()
    W, X = O.gen_q16(0x6E5 ^ (m * k + nb), m * k, nb * k, shift=0)
    want = O.gemv_q16_batched(W, X, m, k, nb).reshape(nb, m)
    need = L.det_gemv_workspace_bytes(m, k, nb)
    assert (need > 0) == (nb >= 2 and k % 512 == 0)
    s = M.Stream()
    dW, dX, dY = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(X), M.DeviceBuffer(nb * m * 4)
    ws = M.DeviceBuffer(max(need, 256))
    for ws_ptr, ws_bytes in ((ws.ptr, need), (ws.ptr, need - 1), (None, 0)):
        for rep in range(2):
            note(f"det_gemv_q16_ws_dev {m}x{k} nb={nb} ws_bytes={ws_bytes} rep={rep}")
            ws.fill(0x3C + rep)
            dY.fill(0xA5)
            M.check(L.det_gemv_q16_ws_dev(dW.ptr, dX.ptr, dY.ptr, m, k, nb, ws_ptr, ws_bytes, s.ptr))
            s.sync()
            np.testing.assert_array_equal(dY.to_array(np.int32, (nb, m)), want)
    assert L.det_gemv_q16_ws_dev(dW.ptr, dX.ptr, None, m, k, nb, ws.ptr, need, s.ptr) == M.DET_ERR_ARG
    assert L.det_gemv_q16_ws_dev(dW.ptr, dX.ptr, dY.ptr, -1, k, nb, ws.ptr, need, s.ptr) == M.DET_ERR_ARG
    for buf in (dW, dX, dY, ws):
        buf.free()
    s.destroy()


@pytest.mark.parametrize("m,k", [(1, 1), (7, 9), (256, 256), (300, 1001), (4096, 4096)])
def test_gemv_i16_shapes(m, k):
    W, x = O.gen_i16(0xDEADBEEF ^ (m * 3 + k), m * k, k)
    note(f"det_gemv_i16 {m}x{k}")
    np.testing.assert_array_equal(M.det_gemv_i16(W.reshape(m, k), x), O.gemv_i16(W, x, m, k))


# ------------------------------------------------------------------ device-pointer API

def test_dev_api_poisoned_outputs_and_run_to_run():
    m, k, n = 320, 448, 192
    a, b = O.gen_i8(0xD0D0, m * k, k * n)
    want = O.gemm_i8(a, b, m, k, n)
    da, db = M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b)
    dc = M.DeviceBuffer(m * n * 4)
    s = M.Stream()
    for rep in range(16):
        dc.fill(0xA5)
        note(f"det_matmul_i8_dev rep={rep}")
        M.check(M.lib().det_matmul_i8_dev(da.ptr, db.ptr, dc.ptr, m, k, n, s.ptr))
        s.sync()
        np.testing.assert_array_equal(dc.to_array(np.int32, (m, n)), want)
    m, k, n = 1040, 200, 1040   # a Q16 shape on the limb kernel (which needs the workspace)
    aq, bq = O.gen_q16_sat(0xD0D1, m * k, k * n)
    wq = O.gemm_q16(aq, bq, m, k, n)
    daq, dbq = M.DeviceBuffer.from_array(aq), M.DeviceBuffer.from_array(bq)
    dc = M.DeviceBuffer(m * n * 4)
    ws_bytes = M.lib().det_workspace_bytes(M.DET_OP_Q16, m, k, n)
    assert ws_bytes > 16
    ws = M.DeviceBuffer(ws_bytes)
    for rep in range(4):
        dc.fill(0xA5)
        note(f"det_matmul_q16_dev rep={rep}")
        M.check(M.lib().det_matmul_q16_dev(daq.ptr, dbq.ptr, dc.ptr, m, k, n, s.ptr))
        s.sync()
        np.testing.assert_array_equal(dc.to_array(np.int32, (m, n)), wq)
        dc.fill(0xA5)
        note(f"det_matmul_ws_dev q16 rep={rep}")
        M.check(M.lib().det_matmul_ws_dev(M.DET_OP_Q16, daq.ptr, dbq.ptr, dc.ptr, m, k, n, ws.ptr, ws_bytes, s.ptr))
        s.sync()
        np.testing.assert_array_equal(dc.to_array(np.int32, (m, n)), wq)
    # a too-small workspace is rejected before any launch
    assert M.lib().det_matmul_ws_dev(M.DET_OP_Q16, daq.ptr, dbq.ptr, dc.ptr, m, k, n, ws.ptr, 16, s.ptr) < 0
    assert "workspace" in M.last_error()
    s.destroy()


@pytest.mark.parametrize("op,m,k,n", [("i16", 64, 5000, 96), ("i16", 300, 1000, 270), ("q16", 64, 5000, 100),
                                      ("q16", 130, 4160, 70)])
def test_ws_dev_exact_workspace_with_garbage(op, m, k, n):
    # the exact reported workspace, refilled with garbage before every call:
    # the preps write every column-sum partial they later read (several
    # 64-row B tiles per partial at these K), nothing relies on zeroed memory
    if op == "i16":
        a, b = O.gen_i16(0x6A5 ^ k, m * k, k * n)
        want, code, dt = O.gemm_i16(a, b, m, k, n), M.DET_OP_I16, np.int16
    else:
        a, b = O.gen_q16_sat(0x6A6 ^ k, m * k, k * n)
        want, code, dt = O.gemm_q16(a, b, m, k, n), M.DET_OP_Q16, np.int32
    ws_bytes = M.lib().det_workspace_bytes(code, m, k, n)
    assert ws_bytes > 0
    da, db = M.DeviceBuffer.from_array(a.astype(dt)), M.DeviceBuffer.from_array(b.astype(dt))
    dc, ws = M.DeviceBuffer(m * n * 4), M.DeviceBuffer(ws_bytes)
    s = M.Stream()
    for rep, fill in enumerate((0xA5, 0x00, 0xFF)):
        ws.fill(fill)
        dc.fill(0x5A)
        note(f"det_matmul_ws_dev {op} {m}x{k}x{n} rep={rep}")
        M.check(M.lib().det_matmul_ws_dev(code, da.ptr, db.ptr, dc.ptr, m, k, n, ws.ptr, ws_bytes, s.ptr))
        s.sync()
        np.testing.assert_array_equal(dc.to_array(np.int32, (m, n)), want.reshape(m, n))
    s.destroy()


def test_invalid_shapes_are_rejected_before_launch():
    c = np.zeros(4, np.int32)
    a = np.zeros(4, np.int8)
    note("invalid shapes")
    assert M.lib().gemmi8(addr(a), addr(a), addr(c), -1, 2, 2) < 0
    assert "dimension" in M.last_error()
    assert M.lib().det_matmul_i8(addr(a), addr(a), addr(c), 1 << 40, 1, 1) < 0


# ------------------------------------------------------------------ BASELINE-size configs

def _sample_rows(m, count=6):
    rng = np.random.default_rng(m)
    rows = sorted(set([0, m - 1] + list(rng.integers(0, m, count))))
    return np.array(rows, np.int64)


def _dev_run(fn, inputs, out_shape, reps=2):
    """Run on device buffers; poison the output each time; all reps must agree."""
    bufs = [M.DeviceBuffer.from_array(x) for x in inputs]
    out = M.DeviceBuffer(int(np.prod(out_shape)) * 4)
    s = M.Stream()
    res = None
    for rep in range(reps):
        out.fill(0xA5)
        M.check(fn(*[b.ptr for b in bufs], out.ptr, s.ptr))
        s.sync()
        got = out.to_array(np.int32, out_shape)
        if res is None:
            res = got
        else:
            np.testing.assert_array_equal(got, res)
    s.destroy()
    for b in bufs + [out]:
        b.free()
    return res


def test_config_int8_4096_cubed():
    m = k = n = 4096
    a, b = M.gen_i8(0xDEADBEEF ^ 0x4096, m * k, k * n)
    note("det_matmul_i8_dev 4096^3")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i8_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n))
    rows = _sample_rows(m)
    np.testing.assert_array_equal(C[rows], O.gemm_i8_rows(a, b, m, k, n, rows))
    cols = _sample_rows(n)
    Bc = np.ascontiguousarray(b.reshape(k, n)[:, cols]).ravel()
    np.testing.assert_array_equal(C[:, cols], O.gemm_i8(a, Bc, m, k, len(cols)))


def test_config_int8_mlp_4096x4096x11008():
    m, k, n = 4096, 4096, 11008
    x = M.gen_i8_gauss(0xDEADBEEF ^ 0x3117, m * k)
    w = M.gen_i8_sym127(0xDEADBEEF ^ 0x3118, k * n)
    note("det_matmul_i8_dev mlp 4096x4096x11008")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i8_dev(pa, pb, pc, m, k, n, s), [x, w], (m, n))
    rows = _sample_rows(m, 4)
    np.testing.assert_array_equal(C[rows], O.gemm_i8_rows(x, w, m, k, n, rows))


def test_config_int8_8192_cubed():
    """The square 8192^3 peak-probe config: sampled rows and columns against
    the oracle, output poisoned before each of two runs."""
    m = k = n = 8192
    a, b = M.gen_i8(0xDEADBEEF ^ 0x8192, m * k, k * n)
    note("det_matmul_i8_dev 8192^3")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i8_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n))
    rows = _sample_rows(m, 4)
    np.testing.assert_array_equal(C[rows], O.gemm_i8_rows(a, b, m, k, n, rows))
    cols = _sample_rows(n, 4)
    Bc = np.ascontiguousarray(b.reshape(k, n)[:, cols]).ravel()
    np.testing.assert_array_equal(C[:, cols], O.gemm_i8(a, Bc, m, k, len(cols)))


def test_config_q16_4096_cubed():
    """Q16 at 4096^3 (the metric's Q16 shape), saturating generator: sampled
    rows against the oracle, two poisoned runs."""
    m = k = n = 4096
    a, b = M.gen_q16_sat(0xDEADBEEF ^ 0x4016, m * k, k * n, 13)
    note("det_matmul_q16_dev 4096^3 (saturating config)")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_q16_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n))
    rows = _sample_rows(m, 5)
    np.testing.assert_array_equal(C[rows], O.gemm_q16_rows(a, b, m, k, n, rows))


def test_determinism_256_runs(canaries):
    """The reference's stability gate (benches/det_gemv_q16_mt.rs:71,
    det_matmul_q16_mt.rs:88: 256 recomputations, one hash): the 64^3 int8 and
    Q16 canaries and the 11922x384 routing-shape GEMV, each computed 256
    times through the reference ABI into fresh poisoned buffers."""
    runs = 256
    w = canaries["workloads"]
    a8, b8 = O.gen_i8(w["gemm-i8-64x64x64"]["seed"], 64 * 64, 64 * 64)
    aq, bq = O.gen_q16(w["gemm-q16-fused-64x64x64"]["seed"], 64 * 64, 64 * 64)
    m, k = 11922, 384
    W, x = O.gen_q16(0xDEADBEEF_00000000 ^ ((m << 20) ^ k), m * k, k)
    want_gemv = h32(O.gemv_q16(W, x, m, k))
    cases = (("gemmi8", a8, b8, 6, w["gemm-i8-64x64x64"]["avx2"]),
             ("gemmqmm", aq, bq, 6, w["gemm-q16-fused-64x64x64"]["avx2"]),
             ("gemvq", W, x, 5, want_gemv))
    for sym, a, b, arity, want in cases:
        note(f"{sym} x{runs} into fresh poisoned buffers")
        fn = getattr(M.lib(), sym)
        hashes = set()
        for rep in range(runs):
            out = np.full(64 * 64 if arity == 6 else m, 0x5A5A5A5A ^ rep, np.int32)
            rc = fn(addr(a), addr(b), addr(out), 64, 64, 64) if arity == 6 else fn(addr(a), addr(b), addr(out), m, k)
            assert rc == 0, (rc, M.last_error())
            hashes.add(h32(out))
        assert hashes == {want}, (sym, len(hashes))


def test_config_q16_1024_cubed():
    m = k = n = 1024
    a, b = M.gen_q16_sat(0xDEADBEEF ^ 0x1016, m * k, k * n, 13)
    note("det_matmul_q16_dev 1024^3 (saturating config)")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_q16_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n))
    np.testing.assert_array_equal(C, O.gemm_q16(a, b, m, k, n))


def test_config_i16_2048_cubed():
    m = k = n = 2048
    a, b = M.gen_i16(0xDEADBEEF ^ 0x2016, m * k, k * n)
    note("det_matmul_i16_dev 2048^3")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i16_dev(pa, pb, pc, m, k, n, s), [a, b], (m, n))
    rows = _sample_rows(m)
    np.testing.assert_array_equal(C[rows], O.gemm_i16_rows(a, b, m, k, n, rows))


@pytest.mark.parametrize("nb", [1, 8])
def test_config_gemv_q16_16384(nb):
    m = k = 16384
    W, X = M.gen_q16(0xDEADBEEF ^ 0x6E3F ^ nb, m * k, nb * k, 15)
    note(f"det_gemv_q16_dev 16384^2 nb={nb}")
    Y = _dev_run(lambda pw, px, py, s: M.lib().det_gemv_q16_dev(pw, px, py, m, k, nb, s), [W, X], (nb, m))
    if nb == 1:
        np.testing.assert_array_equal(Y, O.gemv_q16_batched(W, X, m, k, nb))
    else:
        rows = _sample_rows(m, 64)
        np.testing.assert_array_equal(Y[:, rows], O.gemv_q16_rows(W, X, m, k, nb, rows))


# ------------------------------------------------------------------ operands beyond 2 GiB
# The fast paths address operands through 32-bit buffer offsets and are
# chosen only below 2^31 bytes; a larger operand must take the generic
# (64-bit addressed) variant of the same computation.  One operand of each
# of these calls is 2.5 GiB; outputs are checked on rows sampled across it.

BIG_M = 40960           # x 16384 x 4 bytes = 2.5 GiB of Q16 W / f32 W


def _rows_spread(m, count=12):
    rows = _sample_rows(m, count)
    return np.unique(np.r_[rows, m // 2, (1 << 31) // (4 * 16384) - 1, (1 << 31) // (4 * 16384)])


def test_big_gemv_q16_batch1_and_8():
    m, k = BIG_M, 16384
    W, X = M.gen_q16(0xB16 ^ 1, m * k, 8 * k, 15)
    assert W.nbytes > (1 << 31)
    rows = _rows_spread(m)
    for nb in (1, 8):
        note(f"det_gemv_q16_dev {m}x{k} nb={nb} (W {W.nbytes >> 20} MiB)")
        Y = _dev_run(lambda pw, px, py, s: M.lib().det_gemv_q16_dev(pw, px, py, m, k, nb, s), [W, X[:nb * k]],
                     (nb, m), reps=1)
        np.testing.assert_array_equal(Y[:, rows], O.gemv_q16_rows(W, X[:nb * k], m, k, nb, rows))


def test_big_gemm_i8():
    m, k, n = 65536, 40960, 48            # A = 2.5 GiB
    A, B = M.gen_i8(0xB16 ^ 2, m * k, k * n)
    assert A.nbytes > (1 << 31)
    note(f"det_matmul_i8_dev {m}x{k}x{n} (A {A.nbytes >> 20} MiB)")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i8_dev(pa, pb, pc, m, k, n, s), [A, B], (m, n), reps=1)
    rows = np.unique(np.r_[_sample_rows(m, 12), (1 << 31) // k - 1, (1 << 31) // k])
    np.testing.assert_array_equal(C[rows], O.gemm_i8_rows(A, B, m, k, n, rows))


def test_big_gemm_q16_limb_path():
    m, k, n = BIG_M, 16384, 64            # A = 2.5 GiB: beyond the second-generation kernel's limit
    A, B = M.gen_q16(0xB16 ^ 3, m * k, k * n, 13)
    assert A.nbytes > (1 << 31)
    note(f"det_matmul_q16_dev {m}x{k}x{n} (A {A.nbytes >> 20} MiB)")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_q16_dev(pa, pb, pc, m, k, n, s), [A, B], (m, n), reps=1)
    rows = _rows_spread(m)
    np.testing.assert_array_equal(C[rows], O.gemm_q16_rows(A, B, m, k, n, rows))


def test_big_gemm_i16_limb_path():
    m, k, n = BIG_M, 32768, 48            # A = 2.5 GiB: 2 * M * K >= 2^31 rules out the interleaved-limb kernel
    assert 2 * m * k >= 1 << 31
    A, B = M.gen_i16(0xB16 ^ 5, m * k, k * n)
    note(f"det_matmul_i16_dev {m}x{k}x{n} (A {A.nbytes >> 20} MiB)")
    C = _dev_run(lambda pa, pb, pc, s: M.lib().det_matmul_i16_dev(pa, pb, pc, m, k, n, s), [A, B], (m, n), reps=1)
    rows = np.unique(np.r_[_sample_rows(m, 12), m // 2, (1 << 30) // k - 1, (1 << 30) // k])
    np.testing.assert_array_equal(C[rows], O.gemm_i16_rows(A, B, m, k, n, rows))


def test_big_host_calls_through_the_ring():
    # host-pointer calls whose buffers pass 4 GiB: the pinned ring's pieces
    # then sit at offsets beyond 2^32 and each of its four chunks is reused
    # about seventy times in one call; in (a 4.5 GiB W) and out (a 4.1 GiB C)
    L = M.lib()
    m, k = 73728, 16384
    W, x = M.gen_q16(0xB16 ^ 6, m * k, k, 15)
    assert W.nbytes > (1 << 32)
    y = np.full(m, 0x5A5A5A5A, np.int32)
    note(f"gemvq host {m}x{k} (W {W.nbytes >> 20} MiB through the ring)")
    assert L.gemvq(addr(W), addr(x), addr(y), m, k) == 0
    rows = np.unique(np.r_[_sample_rows(m, 12), (1 << 32) // (4 * k) - 1, (1 << 32) // (4 * k)])
    np.testing.assert_array_equal(y[rows], O.gemv_q16_rows(W, x, m, k, 1, rows).ravel())
    del W
    m, k, n = 33024, 16, 33000
    a, b = O.gen_i8(0xB16 ^ 7, m * k, k * n)
    c = np.empty(m * n, np.int32)
    assert c.nbytes > (1 << 32)
    note(f"gemmi8 host {m}x{k}x{n} (C {c.nbytes >> 20} MiB through the ring)")
    assert L.gemmi8(addr(a), addr(b), addr(c), m, k, n) == 0
    rows = np.unique(np.r_[_sample_rows(m, 12), (1 << 32) // (4 * n) - 1, (1 << 32) // (4 * n)])
    np.testing.assert_array_equal(c.reshape(m, n)[rows], O.gemm_i8_rows(a, b, m, k, n, rows))


def test_big_matmul_rmajor_f32():
    rows_n, cols = BIG_M, 16384           # W = 2.5 GiB
    W, x = M.gen_f32_unit(0xB16 ^ 4, rows_n * cols, cols)
    assert W.nbytes > (1 << 31)
    note(f"det_matmul_rmajor_f32_dev {rows_n}x{cols} (W {W.nbytes >> 20} MiB)")
    dW, dx, dy = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(x), M.DeviceBuffer(rows_n * 4)
    s = M.Stream()
    dy.fill(0xA5)
    M.check(M.lib().det_matmul_rmajor_f32_dev(dW.ptr, dx.ptr, dy.ptr, rows_n, cols, s.ptr))
    s.sync()
    y = dy.to_array(np.float32, (rows_n,))
    for r in _rows_spread(rows_n):
        want = O.matmul_rmajor_f32(W[r * cols:(r + 1) * cols], x, 1, cols)[0]
        assert y[r].view(np.uint32) == np.float32(want).view(np.uint32), r
    s.destroy()
