"""Seeded random-shape sweep over every op of the path, each result against
the CPU oracle: int8 / Q16 / int16 GEMM through det_matmul_ws_dev (device
operands, exactly the reported workspace, bases one element off the 16-byte
grid in a third of the cases) and through the host-pointer det_matmul_*
calls; the Q16 GEMV at batch 1..9, the int16 GEMV, the Q16 / L1 / int16
dots and the strict-FP f32 rows at random lengths; the Q16 FFT at random
sizes and batches.  Shapes mix tiny, odd, near-power-of-two and mid-size
dimensions so that the router's every branch is drawn (tiny direct
kernels, MFMA kernels, repack, K split, limb kernels).  GEMM rows are
sampled (first, last and three random ones); everything else is checked
whole."""
import numpy as np
import pytest

import mind_amd as M
import oracle as O

pytestmark = pytest.mark.gpu

OPS = {"i8": (M.DET_OP_I8, np.int8, O.gemm_i8_rows), "q16": (M.DET_OP_Q16, np.int32, O.gemm_q16_rows),
       "i16": (M.DET_OP_I16, np.int16, O.gemm_i16_rows)}
HOST = {"i8": M.det_matmul_i8, "q16": M.det_matmul_q16, "i16": M.det_matmul_i16}


def _dim(rng):
    r = rng.random()
    if r < 0.3:
        return int(rng.integers(1, 65))
    if r < 0.55:
        return int(rng.integers(65, 700))
    if r < 0.8:
        return int(rng.choice([16, 64, 128, 256, 512, 768, 1024, 1040, 2048])) + int(rng.choice([0, 0, -1, 1, 16, -16]))
    return int(rng.integers(700, 2300))


def _note(msg):
    import sys
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


@pytest.mark.parametrize("seed", [101, 202])
def test_random_gemm_shapes(seed):
    rng = np.random.default_rng(seed)
    L, s = M.lib(), M.Stream()
    done = 0
    while done < 150:
        name = ("i8", "q16", "i16")[int(rng.integers(0, 3))]
        op, dt, rowsf = OPS[name]
        m, k, n = max(1, _dim(rng)), max(1, _dim(rng)), max(1, _dim(rng))
        if m * k + k * n > 6_000_000 or m * n > 4_000_000:
            continue
        sd = int(rng.integers(0, 1 << 30))
        if name == "i8":
            a, b = O.gen_i8(sd, m * k, k * n)
        elif name == "q16":
            a, b = O.gen_q16(sd, m * k, k * n, shift=int(rng.choice([0, 12])))
        else:
            a, b = O.gen_i16(sd, m * k, k * n)
        rows = np.array(sorted(set([0, m - 1] + list(rng.integers(0, m, 3)))), np.int64)
        want = rowsf(a, b, m, k, n, rows)
        host = rng.random() < 0.3
        _note(f"sweep {seed} #{done} {name} {m}x{k}x{n} host={host} gen={sd}")
        if host:
            c = HOST[name](a.reshape(m, k), b.reshape(k, n))
        else:
            off = int(rng.choice([0, 0, 1]))
            da = M.DeviceBuffer.from_array(np.concatenate([np.zeros(off, dt), a]))
            db = M.DeviceBuffer.from_array(np.concatenate([np.zeros(off, dt), b]))
            dc = M.DeviceBuffer(m * n * 4)
            dc.fill(0xA5)
            wsb = L.det_workspace_bytes(op, m, k, n)
            ws = M.DeviceBuffer(max(wsb, 256))
            esz = np.dtype(dt).itemsize
            M.check(L.det_matmul_ws_dev(op, da.ptr + off * esz, db.ptr + off * esz, dc.ptr, m, k, n, ws.ptr, wsb,
                                        s.ptr))
            s.sync()
            c = dc.to_array(np.int32, (m, n))
            for x in (da, db, dc, ws):
                x.free()
        np.testing.assert_array_equal(c[rows], want, err_msg=f"{name} {m}x{k}x{n} host={host} gen={sd}")
        done += 1
    s.destroy()


def test_random_gemv_dot_rows_fft():
    rng = np.random.default_rng(303)
    for i in range(60):   # Q16 GEMV, batch 1..9, and the int16 GEMV
        m, k, nb = max(1, _dim(rng)), max(1, _dim(rng)), int(rng.integers(1, 10))
        W, X = O.gen_q16(1000 + i, m * k, nb * k, shift=int(rng.choice([0, 12])))
        _note(f"sweep gemv #{i} {m}x{k} nb={nb}")
        got = M.det_gemv_q16(W.reshape(m, k), X.reshape(nb, k))
        np.testing.assert_array_equal(got, O.gemv_q16_batched(W, X, m, k, nb).reshape(nb, m))
        W16, x16 = O.gen_i16(2000 + i, m * k, k)
        np.testing.assert_array_equal(M.det_gemv_i16(W16.reshape(m, k), x16), O.gemv_i16(W16, x16, m, k))
    for i in range(60):   # the three integer dots
        n = int(rng.choice([int(rng.integers(0, 40)), int(rng.integers(40, 20000)), int(rng.integers(20000, 300000))]))
        a, b = O.gen_q16(3000 + i, n, n, shift=int(rng.choice([0, 12])))
        _note(f"sweep dots #{i} n={n}")
        assert M.dot_q16(a, b) == O.dot_q16(a, b)
        assert M.dot_l1_q16(a, b) == O.dot_l1_q16(a, b)
        a16, b16 = (a >> 16).astype(np.int16), a.astype(np.int16)
        assert M.dot_i16(a16, b16) == O.dot_i16(a16, b16)
    for i in range(30):   # strict-FP f32 rows
        rows, cols = max(1, _dim(rng)), max(1, _dim(rng))
        W, x = O.gen_f32_unit(4000 + i, rows * cols, cols)
        _note(f"sweep f32 rows #{i} {rows}x{cols}")
        got = M.matmul_rmajor_f32(W.reshape(rows, cols), x)
        assert np.array_equal(got.view(np.uint32), O.matmul_rmajor_f32(W, x, rows, cols).view(np.uint32))
    for i in range(30):   # Q16 FFT
        logn = int(rng.integers(0, 13))
        n, batch = 1 << logn, int(rng.choice([1, int(rng.integers(2, 40)), int(rng.integers(40, 700))]))
        x = rng.integers(-(1 << 30), 1 << 30, (2, batch, n))
        re, im = np.ascontiguousarray(x[0]), np.ascontiguousarray(x[1])
        tw = O.fft_twiddles(n) if n >= 2 else np.zeros(2, np.int64)
        _note(f"sweep fft #{i} n={n} batch={batch}")
        got_r, got_i = M.fft_q16(re, im, tw, logn)
        for f in sorted({0, batch // 2, batch - 1}):
            wr, wi = O.fft_q16(re[f], im[f], tw, logn)
            assert np.array_equal(got_r[f], wr) and np.array_equal(got_i[f], wi), (n, batch, f)
