#!/usr/bin/env python3
"""Benchmark of the deterministic integer GEMM / GEMV hot path on one MI355X.

Headline (the ``value`` of the JSON line): det_matmul_i8 at 4096^3, int8 in,
exact int32 out, in TOP/s (2*M*N*K / time).  A "step" is one call of the
kernel over device-resident synthetic inputs (the reference bench LCG,
benches/det_matmul_i8.rs:221-226).  The secondary configs of the same
metric (Q16.16 GEMM 1024^3 and 4096^3, int16 GEMM 2048^3, Q16 GEMV 16384^2
at batch 1 and 8, the strict-FP f32 row matmul 16384^2, the batched Q16 FFT
(n = 256, 2^18 transforms; Q16-range and +-2^40 inputs), the int8 MLP layer
4096x4096x11008 and the 8192^3 probe)
are timed the same way and reported under "secondary".  --vendor-ref adds,
for context only, the vendor int8 GEMM (torch._int_mm) on the headline shape.

Timing: HIP events recorded on the stream the kernels are launched on,
around exactly K steps after W warm-up steps and --settle seconds (0.5) of
back-to-back running (the clock controller's transient ends within that),
with a device synchronisation on both sides; ms_per_step is the host wall
clock over the same region.
Every timed output is checked bit-exact against the CPU oracle (sampled rows
at these sizes) before its number is reported.

By default the run also times the reference benches' own sweep shapes
(host-pointer call and device-resident, under "reference_sweeps") and the
end-to-end host-pointer calls of the headline shapes (PCIe included, under
"host_abi"); --no-host-abi skips both.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle S] [--only q16_1024,...] [--vendor-ref]
                       [--no-host-abi]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import mind_amd as M  # noqa: E402

METRIC = "int8 & Q16.16 det-GEMM TOPS at 4096³; Q16 GEMV HBM GB/s; bit-exact vs CPU"
PEAK_INT8_TOPS = 5000.0          # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0            # MI355X HBM3E, 8 TB/s
SEED = 0xDEADBEEF


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


SETTLE_S = 0.5                   # back-to-back running before each timed region (--settle)


def time_steps(launch, steps: int, warmup: int, stream, settle: float | None = None) -> tuple[float, float]:
    """Return (event ms per step, wall ms per step) over exactly `steps` launches.

    After the `warmup` launches the workload keeps running back to back for
    SETTLE_S seconds before the timed region: the GPU's clock controller
    takes tens of milliseconds to settle after a burst starts (measured: the
    batched GEMV's calls take ~200 us at first, up to ~260 us a few ms later
    and 203 us from then on), so a short timed region right after a short
    warm-up times that transient, not the sustained rate."""
    for _ in range(warmup):
        launch()
    M.check(M.lib().det_device_sync())
    t_end = time.perf_counter() + (SETTLE_S if settle is None else settle)
    while time.perf_counter() < t_end:
        for _ in range(8):
            launch()
        M.check(M.lib().det_device_sync())
    e0, e1 = M.Event(), M.Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        launch()
    e1.record(stream)
    M.check(M.lib().det_device_sync())
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ev = e0.elapsed_ms(e1) / steps
    e0.destroy(); e1.destroy()
    return ev, wall


def sample_rows(m: int, count: int = 4) -> np.ndarray:
    rng = np.random.default_rng(m + count)
    return np.array(sorted(set([0, m - 1] + list(rng.integers(0, m, count)))), np.int64)


# ---------------------------------------------------------------- workloads

def gemm_workload(kind: str, m: int, k: int, n: int, steps: int, warmup: int, stream, seed_tag: int,
                  check_rows: int = 4, keep_output: bool = False):
    L = M.lib()
    seed = SEED ^ seed_tag
    if kind == "i8":
        a, b = M.gen_i8(seed, m * k, k * n)
    elif kind == "i8_mlp":
        a = M.gen_i8_gauss(seed, m * k)
        b = M.gen_i8_sym127(seed ^ 1, k * n)
    elif kind == "q16":
        a, b = M.gen_q16_sat(seed, m * k, k * n, 13)
    elif kind == "i16":
        a, b = M.gen_i16(seed, m * k, k * n)
    else:
        raise ValueError(kind)
    da, db = M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b)
    dc = M.DeviceBuffer(m * n * 4)
    dc.fill(0xA5)
    op = {"i8": M.DET_OP_I8, "i8_mlp": M.DET_OP_I8, "q16": M.DET_OP_Q16, "i16": M.DET_OP_I16}[kind]
    ws_bytes = L.det_workspace_bytes(op, m, k, n)
    ws = M.DeviceBuffer(ws_bytes) if ws_bytes else None
    sp = stream.ptr

    def launch():
        M.check(L.det_matmul_ws_dev(op, da.ptr, db.ptr, dc.ptr, m, k, n, ws.ptr if ws else None, ws_bytes, sp))

    ev, wall = time_steps(launch, steps, warmup, stream)
    per_launch = None
    if keep_output:   # the headline: also 64 individually timed launches (the reference bench's median)
        e0, e1 = M.Event(), M.Event()
        samples = []
        for _ in range(64):
            e0.record(stream)
            launch()
            e1.record(stream)
            M.check(L.det_device_sync())
            samples.append(e0.elapsed_ms(e1))
        e0.destroy(); e1.destroy()
        samples.sort()
        per_launch = {"median_ms": samples[32], "p10_ms": samples[6], "p90_ms": samples[57]}
    C = dc.to_array(np.int32, (m, n))
    rows = sample_rows(m, check_rows)
    got = C[rows].copy()

    def verify(O):
        """Sampled rows of the timed output against the CPU oracle."""
        fn = {"i8": O.gemm_i8_rows, "i8_mlp": O.gemm_i8_rows, "q16": O.gemm_q16_rows, "i16": O.gemm_i16_rows}[kind]
        return bool(np.array_equal(got, fn(a, b, m, k, n, rows)))

    for buf in (da, db, dc, ws):
        if buf is not None:
            buf.free()
    out = {"ms": ev, "wall_ms": wall, "ops": 2.0 * m * n * k, "verify": verify, "checked_rows": len(rows),
           "per_launch": per_launch}
    if keep_output:
        out["C"], out["A"], out["B"] = C, a, b
    return out


def gemv_workload(m: int, k: int, nb: int, steps: int, warmup: int, stream, seed_tag: int,
                  keep_output: bool = False):
    L = M.lib()
    W, X = M.gen_q16(SEED ^ seed_tag, m * k, nb * k, 15)
    dw, dx = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(X)
    dy = M.DeviceBuffer(m * nb * 4)
    dy.fill(0xA5)
    sp = stream.ptr
    # the caller's workspace (det_gemv_q16_ws_dev), as the GEMMs take theirs
    # through det_matmul_ws_dev: no arena event ordering between calls
    ws_bytes = L.det_gemv_workspace_bytes(m, k, nb)
    ws = M.DeviceBuffer(ws_bytes) if ws_bytes else None

    def launch():
        M.check(L.det_gemv_q16_ws_dev(dw.ptr, dx.ptr, dy.ptr, m, k, nb, ws.ptr if ws else None, ws_bytes, sp))

    ev, wall = time_steps(launch, steps, warmup, stream)
    Y = dy.to_array(np.int32, (nb, m))
    rows = sample_rows(m, 32)
    got = Y[:, rows].copy()
    Wr = np.ascontiguousarray(W.reshape(m, k)[rows]).ravel()

    def verify(O):
        return bool(np.array_equal(got, O.gemv_q16_batched(Wr, X, len(rows), k, nb)))

    for buf in (dw, dx, dy, ws):
        if buf is not None:
            buf.free()
    nbytes = 4.0 * m * k + 4.0 * k * nb + 4.0 * m * nb
    out = {"ms": ev, "wall_ms": wall, "bytes": nbytes, "verify": verify, "checked_rows": len(rows)}
    if keep_output:
        out["W"], out["X"], out["Y"] = W, X, Y
    return out


def f32_rows_workload(rows: int, cols: int, steps: int, warmup: int, stream, seed_tag: int):
    """Strict-FP f32 row-major matmul y = W x (the reference's
    matmul_rmajor_f32 schedule); W and x from the reference f32 generator."""
    L = M.lib()
    W, x = M.gen_f32_unit(SEED ^ seed_tag, rows * cols, cols)
    dw, dx = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(x)
    dy = M.DeviceBuffer(rows * 4)
    dy.fill(0xA5)
    sp = stream.ptr

    def launch():
        M.check(L.det_matmul_rmajor_f32_dev(dw.ptr, dx.ptr, dy.ptr, rows, cols, sp))

    ev, wall = time_steps(launch, steps, warmup, stream)
    y = dy.to_array(np.float32, (rows,))
    sel = sample_rows(rows, 32)
    got = y[sel].copy()
    Wr = np.ascontiguousarray(W.reshape(rows, cols)[sel]).ravel()

    def verify(O):
        want = O.matmul_rmajor_f32(Wr, x, len(sel), cols)
        return bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))

    for buf in (dw, dx, dy):
        buf.free()
    nbytes = 4.0 * rows * cols + 4.0 * cols + 4.0 * rows
    return {"ms": ev, "wall_ms": wall, "bytes": nbytes, "verify": verify, "checked_rows": len(sel)}


def fft_workload(logn: int, batch: int, steps: int, warmup: int, stream, seed_tag: int, amp: int = 65536):
    """Batched Q16.16 FFT (fft256 semantics) of device-resident re / im
    [batch][n], out of place (det_fft_q16_oop_dev): every step transforms the
    same input, whose samples are uniform in [-amp, amp) (65536: harness.c's
    range; 2^40 forces the int64 path)."""
    L = M.lib()
    n = 1 << logn
    rng = np.random.default_rng(SEED ^ seed_tag)
    x = rng.integers(-amp, amp, (2, batch, n)).astype(np.int64)
    tw = M.fft_twiddles(n)
    sre, sim = M.DeviceBuffer.from_array(x[0]), M.DeviceBuffer.from_array(x[1])
    dre, dim_, dtw = M.DeviceBuffer(batch * n * 8), M.DeviceBuffer(batch * n * 8), M.DeviceBuffer.from_array(tw)
    dre.fill(0xA5); dim_.fill(0xA5)
    sp = stream.ptr

    def launch():
        M.check(L.det_fft_q16_oop_dev(sre.ptr, sim.ptr, dre.ptr, dim_.ptr, dtw.ptr, logn, n, batch, sp))

    ev, wall = time_steps(launch, steps, warmup, stream)
    sel = sample_rows(batch, 16)
    got_r = dre.to_array(np.int64, (batch, n))[sel]
    got_i = dim_.to_array(np.int64, (batch, n))[sel]
    x_sel = x[:, sel].copy()

    def verify(O):
        out = [O.fft_q16(x_sel[0][j], x_sel[1][j], tw, logn) for j in range(len(sel))]
        return bool(np.array_equal(np.stack([o[0] for o in out]), got_r) and
                    np.array_equal(np.stack([o[1] for o in out]), got_i))

    for buf in (sre, sim, dre, dim_, dtw):
        buf.free()
    return {"ms": ev, "wall_ms": wall, "bytes": 2.0 * 16 * batch * n, "ffts": batch, "verify": verify,
            "checked_rows": len(sel)}


def cpu_fft_reference(logn: int, seconds: float = 2.0):
    """The reference's C FFT (bench/fft/fft_ref.c, built into oracle/_ref),
    single thread, in place on one fixed buffer like its harness."""
    import oracle as O

    R = O.fft_ref_lib()
    if R is None:
        return None
    n = 1 << logn
    re, im = O.fft_input_harness(0x1234567, n)
    tw = O.fft_twiddles(n)
    a, b, t = re.ctypes.data, im.ctypes.data, tw.ctypes.data
    for _ in range(2000):
        R.fft256_c(a, b, t, logn, n)
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(2000):
            R.fft256_c(a, b, t, logn, n)
        calls += 2000
    dt = time.perf_counter() - t0
    return {"ns_per_fft": round(dt / calls * 1e9, 1), "calls": calls, "cores": 1, "kind": "reference",
            "note": "bench/fft/fft_ref.c compiled -O3 -march=x86-64-v3 into oracle/_ref, called through ctypes "
                    "(the per-call ctypes overhead is included)"}


def host_abi_timings(reps: int = 3) -> dict:
    """End-to-end time of the reference-ABI host-pointer entry points (H2D,
    kernel, D2H on the library stream, synchronous), pageable numpy buffers:
    the PCIe-inclusive rate a drop-in caller sees.  Never the bench value."""
    L = M.lib()
    res = {}

    def timed(fn):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            rc = fn()
            ts.append(time.perf_counter() - t0)
            M.check(rc)
        return sorted(ts)[len(ts) // 2] * 1e3

    m = k = n = 4096
    a, b = M.gen_i8(SEED ^ 0x4096, m * k, k * n)
    c = np.empty(m * n, np.int32)
    ms = timed(lambda: L.gemmi8(a.ctypes.data, b.ctypes.data, c.ctypes.data, m, k, n))
    res["gemmi8_4096"] = {"ms": round(ms, 3), "tops": round(2.0 * m * n * k / ms / 1e9, 1),
                          "pcie_bytes": a.nbytes + b.nbytes + c.nbytes}
    del a, b, c
    m = k = n = 1024
    a, b = M.gen_q16_sat(SEED ^ 0x1016, m * k, k * n, 13)
    c = np.empty(m * n, np.int32)
    ms = timed(lambda: L.gemmqmm(a.ctypes.data, b.ctypes.data, c.ctypes.data, m, k, n))
    res["gemmqmm_1024"] = {"ms": round(ms, 3), "q16_tops": round(2.0 * m * n * k / ms / 1e9, 2),
                           "pcie_bytes": a.nbytes + b.nbytes + c.nbytes}
    del a, b, c
    M_, K_ = 16384, 16384
    W, x = M.gen_q16(SEED ^ 0x6E3F, M_ * K_, K_, 15)
    y = np.empty(M_, np.int32)
    ms = timed(lambda: L.gemvq(W.ctypes.data, x.ctypes.data, y.ctypes.data, M_, K_))
    res["gemvq_16384"] = {"ms": round(ms, 3), "gbs": round(4.0 * M_ * K_ / ms / 1e6, 1), "pcie_bytes": W.nbytes}
    del W, x, y
    Wf, xf = M.gen_f32_unit(SEED ^ 0xF32, M_ * K_, K_)
    yf = np.empty(M_, np.float32)
    ms = timed(lambda: L.mmf32(Wf.ctypes.data, xf.ctypes.data, yf.ctypes.data, M_, K_))
    res["mmf32_16384"] = {"ms": round(ms, 3), "gbs": round(4.0 * M_ * K_ / ms / 1e6, 1), "pcie_bytes": Wf.nbytes}
    del Wf, xf, yf
    tw = M.fft_twiddles(256)
    re = np.random.default_rng(1).integers(-65536, 65536, 256).astype(np.int64)
    im = re[::-1].copy()
    ms = timed(lambda: L.fft256(re.ctypes.data, im.ctypes.data, tw.ctypes.data, 8, 256))
    res["fft256_one"] = {"us": round(ms * 1e3, 1), "note": "one 256-point transform per call (4 KiB each way)"}
    batch = 1 << 18
    R = np.random.default_rng(2).integers(-65536, 65536, (batch, 256)).astype(np.int64)
    I = R[::-1].copy()
    ms = timed(lambda: L.det_fft_q16(R.ctypes.data, I.ctypes.data, tw.ctypes.data, 8, 256, batch))
    res["det_fft_q16_2e18"] = {"ms": round(ms, 3), "ns_per_fft": round(ms * 1e6 / batch, 2),
                               "pcie_bytes": 2 * (R.nbytes + I.nbytes)}
    res["note"] = ("median of %d synchronous calls after one warm-up; pageable host buffers; times include the "
                   "host-to-device and device-to-host copies" % reps)
    return res


# The reference benches' own sweeps: benches/det_matmul_i8.rs:86 and
# det_matmul_q16.rs:82 (n^3, n = 16 .. 512), det_matmul_i16.rs:77 (int16 GEMV
# n x n, n = 64, 256, 512), det_gemv_q16_mt.rs:62 (the GEMV shapes including
# the 11922 x 384 routing shape) and its 512 x 130 anchor (:76-78).  Seeds as
# the benches draw them: the anchor shape 0xDEADBEEF, the others
# 0xDEADBEEF00000000 ^ n (GEMV: ^ (m << 20 ^ k)).
REF_SWEEPS = ([("gemmi8", n) for n in (16, 64, 128, 256, 512)] +
              [("gemmqmm", n) for n in (16, 64, 128, 256, 512)] +
              [("mmi16", n) for n in (64, 256, 512)] +
              [("gemvq", mk) for mk in ((64, 64), (128, 96), (256, 130), (11922, 384), (512, 130))])


def reference_sweeps(stream, steps: int) -> dict:
    """Each shape of the reference benches' sweeps three ways: the host-pointer
    call of the symbol its bench dlsyms (gemmi8, the fused Q16 GEMM under its
    harness name gemmqmm, mmi16, gemvq), timed as its report_gmacs does
    (median of 64 calls after 8 warm-up calls, PCIe copies included:
    benches/det_matmul_i8.rs:363-408); the same work on device-resident
    operands (HIP events over `steps` calls after a 0.1 s settle); and both
    outputs kept for the exactness check against the oracle."""
    L = M.lib()
    sp = stream.ptr
    out = {}
    for sym, shape in REF_SWEEPS:
        if sym == "gemvq":
            m, k = shape
            seed = 0xDEADBEEF if (m, k) == (512, 130) else 0xDEADBEEF00000000 ^ ((m << 20) ^ k)
            W, x = M.gen_q16(seed, m * k, k)
            y = np.empty(m, np.int32)
            host = lambda: L.gemvq(W.ctypes.data, x.ctypes.data, y.ctypes.data, m, k)
            dw, dx, dy = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(x), M.DeviceBuffer(m * 4)
            dev = lambda: M.check(L.det_gemv_q16_ws_dev(dw.ptr, dx.ptr, dy.ptr, m, k, 1, None, 0, sp))
            macs, name, ins, outs = m * k, f"gemvq_{m}x{k}", (W, x), (y, dy, (m,))
        elif sym == "mmi16":
            n = shape
            W, x = M.gen_i16(0xDEADBEEF if n == 256 else 0xDEADBEEF00000000 ^ n, n * n, n)
            y = np.empty(n, np.int32)
            host = lambda: L.mmi16(W.ctypes.data, x.ctypes.data, y.ctypes.data, n, n)
            dw, dx, dy = M.DeviceBuffer.from_array(W), M.DeviceBuffer.from_array(x), M.DeviceBuffer(n * 4)
            dev = lambda: M.check(L.det_gemv_i16_dev(dw.ptr, dx.ptr, dy.ptr, n, n, sp))
            macs, name, ins, outs = n * n, f"mmi16_{n}", (W, x), (y, dy, (n,))
        else:
            n = shape
            seed = 0xDEADBEEF if n == 64 else 0xDEADBEEF00000000 ^ n
            a, b = M.gen_i8(seed, n * n, n * n) if sym == "gemmi8" else M.gen_q16(seed, n * n, n * n)
            op = M.DET_OP_I8 if sym == "gemmi8" else M.DET_OP_Q16
            y = np.empty(n * n, np.int32)
            host = lambda: getattr(L, sym)(a.ctypes.data, b.ctypes.data, y.ctypes.data, n, n, n)
            dw, dx, dy = M.DeviceBuffer.from_array(a), M.DeviceBuffer.from_array(b), M.DeviceBuffer(n * n * 4)
            wsb = L.det_workspace_bytes(op, n, n, n)
            ws = M.DeviceBuffer(wsb) if wsb else None
            dev = lambda: M.check(L.det_matmul_ws_dev(op, dw.ptr, dx.ptr, dy.ptr, n, n, n, ws.ptr if ws else None,
                                                      wsb, sp))
            macs, name, ins, outs = n ** 3, f"{sym}_{n}", (a, b), (y, dy, (n * n,))
        for _ in range(8):
            M.check(host())
        samples = []
        for _ in range(64):
            t0 = time.perf_counter()
            rc = host()
            samples.append(time.perf_counter() - t0)
            M.check(rc)
        host_s = sorted(samples)[32]
        dy.fill(0xA5)
        ev, _ = time_steps(dev, steps, 2, stream, settle=0.1)
        got_dev = dy.to_array(np.int32, outs[2])
        out[name] = {"host_call_us": round(host_s * 1e6, 2), "host_gmac_per_s": round(macs / host_s / 1e9, 3),
                     "device_us": round(ev * 1e3, 2), "device_gmac_per_s": round(macs / (ev * 1e-3) / 1e9, 1),
                     "_check": (sym, shape, ins, outs[0].copy(), got_dev)}
        for buf in (dw, dx, dy):
            buf.free()
        if sym in ("gemmi8", "gemmqmm") and ws is not None:
            ws.free()
        log(f"sweep {name}: host call {out[name]['host_call_us']:.1f} us ({out[name]['host_gmac_per_s']:.2f} GMAC/s), "
            f"device {out[name]['device_us']:.2f} us")
    return out


def verify_sweep(O, sym, shape, ins, host_out, dev_out) -> bool:
    """Both outputs of one sweep shape against the whole oracle output."""
    if sym == "gemvq":
        m, k = shape
        want = O.gemv_q16(ins[0], ins[1], m, k)
    elif sym == "mmi16":
        want = O.gemv_i16(ins[0], ins[1], shape, shape)
    elif sym == "gemmi8":
        want = O.gemm_i8(ins[0], ins[1], shape, shape, shape)
    else:
        want = O.gemm_q16(ins[0], ins[1], shape, shape, shape)
    want = np.asarray(want).ravel()
    return bool(np.array_equal(host_out.ravel(), want) and np.array_equal(dev_out.ravel(), want))


def vendor_int8_child(steps: int, settle_s: float) -> None:
    """Child-process body of --vendor-ref: time the vendor int8 GEMM
    (torch._int_mm, which dispatches to hipBLASLt on ROCm) on the headline
    shape with torch's own events and print one JSON line.  B is passed
    row-major (the reference ABI's layout) and, for comparison, column-major.
    Context only, never part of the product path; it runs in its own process
    because torch bundles its own HIP runtime."""
    import torch
    out = {"impl": "torch._int_mm (hipBLASLt)", "torch": torch.__version__}
    m = k = n = 4096
    a = torch.randint(-128, 128, (m, k), dtype=torch.int8, device="cuda")
    b = torch.randint(-128, 128, (k, n), dtype=torch.int8, device="cuda")
    for name, bb in (("b_row_major", b), ("b_col_major", b.t().contiguous().t())):
        for _ in range(5):
            torch._int_mm(a, bb)
        torch.cuda.synchronize()
        t_end = time.perf_counter() + settle_s   # the same settle phase as time_steps
        while time.perf_counter() < t_end:
            for _ in range(8):
                torch._int_mm(a, bb)
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            torch._int_mm(a, bb)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / steps * 1e3
        out[name] = {"us": round(us, 2), "tops": round(2.0 * m * n * k / us / 1e6, 1)}
    print(json.dumps(out), flush=True)


def vendor_int8_reference(steps: int, settle_s: float) -> dict:
    """Run vendor_int8_child in a child process.  Called before this process
    makes any HIP call, so the child starts from a process that has not
    touched the GPU."""
    import subprocess
    p = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-child", "--steps", str(steps),
                        "--settle", str(settle_s)],
                       capture_output=True, text=True, timeout=600)
    lines = [x for x in p.stdout.splitlines() if x.startswith("{")]
    if p.returncode != 0 or not lines:
        return {"error": f"vendor child exited {p.returncode}", "stderr_tail": p.stderr[-400:]}
    res = json.loads(lines[-1])
    for name in ("b_row_major", "b_col_major"):
        log(f"vendor {name}: {res[name]['us']:.1f} us  {res[name]['tops']:.1f} TOP/s")
    return res


def measure_peaks(stream) -> dict:
    """Roofline denominators measured on this GPU: int8 MFMA issue rate from
    a register-only MFMA loop, HBM read and copy bandwidth over 1 GiB."""
    L = M.lib()
    sp = stream.ptr
    ops_in = M.DeviceBuffer.from_array(np.arange(128 * 16, dtype=np.uint8))
    blocks, iters = 2048, 4096
    out = M.DeviceBuffer(blocks * 256 * 4)
    # shape 2 cycles 8 operand pairs of random bytes (the data a GEMM sees)
    rnd_in = M.DeviceBuffer.from_array(np.random.default_rng(0x5EED).integers(0, 256, 1024 * 16, dtype=np.uint8))
    mfma_tops = {}
    for shape, per_iter, name, src in ((0, 8 * 16384, "16x16x64", ops_in), (1, 8 * 32768, "32x32x32", ops_in),
                                       (2, 16 * 32768, "32x32x32_random_operands", rnd_in),
                                       (3, 32 * 16384, "16x16x64_random_operands", rnd_in)):
        def mfma():
            M.check(L.det_probe_mfma_i8(src.ptr, out.ptr, blocks, iters, shape, sp))

        ms, _ = time_steps(mfma, 3, 1, stream)
        mfma_tops[name] = round(blocks * 4 * iters * per_iter * 2 / (ms * 1e-3) / 1e12, 1)
    rnd_in.free()
    nbytes = 1 << 30
    src, dst = M.DeviceBuffer(nbytes), M.DeviceBuffer(nbytes)
    src.fill(0x5A)
    red = M.DeviceBuffer(8192 * 4)
    red.fill(0)

    def rd():
        M.check(L.det_probe_read(src.ptr, nbytes, red.ptr, 8192, sp))

    ms_r, _ = time_steps(rd, 5, 2, stream)

    def cp():
        M.check(L.det_copy_dev(dst.ptr, src.ptr, nbytes, sp))

    ms_c, _ = time_steps(cp, 5, 2, stream)
    for b in (ops_in, out, src, dst, red):
        b.free()
    return {"mfma_i8_tops": mfma_tops, "hbm_read_gbs": round(nbytes / (ms_r * 1e-3) / 1e9, 1),
            "hbm_copy_gbs": round(2 * nbytes / (ms_c * 1e-3) / 1e9, 1),
            "note": "register-only int8 MFMA loops (inline asm, 8 independent chains, 32 waves/CU): one constant operand pair "
                    "for all MFMAs, or 8 pairs of random bytes cycled (the clock under int8 MFMA load drops with "
                    "operand bit toggles, so the random-operand rate is the one a GEMM's data can reach); "
                    "1 GiB streaming read; 1 GiB copy (read+write)"}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_int8(A: np.ndarray, B: np.ndarray, C_gpu: np.ndarray, m: int, k: int, n: int) -> dict:
    """The multithreaded CPU restatement of the reference's MT int8 path
    (oracle/det_cpu_mt.c), timed on this host's cores on a bounded row band
    of the same 4096^3 workload."""
    import oracle as O

    L = O.lib()
    budget_s = float(os.environ.get("DET_CPU_BASELINE_SECONDS", "10"))

    def run(rows):
        c = np.empty(rows * n, np.int32)
        t0 = time.perf_counter()
        L.det_cpu_gemm_i8(A.ctypes.data, B.ctypes.data, c.ctypes.data, rows, k, n)
        return time.perf_counter() - t0, c.reshape(rows, n)

    probe = 64
    t, _ = run(probe)
    rows = int(min(m, max(probe, (budget_s / 3) / max(t, 1e-6) * probe)))
    rows = max(probe, rows // 64 * 64)
    # the whole workload may take well under the budget on a wide host:
    # repeat it until the budget is spent (at least 3 calls) and take the median
    times = []
    c = None
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 1000):
        dt, c = run(rows)
        times.append(dt)
    exact = bool(np.array_equal(c, C_gpu[:rows])) and bool(
        np.array_equal(c[[0, rows - 1]], O.gemm_i8_rows(A, B, m, k, n, [0, rows - 1])))
    if not exact:
        raise SystemExit("CPU baseline output differs from the GPU/oracle output")
    med = sorted(times)[len(times) // 2]
    return {"value": 2.0 * rows * n * k / med / 1e12, "unit": "TOP/s", "cores": int(L.det_cpu_threads_for(rows)),
            "kind": "port",
            "sample": f"rows 0..{rows - 1} of the 4096x4096x4096 int8 GEMM (median of {len(times)} calls, "
                      f"{med:.3f} s each, {sum(times):.1f} s in all); "
                      f"oracle/det_cpu_mt.c restatement of the reference MT BLIS int8 path, "
                      f"-O3 -march=x86-64-v3, output equal to the GPU rows",
            "host_cpus": os.cpu_count(), "cpu_model": _cpu_model()}


def _time_median(fn, reps: int) -> float:
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baseline_q16(A: np.ndarray, B: np.ndarray, C_gpu: np.ndarray, m: int, k: int, n: int) -> dict:
    """The MT CPU restatement of the reference's Q16 path (BLIS 4x8 i64
    microkernel) on the whole Q16 workload; output equal to the GPU's."""
    import oracle as O

    L = O.lib()
    c = np.empty(m * n, np.int32)
    run = lambda: L.det_cpu_gemm_q16(A.ctypes.data, B.ctypes.data, c.ctypes.data, m, k, n)
    run()
    if not np.array_equal(c.reshape(m, n), C_gpu):
        raise SystemExit("Q16 CPU baseline output differs from the GPU output")
    t = _time_median(run, 33)
    return {"value": 2.0 * m * n * k / t / 1e12, "unit": "Q16 TOP/s (2*MNK/t)", "gmac_per_s": m * n * k / t / 1e9,
            "cores": int(L.det_cpu_threads_for(m)), "kind": "port",
            "sample": f"the whole {m}x{k}x{n} Q16 GEMM (median of 33, {t * 1e3:.1f} ms each); oracle/det_cpu_mt.c "
                      f"restatement of the reference MT Q16 path, output equal to the GPU output",
            "cpu_model": _cpu_model()}


def cpu_baseline_gemv(W: np.ndarray, x: np.ndarray, y_gpu: np.ndarray, m: int, k: int) -> dict:
    """The MT CPU restatement of the reference's Q16 GEMV row bands on the
    whole batch-1 workload; output equal to the GPU's."""
    import oracle as O

    L = O.lib()
    y = np.empty(m, np.int32)
    run = lambda: L.det_cpu_gemv_q16(W.ctypes.data, x.ctypes.data, y.ctypes.data, m, k)
    run()
    if not np.array_equal(y, y_gpu.ravel()):
        raise SystemExit("GEMV CPU baseline output differs from the GPU output")
    t = _time_median(run, 33)
    nbytes = 4.0 * m * k + 4.0 * k + 4.0 * m
    return {"value": nbytes / t / 1e9, "unit": "GB/s", "ms": t * 1e3, "cores": int(L.det_cpu_threads_for(m)),
            "kind": "port",
            "sample": f"the whole {m}x{k} batch-1 Q16 GEMV (median of 33); oracle/det_cpu_mt.c restatement of "
                      f"__mind_blas_gemv_q16_mt's row bands, output equal to the GPU output",
            "cpu_model": _cpu_model()}


# The reference's published single-thread CPU figures for its own bench
# shapes (docs/benchmarks/RESULTS-mind-vs-rust-2026-06-09.md:45-48, MIND
# column; Intel i7-5930K 3.5 GHz AVX2, one core).
PUBLISHED_ST = {("i8", 256): (12.56, 45), ("i8", 512): (14.17, 46), ("q16", 256): (4.17, 47), ("q16", 512): (4.16, 48)}


def cpu_single_thread(op: str, n: int) -> dict:
    """The reference's CPU bench shape n^3 (seed 0xDEADBEEF00000000 ^ n, the
    bench LCG: benches/det_matmul_i8.rs:431-446, det_matmul_q16.rs:424-437) on
    ONE thread of the MT restatement (the AVX2 vpmaddwd 4x16 int8 / vpmuldq
    4x8 Q16 microkernels), beside the reference's published figure.  Int8
    256^3 is BASELINE config 1."""
    import oracle as O

    L = O.lib()
    seed = 0xDEADBEEF00000000 ^ n
    if op == "i8":
        a, b = O.gen_i8(seed, n * n, n * n)
        fn, want = L.det_cpu_gemm_i8, O.gemm_i8(a, b, n, n, n).ravel()
    else:
        a, b = O.gen_q16(seed, n * n, n * n)
        fn, want = L.det_cpu_gemm_q16, O.gemm_q16(a, b, n, n, n).ravel()
    c = np.empty(n * n, np.int32)
    L.det_cpu_set_threads(1)
    try:
        run = lambda: fn(a.ctypes.data, b.ctypes.data, c.ctypes.data, n, n, n)
        run()
        exact = bool(np.array_equal(c, want))
        reps = 101 if n * n * n * (1 if op == "i8" else 8) <= (1 << 27) else 33
        t = _time_median(run, reps)
    finally:
        L.det_cpu_set_threads(0)
    if not exact:
        raise SystemExit(f"{op} {n}^3 CPU baseline output differs from the oracle")
    pub, line = PUBLISHED_ST[(op, n)]
    return {"value": n ** 3 / t / 1e9, "unit": "GMAC/s", "us": t * 1e6, "cores": 1, "kind": "port",
            "sample": f"{'int8' if op == 'i8' else 'Q16.16'} {n}^3 (median of {reps} calls), one thread, "
                      f"output equal to the oracle",
            "published_reference": {"value": pub, "unit": "GMAC/s", "host": "Intel i7-5930K 3.5 GHz AVX2, 1 core",
                                    "source": f"docs/benchmarks/RESULTS-mind-vs-rust-2026-06-09.md:{line}"},
            "cpu_model": _cpu_model()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="", help="comma list of workloads (default: all)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-peaks", action="store_true", help="skip the roofline probe micro-kernels")
    ap.add_argument("--vendor-ref", action="store_true",
                    help="also time the vendor int8 GEMM (torch._int_mm) on the headline shape, for context")
    ap.add_argument("--vendor-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-host-abi", action="store_true",
                    help="skip the end-to-end host-pointer timings (PCIe included) and the reference sweeps")
    ap.add_argument("--settle", type=float, default=0.5,
                    help="seconds of back-to-back running before each timed region (default %(default)s)")
    args = ap.parse_args()
    global SETTLE_S
    SETTLE_S = max(0.0, args.settle)
    if args.vendor_child:
        vendor_int8_child(args.steps, SETTLE_S)
        return 0

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: every box in this build has one MI355X; sharding this "
              "path over several GPUs (row bands of the output, no collectives) is a design, not run.",
              file=sys.stderr)
        return 2
    # the vendor leg runs first, in a child process, before any HIP call here
    vendor = vendor_int8_reference(args.steps, SETTLE_S) if args.vendor_ref else None

    L = M.lib()
    M.check(L.det_set_device(0))
    info = M.device_info()
    log(f"device {info['name']} CUs={info['cus']} clock={info['clock_khz'] / 1e3:.0f} MHz")
    stream = M.Stream()
    K, W = args.steps, args.warmup
    only = set(x for x in args.only.split(",") if x)

    def want(name):
        return not only or name in only

    # ---- headline: int8 4096^3
    m = k = n = 4096
    log("i8_4096: det_matmul_i8 4096x4096x4096")
    head = gemm_workload("i8", m, k, n, K, W, stream, 0x4096, keep_output=True)
    tops = head["ops"] / (head["ms"] * 1e-3) / 1e12
    log(f"i8_4096: {head['ms'] * 1e3:.1f} us/step  {tops:.1f} TOP/s")

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        t = json.load(open(tpath)).get("i8_4096")
        traffic = t["bytes"] if t else None

    result = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "settle_s": SETTLE_S,
        "ms_per_step": round(head["wall_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic: reference bench LCG (s*1664525+1013904223, (i8)(u32>>16)), seed 0xDEADBEEF^0x4096",
        "config": {"workload": "det_matmul_i8 4096x4096x4096 (A int8 row-major, B int8 KxN row-major, C int32)",
                   "m": m, "k": k, "n": n, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": round(tops / PEAK_INT8_TOPS, 4), "traffic": traffic,
                     "traffic_note": "HBM bytes per launch from rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0 "
                                     "(scales from a 1 GiB copy kernel); algorithmic 100,663,296",
                     "kernel": "det::i8g::t256::gemm_i8_t256_kernel<false, 0>",
                     "algorithmic": "2*M*N*K = 1.374e11 int8 ops per launch (one launch per step)",
                     "event_ms_per_launch": round(head["ms"], 5),
                     "gmac_per_s": round(tops * 500.0, 1),
                     "median_of_64_launches_ms": round(head["per_launch"]["median_ms"], 5),
                     "p10_p90_of_64_launches_ms": [round(head["per_launch"]["p10_ms"], 5),
                                                   round(head["per_launch"]["p90_ms"], 5)]},
        "device": info["name"],
    }

    if not args.no_peaks:
        log("peaks: int8 MFMA probe, HBM read and copy probes")
        result["measured_peaks"] = pk = measure_peaks(stream)
        log(f"peaks: {pk}")
        best = max(pk["mfma_i8_tops"]["16x16x64"], pk["mfma_i8_tops"]["32x32x32"])
        # the int8 GEMM kernels issue v_mfma_i32_16x16x64_i8
        rnd = pk["mfma_i8_tops"]["16x16x64_random_operands"]
        result["roofline"]["measured_peak"] = best
        result["roofline"]["frac_of_measured_peak"] = round(tops / best, 4)
        result["roofline"]["measured_peak_random_operands"] = rnd
        result["roofline"]["frac_of_random_operand_peak"] = round(tops / rnd, 4)

    runs = {"i8_4096": head}
    sec = {}
    if want("q16_1024"):
        log("q16_1024: det_matmul_q16 1024^3 (saturating config)")
        r = runs["q16_1024"] = gemm_workload("q16", 1024, 1024, 1024, K, W, stream, 0x1016, keep_output=True)
        t = r["ops"] / (r["ms"] * 1e-3) / 1e12
        sec["q16_1024"] = {"ms": round(r["ms"], 5), "value": round(t, 3), "unit": "Q16 TOP/s (2*MNK/t)",
                           "gmac_per_s": round(t * 500.0, 1),
                           "limb_mfma_tops": round(15 * t, 2),
                           "frac_of_int8_mfma_peak_limb": round(15 * t / PEAK_INT8_TOPS, 4)}
        log(f"q16_1024: {r['ms'] * 1e3:.1f} us  {t:.2f} TOP/s")
    if want("q16_4096"):
        log("q16_4096: det_matmul_q16 4096^3 (saturating config)")
        r = runs["q16_4096"] = gemm_workload("q16", 4096, 4096, 4096, max(3, K // 4), 1, stream, 0x4016,
                                             check_rows=2)
        t = r["ops"] / (r["ms"] * 1e-3) / 1e12
        sec["q16_4096"] = {"ms": round(r["ms"], 5), "value": round(t, 3), "unit": "Q16 TOP/s (2*MNK/t)",
                           "gmac_per_s": round(t * 500.0, 1),
                           "limb_mfma_tops": round(15 * t, 2),
                           "frac_of_int8_mfma_peak_limb": round(15 * t / PEAK_INT8_TOPS, 4),
                           "residue_valu_note": "the per-term floor needs M*N*K 16-bit residue products on the "
                                                "VALU (1 op per term); gfx950 does not co-issue them with MFMA"}
        log(f"q16_4096: {r['ms'] * 1e3:.1f} us  {t:.2f} TOP/s")
    if want("i16_2048"):
        log("i16_2048: det_matmul_i16 2048^3")
        r = runs["i16_2048"] = gemm_workload("i16", 2048, 2048, 2048, K, W, stream, 0x2016)
        t = r["ops"] / (r["ms"] * 1e-3) / 1e12
        sec["i16_2048"] = {"ms": round(r["ms"], 5), "value": round(t, 3), "unit": "TOP/s",
                           "gmac_per_s": round(t * 500.0, 1),
                           "limb_mfma_tops": round(4 * t, 2),
                           "frac_of_int8_mfma_peak_limb": round(4 * t / PEAK_INT8_TOPS, 4)}
        log(f"i16_2048: {r['ms'] * 1e3:.1f} us  {t:.2f} TOP/s")
    for nb in (1, 8):
        name = f"gemv_q16_16384_b{nb}"
        if want(name):
            log(f"{name}: det_gemv_q16 16384x16384 batch {nb}")
            r = runs[name] = gemv_workload(16384, 16384, nb, K, W, stream, 0x6E3F ^ nb, keep_output=(nb == 1))
            gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
            sec[name] = {"ms": round(r["ms"], 5), "value": round(gbs, 1), "unit": "GB/s",
                         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                      "frac": round(gbs / PEAK_HBM_GBS, 4)}}
            log(f"{name}: {r['ms'] * 1e3:.1f} us  {gbs:.0f} GB/s")
    if want("f32_rows_16384"):
        name = "f32_rows_16384"
        log(f"{name}: det_matmul_rmajor_f32 16384x16384 (strict-FP f32)")
        r = runs[name] = f32_rows_workload(16384, 16384, K, W, stream, 0xF32)
        gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
        sec[name] = {"ms": round(r["ms"], 5), "value": round(gbs, 1), "unit": "GB/s",
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                  "frac": round(gbs / PEAK_HBM_GBS, 4)}}
        log(f"{name}: {r['ms'] * 1e3:.1f} us  {gbs:.0f} GB/s")
    for name, amp in (("fft_q16_256", 65536), ("fft_q16_256_wide", 1 << 40)):
        if not want(name):
            continue
        batch = 1 << 18
        log(f"{name}: det_fft_q16 n=256 x {batch} transforms, inputs in [-{amp}, {amp})")
        r = runs[name] = fft_workload(8, batch, K, W, stream, 0xFF7, amp)
        ns = r["ms"] * 1e6 / r["ffts"]
        gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
        sec[name] = {"ms": round(r["ms"], 5), "ns_per_fft": round(ns, 4), "value": round(10240.0 / ns, 1),
                     "unit": "GFLOP/s-equivalent (5 N log2 N / t, the reference's FFT metric)",
                     "batch": batch, "input_range": amp,
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                  "frac": round(gbs / PEAK_HBM_GBS, 4),
                                  "algorithmic": "read + write of re, im: 32 B per point"}}
        log(f"{name}: {r['ms'] * 1e3:.1f} us  {ns:.3f} ns/FFT  {gbs:.0f} GB/s")
    if want("i8_mlp"):
        log("i8_mlp: det_matmul_i8 4096x4096x11008 (MLP layer)")
        r = runs["i8_mlp_4096x4096x11008"] = gemm_workload("i8_mlp", 4096, 4096, 11008, K, W, stream, 0x3117,
                                                           check_rows=2)
        t = r["ops"] / (r["ms"] * 1e-3) / 1e12
        sec["i8_mlp_4096x4096x11008"] = {"ms": round(r["ms"], 5), "value": round(t, 2), "unit": "TOP/s",
                                         "gmac_per_s": round(t * 500.0, 1),
                                         "frac": round(t / PEAK_INT8_TOPS, 4)}
        log(f"i8_mlp: {r['ms'] * 1e3:.1f} us  {t:.1f} TOP/s")
    if want("i8_8192"):
        log("i8_8192: det_matmul_i8 8192^3 (peak probe)")
        r = runs["i8_8192"] = gemm_workload("i8", 8192, 8192, 8192, max(3, K // 4), 2, stream, 0x8192, check_rows=2)
        t = r["ops"] / (r["ms"] * 1e-3) / 1e12
        sec["i8_8192"] = {"ms": round(r["ms"], 5), "value": round(t, 2), "unit": "TOP/s",
                          "gmac_per_s": round(t * 500.0, 1),
                          "frac": round(t / PEAK_INT8_TOPS, 4)}
        log(f"i8_8192: {r['ms'] * 1e3:.1f} us  {t:.1f} TOP/s")
    # int8 off the headline shape: the reference's own sweep sizes (256, 512),
    # a grid smaller than the chip (2048^3) and a ragged cube (4095^3, K and
    # N off the 16-byte grid: operands repacked into padded panels)
    for nn in (256, 512, 2048, 4095):
        name = f"i8_{nn}"
        if want(name):
            log(f"{name}: det_matmul_i8 {nn}^3")
            r = runs[name] = gemm_workload("i8", nn, nn, nn, K, W, stream, nn, check_rows=2)
            t = r["ops"] / (r["ms"] * 1e-3) / 1e12
            sec[name] = {"ms": round(r["ms"], 5), "value": round(t, 2), "unit": "TOP/s",
                         "gmac_per_s": round(t * 500.0, 1), "frac": round(t / PEAK_INT8_TOPS, 4)}
            log(f"{name}: {r['ms'] * 1e3:.1f} us  {t:.1f} TOP/s")
    result["secondary"] = sec
    sweeps = {}
    if not args.no_host_abi:
        log("reference sweeps: the reference benches' shapes, host-pointer calls and device-resident")
        sweeps = reference_sweeps(stream, K)
    stream.destroy()
    if not args.no_host_abi:
        log("host_abi: reference-ABI host-pointer calls, PCIe copies included")
        result["host_abi"] = host_abi_timings()
        log(f"host_abi: {result['host_abi']}")
    if vendor is not None:
        result["vendor_int8_gemm"] = vendor

    # ---- CPU leg: the oracle checks every timed output (sampled rows), then
    # the MT CPU restatement is timed on a row band of the headline workload.
    if not args.no_cpu_baseline:
        import oracle as O

        checks = {}
        for name, r in runs.items():
            checks[name] = r["verify"](O)
            log(f"oracle check {name}: {'exact' if checks[name] else 'MISMATCH'} ({r['checked_rows']} rows)")
        for name, r in sweeps.items():
            checks[f"sweep_{name}"] = verify_sweep(O, *r.pop("_check"))
            log(f"oracle check sweep {name}: {'exact' if checks['sweep_' + name] else 'MISMATCH'} (whole output, "
                f"host call and device)")
        if sweeps:
            result["reference_sweeps"] = {
                "note": "the reference benches' own sweep shapes (benches/det_matmul_i8.rs:86, det_matmul_q16.rs:82, "
                        "det_matmul_i16.rs:77, det_gemv_q16_mt.rs:62 and its 512x130 anchor): host_call = the "
                        "symbol its bench dlsyms, timed as its report_gmacs (median of 64 synchronous calls after 8, "
                        "pageable buffers, PCIe copies included); device = the same work on device-resident operands "
                        "(HIP events); each output checked whole against the oracle (exact_vs_oracle sweep_*)",
                **sweeps}
        result["exact_vs_oracle"] = checks
        if "fft_q16_256" in sec:
            ref = cpu_fft_reference(8)
            if ref is not None:
                sec["fft_q16_256"]["cpu_reference"] = ref
                log(f"fft cpu reference: {ref['ns_per_fft']} ns/FFT (1 thread)")
        if not all(checks.values()):
            print(json.dumps(result), flush=True)
            raise SystemExit("a timed output differs from the oracle: its number is not valid")
        log("cpu_baseline: MT CPU restatement on a row band of the same workload")
        result["cpu_baseline"] = cpu_baseline_int8(head["A"], head["B"], head["C"], m, k, n)
        log(f"cpu_baseline: {result['cpu_baseline']['value']:.3f} TOP/s on {result['cpu_baseline']['cores']} threads")
        extra = {}
        for op, nn in PUBLISHED_ST:
            key = f"{op}_{nn}_one_thread"
            extra[key] = cpu_single_thread(op, nn)
            log(f"cpu_baseline {op} {nn}^3, 1 thread: {extra[key]['value']:.2f} GMAC/s "
                f"(reference published {extra[key]['published_reference']['value']})")
        if "q16_1024" in runs and "A" in runs["q16_1024"]:
            r = runs["q16_1024"]
            extra["q16_1024"] = cpu_baseline_q16(r["A"], r["B"], r["C"], 1024, 1024, 1024)
            log(f"cpu_baseline q16 1024^3: {extra['q16_1024']['gmac_per_s']:.1f} GMAC/s "
                f"on {extra['q16_1024']['cores']} threads")
        if "gemv_q16_16384_b1" in runs and "W" in runs["gemv_q16_16384_b1"]:
            r = runs["gemv_q16_16384_b1"]
            extra["gemv_q16_16384_b1"] = cpu_baseline_gemv(r["W"], r["X"], r["Y"], 16384, 16384)
            log(f"cpu_baseline gemv 16384^2: {extra['gemv_q16_16384_b1']['value']:.1f} GB/s "
                f"on {extra['gemv_q16_16384_b1']['cores']} threads")
        result["cpu_baselines"] = extra
    else:
        result["exact_vs_oracle"] = None
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
