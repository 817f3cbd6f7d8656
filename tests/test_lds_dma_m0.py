"""The LDS-DMA helpers (dma16 / dma16s in mind_amd/csrc/det_common.h) set M0
in inline assembly.  The compiler treats M0 as a reserved register and
ignores it in an asm clobber list (it warns so), so the helpers are safe
only while the compiler itself keeps no value in M0 across them.  This test
compiles every HIP source to gfx950 assembly with the library's own device
flags (CPU only: hipcc cross-compiles) and checks that every M0 access in
the output is one of the helpers' three-instruction sequences
(s_mov_b32 m0 / s_nop 0 / buffer_load_dwordx4 ... lds): no other
instruction reads or writes M0."""
import concurrent.futures as cf
import glob
import os
import re
import shutil
import subprocess

import pytest

import mind_amd.build as B

SRCS = sorted(glob.glob(os.path.join(B.CSRC, "*.hip")))

pytestmark = pytest.mark.skipif(not os.path.exists(B.HIPCC) and shutil.which("hipcc") is None,
                                reason="hipcc not installed")


def _asm(src, out_dir):
    out = os.path.join(out_dir, os.path.basename(src)[:-4] + ".s")
    r = subprocess.run([B.HIPCC, *B.DEVICE_FLAGS, "--cuda-device-only", "-S", src, "-o", out],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return out


def test_m0_only_in_the_lds_dma_sequences(tmp_path):
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        outs = list(ex.map(lambda s: _asm(s, str(tmp_path)), SRCS))
    m0 = re.compile(r"\bm0\b")
    sequences = 0
    for path in outs:
        ins = []   # instruction lines only (no comments, labels or directives)
        for line in open(path):
            t = line.split(";")[0].strip()
            if t and not t.startswith(".") and not t.endswith(":"):
                ins.append(t)
        for i, t in enumerate(ins):
            if not m0.search(t):
                continue
            where = f"{os.path.basename(path)}: {t!r}"
            assert re.fullmatch(r"s_mov_b32 m0, s\d+", t), "M0 used outside the DMA helpers: " + where
            assert ins[i + 1] == "s_nop 0", where
            assert ins[i + 2].startswith("buffer_load_dwordx4") and ins[i + 2].endswith(" lds"), where
            sequences += 1
    assert sequences > 0   # the DMA kernels are in the build
