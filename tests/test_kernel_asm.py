"""Checks on the gfx950 assembly of every HIP source, compiled on the CPU with
the library's own device flags (hipcc cross-compiles; no GPU needed).

1. M0: the LDS-DMA helpers (dma16 / dma16s in mind_amd/csrc/det_common.h)
   set M0 in inline assembly.  The compiler treats M0 as a reserved register
   and ignores it in an asm clobber list (it warns so), so the helpers are
   safe only while the compiler itself keeps no value in M0 across them:
   every M0 access must be one of the helpers' three-instruction sequences
   (s_mov_b32 m0 / s_nop 0 / buffer_load_dwordx4 ... lds).
2. No GPU code writes through the scalar data cache: no scalar store,
   scalar atomic, or scalar-cache write-back / discard instruction appears
   (s_store_*, s_buffer_store_*, s_scratch_store_*, s_atomic_*,
   s_buffer_atomic_*, s_dcache_wb*, s_dcache_discard*).  Stores go through
   the vector memory path only.

It is a CPU test: it never needs a GPU."""
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


@pytest.fixture(scope="module")
def instructions(tmp_path_factory):
    """{file: [instruction lines]} (comments, labels and directives dropped)."""
    d = str(tmp_path_factory.mktemp("asm"))
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        outs = list(ex.map(lambda s: _asm(s, d), SRCS))
    res = {}
    for path in outs:
        ins = []
        for line in open(path):
            t = line.split(";")[0].strip()
            if t and not t.startswith(".") and not t.endswith(":"):
                ins.append(t)
        res[os.path.basename(path)] = ins
    return res


def test_m0_only_in_the_lds_dma_sequences(instructions):
    m0 = re.compile(r"\bm0\b")
    sequences = 0
    for name, ins in instructions.items():
        for i, t in enumerate(ins):
            if not m0.search(t):
                continue
            where = f"{name}: {t!r}"
            assert re.fullmatch(r"s_mov_b32 m0, s\d+", t), "M0 used outside the DMA helpers: " + where
            assert ins[i + 1] == "s_nop 0", where
            assert ins[i + 2].startswith("buffer_load_dwordx4") and ins[i + 2].endswith(" lds"), where
            sequences += 1
    assert sequences > 0   # the DMA kernels are in the build


def test_no_scalar_cache_writes(instructions):
    bad = re.compile(r"^(s_store_|s_buffer_store_|s_scratch_store_|s_atomic_|s_buffer_atomic_|s_dcache_wb|"
                     r"s_dcache_discard)")
    found = [(name, t) for name, ins in instructions.items() for t in ins if bad.match(t)]
    assert not found, found[:10]
    assert sum(len(v) for v in instructions.values()) > 10000   # the kernels were really compiled
