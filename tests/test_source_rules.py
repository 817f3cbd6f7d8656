"""Static checks that the library's sources keep the rules this build runs
under (CPU only, reads the sources):

* no HIP call that is unsafe on these GPU boxes or under graph capture:
  no hipHostRegister (pinned memory is allocated with hipHostMalloc), no
  stream priorities, no uncached device memory, no IPC handles, no
  hipMemsetAsync (memory that must start at zero is cleared by a kernel);
  the one hipMemset is the synchronous harness fill det_memset_dev;
* every device compile carries -packed-fp32-ops;
* gfx950 code only: no platform dual paths (__HIP_PLATFORM_* tests);
* the product never touches the oracle: nothing under mind_amd/ imports,
  loads or names the CPU checker (oracle/, liboracle_det, the reference
  builds in oracle/_ref)."""
import glob
import os
import re

import mind_amd.build as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = glob.glob(os.path.join(ROOT, "mind_amd", "csrc", "*"))
PKG = CSRC + glob.glob(os.path.join(ROOT, "mind_amd", "*.py")) + glob.glob(os.path.join(ROOT, "mind_amd", "shim", "*"))


def _text(path):
    return open(path, encoding="utf-8", errors="replace").read()


def test_no_unsafe_hip_calls():
    banned = ["hipHostRegister", "hipStreamCreateWithPriority", "hipExtMallocWithFlags", "hipDeviceMallocUncached",
              "hipIpcOpenMemHandle", "hipMemsetAsync", "hipMemsetD8Async", "hipMemsetD32Async"]
    hits = [(os.path.basename(p), b) for p in CSRC for b in banned if re.search(r"\b" + b + r"\s*\(", _text(p))]
    assert not hits, hits
    memsets = [(os.path.basename(p), m.start()) for p in CSRC for m in re.finditer(r"\bhipMemset\s*\(", _text(p))]
    assert len(memsets) == 1 and memsets[0][0] == "det_abi.hip", memsets
    abi = _text(os.path.join(ROOT, "mind_amd", "csrc", "det_abi.hip"))
    fill = abi[abi.index("int64_t det_memset_dev("):]
    assert fill.index("hipMemset(") < fill.index("\n}"), "hipMemset outside det_memset_dev"


def test_device_flags_keep_packed_fp32_off():
    f = B.DEVICE_FLAGS
    i = f.index("-packed-fp32-ops")
    assert f[i - 3:i] == ["-Xclang", "-target-feature", "-Xclang"], f
    assert f"--offload-arch={B.ARCH}" in f and B.ARCH == "gfx950"


def test_no_platform_dual_paths():
    hits = [os.path.basename(p) for p in CSRC if re.search(r"__HIP_PLATFORM_|__CUDA_ARCH__|__NVCC__", _text(p))]
    assert not hits, hits


def test_product_never_touches_the_oracle():
    pat = re.compile(r"\bimport\s+oracle\b|\bfrom\s+oracle\b|liboracle|oracle/_ref|det_oracle|det_cpu_mt")
    hits = [os.path.relpath(p, ROOT) for p in PKG if os.path.isfile(p) and pat.search(_text(p))]
    assert not hits, hits
