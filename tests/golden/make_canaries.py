"""Write tests/golden/canaries.json from the reference's committed golden data.

Run in the build container only (it reads /root/reference, which the GPU box
does not have).  It copies DATA, not code: for each hot-path workload the
generator/seed/shape fields of tests/cross_substrate_identity/<id>/manifest.toml
and the avx2 / neon SHA-256 lines of reference_hashes.toml, plus the four
expected digest words embedded in bench/matmul_det_bench.mind:98-101, and
the pinned output hash of the Q16 FFT harness (bench/fft/harness.c:10, also
README.md / RESULTS-fft-2026-06-15.md) with the input parameters of its
harness.c:73-78 signal.
"""
import json
import os
import re
import sys

REF = os.environ.get("MIND_REF", "/root/reference")
IDS = [
    "gemm-i8-64x64x64", "gemm-i8-mt-64x64x64", "gemm-i8-vnni-64x64x64",
    "gemm-q16-64x64x64", "gemm-q16-fused-64x64x64",
    "gemv-q16-256x256", "gemv-i16-256x256",
    "dot-i16-4096", "dot-l2-q16", "dot-l1-q16",
    "dot-f32-v-4093", "matmul-f32-v-64x64",
]


def kv(text):
    out = {}
    for line in text.splitlines():
        line = line.split("#", 1)[0].strip()
        m = re.match(r"^([A-Za-z_0-9]+)\s*=\s*(.+)$", line)
        if m:
            v = m.group(2).strip()
            out[m.group(1)] = v.strip('"') if v.startswith('"') else int(v) if v.isdigit() else v
    return out


def main():
    base = os.path.join(REF, "tests", "cross_substrate_identity")
    res = {"source": "star-ga/mind v0.10.2 tests/cross_substrate_identity/*/{manifest,reference_hashes}.toml",
           "workloads": {}}
    for wid in IDS:
        man = kv(open(os.path.join(base, wid, "manifest.toml")).read())
        hashes = kv(open(os.path.join(base, wid, "reference_hashes.toml")).read())
        keep = {k: man[k] for k in ("seed", "m", "k", "n", "rows", "cols", "length", "dtype", "symbol",
                                    "output_encoding") if k in man}
        keep["avx2"] = hashes["avx2"]
        keep["neon"] = hashes["neon"]
        res["workloads"][wid] = keep
    src = open(os.path.join(REF, "bench", "matmul_det_bench.mind")).read()
    words = [int(x) for x in re.findall(r"let e[0-3]: i64 = (-?\d+);", src)]
    assert len(words) == 4, words
    res["matmul_det_bench_256"] = {"source": "bench/matmul_det_bench.mind:98-101",
                                   "fill_a": "((i+1)%7)-3", "fill_b": "((i+2)%7)-3", "n": 256,
                                   "digest_words_le_i64": words}
    harness = open(os.path.join(REF, "bench", "fft", "harness.c")).read()
    pinned = re.search(r"must be YES, hash ([0-9a-f]{16})", harness).group(1)
    seed = int(re.search(r"uint64_t s = (0x[0-9a-fA-F]+);", harness).group(1), 16)
    readme = open(os.path.join(REF, "bench", "fft", "README.md")).read()
    assert pinned in readme, "harness hash not repeated in README.md"
    res["fft_q16_256_harness"] = {
        "source": "bench/fft/harness.c:10, :50-53, :64-87; README.md",
        "logn": 8, "n": 256, "seed": seed,
        "input": "64-bit LCG s = s*6364136223846793005 + 1442695040888963407; per i: re = s % 131072 - 65536, "
                 "then im likewise",
        "twiddles": "tw[2k] = llround(cos(-2 pi k / n) * 65536), tw[2k+1] = llround(sin(..) * 65536), k < n/2",
        "hash": "fnv1a64(re bytes) ^ fnv1a64(im bytes), little-endian int64",
        "fnv_xor": pinned}
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "canaries.json")
    json.dump(res, open(out, "w"), indent=1)
    print("wrote", out)


if __name__ == "__main__":
    sys.exit(main())
