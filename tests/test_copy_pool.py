"""CPU checks of the host-pointer entry points' threaded host copy
(mind_amd/csrc/det_copy_pool.h, used by det_abi.hip for the pinned staging
and the pinned ring): tests/cpu_checks/copy_pool_check.cpp built with g++ and
run plainly and under ThreadSanitizer (host code only).  Every copy must be
exact with its guard bytes untouched, from three caller threads at once and
across stop / restart of the pool, and ThreadSanitizer must report nothing."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cpu_checks", "copy_pool_check.cpp")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")


def _build(tmp_path, name, flags):
    exe = str(tmp_path / name)
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", *flags, SRC, "-o", exe, "-pthread"],
                       capture_output=True, text=True, timeout=180)
    return exe, r


def test_copy_pool_exact(tmp_path):
    exe, r = _build(tmp_path, "copy_pool_check", ["-O2"])
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([exe, "4", "24"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and "bad=0" in out.stdout, out.stdout + out.stderr[-2000:]


def test_copy_pool_thread_sanitizer(tmp_path):
    exe, r = _build(tmp_path, "copy_pool_check_tsan", ["-O1", "-g", "-fsanitize=thread"])
    if r.returncode != 0 and "tsan" in r.stderr.lower():
        pytest.skip("ThreadSanitizer runtime not available: " + r.stderr[-300:])
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    out = subprocess.run([exe, "2", "12"], capture_output=True, text=True, timeout=300, env=env)
    assert "ThreadSanitizer" not in out.stderr, out.stderr[-4000:]
    assert out.returncode == 0 and "bad=0" in out.stdout, out.stdout + out.stderr[-2000:]
