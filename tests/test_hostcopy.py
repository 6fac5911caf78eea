"""CPU tests of the staging copy pool (manifesto_amd/csrc/hostcopy.cpp):
tests/hostcopy_check.cpp built with g++ against the pool's source, plain and
under ThreadSanitizer, and run with 1, 3 and 8 copy threads.  The pool
splits every upload's, download's and SafeTensors read's host copy; the GPU
tests cover it end to end."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "manifesto_amd", "csrc")


def build(tmp_path, extra):
    exe = tmp_path / ("check" + ("_tsan" if extra else ""))
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I", CSRC,
           "-I", os.path.join(ROOT, "include"), *extra, os.path.join(ROOT, "tests", "hostcopy_check.cpp"),
           os.path.join(CSRC, "hostcopy.cpp"), "-o", str(exe), "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail(r.stderr[-3000:])
    return exe


@pytest.mark.parametrize("sanitize", [False, True], ids=["plain", "tsan"])
def test_copy_pool(tmp_path, sanitize):
    exe = build(tmp_path, ["-fsanitize=thread"] if sanitize else [])
    for threads in ("1", "3", "8"):
        env = dict(os.environ, MFH_COPY_THREADS=threads, TSAN_OPTIONS="halt_on_error=1")
        r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
        assert r.returncode == 0, (threads, r.stdout[-2000:], r.stderr[-4000:])
        assert f"threads {threads}" in r.stdout and "concurrent ok" in r.stdout, r.stdout
