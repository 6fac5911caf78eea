"""The C ABI from a plain C99 host (tests/c_client.c), with no Python or
torch in the process that uses the GPU: the dequantising upload, resident
axpy, and an optimised, HIP-lowered graph run as Backend.CallGraph, each
result downloaded and checked bit for bit against the oracle here."""
import os
import subprocess

import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

from gpu_util import log

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
INCLUDE = os.path.join(os.path.dirname(HERE), "include")


def test_c_host_uploads_axpys_and_calls_a_graph(tmp_path):
    lib_dir = os.path.dirname(M.LIB_PATH)
    exe = tmp_path / "c_client"
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", INCLUDE, os.path.join(HERE, "c_client.c"),
                        "-o", str(exe), "-L", lib_dir, "-l:" + os.path.basename(M.LIB_PATH),
                        f"-Wl,-rpath,{lib_dir}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    rng = np.random.default_rng(0x5EED + 42)
    codes = np.tile(np.arange(256, dtype=np.uint8), 64)
    n = 100003  # odd: every vector path has a tail
    x = rng.normal(0, 2, n).astype(np.float32)
    y = rng.normal(0, 2, n).astype(np.float32)
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    src.write_bytes(np.array([codes.size, n], np.int64).tobytes() + codes.tobytes() + x.tobytes() + y.tobytes())
    log(f"c_client: {codes.size} codes, n = {n}")
    run = subprocess.run([str(exe), str(src), str(dst)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    raw = dst.read_bytes()
    assert len(raw) == codes.size * 2 + n * 8
    q = np.frombuffer(raw[:codes.size * 2], np.uint16)
    y_after = np.frombuffer(raw[codes.size * 2:codes.size * 2 + n * 4], np.float32)
    r_out = np.frombuffer(raw[codes.size * 2 + n * 4:], np.float32)
    assert np.array_equal(q, O.dequant_fp8(codes, O.F8E4M3, 0.5, O.BFLOAT16))
    want_y = O.axpy_f32(y, x, 0.75)
    assert np.array_equal(y_after.view(np.uint32), want_y.view(np.uint32))
    s = x * np.float32(0.5) + want_y  # Mul then Add, each rounded to f32
    want_r = np.where(s < 0, np.float32(0), s).astype(np.float32)  # relu as evalCPU: v < 0 ? 0 : v
    assert np.array_equal(r_out.view(np.uint32), want_r.view(np.uint32))
