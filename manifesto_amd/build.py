"""Builds manifesto_amd/libmfh.so for gfx950 with hipcc.

Every source is compiled with -ffp-contract=off (the reference's Go code never
contracts a*b+c) and with packed-FP32 instructions disabled.  Kernel arguments
are preloaded into SGPRs (gfx950 firmware loads them at wave launch; the code
object keeps a prologue that loads them itself for firmware that does not),
which takes a scalar load off the start of every wave.  The JIT prelude
(codec.hpp + devmath.hpp + fusion_io.hpp) is embedded into the library as a
string so that generated kernels see exactly the code the ahead-of-time
kernels use.

Run: python3 -m manifesto_amd.build   (or __graft_entry__.build())
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmfh.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["runtime.cpp", "dequant.hip", "hostmath.hip", "scratch.hip", "fusion.cpp", "graph.cpp", "plan.cpp",
           "hostcopy.cpp",
           "backend.cpp", "safetensors.cpp"]
PRELUDE_PARTS = ["codec.hpp", "devmath.hpp", "fusion_io.hpp"]

COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I", BUILD, "-I", os.path.join(os.path.dirname(HERE), "include"),
]


def _write_prelude() -> None:
    text = ""
    for part in PRELUDE_PARTS:
        with open(os.path.join(CSRC, part)) as f:
            text += f"// ---- {part} ----\n" + f.read() + "\n"
    delim = "MFHPRELUDE"
    assert f"){delim}\"" not in text
    body = f'static const char kPrelude[] = R"{delim}(\n{text}){delim}";\n'
    path = os.path.join(BUILD, "mfh_prelude.inc")
    old = open(path).read() if os.path.exists(path) else None
    if old != body:
        with open(path, "w") as f:
            f.write(body)


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *COMMON_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    _write_prelude()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           "-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
