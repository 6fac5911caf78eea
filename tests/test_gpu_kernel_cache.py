"""A kernel read back from the compiled-kernel directory runs like the one
hiprtc compiled: two fresh processes launch the same fused kernel, the first
compiling and storing it, the second reading it from the directory, and both
outputs match the oracle bit for bit."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle as O

from gpu_util import log

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

STEP = r"""
import json, sys
import numpy as np
sys.path.insert(0, {root!r})
import manifesto_amd as M
from manifesto_amd.backend import Backend
from oracle import N_ADD, N_MUL, N_RELU, N_SUB, flatten
src, dst = sys.argv[1], sys.argv[2]
x, y = np.fromfile(src, np.float32).reshape(2, -1)
n = x.size
tree = (N_ADD, (N_RELU, (N_SUB, (N_MUL, ("in", 0), ("in", 1)), ("in", 1))), ("in", 0))
k = M.FusedKernel(flatten(tree), [(M.FLOAT32, M.OPERAND_FULL, 0)] * 2, M.FLOAT32, "cache_gpu")
b = Backend(0)
tx, ty = b.upload([n], M.FLOAT32, x), b.upload([n], M.FLOAT32, y)
to = b.upload([n], M.FLOAT32, np.zeros(n, np.float32))
k.launch([tx.dispatch_pointer(), ty.dispatch_pointer()], to.dispatch_pointer(), n)
M.stream_sync(0)
open(dst, "wb").write(bytes(b.download(to)[1]))
for t in (tx, ty, to):
    t.release()
b.release()
print(json.dumps(M.fusion_cache_stats()))
"""


def test_kernel_from_the_directory_matches_the_oracle(tmp_path):
    from oracle import N_ADD, N_MUL, N_RELU, N_SUB, flatten
    rng = np.random.default_rng(0x5EED + 7)
    n = 1000003
    x = rng.normal(0, 3, n).astype(np.float32)
    y = rng.normal(0, 3, n).astype(np.float32)
    src = tmp_path / "in.bin"
    np.stack([x, y]).tofile(src)
    tree = (N_ADD, (N_RELU, (N_SUB, (N_MUL, ("in", 0), ("in", 1)), ("in", 1))), ("in", 0))
    want = O.run(flatten(tree), [x, y], n).view(np.uint32)
    cache = tmp_path / "kernels"
    cache.mkdir()
    env = dict(os.environ, MFH_KERNEL_CACHE_DIR=str(cache))
    stats = []
    for step in range(2):
        dst = tmp_path / f"out{step}.bin"
        log(f"kernel cache: process {step + 1} of 2, n = {n}")
        p = subprocess.run([sys.executable, "-c", STEP.format(root=ROOT), str(src), str(dst)], env=env,
                           capture_output=True, text=True, timeout=120, cwd=ROOT)
        assert p.returncode == 0, p.stderr
        stats.append(json.loads(p.stdout.strip().splitlines()[-1]))
        got = np.fromfile(dst, np.uint32)
        np.testing.assert_array_equal(got, want)
    assert stats == [[1, 0], [0, 1]]
