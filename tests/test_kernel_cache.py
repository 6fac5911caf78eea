"""The compiled-kernel directory (mfh_fusion_cache_dir): a kernel compiled in
one process is read back by the next instead of being compiled again, and a
file that does not match the compile exactly (corrupted, truncated, another
source) costs a compile and nothing else.  Compiling needs no GPU, so each
step runs in a fresh CPU process."""
import json
import os
import subprocess
import sys

import pytest

import manifesto_amd as M
from oracle import N_ADD, N_MUL, N_SIGMOID, N_SUB, flatten

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

STEP = r"""
import json, sys, time
sys.path.insert(0, {root!r})
import manifesto_amd as M
from oracle import flatten
trees = json.loads(sys.argv[1])
out = []
for tree, port in trees:
    def tup(t):
        return tuple(tup(x) if isinstance(x, list) else x for x in t)
    t0 = time.perf_counter()
    k = M.FusedKernel(flatten(tup(tree)), [(M.FLOAT32, M.OPERAND_FULL, 0)] * 2, M.FLOAT32, port)
    out.append({{"ms": (time.perf_counter() - t0) * 1e3, "source": k.source}})
print(json.dumps({{"kernels": out, "stats": M.fusion_cache_stats()}}))
"""

FMS = [N_SUB, [N_MUL, ["in", 0], ["in", 1]], ["in", 0]]
SIG = [N_ADD, [N_SIGMOID, ["in", 0]], ["in", 1]]


def run(cache_dir, trees):
    env = dict(os.environ)
    env.pop("MFH_KERNEL_CACHE_DIR", None)
    if cache_dir is not None:
        env["MFH_KERNEL_CACHE_DIR"] = str(cache_dir)
    p = subprocess.run([sys.executable, "-c", STEP.format(root=ROOT), json.dumps(trees)], env=env,
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert p.returncode == 0, p.stderr
    return json.loads(p.stdout.strip().splitlines()[-1])


def files(d):
    return sorted(f for f in os.listdir(d) if f.endswith(".hsaco"))


def test_second_process_reads_the_kernel_back(tmp_path):
    first = run(tmp_path, [[FMS, "cache_fms"]])
    assert first["stats"] == [1, 0]
    assert len(files(tmp_path)) == 1
    second = run(tmp_path, [[FMS, "cache_fms"]])
    assert second["stats"] == [0, 1]
    assert second["kernels"][0]["source"] == first["kernels"][0]["source"]
    # another kernel is compiled and stored beside it; the first is still read
    third = run(tmp_path, [[SIG, "cache_sig"], [FMS, "cache_fms"]])
    assert third["stats"] == [1, 1]
    assert len(files(tmp_path)) == 2
    assert not [f for f in os.listdir(tmp_path) if ".tmp." in f]


@pytest.mark.parametrize("damage", ["flip", "truncate", "empty", "garbage"])
def test_a_damaged_file_is_compiled_again_and_replaced(tmp_path, damage):
    run(tmp_path, [[FMS, "cache_fms"]])
    (name,) = files(tmp_path)
    path = tmp_path / name
    good = path.read_bytes()
    data = bytearray(good)
    if damage == "flip":
        data[len(data) - 200] ^= 0x10  # inside the code object
    elif damage == "truncate":
        data = data[:len(data) - 100]
    elif damage == "empty":
        data = bytearray()
    else:
        data = bytearray(b"MFHKODE1" + os.urandom(4000))
    path.write_bytes(bytes(data))
    again = run(tmp_path, [[FMS, "cache_fms"]])
    assert again["stats"] == [1, 0]
    assert path.read_bytes() == good  # rewritten whole
    assert run(tmp_path, [[FMS, "cache_fms"]])["stats"] == [0, 1]


def test_a_file_for_another_source_is_not_used(tmp_path):
    # the file of one kernel placed under the name of another: the byte-for-byte
    # source check refuses it
    run(tmp_path, [[FMS, "cache_fms"]])
    (fms_name,) = files(tmp_path)
    other = tmp_path / "other"
    other.mkdir()
    run(other, [[SIG, "cache_sig"]])
    (sig_name,) = files(other)
    (other / sig_name).write_bytes((tmp_path / fms_name).read_bytes())
    assert run(other, [[SIG, "cache_sig"]])["stats"] == [1, 0]


def test_off_or_unwritable_directory_still_compiles(tmp_path):
    assert run(None, [[FMS, "cache_fms"]])["stats"] == [1, 0]
    missing = tmp_path / "does_not_exist"
    assert run(missing, [[FMS, "cache_fms"]])["stats"] == [1, 0]
    assert not missing.exists()


def test_directory_set_through_the_abi(tmp_path):
    M.fusion_cache_dir(tmp_path)
    try:
        before = M.fusion_cache_stats()
        M.FusedKernel(flatten((N_MUL, ("in", 0), ("const", 3.25))), [(M.FLOAT32, M.OPERAND_FULL, 0)], M.FLOAT32,
                      "cache_abi")
        compiles, hits = M.fusion_cache_stats()
        assert (compiles - before[0], hits - before[1]) == (1, 0)
        assert len(files(tmp_path)) == 1
    finally:
        M.fusion_cache_dir(None)
    M.FusedKernel(flatten((N_MUL, ("in", 0), ("const", 4.25))), [(M.FLOAT32, M.OPERAND_FULL, 0)], M.FLOAT32,
                  "cache_abi_off")
    assert len(files(tmp_path)) == 1
