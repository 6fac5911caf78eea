"""GPU tests of the SafeTensors streaming loader (mfh_safetensors_load): tensors
go from the file through the backend's pinned staging ring onto the device,
FP8 / I4 dequantised there; results are checked bit for bit against the
oracle on the same bytes."""
import json
import struct
import time

import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd.backend import Backend
from manifesto_amd.safetensors import SafeTensorsFile
import oracle as O

from gpu_util import log

pytestmark = pytest.mark.gpu


def write(path, entries):
    """entries: name -> (dtype string, shape, bytes)."""
    header, blobs, at = {}, [], 0
    for name, (dt, shape, raw) in entries.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [at, at + len(raw)]}
        blobs.append(raw)
        at += len(raw)
    text = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)
    return path


@pytest.fixture(scope="module")
def backend():
    b = Backend(0)
    yield b
    b.release()


def test_load_every_supported_dtype(backend, tmp_path):
    rng = np.random.default_rng(0)
    f32 = rng.normal(0, 1, (64, 33)).astype(np.float32)
    bf16 = O.f32_to_bf16(rng.normal(0, 1, 999).astype(np.float32))
    f16 = O.f32_to_f16(rng.normal(0, 1, 1000).astype(np.float32))
    codes = rng.integers(0, 256, 12 * (1 << 20) + 5, dtype=np.uint8)  # several staging chunks
    e5 = rng.integers(0, 256, 4096, dtype=np.uint8)
    i4 = rng.integers(0, 256, 1 << 20, dtype=np.uint8)
    path = write(tmp_path / "m.safetensors", {
        "f32": ("F32", f32.shape, f32.tobytes()), "bf16": ("BF16", [999], bf16.tobytes()),
        "f16": ("F16", [10, 100], f16.tobytes()), "q": ("F8_E4M3", [codes.size], codes.tobytes()),
        "k": ("F8_E5M2", [64, 64], e5.tobytes()), "w4": ("I4", [1024, 2048], i4.tobytes())})
    f = SafeTensorsFile(path)
    cases = {"f32": (M.FLOAT32, f32.tobytes()), "bf16": (M.BFLOAT16, bf16.tobytes()),
             "f16": (M.FLOAT16, f16.tobytes()),
             "q": (M.BFLOAT16, O.bytes_to_bf16(O.F8E4M3, codes).tobytes()),
             "k": (M.BFLOAT16, O.bytes_to_bf16(O.F8E5M2, e5).tobytes()),
             "w4": (M.BFLOAT16, O.bytes_to_bf16(O.INT4, i4).tobytes())}
    for name, (dt, want) in cases.items():
        t = f.load(name, backend)
        assert t.shape() == f.index()[name].shape
        got_dt, raw = backend.download(t)
        assert got_dt == dt and raw == want, name
        t.release()
        log(f"safetensors load {name} ok")


def test_load_scaled_fp8_and_grouped_int4(backend, tmp_path):
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 256, (4096, 1024), dtype=np.uint8)
    scale = np.array([0.0125], np.float32)
    rows, cols, group = 512, 4096, 128
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    s16 = O.f32_to_f16(rng.uniform(0.005, 0.02, rows * cols // group).astype(np.float32))
    bscale = O.f32_to_bf16(np.array([0.5], np.float32))
    path = write(tmp_path / "s.safetensors", {
        "w": ("F8_E4M3", codes.shape, codes.tobytes()), "w_scale": ("F32", [], scale.tobytes()),
        "w_bscale": ("BF16", [1], bscale.tobytes()),
        "q": ("I4", [rows, cols], packed.tobytes()), "q_scales": ("F16", [rows, cols // group], s16.tobytes())})
    f = SafeTensorsFile(path)
    t = f.load("w", backend, scale="w_scale")
    np.testing.assert_array_equal(np.frombuffer(backend.download(t)[1], np.uint16),
                                  O.dequant_fp8(codes.reshape(-1), O.F8E4M3, 0.0125, O.BFLOAT16))
    t = f.load("w", backend, scale="w_bscale")
    np.testing.assert_array_equal(np.frombuffer(backend.download(t)[1], np.uint16),
                                  O.dequant_fp8(codes.reshape(-1), O.F8E4M3, 0.5, O.BFLOAT16))
    t = f.load("q", backend, scale="q_scales", group=group)
    np.testing.assert_array_equal(np.frombuffer(backend.download(t)[1], np.uint16),
                                  O.dequant_int4(packed, rows * cols, s16, O.FLOAT16, group, O.BFLOAT16))
    with pytest.raises(M.MFHError, match="need"):
        f.load("q", backend, scale="q_scales", group=64)  # wrong number of scales for the group


def test_load_errors(backend, tmp_path):
    path = write(tmp_path / "e.safetensors", {
        "ids": ("I64", [4], np.arange(4, dtype=np.int64).tobytes()),
        "short": ("F32", [8], b"\0" * 16)})
    f = SafeTensorsFile(path)
    with pytest.raises(M.MFHError) as e:
        f.load("ids", backend)
    assert e.value.code == -2
    with pytest.raises(M.MFHError) as e:
        f.load("short", backend)  # 16 bytes for 8 f32
    assert e.value.code == -3
    with pytest.raises(M.MFHError, match="missing tensor"):
        f.load("nope", backend)


def test_load_many_grouped_int4_tensors(backend, tmp_path):
    # Int4 weights with their group scales, tensor after tensor: the scales
    # stream through the pinned ring beside the nibbles, so a load allocates
    # nothing but its output and runs at the PCIe rate of the packed bytes.
    rng = np.random.default_rng(2)
    rows, cols, group = 14336, 4096, 128
    entries, want = {}, {}
    for k in range(4):
        packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
        s16 = O.f32_to_f16(rng.uniform(0.005, 0.02, rows * cols // group).astype(np.float32))
        entries[f"w{k}"] = ("I4", [rows, cols], packed.tobytes())
        entries[f"w{k}_scales"] = ("F16", [rows, cols // group], s16.tobytes())
        want[f"w{k}"] = (packed, s16)
    f = SafeTensorsFile(write(tmp_path / "many.safetensors", entries))
    f.load("w0", backend, scale="w0_scales", group=group).release()  # staging ring and page cache warm
    t0 = time.perf_counter()
    tensors = [f.load(f"w{k}", backend, scale=f"w{k}_scales", group=group) for k in range(4)]
    dt = time.perf_counter() - t0
    src_bytes = 4 * (rows * cols // 2 + rows * cols // group * 2)
    log(f"safetensors: 4 grouped Int4 tensors [{rows},{cols}] in {dt * 1e3:.1f} ms, "
        f"{src_bytes / dt / 1e9:.1f} GB/s of file bytes")
    for k, t in enumerate(tensors):
        packed, s16 = want[f"w{k}"]
        got = np.frombuffer(backend.download(t)[1], np.uint16)
        np.testing.assert_array_equal(got, O.dequant_int4(packed, rows * cols, s16, O.FLOAT16, group, O.BFLOAT16))
        t.release()


def test_async_loads_back_to_back(backend, tmp_path):
    # Loads queued one after another without a wait: the staging ring runs
    # on across tensor boundaries (tensors of 1, 2 and 3 chunks, so the next
    # load starts on either slot), a download and a synchronous load come in
    # between, and every tensor matches the oracle and its synchronous load.
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 256, 40 * (1 << 20) + 3, dtype=np.uint8)   # 3 chunks
    f32 = rng.normal(0, 1, 5 * (1 << 20) + 7).astype(np.float32)        # 2 chunks
    bf16 = O.f32_to_bf16(rng.normal(0, 1, 1001).astype(np.float32))     # 1 chunk
    e5 = rng.integers(0, 256, 17 * (1 << 20), dtype=np.uint8)           # 2 chunks
    rows, cols, group = 2048, 4096, 128
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    s16 = O.f32_to_f16(rng.uniform(0.005, 0.02, rows * cols // group).astype(np.float32))
    scale = np.array([0.0125], np.float32)
    f = SafeTensorsFile(write(tmp_path / "a.safetensors", {
        "q": ("F8_E4M3", [codes.size], codes.tobytes()), "q_scale": ("F32", [], scale.tobytes()),
        "f": ("F32", [f32.size], f32.tobytes()), "b": ("BF16", [1001], bf16.tobytes()),
        "k": ("F8_E5M2", [e5.size], e5.tobytes()),
        "w": ("I4", [rows, cols], packed.tobytes()), "w_scales": ("F16", [rows, cols // group], s16.tobytes())}))
    want = {"q": O.dequant_fp8(codes, O.F8E4M3, 0.0125, O.BFLOAT16).tobytes(), "f": f32.tobytes(),
            "b": bf16.tobytes(), "k": O.bytes_to_bf16(O.F8E5M2, e5).tobytes(),
            "w": O.dequant_int4(packed, rows * cols, s16, O.FLOAT16, group, O.BFLOAT16).tobytes()}
    scales = {"q": ("q_scale", 0), "w": ("w_scales", group)}
    order = ["q", "b", "f", "w", "k", "q", "w", "b", "f"]
    tensors = []
    for i, name in enumerate(order):
        sc, g = scales.get(name, (None, 0))
        tensors.append((name, f.load_async(name, backend, scale=sc, group=g)))
        if i == 4:
            # a download and a synchronous load between queued loads
            assert backend.download(tensors[1][1])[1] == want["b"]
            t = f.load("f", backend)
            assert backend.download(t)[1] == want["f"]
            t.release()
    for name, t in tensors:
        assert t.state() in (0, 1)  # ready or pending
    for name, t in tensors:
        t.sync()
        assert t.state() == 0
        assert backend.download(t)[1] == want[name], name
        t.release()
    log("safetensors: async loads back to back match the oracle")


@pytest.mark.parametrize("group, n", [(7, 40 * (1 << 20) + 5), (1, 14 * (1 << 20) + 1), (96, 33 * (1 << 20) + 2),
                                      (4096, 3 * (1 << 22) + 77)])
def test_grouped_int4_across_staging_chunks(backend, tmp_path, group, n):
    # chunks hold whole groups and whole bytes, odd and tiny groups included,
    # with a partial last group
    rng = np.random.default_rng(group)
    packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    scales = rng.uniform(-0.05, 0.05, -(-n // group)).astype(np.float32)
    f = SafeTensorsFile(write(tmp_path / "g.safetensors", {
        "q": ("I4", [n], packed.tobytes()), "qs": ("F32", [scales.size], scales.tobytes())}))
    t = f.load("q", backend, scale="qs", group=group)
    got = np.frombuffer(backend.download(t)[1], np.uint16)
    np.testing.assert_array_equal(got, O.dequant_int4(packed, n, scales, O.FLOAT32, group, O.BFLOAT16))
    t.release()
    t = backend.upload_int4([n], packed, scales, O.FLOAT32, group)
    np.testing.assert_array_equal(np.frombuffer(backend.download(t)[1], np.uint16), got)
    t.release()


def test_scale_for_a_tensor_stored_as_written_is_refused(backend, tmp_path):
    f = SafeTensorsFile(write(tmp_path / "a.safetensors", {
        "w": ("BF16", [4], O.f32_to_bf16(np.ones(4, np.float32)).tobytes()),
        "s": ("F32", [1], np.array([2.0], np.float32).tobytes())}))
    with pytest.raises(M.MFHError, match="stored as written") as e:
        f.load("w", backend, scale="s")
    assert e.value.code == -1


def test_truncated_tensor_fails_from_a_copy_thread(backend, tmp_path):
    # A tensor whose bytes end early: the staging chunk that crosses the end
    # of the file is read in pieces by several host threads, and the piece
    # that hits EOF reports it on the calling thread.  A whole tensor loads
    # after it from the same backend.
    n = (40 << 20) // 4
    body = np.arange(n, dtype=np.float32).tobytes()
    header = {"w": {"dtype": "F32", "shape": [n], "data_offsets": [0, len(body)]}}
    text = json.dumps(header).encode()
    path = tmp_path / "cut.safetensors"
    path.write_bytes(struct.pack("<Q", len(text)) + text + body[:30 << 20])
    f = SafeTensorsFile(path)
    with pytest.raises(M.MFHError, match='safetensors read "w": unexpected EOF'):
        f.load("w", backend)
    good = SafeTensorsFile(write(tmp_path / "whole.safetensors", {"w": ("F32", [n], body)}))
    t = good.load("w", backend)
    assert backend.download(t)[1] == body
    t.release()
