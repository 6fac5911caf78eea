"""GPU tests of the SafeTensors streaming loader (mfh_safetensors_load): tensors
go from the file through the backend's pinned staging ring onto the device,
FP8 / I4 dequantised there; results are checked bit for bit against the
oracle on the same bytes."""
import json
import struct

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
