"""CPU tests of the SafeTensors index and reads (include/mfh_safetensors.h),
against weights/reader.go:14-109 and, for files written by the `safetensors`
package, against that package's own view of the same file."""
import json
import struct

import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd.safetensors import SafeTensorsFile
import oracle as O


def write_raw(path, header: dict | str, data: bytes = b"", length=None):
    text = header if isinstance(header, str) else json.dumps(header)
    raw = text.encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw) if length is None else length))
        f.write(raw)
        f.write(data)
    return path


def test_index_matches_the_safetensors_package(tmp_path):
    torch = pytest.importorskip("torch")
    from safetensors import safe_open
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(0)
    tensors = {
        "model.embed.weight": torch.randn(7, 5, generator=g),
        "layers.0.mlp.gate.weight": torch.randn(4, 3, generator=g).to(torch.bfloat16),
        "layers.0.mlp.up.weight": torch.randn(4, 3, generator=g).to(torch.float16),
        "layers.0.q.weight": torch.randn(16, 8, generator=g).to(torch.float8_e4m3fn),
        "layers.0.k.weight": torch.randn(8, 8, generator=g).to(torch.float8_e5m2),
        "layers.0.q.weight_scale": torch.tensor(0.0125),
        "positions": torch.arange(11, dtype=torch.int64),
    }
    path = tmp_path / "w.safetensors"
    save_file(tensors, str(path), metadata={"format": "pt"})
    f = SafeTensorsFile(path)
    index = f.index()
    assert set(index) == set(tensors)
    header_len = struct.unpack("<Q", open(path, "rb").read(8))[0]
    assert f.data_base() == header_len + 8  # the second result of IndexReader
    want_dtype = {torch.float32: ("F32", M.FLOAT32), torch.bfloat16: ("BF16", M.BFLOAT16),
                  torch.float16: ("F16", M.FLOAT16), torch.float8_e4m3fn: ("F8_E4M3", M.F8E4M3),
                  torch.float8_e5m2: ("F8_E5M2", M.F8E5M2), torch.int64: ("I64", M.INT64)}
    with safe_open(str(path), "pt") as ref:
        for name, t in tensors.items():
            meta = index[name]
            assert (meta.dtype, meta.parsed) == want_dtype[t.dtype]
            assert meta.shape == list(t.shape)
            raw = f.read(name)
            assert len(raw) == meta.data_offsets[1] - meta.data_offsets[0]
            got = ref.get_tensor(name)
            assert raw == got.contiguous().reshape(-1).view(torch.uint8).numpy().tobytes()


def test_index_reader_semantics(tmp_path):
    data = bytes(range(64))
    header = ('{"__metadata__": {"k": "v"}, "a": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]},'
              ' "b\\u00e9\\"": {"DType": "fp8-e4m3", "Shape": [16], "DATA_OFFSETS": [16, 32], "extra": [1, {"x": null}]},'
              ' "s": {"dtype": "BF16", "shape": [], "data_offsets": [32, 34]},'
              ' "q": {"dtype": "I4", "shape": [3, 5], "data_offsets": [34, 42]},'
              ' "u": {"dtype": "strange", "shape": [1], "data_offsets": [42, 43]},'
              ' "a": {"dtype": "U8", "shape": [4], "data_offsets": [60, 64]}}')
    f = SafeTensorsFile(write_raw(tmp_path / "h.safetensors", header, data))
    index = f.index()
    assert list(index) == ["a", 'bé"', "s", "q", "u"]  # header order; "__metadata__" skipped
    assert index["a"].dtype == "U8" and index["a"].parsed == M.UINT8  # a repeated key keeps the last value
    assert f.read("a") == data[60:64]
    assert index['bé"'].parsed == M.F8E4M3 and index['bé"'].shape == [16]  # case-insensitive fields
    assert index["s"].shape == [] and f.read("s") == data[32:34]
    assert index["q"].parsed == M.INT4 and f.read("q") == data[34:42]
    assert index["u"].dtype == "strange" and index["u"].parsed == 0  # kept, parsed as Invalid
    with pytest.raises(M.MFHError, match='safetensors: missing tensor "nope"'):
        f.read("nope")


def test_dtype_parse_aliases(tmp_path):
    # dtype.Parse (dtype/dtype.go:242-287)
    names = {"F8_E4M3": M.F8E4M3, " fp8_e5m2 ": M.F8E5M2, "bfloat16": M.BFLOAT16, "Half": M.FLOAT16,
             "double": M.FLOAT64, "INT4": M.INT4, "ubyte": M.UINT8, "B1": 16, "f-32": M.FLOAT32, "F8E4M3FN": 0}
    header = {f"t{i}": {"dtype": n, "shape": [0], "data_offsets": [0, 0]} for i, n in enumerate(names)}
    index = SafeTensorsFile(write_raw(tmp_path / "d.safetensors", header)).index()
    for i, (n, want) in enumerate(names.items()):
        assert index[f"t{i}"].parsed == want, n


@pytest.mark.parametrize("header, length, match", [
    ("{", None, "safetensors index"),
    ('[1, 2]', None, "header is not an object"),
    ('{"a": 1}', None, 'safetensors tensor "a"'),
    ('{"a": {"shape": [1.5], "dtype": "F32", "data_offsets": [0, 4]}}', None, "non-integer"),
    ('{"a": {"dtype": "F32", "data_offsets": 4}}', None, "data_offsets is not an array"),
    ('{"a": {"dtype": "F32", "data_offsets": [0, true]}}', None, "data_offsets holds a non-integer"),
    ('{"a": {"dtype": 7}}', None, "dtype is not a string"),
    ('{}', 10 ** 6, "unexpected EOF"),
    ('{} trailing', None, "trailing data"),
    # numbers as JSON's grammar (and Go's scanner) has them
    ('{"a": {"shape": [01]}}', None, "safetensors index"),
    ('{"a": {"shape": [1.]}}', None, "bad number"),
    ('{"a": {"shape": [1e]}}', None, "bad number"),
    ('{"a": {"shape": [-]}}', None, "bad number"),
    ('{"__metadata__": {"k": 1-2}}', None, "safetensors index"),
])
def test_index_errors(tmp_path, header, length, match):
    path = write_raw(tmp_path / "bad.safetensors", header, length=length)
    with pytest.raises(M.MFHError, match=match):
        SafeTensorsFile(path)


def test_entries_decode_as_json_unmarshal_fills_tensor_meta(tmp_path):
    # weights/reader.go:13-17,64-68: null leaves a field as it was (a nil
    # shape), data_offsets fills [2]int64 with missing elements zero and
    # extra ones skipped, unknown fields and a null entry decode to zeros
    header = ('{"a": {"dtype": "F32", "data_offsets": [4]},'
              ' "b": {"dtype": null, "shape": [null, 3], "data_offsets": [0, 4, "x", {}]},'
              ' "c": null,'
              ' "d": {"DType": "U8", "Shape": [2], "extra": [1, 2], "data_offsets": [null, 2]},'
              ' "e": {"dtype": "U8", "dtype": null, "shape": [5], "shape": null, "data_offsets": [1, 3],'
              ' "data_offsets": [2]}}')
    assert SafeTensorsFile(write_raw(tmp_path / "n.safetensors", " null ")).index() == {}
    index = SafeTensorsFile(write_raw(tmp_path / "m.safetensors", header, b"\0" * 8)).index()
    got = {k: (v.dtype, v.shape, list(v.data_offsets)) for k, v in index.items()}
    assert got == {"a": ("F32", [], [4, 0]), "b": ("", [0, 3], [0, 4]), "c": ("", [], [0, 0]),
                   "d": ("U8", [2], [0, 2]), "e": ("U8", [], [2, 0])}


def test_truncated_file_and_out_of_range_reads(tmp_path):
    (tmp_path / "short.safetensors").write_bytes(b"\x01\x02")
    with pytest.raises(M.MFHError, match="safetensors index: unexpected EOF"):
        SafeTensorsFile(tmp_path / "short.safetensors")
    f = SafeTensorsFile(write_raw(tmp_path / "r.safetensors",
                                  {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]},
                                   "b": {"dtype": "F32", "shape": [1], "data_offsets": [8, 4]}}, b"\0" * 12))
    with pytest.raises(M.MFHError, match='safetensors read "a": unexpected EOF'):
        f.read("a")
    with pytest.raises(M.MFHError, match='safetensors read "b": bad data_offsets'):
        f.read("b")
    # offsets near INT64_MAX: an EOF, not a wrapped sum that reads elsewhere
    big = (1 << 63) - 1
    g = SafeTensorsFile(write_raw(tmp_path / "big.safetensors",
                                  {"c": {"dtype": "U8", "shape": [1], "data_offsets": [big - 1, big]},
                                   "d": {"dtype": "U8", "shape": [1], "data_offsets": [0, big]}}, b"\0" * 4))
    for name in ("c", "d"):
        with pytest.raises(M.MFHError, match=f'safetensors read "{name}": unexpected EOF'):
            g.read(name)
    with pytest.raises(M.MFHError):
        SafeTensorsFile(tmp_path / "missing.safetensors")


def test_load_requires_a_device(tmp_path):
    if M.lib().mfh_init(0) == 0:
        pytest.skip("a GPU is present; loads are covered by the GPU tests")
    f = SafeTensorsFile(write_raw(tmp_path / "l.safetensors", {"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}},
                                  b"\0" * 4))
    assert O.FLOAT32 == M.FLOAT32
    from manifesto_amd.backend import Backend
    with pytest.raises(M.MFHError):
        Backend(0)
    assert f.read("a") == b"\0" * 4


def test_scale_for_a_tensor_stored_as_written_is_refused(tmp_path):
    # Checked from the index before any device work, so it needs no GPU: a
    # scale names nothing to multiply for an F32/F16/BF16 tensor.
    import ctypes
    from manifesto_amd import safetensors as S
    f = SafeTensorsFile(write_raw(tmp_path / "s.safetensors", {
        "w": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]},
        "s": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\0" * 8))
    h = ctypes.c_void_p()
    rc = S._L().mfh_safetensors_load(f._h, b"w", None, b"s", 0, ctypes.byref(h))
    assert rc == -1 and "stored as written" in M.last_error()
    assert not h.value


def test_header_parser_survives_mutated_headers(tmp_path):
    # Every mutation of a valid header (bytes flipped, dropped, duplicated or
    # cut, the stated length off by a few bytes) either indexes or raises
    # MFHError; none may crash the process or read past the header.
    rng = np.random.default_rng(31)
    base = json.dumps({"__metadata__": {"format": "pt"},  # the key's escapes: \u00e9 and a surrogate pair
                       "w\u00e9\U0001f600": {"dtype": "F8_E4M3", "shape": [2, 3], "data_offsets": [0, 6]},
                       "s": {"dtype": "F32", "shape": [], "data_offsets": [6, 10]},
                       "n": {"dtype": "I4", "shape": [4], "data_offsets": [10, 12]}}).encode()
    assert b"\\ud83d\\ude00" in base
    data = bytes(range(12))
    seen = {"ok": 0, "error": 0}
    for trial in range(400):
        raw = bytearray(base)
        for _ in range(int(rng.integers(1, 4))):
            kind = int(rng.integers(0, 4))
            at = int(rng.integers(0, len(raw)))
            if kind == 0:
                raw[at] = int(rng.integers(0, 256))
            elif kind == 1 and len(raw) > 1:
                del raw[at]
            elif kind == 2:
                raw[at:at] = raw[at:at + int(rng.integers(1, 8))]
            else:
                raw = raw[:at]
        length = len(raw) + int(rng.integers(-3, 4)) if trial % 5 == 0 else len(raw)
        path = tmp_path / f"m{trial}.safetensors"
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", max(0, length)))
            f.write(bytes(raw))
            f.write(data)
        try:
            f = SafeTensorsFile(str(path))
            for name in f.index():
                try:
                    f.read(name)
                except M.MFHError:
                    pass
            seen["ok"] += 1
        except M.MFHError:
            seen["error"] += 1
    assert seen["ok"] > 0 and seen["error"] > 0, seen


def test_names_unquoted_like_encoding_json(tmp_path):
    # encoding/json replaces invalid UTF-8 bytes and unpaired surrogate
    # escapes with U+FFFD instead of failing; a high surrogate followed by
    # an escape that is not a low surrogate leaves that escape to be read on
    # its own
    raw = ('{"a\\ud83d\\ude00": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]},'
           ' "b\\udc00x": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]},'
           ' "c\\ud800\\u0041": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]},'
           ' "d\\ud800": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]},').encode()
    raw += b' "e\xff\xc0\x80\xed\xa0\x80z\xc3\xa9": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}'
    path = tmp_path / "names.safetensors"
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        f.write(b"\x07")
    names = list(SafeTensorsFile(str(path)).index())
    # \xff: one U+FFFD; \xc0\x80 (overlong): two; \xed\xa0\x80 (a surrogate
    # in UTF-8): three, one per byte; then "z" and a valid e-acute
    assert names == ["a\U0001f600", "b�x", "c�A", "d�", "e" + "�" * 6 + "zé"]
