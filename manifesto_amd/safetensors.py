"""SafeTensors reader and streaming loader of the mfh ABI
(include/mfh_safetensors.h), mirroring weights/reader.go (IndexFile,
ReadTensor) and loading tensors onto a HIP Backend without staging the file
in host memory.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from .abi import check, lib
from .backend import Backend, Tensor, _L as _backend_L


class _Meta(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype_name", ctypes.c_char_p), ("dtype", ctypes.c_uint8),
                ("reserved", ctypes.c_uint8 * 3), ("rank", ctypes.c_int32), ("begin", ctypes.c_int64),
                ("end", ctypes.c_int64)]


_declared = False


def _L():
    global _declared
    L = lib()
    if not _declared:
        c = ctypes
        vp, i32, i64, sz, cp = c.c_void_p, c.c_int32, c.c_int64, c.c_size_t, c.c_char_p
        sig = {
            "mfh_safetensors_open": (c.c_int, [cp, c.POINTER(vp)]),
            "mfh_safetensors_close": (c.c_int, [vp]),
            "mfh_safetensors_data_base": (i64, [vp]),
            "mfh_safetensors_count": (i32, [vp]),
            "mfh_safetensors_entry": (c.c_int, [vp, i32, c.POINTER(_Meta), c.POINTER(i64), i32]),
            "mfh_safetensors_find": (i32, [vp, cp]),
            "mfh_safetensors_read": (c.c_int, [vp, cp, vp, sz, c.POINTER(sz)]),
            "mfh_safetensors_load": (c.c_int, [vp, cp, vp, cp, i64, c.POINTER(vp)]),
            "mfh_safetensors_load_async": (c.c_int, [vp, cp, vp, cp, i64, c.POINTER(vp)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _declared = True
    return L


@dataclass
class TensorMeta:
    """weights.TensorMeta (weights/reader.go:14-18) plus the parsed dtype."""
    dtype: str
    shape: list
    data_offsets: tuple
    parsed: int


class SafeTensorsFile:
    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(_L().mfh_safetensors_open(str(path).encode(), ctypes.byref(h)))
        self._h = h

    def data_base(self) -> int:
        return _L().mfh_safetensors_data_base(self._h)

    def index(self) -> dict:
        """IndexFile: name -> TensorMeta (in header order)."""
        L = _L()
        out = {}
        for i in range(L.mfh_safetensors_count(self._h)):
            m = _Meta()
            dims = (ctypes.c_int64 * 64)()
            check(L.mfh_safetensors_entry(self._h, i, ctypes.byref(m), dims, 64))
            out[m.name.decode()] = TensorMeta(m.dtype_name.decode(), list(dims[:m.rank]), (m.begin, m.end), m.dtype)
        return out

    def read(self, name: str) -> bytes:
        """ReadTensor: the raw bytes of one entry."""
        L = _L()
        n = ctypes.c_size_t()
        check(L.mfh_safetensors_read(self._h, name.encode(), None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(1, n.value))
        check(L.mfh_safetensors_read(self._h, name.encode(), buf, n.value, ctypes.byref(n)))
        return buf.raw[:n.value]

    def _load(self, fn, name, backend, scale, group) -> Tensor:
        _backend_L()
        h = ctypes.c_void_p()
        check(fn(self._h, name.encode(), backend._h, scale.encode() if scale else None, group, ctypes.byref(h)))
        return Tensor(backend, h)

    def load(self, name: str, backend: Backend, scale: str | None = None, group: int = 0) -> Tensor:
        """Streams one tensor onto `backend` (FP8 / I4 dequantised)."""
        return self._load(_L().mfh_safetensors_load, name, backend, scale, group)

    def load_async(self, name: str, backend: Backend, scale: str | None = None, group: int = 0) -> Tensor:
        """The same load, returned once the file has been read; the tensor is
        pending until its transfer and dequant have run (Tensor.sync)."""
        return self._load(_L().mfh_safetensors_load_async, name, backend, scale, group)

    def close(self) -> None:
        if getattr(self, "_h", None):
            _L().mfh_safetensors_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
