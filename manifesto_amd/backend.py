"""HIP tensor backend of the mfh ABI (include/mfh_backend.h): tensor.Backend /
tensor.Tensor over device memory, dequantising uploads and the resident axpy
(runtime/axpy.go:44-93).  Names follow the reference's Go API; every call
runs in libmfh.so.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import abi
from .abi import check, lib

STATE_READY, STATE_PENDING, STATE_MUTATING, STATE_CLOSED = 0, 1, 2, 3
ERR_SHAPE_INVALID, ERR_TENSOR_CLOSED, ERR_LAYOUT_UNSUPPORTED = -8, -9, -10
LAYOUT_DENSE = 0


class Capabilities(ctypes.Structure):
    """tensor.Capabilities (tensor/backend.go:80-110)."""
    _fields_ = [("max_bytes", ctypes.c_int64), ("supports_async", ctypes.c_int32),
                ("supports_sparse", ctypes.c_int32), ("supports_autograd", ctypes.c_int32),
                ("native_alignment", ctypes.c_int32), ("numa_nodes", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


_declared = False


def _L():
    global _declared
    L = lib()
    if not _declared:
        c = ctypes
        vp, i32, i64, u8, sz = c.c_void_p, c.c_int32, c.c_int64, c.c_uint8, c.c_size_t
        shp = c.POINTER(i64)
        sig = {
            "mfh_backend_open": (c.c_int, [c.c_int, c.POINTER(vp)]),
            "mfh_backend_location": (c.c_char_p, [vp]),
            "mfh_backend_supported_dtypes": (i32, [vp, c.POINTER(u8), i32]),
            "mfh_backend_supported_layouts": (i32, [vp, c.POINTER(u8), i32]),
            "mfh_backend_capabilities": (c.c_int, [vp, c.POINTER(Capabilities)]),
            "mfh_backend_upload": (c.c_int, [vp, shp, i32, u8, vp, sz, c.POINTER(vp)]),
            "mfh_backend_upload_async": (c.c_int, [vp, shp, i32, u8, vp, sz, c.POINTER(vp)]),
            "mfh_backend_upload_sparse": (c.c_int, [vp]),
            "mfh_backend_upload_fp8": (c.c_int, [vp, shp, i32, u8, vp, sz, c.c_float, u8, c.POINTER(vp)]),
            "mfh_backend_upload_int4": (c.c_int, [vp, shp, i32, vp, sz, vp, u8, i64, u8, c.POINTER(vp)]),
            "mfh_backend_upload_fp8_async": (c.c_int, [vp, shp, i32, u8, vp, sz, c.c_float, u8, c.POINTER(vp)]),
            "mfh_backend_upload_int4_async": (c.c_int, [vp, shp, i32, vp, sz, vp, u8, i64, u8, c.POINTER(vp)]),
            "mfh_backend_download": (c.c_int, [vp, vp, c.POINTER(u8), vp, sz, c.POINTER(sz)]),
            "mfh_backend_close": (c.c_int, [vp]),
            "mfh_backend_release": (c.c_int, [vp]),
            "mfh_tensor_dtype": (u8, [vp]),
            "mfh_tensor_len": (i64, [vp]),
            "mfh_tensor_bytes": (i64, [vp]),
            "mfh_tensor_shape": (i32, [vp, shp, i32]),
            "mfh_tensor_location": (c.c_char_p, [vp]),
            "mfh_tensor_state": (i32, [vp]),
            "mfh_tensor_dispatch_pointer": (vp, [vp]),
            "mfh_tensor_sync": (c.c_int, [vp]),
            "mfh_tensor_slice": (c.c_int, [vp, i64, i64, c.POINTER(vp)]),
            "mfh_tensor_reshape": (c.c_int, [vp, shp, i32, c.POINTER(vp)]),
            "mfh_tensor_close": (c.c_int, [vp]),
            "mfh_tensor_release": (c.c_int, [vp]),
            "mfh_axpy_onto_resident": (c.c_int, [vp, vp, vp, c.c_float]),
            "mfh_backend_graph_call": (c.c_int, [vp, vp, c.POINTER(c.c_char_p), c.POINTER(vp), i32,
                                                 c.POINTER(c.c_char_p), i32, c.POINTER(vp)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _declared = True
    return L


def _shape(dims):
    dims = [int(d) for d in dims]
    return (ctypes.c_int64 * max(1, len(dims)))(*dims), len(dims)


def _buf(data) -> tuple:
    """(pointer, nbytes, keep-alive) of bytes / bytearray / numpy data."""
    a = np.ascontiguousarray(data) if isinstance(data, np.ndarray) else np.frombuffer(bytes(data), dtype=np.uint8)
    return (a.ctypes.data if a.nbytes else None), a.nbytes, a


class Tensor:
    """A device-resident tensor (tensor.Tensor) owned by a Backend."""

    def __init__(self, backend, handle):
        self._backend = backend
        self._h = handle

    def dtype(self) -> int:
        return _L().mfh_tensor_dtype(self._h)

    def len(self) -> int:
        return _L().mfh_tensor_len(self._h)

    def bytes(self) -> int:
        return _L().mfh_tensor_bytes(self._h)

    def shape(self) -> list:
        L = _L()
        n = L.mfh_tensor_shape(self._h, None, 0)
        dims = (ctypes.c_int64 * max(1, n))()
        L.mfh_tensor_shape(self._h, dims, n)
        return list(dims[:n])

    def location(self) -> str:
        return _L().mfh_tensor_location(self._h).decode()

    def state(self) -> int:
        return _L().mfh_tensor_state(self._h)

    def dispatch_pointer(self) -> int:
        return _L().mfh_tensor_dispatch_pointer(self._h) or 0

    def sync(self) -> None:
        check(_L().mfh_tensor_sync(self._h))

    def slice(self, start: int, length: int) -> "Tensor":
        h = ctypes.c_void_p()
        check(_L().mfh_tensor_slice(self._h, start, length, ctypes.byref(h)))
        return Tensor(self._backend, h)

    def reshape(self, dims) -> "Tensor":
        arr, rank = _shape(dims)
        h = ctypes.c_void_p()
        check(_L().mfh_tensor_reshape(self._h, arr, rank, ctypes.byref(h)))
        return Tensor(self._backend, h)

    def raw_bytes(self):
        """Tensor.RawBytes: (dtype, bytes) through Backend.Download."""
        return self._backend.download(self)

    def close(self) -> None:
        check(_L().mfh_tensor_close(self._h))

    def release(self) -> None:
        if self._h:
            _L().mfh_tensor_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Backend:
    """tensor.Backend for HIP device memory (Location "hip")."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(_L().mfh_backend_open(device, ctypes.byref(h)))
        self._h = h

    def location(self) -> str:
        return _L().mfh_backend_location(self._h).decode()

    def supported_dtypes(self) -> list:
        arr = (ctypes.c_uint8 * 32)()
        n = _L().mfh_backend_supported_dtypes(self._h, arr, 32)
        return list(arr[:n])

    def supported_layouts(self) -> list:
        arr = (ctypes.c_uint8 * 8)()
        n = _L().mfh_backend_supported_layouts(self._h, arr, 8)
        return list(arr[:n])

    def capabilities(self) -> Capabilities:
        caps = Capabilities()
        check(_L().mfh_backend_capabilities(self._h, ctypes.byref(caps)))
        return caps

    def _upload(self, fn, dims, dtype, data):
        arr, rank = _shape(dims)
        ptr, nbytes, keep = _buf(data)
        h = ctypes.c_void_p()
        check(fn(self._h, arr, rank, dtype, ptr, nbytes, ctypes.byref(h)))
        del keep
        return Tensor(self, h)

    def upload(self, dims, dtype: int, data) -> Tensor:
        return self._upload(_L().mfh_backend_upload, dims, dtype, data)

    def upload_async(self, dims, dtype: int, data) -> Tensor:
        return self._upload(_L().mfh_backend_upload_async, dims, dtype, data)

    def upload_sparse(self):
        check(_L().mfh_backend_upload_sparse(self._h))

    def upload_fp8(self, dims, fp8_dtype: int, codes, scale: float, out_dtype: int = abi.BFLOAT16,
                   queued: bool = False) -> Tensor:
        """Scaled FP8 upload; `queued` returns once the codes are staged and
        every chunk is queued (the tensor pending until it has run)."""
        fn = _L().mfh_backend_upload_fp8_async if queued else _L().mfh_backend_upload_fp8
        arr, rank = _shape(dims)
        ptr, nbytes, keep = _buf(codes)
        h = ctypes.c_void_p()
        check(fn(self._h, arr, rank, fp8_dtype, ptr, nbytes, scale, out_dtype, ctypes.byref(h)))
        return Tensor(self, h)

    def upload_int4(self, dims, packed, scales, scale_dtype: int, group: int,
                    out_dtype: int = abi.BFLOAT16, queued: bool = False) -> Tensor:
        """Int4 upload with per-group scales; `queued` as for upload_fp8."""
        fn = _L().mfh_backend_upload_int4_async if queued else _L().mfh_backend_upload_int4
        arr, rank = _shape(dims)
        ptr, nbytes, keep = _buf(packed)
        sptr, _, skeep = _buf(scales)
        h = ctypes.c_void_p()
        check(fn(self._h, arr, rank, ptr, nbytes, sptr, scale_dtype, group, out_dtype, ctypes.byref(h)))
        return Tensor(self, h)

    def download(self, tensor: Tensor, out=None):
        """Backend.Download: (storage dtype, bytes).  The bytes are a
        bytearray the call fills (or `out`, a writable buffer of at least the
        tensor's size, reused as is)."""
        L = _L()
        n = max(0, tensor.len()) * max(1, _size(tensor.dtype()))
        if out is None:
            out = bytearray(n)
        view = memoryview(out).cast("B")
        if view.nbytes < n:
            raise ValueError(f"download: buffer holds {view.nbytes} bytes, need {n}")
        ptr = (ctypes.c_char * max(1, view.nbytes)).from_buffer(view) if n else None
        dt, got = ctypes.c_uint8(), ctypes.c_size_t()
        check(L.mfh_backend_download(self._h, tensor._h, ctypes.byref(dt), ptr, view.nbytes, ctypes.byref(got)))
        return dt.value, out if got.value == view.nbytes else view[:got.value]

    def axpy_onto_resident(self, y: Tensor, x: Tensor, alpha: float) -> Tensor:
        check(_L().mfh_axpy_onto_resident(self._h, y._h, x._h, alpha))
        return y

    def graph_call(self, graph, inputs: dict, output_keys) -> dict:
        """runtime.Backend.CallGraph over resident tensors: `inputs` maps
        graph input names to Tensors; returns {key: Tensor} with one new flat
        tensor of this backend per output key, pending until the call has
        run."""
        names = list(inputs)
        keys = list(output_keys)
        c_names = (ctypes.c_char_p * max(1, len(names)))(*[n.encode() for n in names])
        c_ins = (ctypes.c_void_p * max(1, len(names)))(*[inputs[n]._h for n in names])
        c_keys = (ctypes.c_char_p * max(1, len(keys)))(*[k.encode() for k in keys])
        c_outs = (ctypes.c_void_p * max(1, len(keys)))()
        check(_L().mfh_backend_graph_call(self._h, graph._h, c_names, c_ins, len(names), c_keys, len(keys), c_outs))
        return {k: Tensor(self, c_outs[j]) for j, k in enumerate(keys)}

    def close(self) -> None:
        check(_L().mfh_backend_close(self._h))

    def release(self) -> None:
        if getattr(self, "_h", None):
            _L().mfh_backend_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


def _size(dtype: int) -> int:
    return {abi.FLOAT64: 8, abi.FLOAT32: 4, abi.FLOAT16: 2, abi.BFLOAT16: 2, abi.F8E4M3: 1, abi.F8E5M2: 1,
            abi.INT64: 8, abi.INT32: 4, abi.INT16: 2, abi.INT8: 1, abi.UINT64: 8, abi.UINT32: 4,
            abi.UINT16: 2, abi.UINT8: 1}.get(dtype, 0)
