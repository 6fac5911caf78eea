"""ctypes binding of the mfh C ABI (include/mfh.h).

Device buffers are passed as integer device pointers (for example
``torch.Tensor.data_ptr()``) and streams as ``hipStream_t`` integers (for
example ``torch.cuda.current_stream().cuda_stream``); 0 means the null stream.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmfh.so")

FLOAT64, FLOAT32, FLOAT16, BFLOAT16, F8E4M3, F8E5M2 = 1, 2, 3, 4, 5, 6
INT64, INT32, INT16, INT8, INT4 = 7, 8, 9, 10, 11
UINT64, UINT32, UINT16, UINT8 = 12, 13, 14, 15

OPERAND_FULL, OPERAND_PERIODIC, OPERAND_SCALAR = 0, 1, 2
FUSION_PRECISE = 1
FUSION_SHORT_QUOTIENT = 2
FUSION_NO_ROUNDING_TEST = 4

MFH_OK = 0


class MFHError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"mfh error {code}: {message}")
        self.code = code


class AstNode(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("input_index", ctypes.c_int32), ("value", ctypes.c_double)]


class Operand(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_uint8), ("mode", ctypes.c_uint8),
                ("reserved", ctypes.c_uint8 * 6), ("period", ctypes.c_int64)]


_lib = None


def lib():
    """Loads libmfh.so; raises if it has not been built (no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MFHError(-6, f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        try:
            # torch ships its own libamdhip64.so.7 / libhiprtc.so.7; loading it
            # first makes libmfh bind to those same copies (one HIP runtime
            # per process) instead of a second set from /opt/rocm/lib.
            import torch  # noqa: F401
        except ImportError:
            pass
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    c = ctypes
    vp, i64, i32, u8, f32 = c.c_void_p, c.c_int64, c.c_int32, c.c_uint8, c.c_float
    sig = {
        "mfh_version": (c.c_int, []),
        "mfh_init": (c.c_int, [c.c_int]),
        "mfh_shutdown": (c.c_int, []),
        "mfh_last_error": (c.c_char_p, []),
        "mfh_take_sticky_error": (c.c_int, [vp]),
        "mfh_capabilities": (c.c_int, [c.POINTER(i64), c.POINTER(i32), c.POINTER(i32)]),
        "mfh_alloc": (c.c_int, [c.POINTER(vp), c.c_size_t]),
        "mfh_free": (c.c_int, [vp]),
        "mfh_memcpy_h2d": (c.c_int, [vp, vp, c.c_size_t, vp]),
        "mfh_memcpy_d2h": (c.c_int, [vp, vp, c.c_size_t, vp]),
        "mfh_stream_sync": (c.c_int, [vp]),
        "mfh_set_launch_config": (c.c_int, [c.c_char_p, i32, i32]),
        "mfh_get_launch_config": (c.c_int, [c.c_char_p, c.POINTER(i32), c.POINTER(i32)]),
        "mfh_set_launch_threads": (c.c_int, [c.c_char_p, i32]),
        "mfh_get_launch_threads": (c.c_int, [c.c_char_p, c.POINTER(i32)]),
        "mfh_axpy": (None, [vp, vp, i64, f32, u8, vp]),
        "mfh_scalar_broadcast": (c.c_int, [vp, u8, vp, u8, i64, f32, i32, vp]),
        "mfh_linspace": (c.c_int, [vp, u8, i64, f32, f32, i32, vp]),
        "mfh_convert": (c.c_int, [vp, u8, vp, u8, i64, vp]),
        "mfh_dequant_fp8": (c.c_int, [vp, u8, vp, u8, i64, f32, vp]),
        "mfh_dequant_int4": (c.c_int, [vp, u8, vp, i64, vp, u8, i64, vp]),
        "mfh_fusion_compile": (c.c_int, [c.POINTER(AstNode), i32, c.POINTER(Operand), i32, u8,
                                          c.c_char_p, c.c_uint32, c.POINTER(vp)]),
        "mfh_fusion_source": (c.c_char_p, [vp]),
        "mfh_fusion_kernel_name": (c.c_char_p, [vp]),
        "mfh_fusion_identifier": (c.c_char_p, [vp]),
        "mfh_fusion_num_inputs": (i32, [vp]),
        "mfh_fusion_launch": (c.c_int, [vp, c.POINTER(vp), i32, vp, i64, vp]),
        "mfh_fusion_release": (c.c_int, [vp]),
        "mfh_fusion_cache_dir": (c.c_int, [c.c_char_p]),
        "mfh_fusion_cache_stats": (c.c_int, [c.POINTER(i64), c.POINTER(i64)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def last_error() -> str:
    msg = lib().mfh_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc != MFH_OK:
        raise MFHError(rc, last_error())


def init(device: int = 0) -> None:
    check(lib().mfh_init(device))


def take_sticky_error(stream: int = 0) -> None:
    """Raises the first sticky error left on `stream` (and clears it)."""
    check(lib().mfh_take_sticky_error(stream))


def stream_sync(stream: int = 0) -> None:
    check(lib().mfh_stream_sync(stream))


def set_launch_config(kernel: str, blocks_per_cu: int = 0, items_per_thread: int = 0) -> None:
    """Launch shape of a streaming-kernel family (0 keeps the current value)."""
    check(lib().mfh_set_launch_config(kernel.encode(), blocks_per_cu, items_per_thread))


def get_launch_config(kernel: str):
    bpc, ipt = ctypes.c_int32(), ctypes.c_int32()
    check(lib().mfh_get_launch_config(kernel.encode(), ctypes.byref(bpc), ctypes.byref(ipt)))
    return bpc.value, ipt.value


def set_launch_threads(kernel: str, threads: int) -> None:
    """Threads per workgroup of a kernel family (0 keeps, -1 restores the default)."""
    check(lib().mfh_set_launch_threads(kernel.encode(), threads))


def get_launch_threads(kernel: str) -> int:
    t = ctypes.c_int32()
    check(lib().mfh_get_launch_threads(kernel.encode(), ctypes.byref(t)))
    return t.value


# ---- runtime math / conversion wrappers ------------------------------------

def axpy(y: int, x: int, count: int, alpha: float, dtype: int, stream: int = 0) -> None:
    """axpyDevice.Axpy: no return value; failures surface at stream_sync."""
    lib().mfh_axpy(y, x, count, alpha, dtype, stream)


def dequant_fp8(out: int, out_dtype: int, src: int, fp8_dtype: int, count: int, scale: float,
                stream: int = 0) -> None:
    check(lib().mfh_dequant_fp8(out, out_dtype, src, fp8_dtype, count, scale, stream))


def dequant_int4(out: int, out_dtype: int, packed: int, count: int, scales: int, scale_dtype: int,
                 group: int, stream: int = 0) -> None:
    check(lib().mfh_dequant_int4(out, out_dtype, packed, count, scales, scale_dtype, group, stream))


def convert(out: int, out_dtype: int, src: int, in_dtype: int, count: int, stream: int = 0) -> None:
    check(lib().mfh_convert(out, out_dtype, src, in_dtype, count, stream))


_OPS = {"add": 0, "sub": 1, "mul": 2, "div": 3}


def scalar_broadcast(out: int, out_dtype: int, src: int, in_dtype: int, count: int, scalar: float,
                     op: str, stream: int = 0) -> None:
    check(lib().mfh_scalar_broadcast(out, out_dtype, src, in_dtype, count, scalar, _OPS.get(op, -1), stream))


def linspace(out: int, out_dtype: int, count: int, start: float, stop: float, endpoint: bool = True,
             stream: int = 0) -> None:
    check(lib().mfh_linspace(out, out_dtype, count, start, stop, 1 if endpoint else 0, stream))


# ---- fused kernels -----------------------------------------------------------

def fusion_cache_dir(path) -> None:
    """Keeps compiled kernels in directory `path` between processes (None
    turns it off)."""
    check(lib().mfh_fusion_cache_dir(os.fsencode(path) if path else None))


def fusion_cache_stats() -> tuple:
    """(kernels compiled by hiprtc, kernels read from the cache directory)."""
    compiles, hits = ctypes.c_int64(), ctypes.c_int64()
    check(lib().mfh_fusion_cache_stats(ctypes.byref(compiles), ctypes.byref(hits)))
    return compiles.value, hits.value


class FusedKernel:
    """One compiled FusionAST (the HIP codegen target).

    ``nodes`` is the pre-order list of (type, input_index, value) triples;
    ``operands`` is a list of (dtype, mode, period) triples, one per input.
    """

    def __init__(self, nodes, operands, out_dtype: int, output_port: str | None = None,
                 flags: int = 0):
        arr = (AstNode * len(nodes))(*[AstNode(t, i, v) for (t, i, v) in nodes]) if nodes else None
        ops = (Operand * max(1, len(operands)))()
        for k, (dt, mode, period) in enumerate(operands):
            ops[k].dtype, ops[k].mode, ops[k].period = dt, mode, period
        handle = ctypes.c_void_p()
        port = output_port.encode() if output_port is not None else None
        rc = lib().mfh_fusion_compile(arr, len(nodes), ops, len(operands), out_dtype, port, flags,
                                      ctypes.byref(handle))
        check(rc)
        self._h = handle
        self.n_inputs = len(operands)

    @property
    def source(self) -> str:
        return lib().mfh_fusion_source(self._h).decode()

    @property
    def kernel_name(self) -> str:
        return lib().mfh_fusion_kernel_name(self._h).decode()

    @property
    def identifier(self) -> str:
        return lib().mfh_fusion_identifier(self._h).decode()

    def launch(self, inputs, out: int, count: int, stream: int = 0) -> None:
        ptrs = (ctypes.c_void_p * max(1, len(inputs)))(*inputs)
        check(lib().mfh_fusion_launch(self._h, ptrs, len(inputs), out, count, stream))

    def close(self) -> None:
        if self._h:
            lib().mfh_fusion_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
