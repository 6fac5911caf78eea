"""CPU oracle for manifesto's Go hot path — TEST INFRASTRUCTURE ONLY.

A ctypes binding of ``oracle/liboracle.so``, the C restatement of the
reference's dtype codecs (dtype/fp8.go, dtype/bfloat16.go, dtype/float16.go,
dtype/int4.go), byte-buffer converters (dtype/convert/convert.go), fused-chain
evaluator (codegen/cpu.go:59-214), axpy (runtime/axpy.go:95-194) and host math
(runtime/executor_math.go).  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg import this module, and only as the checker;
the product library never loads it.

Parity status per function (details in oracle.c):
- codecs, converters, axpy, scalar broadcast, linspace, dequant: pinned by
  the reference's golden vectors and by closed forms (tests/test_oracle_*.py):
  FP8 decode over every code, FP8 encode by brute-force nearest-even plus the
  hand-derived subnormal quirks of both formats, scaled FP8 dequant against
  the closed-form value times an f32 scale narrowed by torch / numpy (with
  scales where an f64 product would differ), 16-bit axpy against numpy f32
  arithmetic narrowed by torch / numpy, wide integers against numpy's
  f64 conversion;
- evaluator transcendentals (exp, log, tanh, sigmoid, silu, gelu): pinned to
  <=1 f32 ulp by independent f64 formulas; their last bit follows glibc, not
  Go's math package (which is absent here) — "parity unpinned" in that bit.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

FLOAT64, FLOAT32, FLOAT16, BFLOAT16, F8E4M3, F8E5M2 = 1, 2, 3, 4, 5, 6
INT64, INT32, INT16, INT8, INT4 = 7, 8, 9, 10, 11
UINT64, UINT32, UINT16, UINT8 = 12, 13, 14, 15

# optimizer.NodeType values (optimizer/fusion_ast.go:30-65).
(N_INVALID, N_INPUT, N_CONSTANT, N_ADD, N_SUB, N_MUL, N_DIV, N_MAX, N_MIN,
 N_NEG, N_ABS, N_SQRT, N_EXP, N_LOG, N_RELU, N_SIGMOID, N_TANH, N_SILU, N_GELU,
 N_LEAKY_RELU) = range(20)


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


class _Node(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("input_index", ctypes.c_int32),
                ("value", ctypes.c_double)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    c = ctypes
    vp, i64, i32, f32 = c.c_void_p, c.c_int64, c.c_int, c.c_float
    L.orc_e4m3_to_f32.restype = f32
    L.orc_e4m3_to_f32.argtypes = [c.c_uint8]
    L.orc_e5m2_to_f32.restype = f32
    L.orc_e5m2_to_f32.argtypes = [c.c_uint8]
    L.orc_f32_to_e4m3.restype = c.c_uint8
    L.orc_f32_to_e4m3.argtypes = [f32]
    L.orc_f32_to_e5m2.restype = c.c_uint8
    L.orc_f32_to_e5m2.argtypes = [f32]
    L.orc_f32_to_fp8_buf.restype = None
    L.orc_f32_to_fp8_buf.argtypes = [c.c_void_p, c.c_int64, c.c_int, c.c_void_p]
    L.orc_f32_to_bf16.restype = c.c_uint16
    L.orc_f32_to_bf16.argtypes = [f32]
    L.orc_bf16_to_f32.restype = f32
    L.orc_bf16_to_f32.argtypes = [c.c_uint16]
    L.orc_f16_to_f32.restype = f32
    L.orc_f16_to_f32.argtypes = [c.c_uint16]
    L.orc_f32_to_f16.restype = c.c_uint16
    L.orc_f32_to_f16.argtypes = [f32]
    L.orc_int4_lo.restype = c.c_int8
    L.orc_int4_lo.argtypes = [c.c_uint8]
    L.orc_int4_hi.restype = c.c_int8
    L.orc_int4_hi.argtypes = [c.c_uint8]
    L.orc_logical_elements.argtypes = [i32, i64, c.POINTER(i64)]
    for name in ("orc_bytes_to_f64", "orc_bytes_to_f32", "orc_bytes_to_bf16", "orc_bytes_to_f16", "orc_bytes_to_i8"):
        getattr(L, name).argtypes = [i32, vp, i64, vp]
    L.orc_f32_to_bf16_buf.argtypes = [vp, i64, vp]
    L.orc_f32_to_f16_buf.argtypes = [vp, i64, vp]
    L.orc_dequant_fp8.argtypes = [vp, i64, i32, f32, i32, vp]
    L.orc_dequant_int4.argtypes = [vp, i64, vp, i32, i64, i32, vp]
    L.orc_node_arity.argtypes = [c.c_int32]
    L.orc_run.argtypes = [vp, i32, vp, vp, i32, vp, i64]
    L.orc_eval_unary.restype = f32
    L.orc_eval_unary.argtypes = [c.c_int32, f32]
    L.orc_eval_binary.restype = f32
    L.orc_eval_binary.argtypes = [c.c_int32, f32, f32]
    L.orc_axpy_f32.argtypes = [vp, vp, i64, f32]
    L.orc_axpy_storage.argtypes = [vp, vp, i64, f32, i32]
    L.orc_scalar_broadcast.argtypes = [vp, i64, f32, i32, vp]
    L.orc_linspace.argtypes = [f32, f32, i64, i32, vp]
    L.orc_fold.argtypes = [c.c_int32, vp, i32, vp]


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class OracleError(RuntimeError):
    pass


# -- scalar codecs ---------------------------------------------------------

def e4m3_to_f32(code: int) -> float:
    return lib().orc_e4m3_to_f32(code)


def e5m2_to_f32(code: int) -> float:
    return lib().orc_e5m2_to_f32(code)


def f32_to_e4m3(v: float) -> int:
    return lib().orc_f32_to_e4m3(v)


def f32_to_e5m2(v: float) -> int:
    return lib().orc_f32_to_e5m2(v)


def f32_to_fp8(values: np.ndarray, fmt: int) -> np.ndarray:
    """BytesToFloat8E4M3 / BytesToFloat8E5M2 of f32 values (fmt F8E4M3/F8E5M2)."""
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(values.size, dtype=np.uint8)
    lib().orc_f32_to_fp8_buf(_ptr(values), values.size, fmt, _ptr(out))
    return out


def f32_bits_to_bf16(bits: int) -> int:
    f = np.array([bits], dtype=np.uint32).view(np.float32)[0]
    return lib().orc_f32_to_bf16(float(f))


def f16_to_f32_bits(h: int) -> int:
    out = np.zeros(1, dtype=np.float32)
    raw = np.array([h], dtype=np.uint16)
    lib().orc_bytes_to_f32(FLOAT16, _ptr(raw), 2, _ptr(out))
    return int(out.view(np.uint32)[0])


# -- buffer converters (bit-exact, via arrays so NaN payloads survive) -----

def bytes_to_f32(dtype: int, buf: np.ndarray) -> np.ndarray:
    buf = np.ascontiguousarray(buf).view(np.uint8).reshape(-1)
    n = ctypes.c_int64()
    if lib().orc_logical_elements(dtype, buf.size, ctypes.byref(n)) != 0:
        raise OracleError("bad dtype or byte count")
    out = np.empty(n.value, dtype=np.float32)
    if lib().orc_bytes_to_f32(dtype, _ptr(buf), buf.size, _ptr(out)) != 0:
        raise OracleError("unsupported dtype")
    return out


def bytes_to_f64(dtype: int, buf: np.ndarray) -> np.ndarray:
    buf = np.ascontiguousarray(buf).view(np.uint8).reshape(-1)
    n = ctypes.c_int64()
    if lib().orc_logical_elements(dtype, buf.size, ctypes.byref(n)) != 0:
        raise OracleError("bad dtype or byte count")
    out = np.empty(n.value, dtype=np.float64)
    if lib().orc_bytes_to_f64(dtype, _ptr(buf), buf.size, _ptr(out)) != 0:
        raise OracleError("unsupported dtype")
    return out


def bytes_to_i8(dtype: int, buf: np.ndarray) -> np.ndarray:
    """BytesToInt8 (dtype/convert/convert.go:235-263); NaN gives 0."""
    buf = np.ascontiguousarray(buf).view(np.uint8).reshape(-1)
    n = ctypes.c_int64()
    if lib().orc_logical_elements(dtype, buf.size, ctypes.byref(n)) != 0:
        raise OracleError("bad dtype or byte count")
    out = np.empty(n.value, dtype=np.int8)
    if lib().orc_bytes_to_i8(dtype, _ptr(buf), buf.size, _ptr(out)) != 0:
        raise OracleError("unsupported dtype")
    return out


def int4_encode(values: np.ndarray) -> np.ndarray:
    """Packs int8 values as Int4Pair bytes: int4Encode (dtype/int4.go:60-70)
    clamps each to [-8, 7] and keeps its low nibble; element 2k is the low
    nibble of byte k (dtype/int4.go:12-22).  An odd count leaves the last
    byte's high nibble 0, as a fresh Int4Vector holds it
    (tensor/int4vector.go:74-87)."""
    v = np.asarray(values, dtype=np.int8).reshape(-1)
    nib = (np.clip(v.astype(np.int16), -8, 7) & 0xF).astype(np.uint8)
    if nib.size % 2:
        nib = np.append(nib, np.uint8(0))
    return (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)


def bytes_to_i4(dtype: int, buf: np.ndarray, count: int) -> np.ndarray:
    """BytesToInt8's values of the first `count` elements, packed by
    int4_encode: what mfh_convert writes for an Int4 output."""
    return int4_encode(bytes_to_i8(dtype, buf)[:count])


def bytes_to_bf16(dtype: int, buf: np.ndarray) -> np.ndarray:
    buf = np.ascontiguousarray(buf).view(np.uint8).reshape(-1)
    n = ctypes.c_int64()
    if lib().orc_logical_elements(dtype, buf.size, ctypes.byref(n)) != 0:
        raise OracleError("bad dtype or byte count")
    out = np.empty(n.value, dtype=np.uint16)
    if lib().orc_bytes_to_bf16(dtype, _ptr(buf), buf.size, _ptr(out)) != 0:
        raise OracleError("unsupported dtype")
    return out


def bytes_to_f16(dtype: int, buf: np.ndarray) -> np.ndarray:
    buf = np.ascontiguousarray(buf).view(np.uint8).reshape(-1)
    n = ctypes.c_int64()
    if lib().orc_logical_elements(dtype, buf.size, ctypes.byref(n)) != 0:
        raise OracleError("bad dtype or byte count")
    out = np.empty(n.value, dtype=np.uint16)
    if lib().orc_bytes_to_f16(dtype, _ptr(buf), buf.size, _ptr(out)) != 0:
        raise OracleError("unsupported dtype")
    return out


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(values.size, dtype=np.uint16)
    lib().orc_f32_to_bf16_buf(_ptr(values), values.size, _ptr(out))
    return out


def f32_to_f16(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(values.size, dtype=np.uint16)
    lib().orc_f32_to_f16_buf(_ptr(values), values.size, _ptr(out))
    return out


def encode(values: np.ndarray, dtype: int) -> np.ndarray:
    """Float32AsDTypeBytes (runtime/session.go:431-451) as a typed array."""
    if dtype == FLOAT32:
        return np.ascontiguousarray(values, dtype=np.float32)
    if dtype == BFLOAT16:
        return f32_to_bf16(values)
    if dtype == FLOAT16:
        return f32_to_f16(values)
    raise OracleError(f"unsupported storage dtype {dtype}")


def decode(values: np.ndarray, dtype: int) -> np.ndarray:
    """BytesToFloat32 of a typed storage array."""
    return bytes_to_f32(dtype, np.ascontiguousarray(values))


# -- dequant ----------------------------------------------------------------

_OUT_NP = {FLOAT32: np.float32, BFLOAT16: np.uint16, FLOAT16: np.uint16}


def dequant_fp8(codes: np.ndarray, fp8_dtype: int, scale: float, out_dtype: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    out = np.empty(codes.size, dtype=_OUT_NP[out_dtype])
    if lib().orc_dequant_fp8(_ptr(codes), codes.size, fp8_dtype, scale, out_dtype, _ptr(out)) != 0:
        raise OracleError("dequant_fp8 rejected its arguments")
    return out


def dequant_int4(packed: np.ndarray, n: int, scales: np.ndarray, scale_dtype: int,
                 group: int, out_dtype: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    scales = np.ascontiguousarray(scales)
    out = np.empty(n, dtype=_OUT_NP[out_dtype])
    if lib().orc_dequant_int4(_ptr(packed), n, _ptr(scales), scale_dtype, group,
                              out_dtype, _ptr(out)) != 0:
        raise OracleError("dequant_int4 rejected its arguments")
    return out


# -- evaluator --------------------------------------------------------------

def flatten(tree) -> list:
    """Pre-order flattening of a nested tuple AST.

    ``("in", k)`` is input k, ``("const", v)`` a constant, and
    ``(node_type, child, ...)`` an operator node.
    """
    out = []

    def walk(t):
        if t[0] == "in":
            out.append((N_INPUT, t[1], 0.0))
        elif t[0] == "const":
            out.append((N_CONSTANT, 0, float(t[1])))
        else:
            out.append((t[0], 0, 0.0))
            for ch in t[1:]:
                walk(ch)

    walk(tree)
    return out


def run(nodes, inputs, count: int, periods=None) -> np.ndarray:
    """CPUKernel.Run over f32 arrays (codegen/cpu.go:59-90)."""
    arr = (_Node * len(nodes))(*[_Node(t, i, v) for (t, i, v) in nodes])
    ins = [np.ascontiguousarray(a, dtype=np.float32).reshape(-1) for a in inputs]
    ptrs = (ctypes.c_void_p * max(1, len(ins)))(*[_ptr(a) for a in ins])
    per = np.array(periods if periods is not None else [0] * len(ins), dtype=np.int64)
    if per.size == 0:
        per = np.zeros(1, dtype=np.int64)
    out = np.empty(count, dtype=np.float32)
    rc = lib().orc_run(ctypes.addressof(arr), len(nodes), ctypes.addressof(ptrs),
                       _ptr(per), len(ins), _ptr(out), count)
    if rc != 0:
        raise OracleError("malformed fusion tree or input index out of range")
    return out


def eval_unary(node_type: int, values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    return run([(node_type, 0, 0.0), (N_INPUT, 0, 0.0)], [values], values.size)


def eval_binary(node_type: int, left: np.ndarray, right: np.ndarray) -> np.ndarray:
    left = np.ascontiguousarray(left, dtype=np.float32).reshape(-1)
    right = np.ascontiguousarray(right, dtype=np.float32).reshape(-1)
    return run([(node_type, 0, 0.0), (N_INPUT, 0, 0.0), (N_INPUT, 1, 0.0)],
               [left, right], left.size)


def arity(node_type: int) -> int:
    return lib().orc_node_arity(node_type)


# -- axpy / host math -------------------------------------------------------

def axpy_f32(y: np.ndarray, x: np.ndarray, alpha: float) -> np.ndarray:
    y = np.array(y, dtype=np.float32, copy=True).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    lib().orc_axpy_f32(_ptr(y), _ptr(x), y.size, alpha)
    return y


def axpy_storage(y: np.ndarray, x: np.ndarray, alpha: float, dtype: int) -> np.ndarray:
    y = np.array(y, copy=True).reshape(-1)
    x = np.ascontiguousarray(x).reshape(-1)
    if lib().orc_axpy_storage(_ptr(y), _ptr(x), y.size, alpha, dtype) != 0:
        raise OracleError("unsupported storage dtype")
    return y


def scalar_broadcast(src: np.ndarray, scalar: float, op: str) -> np.ndarray:
    ops = {"add": 0, "sub": 1, "mul": 2, "div": 3}
    if op not in ops:
        raise OracleError(f"unsupported op {op!r}")
    src = np.ascontiguousarray(src, dtype=np.float32).reshape(-1)
    out = np.empty_like(src)
    if lib().orc_scalar_broadcast(_ptr(src), src.size, scalar, ops[op], _ptr(out)) != 0:
        raise OracleError("scalar divisor must be nonzero")
    return out


def linspace(start: float, stop: float, count: int, endpoint: bool = True) -> np.ndarray:
    out = np.empty(max(count, 1), dtype=np.float32)
    if lib().orc_linspace(start, stop, count, 1 if endpoint else 0, _ptr(out)) != 0:
        raise OracleError("count must be positive")
    return out[:count]


def fold(node_type: int, operands) -> float | None:
    ops = np.array(operands, dtype=np.float64)
    out = np.zeros(1, dtype=np.float64)
    if lib().orc_fold(node_type, _ptr(ops), ops.size, _ptr(out)) == 0:
        return None
    return float(out[0])
