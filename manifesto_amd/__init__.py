"""manifesto_amd — MI355X (gfx950) backend for manifesto's data-parallel hot path.

The product is the native library ``libmfh.so`` (HIP kernels for gfx950 and the
C ABI declared in ``include/mfh.h``).  This package is a thin ctypes binding of
that ABI for tests, the bench and Python callers; it has no compute path of its
own and raises if the library is missing.
"""
from __future__ import annotations

import ctypes
import os

from .abi import (  # noqa: F401
    MFHError, lib, LIB_PATH, init, check, last_error,
    FLOAT64, FLOAT32, FLOAT16, BFLOAT16, F8E4M3, F8E5M2, INT64, INT32, INT16, INT8, INT4,
    UINT64, UINT32, UINT16, UINT8,
    OPERAND_FULL, OPERAND_PERIODIC, OPERAND_SCALAR, FUSION_PRECISE, FUSION_SHORT_QUOTIENT, FUSION_NO_ROUNDING_TEST,
    AstNode, Operand, FusedKernel, fusion_cache_dir, fusion_cache_stats,
    axpy, dequant_fp8, dequant_int4, convert, scalar_broadcast, linspace,
    take_sticky_error, stream_sync, set_launch_config, get_launch_config, set_launch_threads, get_launch_threads,
)

__all__ = [name for name in dir() if not name.startswith("_")]
