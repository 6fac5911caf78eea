"""Helpers for the GPU parity tests: device buffers, ulp metrics, oracle runs."""
from __future__ import annotations

import concurrent.futures as cf
import sys

import numpy as np

import oracle as O


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def torch_mod():
    import torch
    return torch


def to_dev(a: np.ndarray, pad: int = 0):
    """Copies a numpy array to the GPU as raw bytes; returns (tensor, ptr)."""
    torch = torch_mod()
    raw = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
    t = torch.empty(raw.size + pad, dtype=torch.uint8, device="cuda")
    if raw.size:
        t[pad:].copy_(torch.from_numpy(raw.copy()))
    return t, t.data_ptr() + pad


def empty_dev(nbytes: int, pad: int = 0):
    torch = torch_mod()
    t = torch.full((nbytes + pad,), 0xA5, dtype=torch.uint8, device="cuda")
    return t, t.data_ptr() + pad


def to_host(t, dtype, pad: int = 0) -> np.ndarray:
    torch = torch_mod()
    torch.cuda.synchronize()
    return t[pad:].cpu().numpy().view(dtype)


def stream() -> int:
    return torch_mod().cuda.current_stream().cuda_stream


def ulp_key(bits: np.ndarray, width: int) -> np.ndarray:
    u = bits.astype(np.int64)
    sign = 1 << (width - 1)
    return np.where(u & sign, sign - u, u)


def ulp_diff(a_bits: np.ndarray, b_bits: np.ndarray, width: int) -> np.ndarray:
    return np.abs(ulp_key(a_bits, width) - ulp_key(b_bits, width))


def is_nan_bits(bits: np.ndarray, width: int) -> np.ndarray:
    if width == 32:
        return (bits.astype(np.uint32) & 0x7FFFFFFF) > 0x7F800000
    if width == 16 and bits.dtype == np.uint16:
        return bits  # unused
    raise ValueError


def nan_mask(bits: np.ndarray, dtype: int) -> np.ndarray:
    b = bits.astype(np.uint32)
    if dtype == O.FLOAT32:
        return (b & 0x7FFFFFFF) > 0x7F800000
    if dtype == O.BFLOAT16:
        return (b & 0x7FFF) > 0x7F80
    if dtype == O.FLOAT16:
        return (b & 0x7FFF) > 0x7C00
    raise ValueError(dtype)


def compare_storage(got: np.ndarray, want: np.ndarray, dtype: int, max_ulp: int, what: str):
    """NaN positions must agree (payloads not compared); elsewhere <= max_ulp."""
    width = 32 if dtype == O.FLOAT32 else 16
    gb = got.view(np.uint32 if width == 32 else np.uint16)
    wb = want.view(np.uint32 if width == 32 else np.uint16)
    gn, wn = nan_mask(gb, dtype), nan_mask(wb, dtype)
    bad = np.flatnonzero(gn != wn)
    assert bad.size == 0, f"{what}: NaN mismatch at {bad[:5]} got={gb[bad[:5]]} want={wb[bad[:5]]}"
    keep = ~wn
    d = ulp_diff(gb[keep], wb[keep], width)
    worst = int(d.max()) if d.size else 0
    if worst > max_ulp:
        i = np.flatnonzero(keep)[int(np.argmax(d))]
        raise AssertionError(f"{what}: {worst} ulp > {max_ulp} at {i}: got {gb[i]:#x} want {wb[i]:#x}")
    return worst


def oracle_run_parallel(nodes, inputs, count: int, periods=None, threads: int = 16,
                        align: int = 4096) -> np.ndarray:
    """CPUKernel.Run split across threads (each chunk starts on a multiple of
    `align`, which every periodic operand's period divides)."""
    periods = periods or [0] * len(inputs)
    out = np.empty(count, dtype=np.float32)
    chunk = max(align, ((count // (threads * 4)) // align + 1) * align)

    def work(start):
        stop = min(count, start + chunk)
        ins = [a if p > 0 else a[start:stop] for a, p in zip(inputs, periods)]
        out[start:stop] = O.run(nodes, ins, stop - start, periods)

    with cf.ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(work, range(0, count, chunk)))
    return out


def nudge(s: np.ndarray, ulps: int, up: bool) -> np.ndarray:
    """s moved by `ulps` f32 ulps toward +Inf (up) or -Inf."""
    t = s.astype(np.float32)
    target = np.float32(np.inf if up else -np.inf)
    for _ in range(ulps):
        t = np.nextafter(t, target)
    return t


def storage_key(bits: np.ndarray, dtype: int) -> np.ndarray:
    width = 32 if dtype == O.FLOAT32 else 16
    return ulp_key(bits.view(np.uint32 if width == 32 else np.uint16), width)


def check_envelope(got, node_value, tail, out_dt, ulps, what, min_exact=0.99):
    """The fused result must equal the reference chain evaluated with one
    transcendental node's value anywhere within `ulps` f32 ulps of the
    reference's (every other operation exact).  `tail` maps node values (f32)
    to encoded outputs with the reference's remaining operations; it must be
    monotone in the node value.  NaN outputs must agree in position."""
    want = tail(node_value)
    lo = tail(nudge(node_value, ulps, up=False))
    hi = tail(nudge(node_value, ulps, up=True))
    gb = got.view(np.uint32 if out_dt == O.FLOAT32 else np.uint16)
    wb = want.view(gb.dtype)
    gn, wn = nan_mask(gb, out_dt), nan_mask(wb, out_dt)
    bad = np.flatnonzero(gn != wn)
    assert bad.size == 0, f"{what}: NaN mismatch at {bad[:5]}"
    keep = ~wn & ~nan_mask(lo.view(gb.dtype), out_dt) & ~nan_mask(hi.view(gb.dtype), out_dt)
    kg, kl, kh = (storage_key(a.view(gb.dtype)[keep], out_dt) for a in (got, lo, hi))
    lo_k, hi_k = np.minimum(kl, kh), np.maximum(kl, kh)
    out = np.flatnonzero((kg < lo_k) | (kg > hi_k))
    if out.size:
        i = np.flatnonzero(keep)[out[0]]
        raise AssertionError(f"{what}: {out.size} results outside the +-{ulps} ulp envelope, first at {i}: "
                             f"got {gb[i]:#x} want {wb[i]:#x} node {node_value[i]!r}")
    exact = float(np.mean(gb == wb))
    assert exact >= min_exact, f"{what}: only {exact:.5f} bit-identical"
    return exact
