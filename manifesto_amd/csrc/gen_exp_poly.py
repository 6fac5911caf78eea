"""Derives the constants of the f32 exponential kernels in devmath.hpp.

e^x = 2^k * e^r with k = rint(x / ln2) and r = x - k*ln2 (Cody & Waite range
reduction, ln2 split into a 16-bit head, so k*head is exact for |k| < 256, and
an f32 tail).  e^r on |r| <= ln2/2 (plus a margin for the f32 rounding of
x/ln2) is a degree-6 polynomial with the constant term pinned to 1, fitted by
weighted least squares on Chebyshev nodes for relative error and rounded to
f32.

2^f on |f| <= 1/2 (the fraction left when the argument is already in log2
units and reduced in f64) is fitted the same way.

Run: python3 gen_exp_poly.py
"""
import math

import numpy as np

F32 = np.float32


def f32_hex(v):
    return "0x%08xu" % int(np.array([v], dtype=np.float32).view(np.uint32)[0])


def split_ln2():
    ln2 = math.log(2.0)
    head = math.floor(ln2 * 2 ** 16) / 2 ** 16  # 16 significant bits
    tail = float(F32(ln2 - head))
    return F32(head), F32(tail)


def fit(degree=6, half_width=0.3466 + 2e-5, nodes=4000):
    k = np.arange(nodes)
    r = half_width * np.cos(np.pi * (k + 0.5) / nodes)
    target = np.expm1(r)  # fit e^r - 1 = r * q(r), q of degree-1
    basis = np.stack([r ** (j + 1) for j in range(degree)], axis=1)
    w = 1.0 / np.exp(r)
    coef, *_ = np.linalg.lstsq(basis * w[:, None], target * w, rcond=None)
    return [F32(c) for c in coef]


def fit_exp2(degree=6, half_width=0.5, nodes=4000):
    k = np.arange(nodes)
    f = half_width * np.cos(np.pi * (k + 0.5) / nodes)
    target = np.expm1(f * math.log(2.0))  # 2^f - 1 = f * q(f)
    basis = np.stack([f ** (j + 1) for j in range(degree)], axis=1)
    w = 1.0 / np.exp2(f)
    coef, *_ = np.linalg.lstsq(basis * w[:, None], target * w, rcond=None)
    return [F32(c) for c in coef]


def horner_f32(coef, r):
    """Evaluates 1 + r*(c1 + r*(c2 + ...)) with f32 fma rounding."""
    r64 = r.astype(np.float64)
    acc = np.full_like(r, coef[-1], dtype=np.float32)
    for c in reversed(coef[:-1]):
        acc = (acc.astype(np.float64) * r64 + float(c)).astype(np.float32)
    return (acc.astype(np.float64) * r64 + 1.0).astype(np.float32)


def main():
    head, tail = split_ln2()
    coef = fit()
    r = np.linspace(-0.3467, 0.3467, 2_000_001).astype(np.float32)
    approx = horner_f32(coef, r).astype(np.float64)
    exact = np.exp(r.astype(np.float64))
    ulp = np.spacing(exact.astype(np.float32)).astype(np.float64)
    err = np.abs(approx - exact) / ulp
    print("ln2 head", f32_hex(head), float(head))
    print("ln2 tail", f32_hex(tail), float(tail))
    for j, c in enumerate(coef, start=1):
        print(f"c{j}", f32_hex(c), repr(float(c)))
    print("max error of e^r in f32 ulps (incl. Horner rounding):", err.max())
    coef2 = fit_exp2()
    f = np.linspace(-0.5, 0.5, 2_000_001).astype(np.float32)
    approx = horner_f32(coef2, f).astype(np.float64)
    exact = np.exp2(f.astype(np.float64))
    err = np.abs(approx - exact) / np.spacing(exact.astype(np.float32)).astype(np.float64)
    for j, c in enumerate(coef2, start=1):
        print(f"2^f c{j}", f32_hex(c), repr(float(c)))
    print("max error of 2^f in f32 ulps (incl. Horner rounding):", err.max())


if __name__ == "__main__":
    main()
