"""Derives the constants of the f32 exponential kernels in devmath.hpp.

e^x = 2^k * e^r with k = rint(x / ln2) and r = x - k*ln2 (Cody & Waite range
reduction, ln2 split into a 16-bit head, so k*head is exact for |k| < 256, and
an f32 tail).  e^r on |r| <= ln2/2 (plus a margin for the f32 rounding of
x/ln2) is a degree-6 polynomial with the constant term pinned to 1, fitted by
weighted least squares on Chebyshev nodes for relative error and rounded to
f32.

2^f on |f| <= 1/2 (the fraction left when the argument is already in log2
units and reduced in f64) is fitted the same way, once with f32 coefficients
(degree 6, within 0.94 f32 ulp; gelu now uses the hardware v_exp_f32
instead, which measured faster and equally accurate) and once with f64
coefficients (degree 8, fitted in 50-digit arithmetic with mpmath; sigmoid).

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


def fit_exp2_f64(degree=8, half_width=0.5, nodes=600):
    """Weighted least squares for 2^f - 1 = f q(f) in 50-digit arithmetic;
    returns the coefficients rounded to f64 and the max relative error of
    the f64 Horner evaluation on a grid."""
    import mpmath as mp
    mp.mp.dps = 50
    xs = [half_width * mp.cos(mp.pi * (k + mp.mpf(0.5)) / nodes) for k in range(nodes)]
    A = mp.matrix(nodes, degree)
    b = mp.matrix(nodes, 1)
    for i, x in enumerate(xs):
        w = 1 / mp.power(2, x)
        for j in range(degree):
            A[i, j] = w * x ** (j + 1)
        b[i] = w * (mp.power(2, x) - 1)
    Q, R = mp.qr(A)
    c = mp.lu_solve(R[:degree, :degree], (Q.T * b)[:degree, 0])
    coef = [float(c[j]) for j in range(degree)]
    worst = 0
    for i in range(4001):
        f = -half_width + 2 * half_width * i / 4000
        acc = coef[-1]
        for cj in reversed(coef[:-1]):
            acc = acc * f + cj
        acc = acc * f + 1.0
        worst = max(worst, abs((mp.mpf(acc) - mp.power(2, mp.mpf(f))) / mp.power(2, mp.mpf(f))))
    return coef, float(mp.log(worst, 2))


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
    try:
        coef64, log2err = fit_exp2_f64()
    except ImportError:
        print("mpmath is not installed: f64 coefficients skipped")
        return
    for j, c in enumerate(coef64, start=1):
        print(f"2^f f64 c{j}", float.hex(c))
    print("log2 of the max relative error of 2^f in f64:", log2err)


if __name__ == "__main__":
    main()
