"""Accuracy of the fused-kernel activation math, measured on the host.

devmath.hpp compiles for the host (MFH_HOST_MATH) with the same f32/f64
operation sequence the gfx950 kernels run, except for two hardware
instructions: the reciprocal is modelled by a correctly rounded division,
which the residual step that follows it makes immaterial, and gelu's
v_exp_f32 by libm's exp2f, which is more accurate (the device gelu is
checked over every f32 input by test_gpu_activation_exhaustive.py).  A
strided sweep over all 2^32 f32 bit patterns is checked against the oracle's
restatement of codegen/cpu.go:186-200: Sigmoid, Exp, Log, Tanh within 1 f32
ulp, Silu and Gelu within 2, the reference forms within 1, NaN exactly where
the reference's is.  The rounding-tested forms that chains streaming f32 and
MFH_FUSION_PRECISE kernels run (mfh_*_cr, the reference form where they flag
an input) must give the reference forms' bit patterns on every swept input.
"""
import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.fixture(scope="module")
def report(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("devmath") / "devmath_accuracy")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread",
                    os.path.join(HERE, "devmath_accuracy.cpp"), os.path.join(ROOT, "oracle", "oracle.c"),
                    "-o", exe, "-lm"], check=True)
    out = subprocess.run([exe, "4099", "8"], check=True, capture_output=True, text=True).stdout
    rows = {}
    for line in out.splitlines():
        name, *fields = line.split()
        rows[name] = {k: float(v) for k, v in (f.split("=") for f in fields)}
    return rows


TOL = {"sigmoid": 1, "silu": 2, "gelu": 2, "exp_ref": 1, "log_ref": 1, "tanh_ref": 1,
       "sigmoid_ref": 1, "silu_ref": 1, "gelu_ref": 1, "sigmoid_p": 1, "silu_p": 1, "gelu_p": 1}


@pytest.mark.parametrize("name", sorted(TOL))
def test_activation_accuracy(report, name):
    row = report[name]
    assert row["samples"] > 1_000_000
    assert row["nan_mismatch"] == 0, row
    assert row["over_tol"] == 0 and row["max_ulp"] <= TOL[name], row
    # the fast forms are mostly exact; the f64 reference forms almost always
    assert row["exact"] > (0.95 if TOL[name] == 2 else 0.98), row


@pytest.mark.parametrize("name", ["sigmoid_p", "silu_p", "gelu_p"])
def test_rounding_tested_forms_reproduce_the_reference_forms(report, name):
    row = report[name]
    assert row["ref_mismatch"] == 0, row
    # The margin of the rounding test, 2^15 f64 ulps, is at least 2^-38 of the
    # value: the f64 value must stay well within it of the exact function
    # (the device's reciprocal adds at most 2^-46 after its Newton step).
    assert row["max_rel_err_log2"] < -39.5, row
    # flagged over all bit patterns: mostly the range tests (tiny, huge and
    # NaN inputs); on data the midpoint test flags about one element in 2^13
    assert row["flagged"] < 0.5, row
