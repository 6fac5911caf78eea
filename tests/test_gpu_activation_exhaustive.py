"""Every f32 input through the device's Sigmoid, Silu and Gelu nodes.

The fused kernels run on the GPU over all 2^32 f32 bit patterns (in chunks)
beside the MFH_FUSION_PRECISE kernels.  A chain that streams f32 evaluates
the three activations in their rounding-tested forms, which must give the
precise kernel's bit pattern on every input.  The forms 16-bit chains use
(f32 Silu and Gelu with the rounding of 1 + E left in the quotient, the f64
Sigmoid without a rounding test) run here through MFH_FUSION_SHORT_QUOTIENT.
The precise kernels, which give the values of the reference's f64 formulas
(codegen/cpu.go:186-200) rounded once, are within one f32 ulp of the oracle
(they differ only where an f64 result sits at an f32 rounding tie that two
f64 libraries round differently).  NaN positions must match.  Every input
where a 16-bit chain's form is `tol` or more ulps from the precise kernel is
then checked against the CPU oracle itself, which it must be within `tol`
of; every other input is within tol - 1 of the precise kernel and so within
tol of the oracle.  This covers the device math the host sweep
(test_devmath_host.py) cannot model: the hardware reciprocals, and gelu's
hardware v_exp_f32.
"""
import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

from gpu_util import log, stream

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28
TOL = {O.N_SIGMOID: 1, O.N_SILU: 2, O.N_GELU: 2}


def ulp_key(bits):
    """Monotone integer key of f32 bit patterns (int32 or int64 tensor/array)."""
    import torch
    if isinstance(bits, np.ndarray):
        b = bits.astype(np.int64)
        return np.where(b < 0, -(b & 0x7FFFFFFF), b)
    b = bits.to(torch.int64)
    return torch.where(b < 0, -(b & 0x7FFFFFFF), b)


CASES = [(O.N_SIGMOID, 0), (O.N_SIGMOID, M.FUSION_SHORT_QUOTIENT), (O.N_SILU, 0), (O.N_SILU, M.FUSION_SHORT_QUOTIENT),
         (O.N_GELU, 0), (O.N_GELU, M.FUSION_SHORT_QUOTIENT)]


@pytest.mark.parametrize("node, flags", CASES)
def test_fast_activation_every_f32_input(node, flags):
    import torch
    M.init(0)
    tol = TOL[node]
    nodes = O.flatten((node, ("in", 0)))
    ops = [(M.FLOAT32, M.OPERAND_FULL, 0)]
    fast_k = M.FusedKernel(nodes, ops, M.FLOAT32, f"exh_fast_{node}", flags)
    precise_k = M.FusedKernel(nodes, ops, M.FLOAT32, f"exh_precise_{node}", M.FUSION_PRECISE)
    fast = torch.empty(CHUNK, dtype=torch.int32, device="cuda")
    precise = torch.empty(CHUNK, dtype=torch.int32, device="cuda")
    hist = torch.zeros(tol + 3, dtype=torch.int64, device="cuda")
    candidates = []
    for c in range((1 << 32) // CHUNK):
        log(f"node {node} flags {flags}: bit patterns [{c * CHUNK:#x}, {(c + 1) * CHUNK:#x})")
        x = (torch.arange(c * CHUNK, (c + 1) * CHUNK, dtype=torch.int64, device="cuda") - (1 << 31)).to(torch.int32)
        fast_k.launch([x.data_ptr()], fast.data_ptr(), CHUNK, stream())
        precise_k.launch([x.data_ptr()], precise.data_ptr(), CHUNK, stream())
        nan_f = (fast & 0x7FFFFFFF) > 0x7F800000
        nan_p = (precise & 0x7FFFFFFF) > 0x7F800000
        bad = int((nan_f != nan_p).sum())
        assert bad == 0, f"node {node}: {bad} NaN mismatches in chunk {c}"
        d = (ulp_key(fast) - ulp_key(precise)).abs()
        d = torch.where(nan_f, torch.zeros_like(d), d)
        hist += torch.bincount(d.clamp(max=tol + 2), minlength=tol + 3)
        idx = torch.nonzero(d >= tol).flatten()
        if idx.numel():
            candidates.append(torch.stack([x[idx], fast[idx]], 1).cpu().numpy())
    h = hist.tolist()
    log(f"node {node} flags {flags}: ulps from the precise form {h} (last bin: {tol + 2} or more)")
    assert sum(h) == 1 << 32
    if not flags:  # a chain that streams f32: the rounding-tested forms
        assert h[0] == 1 << 32, f"node {node}: {(1 << 32) - h[0]} inputs differ from the precise kernel"
    assert h[0] / (1 << 32) > 0.95, f"node {node}: only {h[0] / (1 << 32):.4f} identical to the precise form"
    if not candidates:
        return
    a = np.concatenate(candidates)
    want = O.eval_unary(node, a[:, 0].view(np.float32)).view(np.int32)
    dd = np.abs(ulp_key(a[:, 1]) - ulp_key(want))
    log(f"node {node} flags {flags}: {a.shape[0]} inputs {tol}+ ulps from the precise form, at most {int(dd.max())} from the oracle")
    i = int(np.argmax(dd))
    assert dd.max() <= tol, (f"node {node}: {int(dd.max())} ulp from the oracle at x bits {a[i, 0] & 0xFFFFFFFF:#x}: "
                             f"got {a[i, 1] & 0xFFFFFFFF:#x} want {want[i] & 0xFFFFFFFF:#x}")


@pytest.mark.parametrize("node", [O.N_SIGMOID, O.N_SILU, O.N_GELU, O.N_EXP, O.N_LOG, O.N_TANH])
def test_precise_forms_against_the_oracle(node):
    # The MFH_FUSION_PRECISE forms (and the flagged elements of the fast
    # kernels, which run the same functions) against the CPU oracle itself on
    # every 251st f32 bit pattern: within 1 f32 ulp, identical almost always.
    import torch
    from gpu_util import oracle_run_parallel
    M.init(0)
    nodes = O.flatten((node, ("in", 0)))
    k = M.FusedKernel(nodes, [(M.FLOAT32, M.OPERAND_FULL, 0)], M.FLOAT32, f"precise_{node}", M.FUSION_PRECISE)
    x = (torch.arange(0, 1 << 32, 251, dtype=torch.int64, device="cuda") - (1 << 31)).to(torch.int32)
    out = torch.empty_like(x)
    k.launch([x.data_ptr()], out.data_ptr(), x.numel(), stream())
    got = out.cpu().numpy()
    xs = x.cpu().numpy().view(np.float32)
    log(f"node {node}: {xs.size} inputs through the oracle")
    want = oracle_run_parallel(nodes, [xs], xs.size, align=1).view(np.int32)
    nan_g, nan_w = (got & 0x7FFFFFFF) > 0x7F800000, (want & 0x7FFFFFFF) > 0x7F800000
    assert np.array_equal(nan_g, nan_w), f"node {node}: NaN positions differ"
    d = np.abs(ulp_key(got[~nan_w]) - ulp_key(want[~nan_w]))
    log(f"node {node}: precise form vs oracle: max {int(d.max())} ulp, {float(np.mean(d == 0)):.7f} identical")
    assert d.max() <= 1 and np.mean(d == 0) > 0.9999, f"node {node}: max {int(d.max())} ulp"


@pytest.mark.parametrize("node", [O.N_SIGMOID, O.N_SILU, O.N_GELU])
def test_precise_rounding_test_reproduces_the_reference_forms(node):
    # MFH_FUSION_PRECISE kernels run the rounding-tested f64 forms and the
    # reference forms only where the test flags an element; with
    # MFH_FUSION_NO_ROUNDING_TEST every element runs the reference forms.  The
    # two must give the same bit pattern for every f32 input, NaN payloads
    # included: that checks the test's margin against the device's own
    # arithmetic (its f64 reciprocal among it) on every input.
    import torch
    M.init(0)
    nodes = O.flatten((node, ("in", 0)))
    ops = [(M.FLOAT32, M.OPERAND_FULL, 0)]
    tested = M.FusedKernel(nodes, ops, M.FLOAT32, f"exh_tested_{node}", M.FUSION_PRECISE)
    plain = M.FusedKernel(nodes, ops, M.FLOAT32, f"exh_plain_{node}", M.FUSION_PRECISE | M.FUSION_NO_ROUNDING_TEST)
    a = torch.empty(CHUNK, dtype=torch.int32, device="cuda")
    b = torch.empty(CHUNK, dtype=torch.int32, device="cuda")
    for c in range((1 << 32) // CHUNK):
        log(f"node {node} rounding test: bit patterns [{c * CHUNK:#x}, {(c + 1) * CHUNK:#x})")
        x = (torch.arange(c * CHUNK, (c + 1) * CHUNK, dtype=torch.int64, device="cuda") - (1 << 31)).to(torch.int32)
        tested.launch([x.data_ptr()], a.data_ptr(), CHUNK, stream())
        plain.launch([x.data_ptr()], b.data_ptr(), CHUNK, stream())
        idx = torch.nonzero(a != b).flatten()
        if idx.numel():
            i = idx[:4].cpu().tolist()
            raise AssertionError(f"node {node}: {idx.numel()} inputs differ in chunk {c}, e.g. x bits "
                                 f"{[int(x[j]) & 0xFFFFFFFF for j in i]}: tested {[int(a[j]) & 0xFFFFFFFF for j in i]}"
                                 f" plain {[int(b[j]) & 0xFFFFFFFF for j in i]}")
