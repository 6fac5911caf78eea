"""The CPU oracle against what the mathematics fixes, independently of its code.

Each check uses a different formulation or a library routine, chosen so that a
plausible slip in the restatement (a wrong bias, a dropped tie term, a swapped
nibble, an FMA where the reference has none) fails at least one of them; the
last tests show that on mutated formulas.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
from scipy.special import expit

import oracle as O

F32 = np.float32


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def from_bits(u):
    return np.asarray(u, dtype=np.uint32).view(np.float32)


def ulp_diff(a, b):
    """Distance in f32 ulps on the monotone integer line (NaNs excluded)."""
    def key(x):
        u = bits(x).astype(np.int64)
        return np.where(u & 0x80000000, 0x80000000 - u, u)
    return np.abs(key(a) - key(b))


# --------------------------------------------------------------------------
# FP8: exhaustive over all 256 codes against the OCP closed form.
# --------------------------------------------------------------------------

def e4m3_closed(code):
    s = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 0xF, code & 7
    if e == 0xF and m == 7:
        return None
    if e == 0:
        return s * math.ldexp(m / 8, -6)
    return s * math.ldexp(1 + m / 8, e - 7)


def e5m2_closed(code):
    s = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 2) & 0x1F, code & 3
    if e == 0x1F:
        return s * math.inf if m == 0 else None
    if e == 0:
        return s * math.ldexp(m / 4, -14)
    return s * math.ldexp(1 + m / 4, e - 15)


def test_e4m3_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    got = O.bytes_to_f32(O.F8E4M3, codes)
    for c in range(256):
        want = e4m3_closed(c)
        if want is None:
            # NaN keeps the sign and is the canonical quiet NaN (dtype/fp8.go:43-45)
            assert bits(got[c]) == ((c >> 7) << 31 | 0x7FC00000)
        else:
            assert got[c] == want and math.copysign(1, got[c]) == math.copysign(1, want), c
    finite = [c for c in range(256) if e4m3_closed(c) is not None]
    assert max(abs(e4m3_closed(c)) for c in finite) == 448.0
    assert min(abs(e4m3_closed(c)) for c in finite if e4m3_closed(c) != 0) == 2.0 ** -9


def test_e5m2_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    got = O.bytes_to_f32(O.F8E5M2, codes)
    for c in range(256):
        want = e5m2_closed(c)
        if want is None:
            assert bits(got[c]) == ((c >> 7) << 31 | 0x7FC00000 | ((c & 3) << 21))
        else:
            assert got[c] == want and math.copysign(1, got[c]) == math.copysign(1, want), c


def test_fp8_encode_round_trips_normal_codes():
    # The encoders (dtype/fp8.go:77-136,190-249) invert the decoders on every
    # normal code below the top binade, and keep their documented quirks:
    # 256..448 saturate to 0x7e, and the subnormal branch shifts by one less.
    for c in range(256):
        e = (c >> 3) & 0xF
        if 1 <= e <= 14:
            assert O.f32_to_e4m3(O.e4m3_to_f32(c)) == c
        e5 = (c >> 2) & 0x1F
        if 1 <= e5 <= 30:
            assert O.f32_to_e5m2(O.e5m2_to_f32(c)) == c
    assert O.f32_to_e4m3(256.0) == 0x7E
    assert O.f32_to_e4m3(2.0 ** -7) == 0x08


def nearest_even_code(x, table, mbits):
    """Brute force: the code of the representable value nearest to x, ties to
    the even mantissa; `table` maps positive finite codes to their values."""
    codes = np.array(sorted(table))
    vals = np.array([table[c] for c in codes])
    d = np.abs(vals - x)
    best = np.flatnonzero(d == d.min())
    if best.size == 1:
        return int(codes[best[0]])
    even = [int(codes[b]) for b in best if (codes[b] & ((1 << mbits) - 1)) % 2 == 0]
    return even[0]


@pytest.mark.parametrize("fmt, lo, hi, mbits", [(O.F8E4M3, 2.0 ** -6, 248.0, 3), (O.F8E5M2, 2.0 ** -14, 57344.0, 2)])
def test_fp8_encode_is_nearest_even_in_the_normal_range(fmt, lo, hi, mbits):
    # Independent of the restated algorithm: inside the normal range the
    # encoder must pick the nearest representable value, ties to even.  For
    # E4M3 the range stops below 248, the midpoint into the top binade, which
    # the reference saturates to 0x7e (448) instead of rounding to 256.
    # Inputs: random values, every midpoint between neighbours and one f32 ulp
    # either side of it.
    dec = O.e4m3_to_f32 if fmt == O.F8E4M3 else O.e5m2_to_f32
    table = {c: dec(c) for c in range(0x80) if math.isfinite(dec(c)) and dec(c) > 0}
    table = {c: v for c, v in table.items() if lo <= v <= hi}
    vals = sorted(table.values())
    rng = np.random.default_rng(8)
    xs = list(np.exp(rng.uniform(math.log(lo), math.log(hi), 3000)).astype(np.float32))
    for a, b in zip(vals, vals[1:]):
        m = np.float32((a + b) / 2)
        xs += [m, np.nextafter(m, np.float32(0)), np.nextafter(m, np.float32(np.inf))]
    xs = np.array([x for x in xs if lo <= x < hi], dtype=np.float32)
    assert xs.size > 3000
    got = O.f32_to_fp8(xs, fmt)
    for x, g in zip(xs, got):
        want = nearest_even_code(float(x), table, mbits)
        assert g == want, (float(x), hex(g), hex(want))
        assert O.f32_to_fp8(-np.array([x], np.float32), fmt)[0] == want | 0x80


# --------------------------------------------------------------------------
# Int4: closed form n - 16*(n >= 8), both nibbles, all bytes.
# --------------------------------------------------------------------------

def test_int4_all_bytes():
    buf = np.arange(256, dtype=np.uint8)
    got = O.bytes_to_f64(O.INT4, buf)
    lo = [(b & 15) - 16 * ((b & 15) >= 8) for b in range(256)]
    hi = [(b >> 4) - 16 * ((b >> 4) >= 8) for b in range(256)]
    assert list(got[0::2]) == lo and list(got[1::2]) == hi


# --------------------------------------------------------------------------
# F16: exhaustive decode vs numpy; encode vs numpy's RNE narrowing.
# --------------------------------------------------------------------------

def test_f16_decode_all_codes():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.bytes_to_f32(O.FLOAT16, codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(bits(got[~nan]), bits(ref[~nan]))
    c = codes[nan].astype(np.uint32)
    want = ((c & 0x8000) << 16) | 0x7FC00000 | ((c & 0x3FF) << 13)
    assert np.array_equal(bits(got[nan]), want)


def _f16_probe_inputs(rng):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    h = h[np.isfinite(h)]
    nxt = np.nextafter(h, np.float32(np.inf))
    mids = ((h.astype(np.float64) + np.roll(h, -1).astype(np.float64)) / 2).astype(np.float32)
    rand = from_bits(rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32))
    return np.concatenate([h, nxt, mids, np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(-np.inf)), rand]).astype(np.float32)


def test_f16_encode_matches_numpy_rne():
    x = _f16_probe_inputs(np.random.default_rng(1))
    got = O.f32_to_f16(x)
    nan = np.isnan(x)
    with np.errstate(over="ignore"):
        ref = x[~nan].astype(np.float16).view(np.uint16)
    assert np.array_equal(got[~nan], ref)
    u = bits(x[nan])
    want = ((u >> 16) & 0x8000) | 0x7C00 | 0x0200 | ((u & 0x7FFFFF) >> 13)
    assert np.array_equal(got[nan], want.astype(np.uint16))


# --------------------------------------------------------------------------
# BF16: against torch's RNE narrowing and a compare-based restatement.
# --------------------------------------------------------------------------

def test_bf16_encode_matches_torch_rne():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    u = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2**16, size=4096, dtype=np.uint32) << 16) | 0x8000
    u = np.concatenate([u, ties, ties + 1, ties - 1]).astype(np.uint32)
    x = from_bits(u)
    got = O.f32_to_bf16(x)
    nan = np.isnan(x)
    ref = torch.from_numpy(x[~nan].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[~nan], ref)
    assert np.array_equal(got[nan], ((u[nan] >> 16) | 0x40).astype(np.uint16))
    # Compare-based statement of RNE (not the add-0x7fff trick):
    low, up = u & 0xFFFF, u >> 16
    up2 = up + ((low > 0x8000) | ((low == 0x8000) & ((up & 1) == 1)))
    assert np.array_equal(got[~nan], up2[~nan].astype(np.uint16))


# --------------------------------------------------------------------------
# axpy: IEEE single arithmetic with the product rounded before the add.
# --------------------------------------------------------------------------

def fused_f32(a, x, y):
    """fl32(a*x + y) with one rounding, exactly (the FMA result)."""
    exact = Fraction(float(a)) * Fraction(float(x)) + Fraction(float(y))
    return np.float32(float(exact)) if abs(float(exact)) < 3e38 else np.float32(float(exact))


def test_axpy_is_unfused_ieee():
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, 4096).astype(np.float32)
    y = rng.uniform(-1, 1, 4096).astype(np.float32)
    a = np.float32(0.75)
    got = O.axpy_f32(y, x, float(a))
    ref = (y + (a * x).astype(np.float32)).astype(np.float32)
    assert np.array_equal(bits(got), bits(ref))
    # The unfused and fused results differ on some of these inputs, so this
    # test would catch a contracted (FMA) build.
    a3 = np.float32(1 / 3)
    got3 = O.axpy_f32(y, x, float(a3))
    fused = np.array([float(Fraction(float(a3)) * Fraction(float(xi)) + Fraction(float(yi)))
                      for xi, yi in zip(x, y)]).astype(np.float32)
    assert np.array_equal(bits(got3), bits((y + (a3 * x).astype(np.float32)).astype(np.float32)))
    assert not np.array_equal(bits(got3), bits(fused))


# --------------------------------------------------------------------------
# Evaluator node formulas.
# --------------------------------------------------------------------------

def _probe_f32(rng, n=1 << 16, lo=-20, hi=20):
    v = rng.uniform(lo, hi, n).astype(np.float32)
    specials = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 1e-30, -1e-30, 3e38, -3e38],
                        dtype=np.float32)
    return np.concatenate([v, specials])


def test_arithmetic_nodes_are_ieee_f32():
    rng = np.random.default_rng(4)
    a = _probe_f32(rng)
    b = rng.permutation(a)
    with np.errstate(all="ignore"):
        for t, ref in ((O.N_ADD, a + b), (O.N_SUB, a - b), (O.N_MUL, a * b), (O.N_DIV, a / b)):
            got = O.eval_binary(t, a, b)
            nan = np.isnan(ref)
            assert np.array_equal(np.isnan(got), nan)
            assert np.array_equal(bits(got[~nan]), bits(ref[~nan].astype(np.float32)))
        got = O.eval_unary(O.N_SQRT, np.abs(a))
        assert np.array_equal(bits(got), bits(np.sqrt(np.abs(a))))


def test_select_nodes_keep_signed_zero_and_pick_right_on_nan():
    nan = np.float32(np.nan)
    l = np.array([1, -0.0, nan, 2, 0.0], dtype=np.float32)
    r = np.array([2, 0.0, 3, nan, -0.0], dtype=np.float32)
    mx = O.eval_binary(O.N_MAX, l, r)
    mn = O.eval_binary(O.N_MIN, l, r)
    # l > r ? l : r  /  l < r ? l : r  (codegen/cpu.go:144-163)
    assert bits(mx).tolist() == bits(np.array([2, 0.0, 3, nan, -0.0], dtype=np.float32)).tolist()
    assert bits(mn).tolist() == bits(np.array([1, 0.0, 3, nan, -0.0], dtype=np.float32)).tolist()
    v = np.array([-0.0, -2.0, 3.0], dtype=np.float32)
    assert bits(O.eval_unary(O.N_ABS, v)).tolist() == bits(np.array([-0.0, 2.0, 3.0], np.float32)).tolist()
    assert bits(O.eval_unary(O.N_RELU, v)).tolist() == bits(np.array([-0.0, 0.0, 3.0], np.float32)).tolist()
    lr = O.eval_unary(O.N_LEAKY_RELU, v)
    assert bits(lr).tolist() == bits(np.array([-0.0, np.float32(0.01) * np.float32(-2.0), 3.0], np.float32)).tolist()


def test_transcendental_nodes_within_one_ulp_of_independent_forms():
    rng = np.random.default_rng(5)
    v = _probe_f32(rng, lo=-30, hi=30)
    v = v[np.isfinite(v)]
    d = v.astype(np.float64)
    with np.errstate(all="ignore"):
        cases = {
            O.N_EXP: np.exp(d),
            O.N_TANH: np.tanh(d),
            O.N_SIGMOID: expit(d),
            O.N_SILU: d * expit(d),
        }
        pos = np.abs(v) + np.float32(1e-3)
        log_ref = np.log(pos.astype(np.float64)).astype(np.float32)
    for t, ref in cases.items():
        got = O.eval_unary(t, v)
        ref32 = ref.astype(np.float32)
        ok = np.isfinite(ref32)
        assert ulp_diff(got[ok], ref32[ok]).max() <= 1, t
    assert ulp_diff(O.eval_unary(O.N_LOG, pos), log_ref).max() <= 1


def test_gelu_tanh_form():
    # Where the tanh form does not cancel, it equals v*sigmoid(2*inner).
    v = np.linspace(-5, 10, 200001, dtype=np.float32)
    d = v.astype(np.float64)
    inner = math.sqrt(2 / math.pi) * (d + 0.044715 * d ** 3)
    ref = (d * expit(2 * inner)).astype(np.float32)
    got = O.eval_unary(O.N_GELU, v)
    assert ulp_diff(got, ref).max() <= 1
    # Far left, 1 + tanh(inner) is exactly 0 in f64, so the reference form
    # returns -0 where v*sigmoid would not.
    far = np.array([-7.5, -9.0, -20.0], dtype=np.float32)
    assert bits(O.eval_unary(O.N_GELU, far)).tolist() == [0x80000000] * 3
    assert O.eval_unary(O.N_GELU, np.array([0.0], np.float32))[0] == 0.0


def test_special_values_of_activations():
    s = np.array([0.0, np.inf, -np.inf], dtype=np.float32)
    sig = O.eval_unary(O.N_SIGMOID, s)
    assert sig.tolist() == [0.5, 1.0, 0.0]
    silu = O.eval_unary(O.N_SILU, s)
    assert silu[0] == 0.0 and silu[1] == np.inf and np.isnan(silu[2])
    big = np.array([20.0, 100.0], dtype=np.float32)
    assert O.eval_unary(O.N_SILU, big).tolist() == [20.0, 100.0]


def test_scalar_broadcast_and_linspace_are_f32():
    rng = np.random.default_rng(6)
    x = rng.normal(size=1000).astype(np.float32)
    s = np.float32(1.7)
    assert np.array_equal(O.scalar_broadcast(x, float(s), "div"), (x / s).astype(np.float32))
    out = O.linspace(-3.0, 5.0, 11)
    step = (np.float32(5.0) - np.float32(-3.0)) / np.float32(10)
    ref = (np.float32(-3.0) + np.arange(11, dtype=np.float32) * step).astype(np.float32)
    ref[0], ref[-1] = -3.0, 5.0
    assert np.array_equal(out, ref)
    noend = O.linspace(0.0, 1.0, 4, endpoint=False)
    assert noend.tolist() == [0.0, 0.25, 0.5, 0.75]


# --------------------------------------------------------------------------
# Sensitivity: the checks above fail on plausible mutations.
# --------------------------------------------------------------------------

def test_checks_catch_planted_mistakes(golden):
    # bf16 by truncation misses the golden tie vectors.
    truncated = [int(c["f32_bits"], 16) >> 16 for c in golden["bf16_from_f32"]["cases"]]
    want = [int(c["bf16"], 16) for c in golden["bf16_from_f32"]["cases"]]
    assert truncated != want
    # bf16 rounding half-up (no to-even term) misses them too.
    halfup = [((int(c["f32_bits"], 16) + 0x8000) >> 16) & 0xFFFF for c in golden["bf16_from_f32"]["cases"]]
    assert halfup != want
    # E4M3 with bias 8 (the MI300 fnuz flavour) fails the closed form.
    assert any(math.ldexp(1 + (c & 7) / 8, ((c >> 3) & 15) - 8) != e4m3_closed(c)
               for c in range(1, 0x7F) if (c >> 3) & 15)
    # Swapping the Int4 nibble order fails the golden pair decode.
    pairs = golden["int4"]["decode_f64"][0]
    swapped = []
    for lo, hi in pairs["pairs"]:
        swapped += [hi, lo]
    assert swapped != pairs["values"]
    # gelu written as v*sigmoid(1.702 v) is off by far more than 1 ulp.
    v = np.float32(1.0)
    assert abs(float(v * expit(1.702 * v)) - float(O.eval_unary(O.N_GELU, np.array([v]))[0])) > 1e-4
