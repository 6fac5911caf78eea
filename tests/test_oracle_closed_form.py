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


# --------------------------------------------------------------------------
# Scaled FP8 dequant: closed-form decode, one numpy f32 multiply, then a
# library narrowing (torch bf16, numpy f16).  Nothing here calls the oracle's
# own decode or encode.
# --------------------------------------------------------------------------

# Scales: the config-2 scale, identity, a negative one, products that land in
# f32 denormals, products that overflow f16 / bf16 / f32, signed zeros, and
# scales where a product formed in f64 and rounded once to the output dtype
# differs from the f32 product narrowed (found by search; bf16 for e4m3
# 0x40e22e8b, 0x40f35556, e5m2 0x3ffd2492; f16 for e4m3 0x40f79555, e5m2
# 0x41178aab).
_FP8_SCALE_BITS = [0x3C4CCCCD, 0x3F800000, 0xC0600000, 0x09800000, 0x7149F2CA, 0x7E967699, 0x00000000,
                   0x80000000, 0x40E22E8B, 0x40F35556, 0x3FFD2492, 0x40F79555, 0x41178AAB]


def _closed_values(fmt):
    closed = e4m3_closed if fmt == O.F8E4M3 else e5m2_closed
    vals = [closed(c) for c in range(256)]
    nan = np.array([v is None for v in vals])
    return np.array([0.0 if v is None else v for v in vals], dtype=np.float32), nan


def _torch_bf16_bits(x):
    torch = pytest.importorskip("torch")
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16) \
        .numpy().view(np.uint16)


def _narrow(x, out_dtype):
    with np.errstate(over="ignore"):
        if out_dtype == O.FLOAT32:
            return np.ascontiguousarray(x, dtype=np.float32).copy()
        if out_dtype == O.BFLOAT16:
            return _torch_bf16_bits(x)
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def _as_bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("fmt", [O.F8E4M3, O.F8E5M2])
@pytest.mark.parametrize("out_dtype", [O.FLOAT32, O.BFLOAT16, O.FLOAT16])
def test_dequant_fp8_is_closed_form_times_f32_scale_then_narrowed(fmt, out_dtype):
    codes = np.arange(256, dtype=np.uint8)
    vals, nan = _closed_values(fmt)
    for sb in _FP8_SCALE_BITS:
        scale = from_bits(np.array([sb], np.uint32))[0]
        with np.errstate(over="ignore", invalid="ignore"):
            prod = (vals * scale).astype(np.float32)
        ok = ~nan & ~np.isnan(prod)  # Inf*0 has its own rule below
        want = _as_bits(_narrow(prod, out_dtype))
        got = _as_bits(O.dequant_fp8(codes, fmt, float(scale), out_dtype))
        assert np.array_equal(got[ok], want[ok]), (fmt, out_dtype, hex(sb))


def _nan_narrow(u32, out_dtype):
    """The reference narrowing of a NaN bit pattern (dtype/bfloat16.go:48-50,
    dtype/float16.go:273-278), stated directly."""
    u32 = int(u32)
    if out_dtype == O.FLOAT32:
        return u32
    if out_dtype == O.BFLOAT16:
        return (u32 >> 16) | 0x0040
    return ((u32 >> 16) & 0x8000) | 0x7C00 | 0x0200 | ((u32 & 0x7FFFFF) >> 13)


@pytest.mark.parametrize("out_dtype", [O.FLOAT32, O.BFLOAT16, O.FLOAT16])
def test_dequant_fp8_nan_and_inf_rules(out_dtype):
    # The scale multiply is build-defined with x86 mulss NaN rules made
    # explicit: a NaN code keeps its quieted NaN, a NaN scale propagates
    # quieted, Inf * 0 is the x86 default NaN 0xffc00000.
    def one(code, fmt, scale):
        return int(_as_bits(O.dequant_fp8(np.array([code], np.uint8), fmt, scale, out_dtype))[0])

    for code, bits32 in ((0x7F, 0x7FC00000), (0xFF, 0xFFC00000)):
        for scale in (0.0125, 0.0, -1.0, float("inf"), float("nan")):
            assert one(code, O.F8E4M3, scale) == _nan_narrow(bits32, out_dtype), (hex(code), scale)
    for code, bits32 in ((0x7D, 0x7FE00000), (0x7E, 0x7FC00000), (0x7F, 0x7FE00000), (0xFD, 0xFFE00000)):
        assert one(code, O.F8E5M2, 2.0) == _nan_narrow(bits32, out_dtype), hex(code)
    snan_scale = float(from_bits(np.array([0x7F800001], np.uint32))[0])
    assert one(0x38, O.F8E4M3, snan_scale) == _nan_narrow(0x7FC00001, out_dtype)
    for code in (0x7C, 0xFC):  # e5m2 +-Inf times +-0
        for zero in (0.0, -0.0):
            assert one(code, O.F8E5M2, zero) == _nan_narrow(0xFFC00000, out_dtype)
    for code in (0x00, 0x80):  # +-0 times Inf
        assert one(code, O.F8E4M3, float("inf")) == _nan_narrow(0xFFC00000, out_dtype)
    pinf = {O.FLOAT32: 0x7F800000, O.BFLOAT16: 0x7F80, O.FLOAT16: 0x7C00}[out_dtype]
    assert one(0x7C, O.F8E5M2, 3.0) == pinf
    assert one(0xFC, O.F8E5M2, -3.0) == pinf


# --------------------------------------------------------------------------
# axpy in a 16-bit storage dtype: decode, y + fl32(alpha * x) in f32, narrow.
# --------------------------------------------------------------------------

def _storage_decode(u16, dtype):
    if dtype == O.FLOAT16:
        return u16.view(np.float16).astype(np.float32)
    return (u16.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("dtype", [O.BFLOAT16, O.FLOAT16])
def test_axpy_storage_is_f32_axpy_then_library_narrowing(dtype):
    rng = np.random.default_rng(11)
    n = 1 << 16
    y16 = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    x16 = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    yv, xv = _storage_decode(y16, dtype), _storage_decode(x16, dtype)
    for alpha in (0.75, -1.0 / 3.0, 1e-3, 3e4):
        a = np.float32(alpha)
        with np.errstate(all="ignore"):
            ref32 = (yv + (a * xv).astype(np.float32)).astype(np.float32)
        ok = ~np.isnan(ref32)
        want = _narrow(ref32, dtype)
        got = O.axpy_storage(y16, x16, float(a), dtype)
        assert np.array_equal(got[ok], want[ok]), (dtype, alpha)
        assert ok.mean() > 0.9


# --------------------------------------------------------------------------
# Wide integers: BytesToFloat64 is a correctly rounded conversion,
# BytesToFloat32 goes through it (two roundings; convert.go:132-145).
# --------------------------------------------------------------------------

def _wide_int_probe(np_type):
    info = np.iinfo(np_type)
    rng = np.random.default_rng(12)
    bits = 8 * np.dtype(np_type).itemsize
    r = rng.integers(0, 1 << 62, 1 << 14, dtype=np.uint64)
    r = (r << np.uint64(2)) | rng.integers(0, 4, r.size, dtype=np.uint64)  # all 64 bits random
    r = (r >> np.uint64(64 - bits)).astype(np.dtype(f"u{bits // 8}")).view(np_type)
    edges = [info.min, info.max, 0, 1, -1, (1 << 24) + 1, (1 << 24) + 3, (1 << 31) - 1]
    if bits == 64:
        # exact ties after the f64 rounding: 2^60 + 2^36 + 1 rounds to the
        # even f32 2^60 through f64, to 2^60 + 2^37 when rounded once
        edges += [(1 << 60) + (1 << 36) + 1, (1 << 62) + (1 << 38) + 1, (1 << 53) + 1, (1 << 63) - 1]
    edges = [e for e in edges if info.min <= e <= info.max]
    return np.concatenate([r, np.array([np_type(e) for e in edges], dtype=np_type)])


@pytest.mark.parametrize("np_type, dt", [(np.int32, O.INT32), (np.int64, O.INT64), (np.uint32, O.UINT32),
                                         (np.uint64, O.UINT64)])
def test_wide_ints_convert_through_f64(np_type, dt):
    v = _wide_int_probe(np_type)
    f64 = O.bytes_to_f64(dt, v)
    assert np.array_equal(f64, v.astype(np.float64))
    f32 = O.bytes_to_f32(dt, v)
    assert np.array_equal(bits(f32), bits(v.astype(np.float64).astype(np.float32)))


def test_wide_int_double_rounding_is_kept():
    v = np.array([(1 << 60) + (1 << 36) + 1], dtype=np.int64)
    assert O.bytes_to_f32(O.INT64, v)[0] == np.float32(2.0 ** 60)
    # rounded once it would be the next f32 up: the two-step path is observable
    assert float(Fraction((1 << 60) + (1 << 37))) == float(np.float32(v.astype(np.float32)[0]))
    u = np.array([(1 << 63) + (1 << 39) + 1], dtype=np.uint64)
    assert O.bytes_to_f32(O.UINT64, u)[0] == np.float32(2.0 ** 63)


# --------------------------------------------------------------------------
# E5M2 subnormal encode quirk, values derived by hand from
# dtype/fp8.go:190-249: for an f32 exponent E, the branch shifts the 24-bit
# significand right by 21 - (E + 15), one bit short of the subnormal grid
# (units of 2^-16), so the code is twice the textbook one: [2^-15, 2^-14)
# rounds to 4..7 and clamps to 0x04, [2^-16, 2^-15) gives 1.m * 2 rounded
# half-even (2, 3 or 4), and anything below 2^-16 is zero.
# --------------------------------------------------------------------------

E5M2_SUBNORMAL_QUIRK = [
    (2.0 ** -15, 0x04), (1.5 * 2.0 ** -15, 0x04), (1.99 * 2.0 ** -15, 0x04), (2.0 ** -14, 0x04),
    (2.0 ** -16, 0x02), (1.25 * 2.0 ** -16, 0x02), (1.375 * 2.0 ** -16, 0x03), (1.5 * 2.0 ** -16, 0x03),
    (1.625 * 2.0 ** -16, 0x03), (1.75 * 2.0 ** -16, 0x04), (1.999 * 2.0 ** -16, 0x04),
    (2.0 ** -17, 0x00), (1.999 * 2.0 ** -17, 0x00), (2.0 ** -30, 0x00),
    (-(2.0 ** -16), 0x82), (-(2.0 ** -15), 0x84), (-(2.0 ** -17), 0x80),
]


def test_e5m2_subnormal_encode_quirk():
    for v, code in E5M2_SUBNORMAL_QUIRK:
        assert O.f32_to_e5m2(v) == code, (v, hex(code))
    xs = np.array([v for v, _ in E5M2_SUBNORMAL_QUIRK], np.float32)
    assert O.f32_to_fp8(xs, O.F8E5M2).tolist() == [c for _, c in E5M2_SUBNORMAL_QUIRK]


def _e5m2_nearest_even_subnormal(v):
    """What a textbook encoder gives in the subnormal range (units of 2^-16,
    ties to even, carrying into the normal 0x04)."""
    q = v / 2.0 ** -16
    r = math.floor(q)
    frac = q - r
    if frac > 0.5 or (frac == 0.5 and r % 2 == 1):
        r += 1
    return min(r, 4)


def test_new_checks_catch_planted_mistakes():
    # Planted in restatements written here, never in the product.
    codes = np.arange(256, dtype=np.uint8)
    vals, nan = _closed_values(O.F8E4M3)
    fin = ~nan
    # (1) the product formed in f64 and rounded once to bf16 fails the
    #     composition check at the searched scale
    s = from_bits(np.array([0x40E22E8B], np.uint32))[0]
    p64 = vals[fin].astype(np.float64) * np.float64(s)
    m, e = np.frexp(p64)
    once = (np.ldexp(np.rint(m * 256.0), e - 8).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    want = _narrow((vals[fin] * s).astype(np.float32), O.BFLOAT16)
    assert not np.array_equal(once, want)
    assert np.array_equal(O.dequant_fp8(codes, O.F8E4M3, float(s), O.BFLOAT16)[fin], want)
    # (2) the scale narrowed to bf16 before the multiply fails it at 0.0125
    s = np.float32(0.0125)
    s_bf16 = from_bits(np.array([int(_narrow(np.array([s]), O.BFLOAT16)[0]) << 16], np.uint32))[0]
    early = _narrow((vals[fin] * s_bf16).astype(np.float32), O.BFLOAT16)
    assert not np.array_equal(early, _narrow((vals[fin] * s).astype(np.float32), O.BFLOAT16))
    # (3) nearest-even subnormals fail the hand-derived e5m2 quirk table
    textbook = [_e5m2_nearest_even_subnormal(v) for v, c in E5M2_SUBNORMAL_QUIRK if 0 < v < 2.0 ** -14]
    quirk = [c for v, c in E5M2_SUBNORMAL_QUIRK if 0 < v < 2.0 ** -14]
    assert textbook != quirk
    # (4) a single-rounding int64 -> f32 conversion fails the wide-int check
    v = np.array([(1 << 60) + (1 << 36) + 1], dtype=np.int64)
    assert v.astype(np.float32)[0] != v.astype(np.float64).astype(np.float32)[0]
    # (5) an FMA-contracted 16-bit axpy fails the storage check on some input
    rng = np.random.default_rng(13)
    y = _storage_decode(rng.integers(0, 1 << 16, 4096, dtype=np.uint32).astype(np.uint16), O.FLOAT16)
    x = _storage_decode(rng.integers(0, 1 << 16, 4096, dtype=np.uint32).astype(np.uint16), O.FLOAT16)
    a = np.float32(-1.0 / 3.0)
    ok = np.isfinite(x) & np.isfinite(y) & (np.abs(x) < 1e4) & (np.abs(y) < 1e4)
    fused = np.array([np.float32(float(Fraction(float(a)) * Fraction(float(xi)) + Fraction(float(yi))))
                      for xi, yi in zip(x[ok], y[ok])], dtype=np.float32)
    unfused = (y[ok] + (a * x[ok]).astype(np.float32)).astype(np.float32)
    assert not np.array_equal(_narrow(fused, O.FLOAT16), _narrow(unfused, O.FLOAT16))


# --------------------------------------------------------------------------
# BytesToFloat64 and BytesToInt8 (dtype/convert/convert.go:36-79, 235-263).
# --------------------------------------------------------------------------

def _f32_probe_bits(rng):
    r = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 1, 0x807FFFFF, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x7F800001,
                        0xFFBFFFFF, 0x7FC00000, 0xFFC12345, 0x00800000], dtype=np.uint32)
    return np.concatenate([r, special])


def test_f32_to_f64_matches_the_hardware_widening():
    # numpy widens with the host's cvtss2sd, the instruction Go's float64(f32)
    # compiles to on amd64: exact for numbers, NaN quieted with its payload.
    u = _f32_probe_bits(np.random.default_rng(14))
    with np.errstate(invalid="ignore"):
        ref = u.view(np.float32).astype(np.float64).view(np.uint64)
    got = O.bytes_to_f64(O.FLOAT32, u).view(np.uint64)
    assert np.array_equal(got, ref)
    # every 16-bit and FP8 code: the f64 value of the Float32() decode
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for dt in (O.FLOAT16, O.BFLOAT16):
        with np.errstate(invalid="ignore"):
            want = O.bytes_to_f32(dt, h).astype(np.float64).view(np.uint64)
        assert np.array_equal(O.bytes_to_f64(dt, h).view(np.uint64), want)
    codes = np.arange(256, dtype=np.uint8)
    for dt in (O.F8E4M3, O.F8E5M2):
        with np.errstate(invalid="ignore"):
            want = O.bytes_to_f32(dt, codes).astype(np.float64).view(np.uint64)
        assert np.array_equal(O.bytes_to_f64(dt, codes).view(np.uint64), want)


def _i8_closed(d):
    """Saturate then truncate toward zero, NaN to 0, with numpy's own clip and trunc."""
    d = np.asarray(d, dtype=np.float64)
    with np.errstate(invalid="ignore"):
        t = np.clip(np.trunc(np.where(np.isnan(d), 0.0, d)), -128, 127)
    return t.astype(np.int8)


BYTES_TO_I8_EDGES = [0.0, -0.0, 0.999, -0.999, 1.0, -1.0, 1.9999999999, -1.9999999999, 126.9, 127.0, 127.5, 127.999,
                     128.0, 128.5, 1e30, -127.9, -128.0, -128.5, -128.999, -129.0, -1e30, float("inf"), float("-inf"),
                     float("nan"), -float("nan")]


def test_bytes_to_i8_is_saturate_then_truncate():
    rng = np.random.default_rng(15)
    d = np.concatenate([np.array(BYTES_TO_I8_EDGES), rng.uniform(-300, 300, 1 << 16), rng.normal(0, 50, 1 << 16)])
    assert np.array_equal(O.bytes_to_i8(O.FLOAT64, d), _i8_closed(d))
    f = d.astype(np.float32)
    assert np.array_equal(O.bytes_to_i8(O.FLOAT32, f), _i8_closed(f))
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for dt in (O.FLOAT16, O.BFLOAT16):
        assert np.array_equal(O.bytes_to_i8(dt, h), _i8_closed(O.bytes_to_f64(dt, h)))
    codes = np.arange(256, dtype=np.uint8)
    for dt in (O.F8E4M3, O.F8E5M2, O.INT8, O.UINT8):
        assert np.array_equal(O.bytes_to_i8(dt, codes), _i8_closed(O.bytes_to_f64(dt, codes)))
    assert O.bytes_to_i8(O.INT4, codes).tolist() == O.bytes_to_f64(O.INT4, codes).astype(np.int8).tolist()
    for np_type, dt in ((np.int16, O.INT16), (np.uint16, O.UINT16), (np.int32, O.INT32), (np.uint32, O.UINT32),
                        (np.int64, O.INT64), (np.uint64, O.UINT64)):
        v = _wide_int_probe(np_type)
        v = np.concatenate([v, np.array([np_type(x) for x in (0, 1, 127, 128, 200, 255)], dtype=np_type)])
        if np.iinfo(np_type).min < 0:
            v = np.concatenate([v, np.array([-1, -127, -128, -129, -1000], dtype=np_type)])
        want = np.clip(v.astype(np.float64), -128, 127).astype(np.int8)  # integers: saturation only
        assert np.array_equal(O.bytes_to_i8(dt, v), want), np_type


def test_bytes_to_i8_checks_catch_planted_mistakes():
    d = np.array(BYTES_TO_I8_EDGES)
    ok = ~np.isnan(d)
    want = _i8_closed(d)
    with np.errstate(invalid="ignore"):
        # rounding to nearest instead of truncating
        assert not np.array_equal(np.clip(np.rint(d[ok]), -128, 127).astype(np.int8), want[ok])
        # wrapping instead of saturating
        assert not np.array_equal(np.trunc(d[ok & (np.abs(d) < 1e9)]).astype(np.int64).astype(np.int8),
                                  want[ok & (np.abs(d) < 1e9)])
        # truncating the f32 value of an f64 input (1.9999999999 becomes 2)
        assert not np.array_equal(_i8_closed(d.astype(np.float32)), want)


# --------------------------------------------------------------------------
# Int4 encode (dtype/int4.go:60-70): int8 -> clamp to [-8, 7] -> nibble,
# low nibble first.  Pinned by decoding the packed bytes with the oracle's
# Int4 decode (itself pinned by the golden pair vectors above) and checking
# the clamp against plain integer bounds, for every int8 value in both
# nibble positions.
# --------------------------------------------------------------------------

def test_int4_encode_every_int8_value():
    v = np.arange(-128, 128, dtype=np.int16).astype(np.int8)
    want = np.minimum(np.maximum(v.astype(np.int16), -8), 7)
    zero = np.zeros_like(v)
    for slot, pairs in ((0, np.stack([v, zero], axis=1)), (1, np.stack([zero, v], axis=1))):
        back = O.bytes_to_i8(O.INT4, O.int4_encode(pairs.reshape(-1))).astype(np.int16).reshape(-1, 2)
        np.testing.assert_array_equal(back[:, slot], want)  # every value as the low, then the high nibble
        np.testing.assert_array_equal(back[:, 1 - slot], 0)
    # an odd count: the last byte's high nibble is 0
    assert O.int4_encode(np.array([3, -2, 7], np.int8)).tolist() == [0xE3, 0x07]
    # planted: wrapping instead of clamping (v & 0xF) decodes -100 as -4, not -8
    wrapped = (np.array([-100], np.int16) & 0xF).astype(np.uint8)
    assert O.bytes_to_i8(O.INT4, wrapped).tolist() != [-8]


def test_bytes_to_i4_follows_bytes_to_i8():
    # the float path: BytesToInt8's saturate-then-truncate, then the clamp
    f = np.array([0.0, -0.0, 0.9, -0.9, 7.99, -8.99, 8.0, -9.0, 1e9, -1e9, np.nan, np.inf, -np.inf, 3.5],
                 dtype=np.float32)
    got = O.bytes_to_i8(O.INT4, O.bytes_to_i4(O.FLOAT32, f, f.size))[:f.size].tolist()
    assert got == [0, 0, 0, 0, 7, -8, 7, -8, 7, -8, 0, 7, -8, 3]


# --------------------------------------------------------------------------
# Build-defined extensions of the reference, pinned by the reference's own
# semantics.  Broadcast: CPUKernel.Run requires every input to hold at least
# `count` values (codegen/cpu.go:78-85), so a periodic or scalar operand must
# give exactly what the same chain gives on its pre-expanded copy.  Int4 group
# scale: decodeInt4ToFloat64 (dtype/convert/decoders.go:262-289) gives the
# signed nibble, low nibble first, and the build multiplies it by the f32 value
# of scale[i // group] once, then narrows like float32VectorBytes.
# --------------------------------------------------------------------------

CONFIG4_CHAIN = (O.N_ADD, (O.N_GELU, (O.N_MUL, (O.N_ADD, ("in", 0), ("in", 1)), ("in", 2))), ("in", 3))


def _expanded(a, period, count):
    """The reference's own operand: `count` values, element e = a[e % period]."""
    return np.resize(np.asarray(a, dtype=np.float32), count)


@pytest.mark.parametrize("count", [4096 * 3, 4096 * 3 + 17, 5])
def test_periodic_operands_equal_their_pre_expanded_copies_config4(count):
    rng = np.random.default_rng(count)
    x = rng.standard_normal(count).astype(np.float32)
    r = rng.standard_normal(count).astype(np.float32)
    bias = rng.normal(0, 0.02, 4096).astype(np.float32)
    s = np.array([1.1], np.float32)
    nodes = O.flatten(CONFIG4_CHAIN)
    got = O.run(nodes, [x, bias, s, r], count, periods=[0, 4096, 1, 0])
    want = O.run(nodes, [x, _expanded(bias, 4096, count), np.full(count, s[0], np.float32), r], count)
    assert np.array_equal(bits(got), bits(want))


def _random_chain(rng, n_inputs, depth):
    if depth == 0 or rng.random() < 0.25:
        return ("in", int(rng.integers(0, n_inputs)))
    op = int(rng.choice([O.N_ADD, O.N_SUB, O.N_MUL, O.N_DIV, O.N_MAX, O.N_MIN, O.N_NEG, O.N_ABS,
                         O.N_RELU, O.N_SILU, O.N_GELU, O.N_SIGMOID, O.N_TANH, O.N_LEAKY_RELU]))
    if O.arity(op) == 2:
        return (op, _random_chain(rng, n_inputs, depth - 1), _random_chain(rng, n_inputs, depth - 1))
    return (op, _random_chain(rng, n_inputs, depth - 1))


def test_periodic_operands_equal_their_pre_expanded_copies_random_chains():
    rng = np.random.default_rng(2024)
    count = 3 * 7 * 64 + 11
    for trial in range(40):
        n_in = int(rng.integers(1, 5))
        nodes = O.flatten(_random_chain(rng, n_in, 4))
        periods = [int(rng.choice([0, 1, 7, 64, 100, count])) for _ in range(n_in)]
        arrays = [rng.normal(0, 2, p if p > 0 else count).astype(np.float32) for p in periods]
        got = O.run(nodes, arrays, count, periods=periods)
        want = O.run(nodes, [_expanded(a, p, count) if p > 0 else a for a, p in zip(arrays, periods)], count)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), (trial, periods)
        assert np.array_equal(bits(got[~nan]), bits(want[~nan])), (trial, periods)


# Scales that reach every branch of the product: exact products, zeros of
# both signs, an f16 subnormal, the largest f16, Inf and NaN.
_INT4_F16_SCALES = np.array([0x2148, 0x251F, 0x3C00, 0xB800, 0x0000, 0x8000, 0x0001, 0x03FF, 0x7BFF, 0x7C00,
                             0xFC00, 0x7E00, 0x7D01], dtype=np.uint16)


def _int4_closed(packed, n, scale_f32, group):
    """(nib - 16 (nib >= 8)) * scale[i // group], low nibble first, in f32."""
    nib = np.empty(2 * packed.size, dtype=np.int64)
    nib[0::2], nib[1::2] = packed & 15, packed >> 4
    q = (nib - 16 * (nib >= 8))[:n].astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        return (q * scale_f32[np.arange(n) // group]).astype(np.float32)


@pytest.mark.parametrize("out_dtype", [O.FLOAT32, O.BFLOAT16, O.FLOAT16])
@pytest.mark.parametrize("group, n", [(128, 128 * 26), (128, 128 * 26 - 37), (96, 96 * 26 + 5), (3, 3 * 26 + 1)])
def test_dequant_int4_is_nibble_times_group_scale_then_narrowed(out_dtype, group, n):
    # Every byte (so all 16 codes on both nibbles) under each special f16
    # scale, one scale per group; a partial last group, odd counts (the last
    # byte's high nibble unused) and groups that are not powers of two.
    groups = -(-n // group)
    scales = np.resize(_INT4_F16_SCALES, groups)
    packed = np.resize(np.arange(256, dtype=np.uint8), (n + 1) // 2)
    np.random.default_rng(group + n).shuffle(packed)
    prod = _int4_closed(packed, n, scales.view(np.float16).astype(np.float32), group)
    got = _as_bits(O.dequant_int4(packed, n, scales, O.FLOAT16, group, out_dtype))
    nan = np.isnan(prod)
    assert np.array_equal(got[~nan], _as_bits(_narrow(prod[~nan], out_dtype)))
    # NaN products keep the x86 multiply's NaN: Inf * 0 is the default NaN
    # 0xffc00000, a NaN scale propagates quieted with its payload
    sf = scales.view(np.uint16).astype(np.uint32)[np.arange(n) // group]
    s32 = scales.view(np.float16).astype(np.float32).view(np.uint32)[np.arange(n) // group]
    want_nan = np.where((sf & 0x7FFF) > 0x7C00, s32 | 0x00400000, 0xFFC00000)
    assert [int(b) for b in got[nan]] == [_nan_narrow(b, out_dtype) for b in want_nan[nan]]


@pytest.mark.parametrize("scale_dtype", [O.FLOAT32, O.BFLOAT16])
def test_dequant_int4_wide_scales(scale_dtype):
    rng = np.random.default_rng(scale_dtype)
    n, group = 128 * 40 + 3, 128
    packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    s32 = rng.uniform(-3, 3, -(-n // group)).astype(np.float32)
    if scale_dtype == O.BFLOAT16:
        scales = _narrow(s32, O.BFLOAT16)
        s32 = (scales.astype(np.uint32) << 16).view(np.float32)
    else:
        scales = s32
    want = _narrow(_int4_closed(packed, n, s32, group), O.BFLOAT16)
    assert np.array_equal(O.dequant_int4(packed, n, scales, scale_dtype, group, O.BFLOAT16), want)


def test_extension_checks_catch_planted_mistakes():
    # Planted in restatements written here, never in the product: each one is
    # told apart from the oracle by the checks above.
    rng = np.random.default_rng(99)
    count = 4096 * 2 + 9
    x = rng.standard_normal(count).astype(np.float32)
    r = rng.standard_normal(count).astype(np.float32)
    bias = rng.normal(0, 0.02, 4096).astype(np.float32)
    s = np.array([1.1], np.float32)
    nodes = O.flatten(CONFIG4_CHAIN)
    periodic = O.run(nodes, [x, bias, s, r], count, periods=[0, 4096, 1, 0])
    # (1) broadcast by e // p (each bias value repeated) instead of e % p
    wrong = np.repeat(bias, -(-count // 4096))[:count]
    assert not np.array_equal(bits(O.run(nodes, [x, wrong, np.full(count, 1.1, np.float32), r], count)),
                              bits(periodic))
    # Int4: every byte, f16 scales that differ per group, group 128
    n, group = 128 * 8 + 3, 128
    packed = np.resize(np.arange(256, dtype=np.uint8), (n + 1) // 2)
    scales = O.f32_to_f16(rng.uniform(0.005, 0.02, -(-n // group)).astype(np.float32))
    sf = scales.view(np.float16).astype(np.float32)
    got = O.dequant_int4(packed, n, scales, O.FLOAT16, group, O.BFLOAT16)
    assert np.array_equal(got, _narrow(_int4_closed(packed, n, sf, group), O.BFLOAT16))
    nib = np.empty(2 * packed.size, dtype=np.int64)
    # (2) the group counted over bytes rather than elements
    nib[0::2], nib[1::2] = packed & 15, packed >> 4
    q = (nib - 16 * (nib >= 8))[:n].astype(np.float32)
    by_bytes = (q * sf[(np.arange(n) // 2) // group]).astype(np.float32)
    assert not np.array_equal(_narrow(by_bytes, O.BFLOAT16), got)
    # (3) the high nibble first
    nib[0::2], nib[1::2] = packed >> 4, packed & 15
    q = (nib - 16 * (nib >= 8))[:n].astype(np.float32)
    assert not np.array_equal(_narrow((q * sf[np.arange(n) // group]).astype(np.float32), O.BFLOAT16), got)
    # (4) unsigned nibbles (no sign extension)
    nib[0::2], nib[1::2] = packed & 15, packed >> 4
    q = nib[:n].astype(np.float32)
    assert not np.array_equal(_narrow((q * sf[np.arange(n) // group]).astype(np.float32), O.BFLOAT16), got)
