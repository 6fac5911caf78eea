"""The CPU oracle against the golden vectors of the reference's own Go tests.

Fixture: tests/golden/reference_vectors.json (values transcribed from
dtype/*_test.go, dtype/convert/convert_test.go, codegen/codegen_test.go,
optimizer/constant_fold_test.go, runtime/axpy_test.go,
runtime/executor_math_test.go).
"""
import math

import numpy as np
import pytest

import oracle as O


def h(s):
    return int(s, 16)


def f32_from_bits(bits):
    return float(np.array([bits], dtype=np.uint32).view(np.float32)[0])


def bits_of_f32(v):
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0])


def test_bf16_rne_golden(golden):
    for case in golden["bf16_from_f32"]["cases"]:
        assert O.f32_bits_to_bf16(h(case["f32_bits"])) == h(case["bf16"]), case["note"]
    for nan in golden["bf16_from_f32"]["nan_inputs_stay_nan"]:
        out = O.f32_bits_to_bf16(h(nan))
        assert (out & 0x7f80) == 0x7f80 and (out & 0x007f) != 0


def test_bf16_bytes_golden(golden):
    g = golden["bf16_bytes"]
    buf = np.array(g["le_bytes_of_1_and_2"], dtype=np.uint8)
    assert list(O.bytes_to_f32(O.BFLOAT16, buf)) == g["decoded_f32"]
    enc = O.f32_to_bf16(np.array(g["decoded_f32"], dtype=np.float32))
    assert list(enc.view(np.uint8)) == g["le_bytes_of_1_and_2"]


def test_e4m3_golden(golden):
    g = golden["e4m3_round_trip"]
    for v in g["values"]:
        assert O.e4m3_to_f32(O.f32_to_e4m3(v)) == pytest.approx(v, abs=g["tolerance"])
    for v, want in g["saturate"]:
        assert O.e4m3_to_f32(O.f32_to_e4m3(v)) == want
    assert O.f32_to_e4m3(float("nan")) == h(g["nan_code"])
    assert math.isnan(O.e4m3_to_f32(h(g["nan_code"])))
    for v, code in g["zero_codes"]:
        assert O.f32_to_e4m3(v) == h(code)


def test_e5m2_golden(golden):
    g = golden["e5m2_round_trip"]
    for v in g["values"]:
        assert O.e5m2_to_f32(O.f32_to_e5m2(v)) == pytest.approx(v, abs=g["tolerance"])
    for v, want in g["overflow_to_inf"]:
        got = O.e5m2_to_f32(O.f32_to_e5m2(v))
        assert math.isinf(got) and (got > 0) == (want == "+inf")
    assert math.isinf(O.e5m2_to_f32(O.f32_to_e5m2(float("inf"))))
    assert math.isnan(O.e5m2_to_f32(O.f32_to_e5m2(float("nan"))))


def test_f16_golden(golden):
    g = golden["f16"]
    for bits, want in g["decode"]:
        raw = np.array([h(bits)], dtype=np.uint16)
        assert O.bytes_to_f32(O.FLOAT16, raw)[0] == want
    for v, bits in g["encode"]:
        assert O.f32_to_f16(np.array([v], dtype=np.float32))[0] == h(bits)
    enc = O.f32_to_f16(np.array([np.inf, -np.inf], dtype=np.float32))
    assert list(enc) == [h(g["inf_bits"]["pos"]), h(g["inf_bits"]["neg"])]
    for bits in (g["quiet_nan_bits"], g["signaling_nan_bits"]):
        raw = np.array([h(bits)], dtype=np.uint16)
        assert math.isnan(O.bytes_to_f32(O.FLOAT16, raw)[0])


def pack_pair(lo, hi):
    clamp = lambda v: max(-8, min(7, v)) & 0xF  # noqa: E731  (int4Encode, dtype/int4.go:60-70)
    return clamp(lo) | (clamp(hi) << 4)


def test_int4_golden(golden):
    g = golden["int4"]
    for lo, hi in g["pairs"]:
        b = pack_pair(lo, hi)
        assert (O.lib().orc_int4_lo(b), O.lib().orc_int4_hi(b)) == (lo, hi)
    for lo, hi, want_lo, want_hi in g["clamp"]:
        b = pack_pair(lo, hi)
        assert (O.lib().orc_int4_lo(b), O.lib().orc_int4_hi(b)) == (want_lo, want_hi)
    for case in g["decode_f64"]:
        buf = np.array([pack_pair(lo, hi) for lo, hi in case["pairs"]], dtype=np.uint8)
        assert list(O.bytes_to_f64(O.INT4, buf)) == case["values"]


def test_convert_golden(golden):
    g = golden["convert"]
    f = np.array(g["f32_to_f64_lossless"], dtype=np.float32)
    assert list(O.bytes_to_f64(O.FLOAT32, f)) == [float(x) for x in f]
    bf = O.f32_to_bf16(np.array(g["bf16_to_f64_within_1e-2"], dtype=np.float32))
    assert O.bytes_to_f64(O.BFLOAT16, bf) == pytest.approx(g["bf16_to_f64_within_1e-2"], abs=1e-2)
    i8 = np.array(g["int8_bytes"], dtype=np.uint8)
    assert list(O.bytes_to_f64(O.INT8, i8)) == g["int8_values"]
    rt = np.array(g["f32_round_trip"], dtype=np.float32)
    assert list(O.bytes_to_f32(O.FLOAT32, rt)) == g["f32_round_trip"]
    rb = O.bytes_to_bf16(O.FLOAT32, np.array(g["bf16_round_trip_within_1e-2"], dtype=np.float32))
    assert O.bytes_to_f32(O.BFLOAT16, rb) == pytest.approx(g["bf16_round_trip_within_1e-2"], abs=1e-2)
    with pytest.raises(O.OracleError):
        O.bytes_to_f64(16, np.array([1], dtype=np.uint8))  # Bool is rejected (convert_test.go:70-75)


def test_bytes_to_int8_golden(golden):
    g = golden["bytes_to_int8"]
    for case in (g["truncate"], g["saturate"]):
        f = np.array(case["f32"], dtype=np.float32)
        assert O.bytes_to_i8(O.FLOAT32, f).tolist() == case["i8"]


def test_evaluator_golden(golden):
    g = golden["evaluator"]
    nodes = O.flatten((O.N_RELU, (O.N_ADD, ("in", 0), ("in", 1))))
    out = O.run(nodes, [g["relu_add"]["x"], g["relu_add"]["y"]], 4)
    assert list(out) == g["relu_add"]["expected"]
    with pytest.raises(O.OracleError):  # a node addressing a missing input (codegen_test.go:52-56)
        O.run(nodes, [g["relu_add"]["x"]], 2)
    xs = np.array(g["activation_inputs"], dtype=np.float32)
    tol = g["activation_tolerance"]
    sig = O.eval_unary(O.N_SIGMOID, xs)
    assert sig == pytest.approx([1 / (1 + math.exp(-float(v))) for v in xs], abs=tol)
    th = O.eval_unary(O.N_TANH, xs)
    assert th == pytest.approx([math.tanh(float(v)) for v in xs], abs=tol)


def test_constant_fold_golden(golden):
    g = golden["constant_fold"]
    v, tol = g["operand"], g["tolerance"]
    assert O.fold(O.N_EXP, [v]) == pytest.approx(math.exp(v), abs=tol)
    assert O.fold(O.N_TANH, [v]) == pytest.approx(math.tanh(v), abs=tol)
    assert O.fold(O.N_SIGMOID, [v]) == pytest.approx(1 / (1 + math.exp(-v)), abs=tol)
    assert O.fold(O.N_DIV, [1.0, 0.0]) is None  # division by zero is not folded


def test_axpy_golden(golden):
    g = golden["axpy"]
    assert list(O.axpy_f32(g["y"], g["x"], g["alpha"])) == g["expected"]
    y = O.f32_to_bf16(np.array(g["y"], dtype=np.float32))
    x = O.f32_to_bf16(np.array(g["x"], dtype=np.float32))
    out = O.axpy_storage(y, x, g["alpha"], O.BFLOAT16)
    assert list(O.bytes_to_f32(O.BFLOAT16, out)) == g["expected"]


def test_linspace_scalar_broadcast_golden(golden):
    g = golden["linspace_scalar_broadcast"]
    ls = g["linspace"]
    sig = O.linspace(ls["start"], ls["stop"], ls["count"])
    for i, v in g["sigmas"]["exact"]:
        assert sig[i] == v
    for i, v in g["sigmas"]["approx"]:
        assert sig[i] == pytest.approx(v, abs=g["sigmas"]["tolerance"])
    sb = g["scalar_broadcast"]
    ts = O.scalar_broadcast(sig, sb["scalar"], sb["op"])
    for i, v in g["timesteps"]["exact"]:
        assert ts[i] == v
    for i, v in g["timesteps"]["approx"]:
        assert ts[i] == pytest.approx(v, abs=g["timesteps"]["tolerance"])
    with pytest.raises(O.OracleError):
        O.scalar_broadcast(sig, 0.0, "div")
    with pytest.raises(O.OracleError):
        O.linspace(0.0, 1.0, 0)


def test_int4_pair_golden(golden):
    # NewInt4Pair packs the clamped low and high nibbles; Lo/Hi sign-extend
    # them back (the oracle's Int4 decode), so each pair's byte decodes to
    # the reference's expected values.
    g = golden["int4_pair"]
    for (lo, hi), want in zip(g["pairs"], g["lo_hi"]):
        packed = O.int4_encode(np.array([lo, hi], np.int8))
        assert packed.size == 1
        assert O.bytes_to_i8(O.INT4, packed).tolist() == want
    for key, slot in (("with_lo", 0), ("with_hi", 1)):
        case = g[key]
        vals = list(case["pair"])
        vals[slot] = case["value"]  # WithLo/WithHi replace one nibble of the pair
        assert O.bytes_to_i8(O.INT4, O.int4_encode(np.array(vals, np.int8))).tolist() == case["lo_hi"]
