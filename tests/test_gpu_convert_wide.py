"""GPU parity of mfh_convert's f64, i8 and i4 outputs: BytesToFloat64
(dtype/convert/convert.go:36-79, decoders.go), BytesToInt8 (:235-263) and
BytesToInt8 through int4Encode (dtype/int4.go:60-70),
bit for bit against the CPU oracle on every 16-bit, FP8, Int4 and byte code,
random wide sources with their edge values, tails and misaligned buffers, and
over every f32 input against closed forms evaluated with torch on the device.
"""
import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

from gpu_util import empty_dev, log, stream, to_dev, to_host

pytestmark = pytest.mark.gpu

OUT_NP = {O.FLOAT64: np.uint64, O.INT8: np.int8, O.F8E4M3: np.uint8}
OUT_SIZE = {O.FLOAT64: 8, O.INT8: 1, O.F8E4M3: 1}
ORACLE = {O.FLOAT64: lambda dt, a: O.bytes_to_f64(dt, a).view(np.uint64), O.INT8: O.bytes_to_i8}
NP_OF = {O.FLOAT64: np.float64, O.FLOAT32: np.float32, O.INT64: np.int64, O.INT32: np.int32, O.INT16: np.int16,
         O.INT8: np.int8, O.UINT64: np.uint64, O.UINT32: np.uint32, O.UINT16: np.uint16, O.UINT8: np.uint8,
         O.FLOAT16: np.uint16, O.BFLOAT16: np.uint16, O.F8E4M3: np.uint8, O.F8E5M2: np.uint8}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def convert(a, in_dt, out_dt, n, pad_in=0, pad_out=0):
    src, sp = to_dev(a, pad=pad_in)
    out, op = empty_dev(n * OUT_SIZE[out_dt], pad=pad_out)
    M.convert(op, out_dt, sp, in_dt, n, stream())
    return to_host(out, OUT_NP[out_dt], pad=pad_out)


def check(got, want, what):
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:4]}: got {got[bad[:4]]} want {want[bad[:4]]}"


@pytest.mark.parametrize("out_dt", [O.FLOAT64, O.INT8])
@pytest.mark.parametrize("in_dt", [O.FLOAT16, O.BFLOAT16, O.F8E4M3, O.F8E5M2, O.INT8, O.UINT8, O.INT16, O.UINT16,
                                   O.INT4])
def test_every_code(in_dt, out_dt):
    if in_dt in (O.FLOAT16, O.BFLOAT16, O.INT16, O.UINT16):
        a = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(NP_OF[in_dt])
        n = a.size
    else:
        a = np.tile(np.arange(256, dtype=np.uint8), 3)
        n = a.size * (2 if in_dt == O.INT4 else 1)
    got = convert(a, in_dt, out_dt, n)
    check(got, ORACLE[out_dt](in_dt, a), f"{in_dt}->{out_dt}")


def wide_source(in_dt, n, rng):
    np_dt = NP_OF[in_dt]
    a = rng.integers(0, 256, size=8 * n, dtype=np.uint8).view(np_dt)[:n].copy()
    if in_dt in (O.FLOAT64, O.FLOAT32):
        f = np.array([0.0, -0.0, 0.999, -0.999, 1.9999999999, -1.9999999999, 127.0, 127.5, 128.0, -128.0, -128.5,
                      -129.0, 1e30, -1e30, np.inf, -np.inf, np.nan, 1e-300, -5e-324], dtype=np.float64)
        with np.errstate(over="ignore", under="ignore", invalid="ignore"):
            edges = f.astype(np_dt)
        specials = np.array([0x7F800001, 0xFFC12345, 0x00000001, 0x807FFFFF], np.uint32).view(np.float32)
        if in_dt == O.FLOAT32:
            edges = np.concatenate([edges, specials])
        else:
            edges = np.concatenate([edges, np.array([0x7FF0000000000001, 0xFFF8123456789ABC], np.uint64)
                                    .view(np.float64)])
        # values spread over the int8 range and past it
        spread = rng.uniform(-300, 300, n // 4).astype(np_dt)
        a = np.concatenate([a, edges, spread])
    else:
        info = np.iinfo(np_dt)
        edges = [0, 1, 127, 128, 255, info.max, info.min]
        if info.min < 0:
            edges += [-1, -127, -128, -129]
        if info.bits == 64:
            edges += [(1 << 53) + 1, (1 << 60) + (1 << 36) + 1]
        edges = np.array([np_dt(e) for e in edges if info.min <= e <= info.max], dtype=np_dt)
        a = np.concatenate([a, edges])
    return a


@pytest.mark.parametrize("out_dt", [O.FLOAT64, O.INT8])
@pytest.mark.parametrize("in_dt", [O.FLOAT64, O.FLOAT32, O.INT64, O.INT32, O.UINT64, O.UINT32])
@pytest.mark.parametrize("n, pad", [(50001, 0), (50001, 1), (50001, 8), (7, 0), (3, 2)])
def test_wide_sources_tails_misaligned(in_dt, out_dt, n, pad):
    # aligned buffers take whole items plus an element tail; a source or an
    # output off its alignment runs the element loop
    a = wide_source(in_dt, n, np.random.default_rng(in_dt * 11 + n + pad))
    got = convert(a, in_dt, out_dt, a.size, pad_in=pad, pad_out=pad % 3)
    check(got, ORACLE[out_dt](in_dt, a), f"{in_dt}->{out_dt} n={a.size} pad={pad}")


@pytest.mark.parametrize("out_pad", [0, 1, 2, 8, 16])
@pytest.mark.parametrize("in_dt", [O.FLOAT16, O.INT16])
def test_int8_from_2byte_sources_every_output_alignment(in_dt, out_pad):
    # 2-byte sources write one 8-byte store per 16-byte source piece when the
    # output is 8-byte aligned and run the 16-element items otherwise
    n = 3 * 4096 + 37
    a = np.random.default_rng(out_pad).integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16).view(NP_OF[in_dt])
    got = convert(a, in_dt, O.INT8, n, pad_out=out_pad)
    check(got, O.bytes_to_i8(in_dt, a), f"{in_dt}->i8 out_pad={out_pad}")
    got8 = convert(a, in_dt, O.F8E4M3, n, pad_out=out_pad)
    want8 = O.f32_to_fp8(O.bytes_to_f32(in_dt, a), O.F8E4M3)
    assert np.array_equal(got8.view(np.uint8), want8), f"{in_dt}->e4m3 out_pad={out_pad}"


def test_golden_bytes_to_int8(golden):
    g = golden["bytes_to_int8"]
    for case in (g["truncate"], g["saturate"]):
        f = np.array(case["f32"], dtype=np.float32)
        assert convert(f, O.FLOAT32, O.INT8, f.size).tolist() == case["i8"]


def test_every_f32_input_to_f64_and_i8():
    # All 2^32 f32 bit patterns.  f64: exact widening on the bits (normals
    # re-biased, denormals as m * 2^-149 computed in f64 on the device, NaN
    # quieted with its payload); i8: torch's trunc and clamp, NaN to 0.
    torch = __import__("torch")
    chunk = 1 << 28
    src = torch.empty(chunk, dtype=torch.int32, device="cuda")
    out64 = torch.empty(chunk, dtype=torch.int64, device="cuda")
    out8 = torch.empty(chunk, dtype=torch.int8, device="cuda")
    s = stream()
    for start in range(0, 1 << 32, chunk):
        b = torch.arange(start, start + chunk, dtype=torch.int64, device="cuda")
        src.copy_(b.to(torch.int32))
        M.convert(out64.data_ptr(), O.FLOAT64, src.data_ptr(), O.FLOAT32, chunk, s)
        M.convert(out8.data_ptr(), O.INT8, src.data_ptr(), O.FLOAT32, chunk, s)
        sign = (b >> 31) << 63
        e = (b >> 23) & 0xFF
        m = b & 0x7FFFFF
        normal = sign | ((e + 896) << 52) | (m << 29)
        den = (m.to(torch.float64) * 2.0 ** -149).view(torch.int64) | sign
        special = sign | 0x7FF0000000000000 | ((m != 0).to(torch.int64) << 51) | (m << 29)
        want64 = torch.where(e == 0xFF, special, torch.where(e == 0, den, normal))
        bad = torch.nonzero(out64 != want64).flatten()
        assert bad.numel() == 0, f"f32->f64 at input {int(b[bad[0]]):#010x}: got {int(out64[bad[0]]):#x}"
        x = src.view(torch.float32)
        t = torch.clamp(torch.trunc(x), -128, 127)
        want8 = torch.where(torch.isnan(x), torch.zeros_like(t), t).to(torch.int8)
        bad = torch.nonzero(out8 != want8).flatten()
        assert bad.numel() == 0, f"f32->i8 at input {int(b[bad[0]]):#010x}: got {int(out8[bad[0]])}"
        log(f"f32->f64, i8: inputs {start:#x}.. ok")
    # a sample of the same inputs against the CPU oracle
    rng = np.random.default_rng(16)
    u = rng.integers(0, 2 ** 32, 1 << 16, dtype=np.uint64).astype(np.uint32)
    check(convert(u, O.FLOAT32, O.FLOAT64, u.size), O.bytes_to_f64(O.FLOAT32, u).view(np.uint64), "f32->f64 sample")
    check(convert(u, O.FLOAT32, O.INT8, u.size), O.bytes_to_i8(O.FLOAT32, u), "f32->i8 sample")


def test_rejects_unsupported_outputs():
    src, sp = to_dev(np.zeros(64, np.uint8))
    out, op = empty_dev(256)
    for bad in (O.INT16, O.INT32, O.UINT8, 16):
        with pytest.raises(M.MFHError, match="is not f64/f32/bf16/f16/fp8/i8/i4"):
            M.convert(op, bad, sp, O.FLOAT32, 16, stream())


# ---- Int4 output: BytesToInt8's value through int4Encode (dtype/int4.go:60-70) ----

def convert_i4(a, in_dt, n, pad_in=0, pad_out=0):
    src, sp = to_dev(a, pad=pad_in)
    out, op = empty_dev((n + 1) // 2, pad=pad_out)
    M.convert(op, O.INT4, sp, in_dt, n, stream())
    return to_host(out, np.uint8, pad=pad_out)


@pytest.mark.parametrize("in_dt", [O.FLOAT16, O.BFLOAT16, O.F8E4M3, O.F8E5M2, O.INT8, O.UINT8, O.INT16, O.UINT16,
                                   O.INT4])
def test_int4_from_every_code(in_dt):
    if in_dt in (O.FLOAT16, O.BFLOAT16, O.INT16, O.UINT16):
        a = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(NP_OF[in_dt])
        n = a.size
    else:
        # 41 copies: two whole 4 KiB wave chunks of 8-bit codes and a tail
        a = np.tile(np.arange(256, dtype=np.uint8), 41)
        n = a.size * (2 if in_dt == O.INT4 else 1)
    check(convert_i4(a, in_dt, n), O.bytes_to_i4(in_dt, a, n), f"{in_dt}->i4")


@pytest.mark.parametrize("in_dt", [O.FLOAT64, O.FLOAT32, O.INT64, O.INT32, O.UINT64, O.UINT32])
@pytest.mark.parametrize("n, pad", [(50001, 0), (50001, 1), (50000, 16), (7, 0), (1, 2), (33, 0)])
def test_int4_wide_sources_odd_counts_misaligned(in_dt, n, pad):
    # 32-element items into 16-byte stores when the output is 16-byte
    # aligned, the byte loop otherwise and for the tail; an odd count's last
    # high nibble is 0
    a = wide_source(in_dt, n, np.random.default_rng(in_dt * 13 + n + pad))
    for m in (a.size, a.size - 1):  # both parities of the count
        got = convert_i4(a, in_dt, m, pad_in=pad, pad_out=pad % 3)
        check(got, O.bytes_to_i4(in_dt, a, m), f"{in_dt}->i4 n={m} pad={pad}")


def test_golden_int4_pairs(golden):
    g = golden["int4_pair"]
    vals = np.array([v for pair in g["pairs"] for v in pair], np.int8)
    got = convert_i4(vals, O.INT8, vals.size)
    assert O.bytes_to_i8(O.INT4, got).reshape(-1, 2).tolist() == g["lo_hi"]
