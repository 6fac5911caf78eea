"""GPU parity of FP8 encoding (mfh_convert to Float8E4M3 / Float8E5M2) against
the oracle's restatement of BytesToFloat8E4M3 / BytesToFloat8E5M2
(dtype/convert/convert.go:194-232, dtype/fp8.go:77-136,190-249): bit-exact on
every f32 bit pattern, every 16-bit code, every FP8 code of the other format,
every Int4 nibble and the other numeric dtypes, with tails and unaligned
buffers.
"""
import concurrent.futures as cf

import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

from gpu_util import empty_dev, log, stream, to_dev, to_host

pytestmark = pytest.mark.gpu

FMTS = [O.F8E4M3, O.F8E5M2]


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def encode_dev(values, in_dt, fmt, count=None, pad=0, out_pad=0):
    count = values.size if count is None else count
    src, sp = to_dev(values, pad=pad)
    out, op = empty_dev(count, pad=out_pad)
    M.convert(op, fmt, sp, in_dt, count, stream())
    return to_host(out, np.uint8, pad=out_pad)[:count]


def check(got, want, what, inputs=None):
    bad = np.flatnonzero(got != want)
    if bad.size:
        i = bad[0]
        src = f" input {inputs[i]!r}" if inputs is not None else ""
        raise AssertionError(f"{what}: {bad.size} mismatches, first at {i}:{src} got {got[i]:#04x} want {want[i]:#04x}")


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_every_f32_input(fmt):
    torch = __import__("torch")
    chunk = 1 << 28
    src = torch.empty(chunk, dtype=torch.int32, device="cuda")
    out = torch.empty(chunk, dtype=torch.uint8, device="cuda")
    for start in range(0, 1 << 32, chunk):
        host = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32)
        src.copy_(torch.from_numpy(host.view(np.int32)))
        M.convert(out.data_ptr(), fmt, src.data_ptr(), O.FLOAT32, chunk, stream())
        got = out.cpu().numpy()
        x = host.view(np.float32)
        parts = np.array_split(np.arange(chunk), 16)
        with cf.ThreadPoolExecutor(16) as ex:
            want = np.concatenate(list(ex.map(lambda ix: O.f32_to_fp8(x[ix[0]:ix[-1] + 1], fmt), parts)))
        check(got, want, f"f32->fmt{fmt} from {start:#x}", host)
        log(f"f32->fmt{fmt}: inputs {start:#x}.. ok")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("in_dt", [O.BFLOAT16, O.FLOAT16])
def test_encode_every_16bit_code(fmt, in_dt):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = encode_dev(codes, in_dt, fmt)
    want = O.f32_to_fp8(O.bytes_to_f32(in_dt, codes), fmt)
    check(got, want, f"{in_dt}->fmt{fmt}", codes)


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_fp8_and_int4_sources(fmt):
    codes = np.arange(256, dtype=np.uint8)
    for src_fmt in FMTS:
        got = encode_dev(codes, src_fmt, fmt)
        want = O.f32_to_fp8(O.bytes_to_f32(src_fmt, codes), fmt)
        check(got, want, f"fmt{src_fmt}->fmt{fmt}", codes)
    # Int4: every byte, both nibbles, and an odd count (the last byte's low
    # nibble only)
    got = encode_dev(codes, O.INT4, fmt, count=511)
    want = O.f32_to_fp8(O.bytes_to_f32(O.INT4, codes)[:511], fmt)
    check(got, want, f"int4->fmt{fmt}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("in_dt, np_dt", [
    (O.FLOAT64, np.float64), (O.INT8, np.int8), (O.INT16, np.int16), (O.INT32, np.int32), (O.INT64, np.int64),
    (O.UINT8, np.uint8), (O.UINT16, np.uint16), (O.UINT32, np.uint32), (O.UINT64, np.uint64)])
def test_encode_other_numeric_sources(fmt, in_dt, np_dt):
    rng = np.random.default_rng(in_dt * 10 + fmt)
    if np_dt == np.float64:
        x = np.concatenate([rng.normal(0, 100, 3000), rng.normal(0, 1e-3, 3000), np.exp(rng.uniform(-40, 40, 3000)),
                            [0.0, -0.0, np.inf, -np.inf, np.nan, 448.0, 447.9999, 448.0001, 57344.0, 1e300, -1e-300]])
        x = x.astype(np.float64)
    else:
        info = np.iinfo(np_dt)
        x = np.concatenate([rng.integers(info.min, info.max, 9000, dtype=np_dt, endpoint=True),
                            np.array([info.min, info.max, 0, 1], dtype=np_dt)])
    got = encode_dev(x, in_dt, fmt)
    want = O.f32_to_fp8(O.bytes_to_f32(in_dt, x), fmt)
    check(got, want, f"{np_dt.__name__}->fmt{fmt}", x)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("in_dt", [O.FLOAT32, O.BFLOAT16])
@pytest.mark.parametrize("n, pad, out_pad", [(1, 0, 0), (15, 0, 0), (16, 0, 0), (17, 0, 0), (1000003, 0, 0),
                                             (4096, 2, 1), (4097, 0, 3), (40000, 0, 8)])
def test_encode_tails_and_misaligned(fmt, in_dt, n, pad, out_pad):
    rng = np.random.default_rng(n)
    v = (rng.normal(0, 64, n) * np.exp(rng.uniform(-8, 4, n))).astype(np.float32)
    x = v if in_dt == O.FLOAT32 else O.f32_to_bf16(v)
    elem = 4 if in_dt == O.FLOAT32 else 2
    got = encode_dev(x, in_dt, fmt, pad=pad * elem, out_pad=out_pad)
    want = O.f32_to_fp8(O.bytes_to_f32(in_dt, x), fmt)
    check(got, want, f"n={n} pad={pad} out_pad={out_pad}")
