"""GPU parity: FP8 / Int4 dequantisation and dtype conversion, bit-exact
against the CPU oracle (dtype/fp8.go, dtype/int4.go, dtype/convert/*.go)."""
import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

from gpu_util import (compare_storage, empty_dev, log, stream, to_dev, to_host)

pytestmark = pytest.mark.gpu

OUT_NP = {O.FLOAT32: np.float32, O.BFLOAT16: np.uint16, O.FLOAT16: np.uint16}
OUT_SIZE = {O.FLOAT32: 4, O.BFLOAT16: 2, O.FLOAT16: 2}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def bits_equal(got, want, what):
    g = got.view(np.uint32 if got.dtype == np.float32 else got.dtype)
    w = want.view(np.uint32 if want.dtype == np.float32 else want.dtype)
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:4]}: got {g[bad[:4]]} want {w[bad[:4]]}"


FP8_SCALES = [1.0, 0.0125, -3.5, 2.0 ** -140, 1e30, 0.0, -0.0, np.inf, -np.inf, np.nan]


@pytest.mark.parametrize("fmt", [O.F8E4M3, O.F8E5M2])
@pytest.mark.parametrize("out_dt", [O.BFLOAT16, O.FLOAT32, O.FLOAT16])
def test_fp8_every_code_every_scale(fmt, out_dt):
    codes = np.tile(np.arange(256, dtype=np.uint8), 17)[: 4096 + 13]
    for scale in FP8_SCALES:
        log(f"fp8 fmt={fmt} out={out_dt} scale={scale}")
        scale32 = float(np.float32(scale))
        src, sp = to_dev(codes)
        out, op = empty_dev(codes.size * OUT_SIZE[out_dt])
        M.dequant_fp8(op, out_dt, sp, fmt, codes.size, scale32, stream())
        got = to_host(out, OUT_NP[out_dt])
        want = O.dequant_fp8(codes, fmt, scale32, out_dt)
        bits_equal(got, want, f"fp8 fmt={fmt} out={out_dt} scale={scale}")


def test_fp8_config2_full_size():
    # e4m3 [4096, 14336], every code, scale 0.0125 -> bf16.
    rng = np.random.default_rng(0x5EED + 2)
    codes = rng.integers(0, 256, size=4096 * 14336, dtype=np.uint8)
    log("fp8 config 2 full size")
    src, sp = to_dev(codes)
    out, op = empty_dev(codes.size * 2)
    M.dequant_fp8(op, O.BFLOAT16, sp, O.F8E4M3, codes.size, 0.0125, stream())
    got = to_host(out, np.uint16)
    table = O.dequant_fp8(np.arange(256, dtype=np.uint8), O.F8E4M3, 0.0125, O.BFLOAT16)
    bits_equal(got, table[codes], "config 2 vs per-code table")
    head = O.dequant_fp8(codes[: 1 << 20], O.F8E4M3, 0.0125, O.BFLOAT16)
    bits_equal(got[: 1 << 20], head, "config 2 head vs oracle")
    assert table[0x7F] == 0x7FC0 and table[0xFF] == 0xFFC0 and table[0] == 0 and table[0x80] == 0x8000


@pytest.mark.parametrize("pad", [0, 1, 3])
@pytest.mark.parametrize("n", [1, 15, 16, 17, 4095, 100003])
def test_fp8_tails_and_misaligned(pad, n):
    rng = np.random.default_rng(n + pad)
    codes = rng.integers(0, 256, size=n, dtype=np.uint8)
    src, sp = to_dev(codes, pad=pad)
    out, op = empty_dev(n * 2, pad=2 * pad)
    M.dequant_fp8(op, O.BFLOAT16, sp, O.F8E5M2, n, -0.75, stream())
    got = to_host(out, np.uint16, pad=2 * pad)
    bits_equal(got, O.dequant_fp8(codes, O.F8E5M2, -0.75, O.BFLOAT16), f"n={n} pad={pad}")


def int4_case(n, group, scale_dt, out_dt, scales_f32, rng, pad=0):
    packed = rng.integers(0, 256, size=(n + 1) // 2, dtype=np.uint8)
    ngroups = (n + group - 1) // group
    s = scales_f32[:ngroups]
    if scale_dt == O.FLOAT16:
        s_store = O.f32_to_f16(s)
    elif scale_dt == O.BFLOAT16:
        s_store = O.f32_to_bf16(s)
    else:
        s_store = s.astype(np.float32)
    src, pp = to_dev(packed, pad=pad)
    sc, scp = to_dev(s_store)
    out, op = empty_dev(n * OUT_SIZE[out_dt], pad=pad * OUT_SIZE[out_dt])
    M.dequant_int4(op, out_dt, pp, n, scp, scale_dt, group, stream())
    got = to_host(out, OUT_NP[out_dt], pad=pad * OUT_SIZE[out_dt])
    want = O.dequant_int4(packed, n, s_store, scale_dt, group, out_dt)
    bits_equal(got, want, f"int4 n={n} group={group} sdt={scale_dt} out={out_dt} pad={pad}")


@pytest.mark.parametrize("group", [128, 32, 64, 7, 1, 4096])
@pytest.mark.parametrize("scale_dt", [O.FLOAT16, O.FLOAT32, O.BFLOAT16])
@pytest.mark.parametrize("out_dt", [O.BFLOAT16, O.FLOAT32, O.FLOAT16])
def test_int4_groups_and_dtypes(group, scale_dt, out_dt):
    rng = np.random.default_rng(group * 31 + scale_dt * 7 + out_dt)
    n = 32 * 1024 + 7
    scales = rng.uniform(-0.05, 0.05, size=n // group + 2).astype(np.float32)
    log(f"int4 group={group} sdt={scale_dt} out={out_dt}")
    int4_case(n, group, scale_dt, out_dt, scales, rng)


@pytest.mark.parametrize("group, n", [(8192, 5 * 8192 + 4099), (1 << 21, 3 * (1 << 21) + 4099),
                                      (1 << 22, (1 << 23) + 8), (1 << 23, (1 << 23) - 24)])
def test_int4_groups_larger_than_a_chunk(group, n):
    # A workgroup's chunk spans 4096 elements (bf16 out), so these groups
    # start mid-chunk (8192) or take the large-group form of the scale index
    # (past 2^20 elements), with partial last groups.
    rng = np.random.default_rng(group + n)
    scales = rng.uniform(-0.05, 0.05, size=n // group + 2).astype(np.float32)
    log(f"int4 group={group} n={n}")
    for out_dt in (O.BFLOAT16, O.FLOAT32):
        int4_case(n, group, O.FLOAT16, out_dt, scales, rng)


def test_int4_every_nibble_and_special_scales():
    rng = np.random.default_rng(11)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 6e-8, 65504.0, -1.5, 1e-45, 3e38],
                        dtype=np.float32)
    for out_dt in (O.BFLOAT16, O.FLOAT32, O.FLOAT16):
        for scale_dt in (O.FLOAT32, O.FLOAT16):
            packed = np.tile(np.arange(256, dtype=np.uint8), 20)
            n = packed.size * 2
            group = 512
            scales = np.resize(specials, n // group)
            s_store = O.f32_to_f16(scales) if scale_dt == O.FLOAT16 else scales
            src, pp = to_dev(packed)
            sc, scp = to_dev(s_store)
            out, op = empty_dev(n * OUT_SIZE[out_dt])
            M.dequant_int4(op, out_dt, pp, n, scp, scale_dt, group, stream())
            got = to_host(out, OUT_NP[out_dt])
            bits_equal(got, O.dequant_int4(packed, n, s_store, scale_dt, group, out_dt),
                       f"int4 specials out={out_dt} sdt={scale_dt}")


@pytest.mark.parametrize("pad", [1, 2])
def test_int4_misaligned_odd(pad):
    rng = np.random.default_rng(pad)
    int4_case(4097, 128, O.FLOAT16, O.BFLOAT16, rng.uniform(0.005, 0.02, 64).astype(np.float32), rng, pad=pad)


def test_int4_config5_full_size():
    # [14336, 4096] nibbles, f16 scale per 128, U[0.005, 0.02] -> bf16.
    rng = np.random.default_rng(0x5EED + 5)
    n = 14336 * 4096
    log("int4 config 5 full size")
    scales = rng.uniform(0.005, 0.02, size=n // 128).astype(np.float32)
    int4_case(n, 128, O.FLOAT16, O.BFLOAT16, scales, rng)


def test_int4_golden_pairs(golden):
    # convert_test.go:56-67: pairs (1,-2), (-8,7) -> [1,-2,-8,7] (scale 1 via mfh_convert).
    packed = np.array([0xE1, 0x78], dtype=np.uint8)
    src, sp = to_dev(packed)
    out, op = empty_dev(16)
    M.convert(op, O.FLOAT32, sp, O.INT4, 4, stream())
    assert to_host(out, np.float32).tolist() == [1.0, -2.0, -8.0, 7.0]


@pytest.mark.parametrize("in_dt", [O.BFLOAT16, O.FLOAT16])
@pytest.mark.parametrize("out_dt", [O.FLOAT32, O.BFLOAT16, O.FLOAT16])
def test_convert_every_16bit_code(in_dt, out_dt):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    src, sp = to_dev(codes)
    out, op = empty_dev(codes.size * OUT_SIZE[out_dt])
    M.convert(op, out_dt, sp, in_dt, codes.size, stream())
    got = to_host(out, OUT_NP[out_dt])
    conv = {O.FLOAT32: O.bytes_to_f32, O.BFLOAT16: O.bytes_to_bf16, O.FLOAT16: O.bytes_to_f16}[out_dt]
    bits_equal(got, conv(in_dt, codes), f"convert {in_dt}->{out_dt}")


def f32_probe(rng):
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1000, 0x0FFF, 0x2000, 0x3000], dtype=np.uint32)
    grid = (hi[:, None] | lows[None, :]).reshape(-1)
    rand = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([grid, rand]).view(np.float32)


@pytest.mark.parametrize("out_dt", [O.BFLOAT16, O.FLOAT16])
def test_convert_f32_narrowing_every_input(out_dt):
    # All 2^32 f32 bit patterns through mfh_convert (the gfx950 conversion
    # instructions it uses must reproduce the Go rules everywhere: NaN
    # payloads, ties, denormals, overflow).
    import concurrent.futures as cf
    torch = __import__("torch")
    chunk = 1 << 28
    narrow = O.f32_to_bf16 if out_dt == O.BFLOAT16 else O.f32_to_f16
    src = torch.empty(chunk, dtype=torch.int32, device="cuda")
    out = torch.empty(chunk, dtype=torch.int16, device="cuda")
    for start in range(0, 1 << 32, chunk):
        host = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32)
        src.copy_(torch.from_numpy(host.view(np.int32)))
        M.convert(out.data_ptr(), out_dt, src.data_ptr(), O.FLOAT32, chunk, stream())
        got = out.cpu().numpy().view(np.uint16)
        x = host.view(np.float32)
        parts = np.array_split(np.arange(chunk), 16)
        with cf.ThreadPoolExecutor(16) as ex:
            want = np.concatenate(list(ex.map(lambda ix: narrow(x[ix[0]:ix[-1] + 1]), parts)))
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"f32->{out_dt}: input {host[bad[0]]:#010x} gave {got[bad[0]]:#06x}, want {want[bad[0]]:#06x}"
        log(f"f32->{out_dt}: inputs {start:#x}.. ok")


@pytest.mark.parametrize("out_dt", [O.BFLOAT16, O.FLOAT16])
def test_convert_f32_narrowing_rounding_classes(out_dt):
    # Every sign/exponent/top-mantissa pattern with the low bits at each
    # rounding class (ties, just above/below, NaN payloads, subnormals).
    x = f32_probe(np.random.default_rng(3))
    for pad in (0, 4):
        src, sp = to_dev(x, pad=pad)
        out, op = empty_dev(x.size * 2, pad=pad)
        M.convert(op, out_dt, sp, O.FLOAT32, x.size - (pad // 4), stream())
        got = to_host(out, np.uint16, pad=pad)[: x.size - (pad // 4)]
        want = (O.f32_to_bf16 if out_dt == O.BFLOAT16 else O.f32_to_f16)(x[: x.size - (pad // 4)])
        bits_equal(got, want, f"f32->{out_dt} pad={pad}")


@pytest.mark.parametrize("in_dt, np_dt", [
    (O.FLOAT64, np.float64), (O.FLOAT32, np.float32), (O.INT8, np.int8), (O.INT16, np.int16),
    (O.INT32, np.int32), (O.INT64, np.int64), (O.UINT8, np.uint8), (O.UINT16, np.uint16),
    (O.UINT32, np.uint32), (O.UINT64, np.uint64)])
@pytest.mark.parametrize("out_dt", [O.FLOAT32, O.BFLOAT16, O.FLOAT16])
@pytest.mark.parametrize("n, pad", [(50001, 0), (50001, 1), (7, 0), (3, 0)])
def test_convert_other_numeric_dtypes(in_dt, np_dt, out_dt, n, pad):
    # aligned sources take whole 16-byte output items plus an element tail;
    # a source one byte off its alignment runs the element loop
    rng = np.random.default_rng(in_dt * 7 + n)
    raw = rng.integers(0, 256, size=8 * n, dtype=np.uint8)
    a = raw.view(np_dt)[:n]
    if in_dt == O.FLOAT64 and n > 10:
        a = np.concatenate([a, np.array([np.nan, -np.inf, 1e300, -1e-320, 0.1], dtype=np.float64)])
    if in_dt == O.FLOAT32 and n > 10:  # NaN payloads and denormals pass through unchanged
        a = np.concatenate([a, np.array([0x7FC00001, 0xFF800000, 0x00000001, 0x80000000], np.uint32).view(np.float32)])
    src, sp = to_dev(a, pad=pad)
    out, op = empty_dev(a.size * OUT_SIZE[out_dt])
    M.convert(op, out_dt, sp, in_dt, a.size, stream())
    got = to_host(out, OUT_NP[out_dt])
    conv = {O.FLOAT32: O.bytes_to_f32, O.BFLOAT16: O.bytes_to_bf16, O.FLOAT16: O.bytes_to_f16}[out_dt]
    bits_equal(got, conv(in_dt, a), f"convert {in_dt}->{out_dt} n={n} pad={pad}")


@pytest.mark.parametrize("fmt", [O.F8E4M3, O.F8E5M2])
def test_convert_fp8_is_bytes_to_bfloat16(fmt):
    codes = np.arange(256, dtype=np.uint8)
    src, sp = to_dev(codes)
    out, op = empty_dev(512)
    M.convert(op, O.BFLOAT16, sp, fmt, 256, stream())
    bits_equal(to_host(out, np.uint16), O.bytes_to_bf16(fmt, codes), f"BytesToBFloat16({fmt})")


def test_dequant_rejects_bad_arguments():
    src, sp = to_dev(np.zeros(64, np.uint8))
    out, op = empty_dev(256)
    with pytest.raises(M.MFHError, match="not an FP8 dtype"):
        M.dequant_fp8(op, O.BFLOAT16, sp, O.INT8, 64, 1.0)
    with pytest.raises(M.MFHError, match="not f32/bf16/f16"):
        M.dequant_fp8(op, O.INT8, sp, O.F8E4M3, 64, 1.0)
    with pytest.raises(M.MFHError, match="group must be positive"):
        M.dequant_int4(op, O.BFLOAT16, sp, 64, sp, O.FLOAT16, 0)
    M.dequant_fp8(op, O.BFLOAT16, sp, O.F8E4M3, 0, 1.0)  # empty input is a no-op
