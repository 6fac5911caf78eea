"""GPU parity tests past 32-bit element counts.

Every kernel family indexes with 64-bit integers; these tests run one member
of each at a size past 2^31 elements (Int4 past 2^32 nibbles), with a ragged
tail, so that an offset or a grid computed in 32 bits would corrupt or skip
data.  The inputs are generated on the device and the results are checked on
the device in chunks:
  * FP8: the output of each element depends only on its code, so the oracle
    computes the 256-entry table and every output must equal table[code];
  * Int4, axpy and the arithmetic fused chain: the expected values are exact
    IEEE f32 operations (an exact int4 * f16-scale product, an unfused
    multiply then add, Mul then Add) followed by round-to-nearest-even to
    bf16, computed with torch's f32 arithmetic and its f32 -> bf16 cast (the
    CPU tests pin that cast against the oracle's bf16 rule).
"""
import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

from gpu_util import log, stream

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28


@pytest.fixture(scope="module")
def torch():
    import torch as t
    M.init(0)
    if t.cuda.get_device_properties(0).total_memory < (96 << 30):
        pytest.skip("needs a device with at least 96 GiB")
    yield t
    t.cuda.empty_cache()


def chunks(n):
    for lo in range(0, n, CHUNK):
        yield lo, min(n, lo + CHUNK)


def test_fp8_past_2_31(torch):
    n = (1 << 31) + 4099
    log(f"fp8 e4m3 -> bf16, n = {n}")
    g = torch.Generator(device="cuda").manual_seed(31)
    codes = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
    out = torch.empty(n, dtype=torch.int16, device="cuda")
    M.dequant_fp8(out.data_ptr(), M.BFLOAT16, codes.data_ptr(), M.F8E4M3, n, 0.0125, stream())
    table = O.dequant_fp8(np.arange(256, dtype=np.uint8), O.F8E4M3, 0.0125, O.BFLOAT16)
    table = torch.from_numpy(table.view(np.int16).copy()).cuda()
    for lo, hi in chunks(n):
        want = torch.index_select(table, 0, codes[lo:hi].int())
        assert torch.equal(out[lo:hi], want), f"fp8 mismatch in [{lo}, {hi})"


def test_int4_past_2_32(torch):
    n, group = (1 << 32) + 262, 128  # the last group is partial
    nbytes, ngroups = (n + 1) // 2, -(-n // group)
    log(f"int4 -> bf16, n = {n} nibbles, group {group}")
    g = torch.Generator(device="cuda").manual_seed(32)
    packed = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=g)
    scales = (torch.rand(ngroups, device="cuda", generator=g) * 0.015 + 0.005).to(torch.float16)
    out = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    M.dequant_int4(out.data_ptr(), M.BFLOAT16, packed.data_ptr(), n, scales.data_ptr(), M.FLOAT16, group,
                   stream())
    for lo, hi in chunks(n):  # CHUNK is a multiple of the group and of 2
        b = packed[lo // 2:(hi + 1) // 2].to(torch.int16)
        nib = torch.stack([b & 15, b >> 4], dim=1).reshape(-1)[:hi - lo]
        q = (nib - 16 * (nib >= 8).to(torch.int16)).float()
        s = scales[lo // group:-(-hi // group)].float().repeat_interleave(group)[:hi - lo]
        want = (q * s).to(torch.bfloat16)
        assert torch.equal(out[lo:hi].view(torch.int16), want.view(torch.int16)), f"int4 mismatch in [{lo}, {hi})"


def test_axpy_past_2_31(torch):
    n = (1 << 31) + 3
    log(f"axpy f32, n = {n}")
    g = torch.Generator(device="cuda").manual_seed(33)
    x = torch.rand(n, device="cuda", generator=g) * 2 - 1
    y = torch.rand(n, device="cuda", generator=g) * 2 - 1
    y0 = y.clone()
    M.axpy(y.data_ptr(), x.data_ptr(), n, 0.75, M.FLOAT32, stream())
    for lo, hi in chunks(n):
        product = x[lo:hi] * 0.75  # rounded, then the add: no contraction
        want = y0[lo:hi] + product
        assert torch.equal(y[lo:hi].view(torch.int32), want.view(torch.int32)), f"axpy mismatch in [{lo}, {hi})"


def test_fused_chain_past_2_31(torch):
    n = (1 << 31) + 5
    log(f"fused Add(Mul(in0, in1), in2) bf16, n = {n}")
    nodes = O.flatten((O.N_ADD, (O.N_MUL, ("in", 0), ("in", 1)), ("in", 2)))
    k = M.FusedKernel(nodes, [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 3, M.BFLOAT16, "large_chain")
    g = torch.Generator(device="cuda").manual_seed(34)
    a, b, c = (torch.randn(n, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    out = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    k.launch([a.data_ptr(), b.data_ptr(), c.data_ptr()], out.data_ptr(), n, stream())
    for lo, hi in chunks(n):
        product = a[lo:hi].float() * b[lo:hi].float()
        want = (product + c[lo:hi].float()).to(torch.bfloat16)
        assert torch.equal(out[lo:hi].view(torch.int16), want.view(torch.int16)), f"chain mismatch in [{lo}, {hi})"


def test_int4_encode_round_trip_past_2_31(torch):
    # int8 -> Int4 (int4Encode's clamp) -> int8 again over an odd count past
    # 2^31: the round trip must give every value clamped to [-8, 7] and the
    # last byte's high nibble must stay 0
    n = (1 << 31) + 7
    log(f"int8 -> int4 -> int8, n = {n}")
    g = torch.Generator(device="cuda").manual_seed(35)
    v = torch.randint(-128, 128, (n,), dtype=torch.int8, device="cuda", generator=g)
    packed = torch.empty((n + 1) // 2, dtype=torch.uint8, device="cuda")
    back = torch.empty(n, dtype=torch.int8, device="cuda")
    M.convert(packed.data_ptr(), M.INT4, v.data_ptr(), M.INT8, n, stream())
    M.convert(back.data_ptr(), M.INT8, packed.data_ptr(), M.INT4, n, stream())
    for lo, hi in chunks(n):
        want = torch.clamp(v[lo:hi], -8, 7)
        assert torch.equal(back[lo:hi], want), f"int4 round trip mismatch in [{lo}, {hi})"
    assert int(packed[-1]) >> 4 == 0


@pytest.mark.parametrize("in_dt", [M.BFLOAT16, M.FLOAT64, M.INT8])
def test_casts_to_f32_past_2_31(torch, in_dt):
    # bf16 -> f32 (k_convert16_vec), f64 -> f32 (k_narrow_f64_vec) and
    # int8 -> f32 (k_convert_vec, two items per thread) over an odd count past
    # 2^31: each is exact or one IEEE rounding (f64 -> f32 of finite values is
    # round-to-nearest-even, which torch's cast also does)
    n = (1 << 31) + 5
    log(f"cast {in_dt} -> f32, n = {n}")
    g = torch.Generator(device="cuda").manual_seed(36 + in_dt)
    if in_dt == M.INT8:
        src = torch.randint(-128, 128, (n,), dtype=torch.int8, device="cuda", generator=g)
    else:
        tdt = torch.bfloat16 if in_dt == M.BFLOAT16 else torch.float64
        src = torch.randn(n, dtype=torch.float32, device="cuda", generator=g).to(tdt)
        if in_dt == M.FLOAT64:
            src.mul_(1.0 + 2.0 ** -30)  # bits below f32 precision, so the narrowing rounds
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    M.convert(out.data_ptr(), M.FLOAT32, src.data_ptr(), in_dt, n, stream())
    for lo, hi in chunks(n):
        want = src[lo:hi].float()
        assert torch.equal(out[lo:hi].view(torch.int32), want.view(torch.int32)), f"{in_dt} mismatch in [{lo}, {hi})"
    del src, out
    torch.cuda.empty_cache()
