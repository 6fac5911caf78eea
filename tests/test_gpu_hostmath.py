"""GPU parity: axpy, scalar broadcast and linspace against the oracle
(runtime/axpy.go, runtime/executor_math.go)."""
import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

from gpu_util import empty_dev, log, stream, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def test_axpy_golden(golden):
    g = golden["axpy"]
    for dt in (O.FLOAT32, O.BFLOAT16, O.FLOAT16):
        y = O.encode(np.array(g["y"], np.float32), dt)
        x = O.encode(np.array(g["x"], np.float32), dt)
        yt, yp = to_dev(y)
        xt, xp = to_dev(x)
        M.axpy(yp, xp, 3, g["alpha"], dt, stream())
        M.stream_sync(stream())
        got = O.decode(to_host(yt, y.dtype), dt)
        assert got.tolist() == g["expected"], dt


def test_axpy_config1_full_size():
    # f32, N = 2^24, alpha = 0.75, x, y ~ U[-1, 1].
    rng = np.random.default_rng(0x5EED + 1)
    n = 1 << 24
    x = rng.uniform(-1, 1, n).astype(np.float32)
    y = rng.uniform(-1, 1, n).astype(np.float32)
    log("axpy config 1")
    yt, yp = to_dev(y)
    xt, xp = to_dev(x)
    M.axpy(yp, xp, n, 0.75, O.FLOAT32, stream())
    M.stream_sync(stream())
    got = to_host(yt, np.float32)
    want = O.axpy_f32(y, x, 0.75)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dt", [O.FLOAT32, O.BFLOAT16, O.FLOAT16])
@pytest.mark.parametrize("n, pad", [(1, 0), (7, 0), (4097, 0), (100003, 2), (65536, 1)])
def test_axpy_storage_dtypes_tails(dt, n, pad):
    rng = np.random.default_rng(n * 3 + dt)
    x = O.encode(rng.normal(0, 3, n).astype(np.float32), dt)
    y = O.encode(rng.normal(0, 3, n).astype(np.float32), dt)
    pad_bytes = pad * y.itemsize  # whole elements: breaks 16-byte alignment only
    yt, yp = to_dev(y, pad=pad_bytes)
    xt, xp = to_dev(x, pad=pad_bytes)
    M.axpy(yp, xp, n, -1.3, dt, stream())
    M.stream_sync(stream())
    got = to_host(yt, y.dtype, pad=pad_bytes)
    want = O.axpy_storage(y, x, -1.3, dt)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (dt, n, pad)


def test_axpy_specials_keep_reference_bits():
    vals = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, 3e38, -3e38, 1.0], np.float32)
    x = np.resize(vals, 4096).astype(np.float32)
    y = np.roll(x, 3)
    for dt in (O.FLOAT32, O.BFLOAT16, O.FLOAT16):
        xs, ys = O.encode(x, dt), O.encode(y, dt)
        yt, yp = to_dev(ys)
        xt, xp = to_dev(xs)
        M.axpy(yp, xp, xs.size, 2.5, dt, stream())
        M.stream_sync(stream())
        got = to_host(yt, ys.dtype)
        want = O.axpy_storage(ys, xs, 2.5, dt)
        gb, wb = got.view(np.uint8), want.view(np.uint8)
        if dt == O.FLOAT32:
            nan = np.isnan(want)
            assert np.array_equal(np.isnan(got), nan)
            assert np.array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])
        else:
            g16, w16 = got.view(np.uint16), want.view(np.uint16)
            lim = 0x7F80 if dt == O.BFLOAT16 else 0x7C00
            nan = (w16 & 0x7FFF) > lim
            assert np.array_equal((g16 & 0x7FFF) > lim, nan)
            assert np.array_equal(g16[~nan], w16[~nan]), dt
        del gb, wb


def test_axpy_errors_are_sticky():
    yt, yp = to_dev(np.zeros(8, np.float32))
    M.axpy(yp, yp, 8, 1.0, O.INT32, stream())  # no error channel at the call
    with pytest.raises(M.MFHError, match="is not f32/bf16/f16"):
        M.stream_sync(stream())
    M.stream_sync(stream())  # the sticky error was consumed


def test_linspace_scalar_broadcast_golden(golden):
    g = golden["linspace_scalar_broadcast"]
    ls = g["linspace"]
    sig, sp = empty_dev(16)
    M.linspace(sp, O.FLOAT32, ls["count"], ls["start"], ls["stop"], True, stream())
    ts, tp = empty_dev(16)
    sb = g["scalar_broadcast"]
    M.scalar_broadcast(tp, O.FLOAT32, sp, O.FLOAT32, 4, sb["scalar"], sb["op"], stream())
    s = to_host(sig, np.float32)
    t = to_host(ts, np.float32)
    assert np.array_equal(s, O.linspace(ls["start"], ls["stop"], ls["count"]))
    assert np.array_equal(t, O.scalar_broadcast(s, sb["scalar"], sb["op"]))
    for i, v in g["timesteps"]["exact"]:
        assert t[i] == v


FLOATS = [O.FLOAT32, O.BFLOAT16, O.FLOAT16]


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("in_dt", FLOATS)
@pytest.mark.parametrize("out_dt", FLOATS)
@pytest.mark.parametrize("n, pad_in, pad_out", [(10007, 0, 0), (8, 0, 0), (3, 0, 0), (4099, 2, 0), (4099, 0, 4),
                                                (4104, 8, 0)])
def test_scalar_broadcast_vs_oracle(op, in_dt, out_dt, n, pad_in, pad_out):
    # 16-byte output items where the buffers allow (an f32 source aligned to
    # 16 bytes, a 16-bit one to the item's 8 or 16), the element loop
    # otherwise and for the tail
    rng = np.random.default_rng(5 + n + pad_in)
    src = O.encode(rng.normal(0, 10, n).astype(np.float32), in_dt)
    st, sp = to_dev(src, pad=pad_in)
    size = 4 if out_dt == O.FLOAT32 else 2
    ot, opp = empty_dev(src.size * size, pad=pad_out)
    M.scalar_broadcast(opp, out_dt, sp, in_dt, src.size, 0.37, op, stream())
    got = to_host(ot, np.float32 if out_dt == O.FLOAT32 else np.uint16, pad=pad_out)
    want = O.encode(O.scalar_broadcast(O.decode(src, in_dt), 0.37, op), out_dt)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def test_scalar_broadcast_and_linspace_reject_like_the_executor():
    st, sp = to_dev(np.ones(4, np.float32))
    with pytest.raises(M.MFHError, match="scalar divisor must be nonzero"):
        M.scalar_broadcast(sp, O.FLOAT32, sp, O.FLOAT32, 4, 0.0, "div")
    with pytest.raises(M.MFHError, match="unsupported op"):
        M.scalar_broadcast(sp, O.FLOAT32, sp, O.FLOAT32, 4, 1.0, "pow")
    with pytest.raises(M.MFHError, match="count must be positive"):
        M.linspace(sp, O.FLOAT32, 0, 0.0, 1.0)


@pytest.mark.parametrize("count, endpoint", [(1, True), (2, True), (11, True), (4, False), (100000, True),
                                             (16777217, True)])
def test_linspace_vs_oracle(count, endpoint):
    ot, opp = empty_dev(count * 4)
    M.linspace(opp, O.FLOAT32, count, -0.0, 7.25, endpoint, stream())
    got = to_host(ot, np.float32)
    want = O.linspace(-0.0, 7.25, count, endpoint)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dt", FLOATS)
@pytest.mark.parametrize("count, pad", [(9, 0), (100003, 0), (100003, 2), (16, 4)])
def test_linspace_every_dtype_and_alignment(dt, count, pad):
    size = 4 if dt == O.FLOAT32 else 2
    ot, opp = empty_dev(count * size, pad=pad)
    M.linspace(opp, dt, count, -3.5, 11.0, True, stream())
    got = to_host(ot, np.float32 if dt == O.FLOAT32 else np.uint16, pad=pad)
    want = O.encode(O.linspace(-3.5, 11.0, count, True), dt)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
