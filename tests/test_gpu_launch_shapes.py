"""GPU tests of launch shapes: every streaming kernel family gives the same
bits under small capped grids (one workgroup per CU, so each workgroup walks
many chunks, with 1, 2 and 4 items per thread) as under its default one-shot
grid, at sizes with ragged tails and on unaligned buffers, at every
workgroup size the family runs (FP8, axpy and the casts 64, 128 and 256
threads; Int4 also 512; generated kernels also 1024).  The default shape
itself is pinned against the oracle here and in the per-family test files."""
import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

from gpu_util import empty_dev, log, stream, to_dev, to_host

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (1, 2), (1, 4), (3, 2), (-1, -1)]  # (workgroups per CU, items per thread); -1: default
# workgroup sizes each ahead-of-time family runs besides its default
THREADS = {"fp8": (64, 128, 256), "int4": (64, 128, 256, 512), "axpy": (64, 128, 256), "axpy16": (64, 128, 256),
           "convert": (64, 128, 256)}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)
    yield
    for fam in ("fp8", "int4", "axpy", "axpy16", "convert", "fused"):
        M.set_launch_config(fam, -1, -1)
        M.set_launch_threads(fam, -1)


def under_shapes(family, run):
    """Runs `run()` (which returns host bytes) under every shape of SHAPES, at
    every workgroup size of THREADS, and checks that all results equal the
    default shape's."""
    M.set_launch_config(family, -1, -1)
    M.set_launch_threads(family, -1)
    want = run()
    try:
        for threads in THREADS.get(family, (-1,)):
            M.set_launch_threads(family, threads)
            for bpc, u in SHAPES:
                M.set_launch_config(family, bpc, u)
                got = run()
                assert got == want, f"{family}: launch shape ({bpc}, {u}) at {threads} threads changed the result"
    finally:
        M.set_launch_config(family, -1, -1)
        M.set_launch_threads(family, -1)
    return want


@pytest.mark.parametrize("out_dt", [M.BFLOAT16, M.FLOAT32])
@pytest.mark.parametrize("offset", [0, 1])
def test_fp8_shapes(out_dt, offset):
    n = 3 * (1 << 20) + 13
    log(f"fp8 shapes out={out_dt} offset={offset} n={n}")
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, n, dtype=np.uint8)
    t, p = to_dev(codes, pad=offset)
    size = 2 if out_dt == M.BFLOAT16 else 4
    o, po = empty_dev(n * size)

    def run():
        M.dequant_fp8(po, out_dt, p, M.F8E4M3, n, 0.0125, stream())
        return to_host(o, np.uint8).tobytes()

    got = under_shapes("fp8", run)
    want = O.dequant_fp8(codes, O.F8E4M3, 0.0125, out_dt)
    assert got == np.ascontiguousarray(want).tobytes()


@pytest.mark.parametrize("offset", [0, 2])
def test_int4_shapes(offset):
    n, group = (1 << 21) + 6, 128
    log(f"int4 shapes offset={offset} n={n}")
    rng = np.random.default_rng(6)
    packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    scales = O.f32_to_f16(rng.uniform(0.005, 0.02, -(-n // group)).astype(np.float32))
    tp, pp = to_dev(packed, pad=offset)
    ts, ps = to_dev(scales)
    o, po = empty_dev(n * 2)

    def run():
        M.dequant_int4(po, M.BFLOAT16, pp, n, ps, M.FLOAT16, group, stream())
        return to_host(o, np.uint8).tobytes()

    got = under_shapes("int4", run)
    want = O.dequant_int4(packed, n, scales, O.FLOAT16, group, O.BFLOAT16)
    assert got == np.ascontiguousarray(want).tobytes()


@pytest.mark.parametrize("dt, family", [(M.FLOAT32, "axpy"), (M.BFLOAT16, "axpy16")])
def test_axpy_shapes(dt, family):
    n = (1 << 20) + 7
    log(f"axpy shapes dt={dt} n={n}")
    rng = np.random.default_rng(7)
    x = rng.uniform(-1, 1, n).astype(np.float32)
    y = rng.uniform(-1, 1, n).astype(np.float32)
    if dt == M.BFLOAT16:
        x, y = O.f32_to_bf16(x), O.f32_to_bf16(y)
    tx, px = to_dev(x)
    ty, py = to_dev(y)

    def run():
        ty.copy_(to_dev(y)[0])  # axpy is in place: start from the same y
        M.axpy(py, px, n, 0.75, dt, stream())
        return to_host(ty, np.uint8).tobytes()

    under_shapes(family, run)


@pytest.mark.parametrize("src_dt, out_dt", [(M.BFLOAT16, M.FLOAT32), (M.FLOAT32, M.BFLOAT16),
                                            (M.FLOAT16, M.BFLOAT16), (M.FLOAT32, M.F8E4M3)])
def test_convert_shapes(src_dt, out_dt):
    n = (1 << 20) + 21
    log(f"convert shapes {src_dt}->{out_dt} n={n}")
    rng = np.random.default_rng(8)
    f = rng.normal(0, 4, n).astype(np.float32)
    src = {M.FLOAT32: f, M.BFLOAT16: O.f32_to_bf16(f), M.FLOAT16: O.f32_to_f16(f)}[src_dt]
    ts, ps = to_dev(src)
    size = {M.FLOAT32: 4, M.BFLOAT16: 2, M.FLOAT16: 2, M.F8E4M3: 1}[out_dt]
    o, po = empty_dev(n * size)

    def run():
        M.convert(po, out_dt, ps, src_dt, n, stream())
        return to_host(o, np.uint8).tobytes()

    under_shapes("convert", run)


def test_fused_shapes():
    # SwiGLU-shaped chain: Mul(Silu(In0), In1) in bf16, and the f16 gelu chain
    # with a periodic bias and a scalar, compiled under each items-per-thread
    from test_abi import flatten, swiglu_nodes, N_ADD, N_GELU, N_MUL
    n = (1 << 20) + 9
    log(f"fused shapes n={n}")
    rng = np.random.default_rng(9)
    a = O.f32_to_bf16(rng.normal(0, 1, n).astype(np.float32))
    b = O.f32_to_bf16(rng.normal(0, 1, n).astype(np.float32))
    ta, pa = to_dev(a)
    tb, pb = to_dev(b)
    o, po = empty_dev(n * 2)
    chain = flatten((N_ADD, (N_GELU, (N_MUL, (N_ADD, ("in", 0), ("in", 1)), ("in", 2))), ("in", 3)))
    rows = 4096
    x = O.f32_to_f16(rng.normal(0, 1, rows * 257).astype(np.float32))
    bias = O.f32_to_f16(rng.normal(0, 0.02, rows).astype(np.float32))
    s = np.array([1.1], np.float32)
    res = O.f32_to_f16(rng.normal(0, 1, x.size).astype(np.float32))
    tx, px = to_dev(x)
    tbias, pbias = to_dev(bias)
    tsc, psc = to_dev(s)
    tr, pr = to_dev(res)
    o2, po2 = empty_dev(x.size * 2)
    ops = [(M.FLOAT16, M.OPERAND_FULL, 0), (M.FLOAT16, M.OPERAND_PERIODIC, rows),
           (M.FLOAT32, M.OPERAND_SCALAR, 0), (M.FLOAT16, M.OPERAND_FULL, 0)]

    def run():
        k1 = M.FusedKernel(swiglu_nodes(), [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, "swiglu_shape")
        k1.launch([pa, pb], po, n, stream())
        k2 = M.FusedKernel(chain, ops, M.FLOAT16, "gelu_shape")
        k2.launch([px, pbias, psc, pr], po2, x.size, stream())
        return to_host(o, np.uint8).tobytes() + to_host(o2, np.uint8).tobytes()

    want = under_shapes("fused", run)
    # workgroup sizes other than the default one wave, one-shot and capped
    try:
        for threads in (128, 256, 1024):
            M.set_launch_threads("fused", threads)
            for bpc, u in ((-1, -1), (1, 2)):
                M.set_launch_config("fused", bpc, u)
                assert run() == want, f"fused: {threads} threads, shape ({bpc}, {u}) changed the result"
    finally:
        M.set_launch_threads("fused", -1)
        M.set_launch_config("fused", -1, -1)
