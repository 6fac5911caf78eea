"""GPU tests of empty inputs: every entry point with a count of 0 returns
MFH_OK and writes nothing (NULL buffers included, as a zero-length copy
allows), except where the reference rejects the call itself: linspace's
count must be positive (runtime/executor_math.go:79-81) and scalar
broadcast checks its op and divisor before it looks at the data
(runtime/executor_math.go:195-234)."""
import numpy as np
import pytest

import manifesto_amd as M
import oracle as O
from manifesto_amd.backend import Backend
from manifesto_amd.graph import Graph, GraphNode

from gpu_util import empty_dev, stream, to_host, torch_mod

pytestmark = pytest.mark.gpu

SENTINEL = np.full(64, 0xA5, np.uint8)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    M.init(0)


def untouched(t):
    assert np.array_equal(to_host(t, np.uint8), SENTINEL)


@pytest.mark.parametrize("out_dt, in_dt", [(O.FLOAT32, O.FLOAT64), (O.BFLOAT16, O.FLOAT32), (O.FLOAT16, O.INT8),
                                           (O.F8E4M3, O.FLOAT32), (O.F8E5M2, O.BFLOAT16), (O.INT8, O.FLOAT32),
                                           (O.INT4, O.INT8), (O.FLOAT64, O.INT4), (O.FLOAT32, O.F8E4M3)])
def test_convert_empty(out_dt, in_dt):
    out, op = empty_dev(64)
    src, sp = empty_dev(64)
    M.convert(op, out_dt, sp, in_dt, 0, stream())
    M.convert(0, out_dt, 0, in_dt, 0, stream())
    untouched(out)


def test_dequant_empty():
    out, op = empty_dev(64)
    src, sp = empty_dev(64)
    M.dequant_fp8(op, O.BFLOAT16, sp, O.F8E5M2, 0, 2.0, stream())
    M.dequant_fp8(0, O.FLOAT32, 0, O.F8E4M3, 0, 1.0, stream())
    M.dequant_int4(op, O.BFLOAT16, sp, 0, sp, O.FLOAT16, 128, stream())
    M.dequant_int4(0, O.FLOAT32, 0, 0, 0, O.FLOAT32, 128, stream())
    untouched(out)
    with pytest.raises(M.MFHError):  # dtypes are still checked
        M.dequant_fp8(op, O.BFLOAT16, sp, O.FLOAT32, 0, 1.0, stream())


@pytest.mark.parametrize("dt", [O.FLOAT32, O.BFLOAT16, O.FLOAT16])
def test_axpy_and_broadcast_empty(dt):
    y, yp = empty_dev(64)
    x, xp = empty_dev(64)
    M.axpy(yp, xp, 0, 2.0, dt, stream())
    M.axpy(0, 0, 0, 2.0, dt, stream())
    M.stream_sync(stream())  # no sticky error either
    M.scalar_broadcast(yp, dt, xp, dt, 0, 3.0, "mul", stream())
    M.scalar_broadcast(0, dt, 0, dt, 0, 3.0, "add", stream())
    untouched(y)
    with pytest.raises(M.MFHError, match="scalar divisor must be nonzero"):
        M.scalar_broadcast(yp, dt, xp, dt, 0, 0.0, "div", stream())
    with pytest.raises(M.MFHError, match="count must be positive"):
        M.linspace(yp, dt, 0, 0.0, 1.0)
    untouched(y)


def test_fused_kernel_and_graph_call_empty():
    torch = torch_mod()
    nodes = O.flatten((O.N_MUL, (O.N_SILU, ("in", 0)), ("in", 1)))
    k = M.FusedKernel(nodes, [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, "empty_swiglu")
    out, op = empty_dev(64)
    a, ap = empty_dev(64)
    k.launch([ap, ap], op, 0, stream())
    k.launch([0, 0], 0, 0, stream())
    untouched(out)
    g = Graph(inputs=["x", "y"], outputs={"e": "e"}, execution_dtype=M.FLOAT32, nodes=[
        GraphNode("a", "math.mul", ["x", "y"]), GraphNode("e", "activation.relu", ["a"])])
    x = torch.empty(0, device="cuda")
    e = torch.empty(0, device="cuda")
    for _ in range(3):  # launch, capture, replay
        g.call({"x": x, "y": x}, {"e": e}, stream())
    torch.cuda.synchronize()


def test_backend_empty_tensor_round_trip():
    b = Backend(0)
    try:
        t = b.upload([0, 4], M.FLOAT32, b"")
        assert t.len() == 0 and t.shape() == [0, 4]
        dt, data = b.download(t)
        assert dt == M.FLOAT32 and bytes(data) == b""
        t.close()
        # every upload form, synchronous and queued, with no elements
        empty = np.zeros(0, np.uint8)
        scales = np.zeros(0, np.float16)
        made = [b.upload_async([0], M.BFLOAT16, b""),
                b.upload_fp8([0, 7], M.F8E4M3, empty, 0.5),
                b.upload_fp8([0], M.F8E5M2, empty, 0.5, M.FLOAT32, queued=True),
                b.upload_int4([3, 0], empty, scales, M.FLOAT16, 128),
                b.upload_int4([0], empty, scales, M.FLOAT16, 128, M.FLOAT16, queued=True)]
        for t in made:
            t.sync()
            assert t.len() == 0 and bytes(b.download(t)[1]) == b""
            t.release()
    finally:
        b.close()
