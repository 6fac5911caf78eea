"""GPU tests of the HIP tensor backend (include/mfh_backend.h): the
tensor.Backend / tensor.Tensor contract (tensor/backend.go:18-68,
tensor/tensor.go:53-130) over device memory, the dequantising uploads
checked bit for bit against the oracle (BytesToBFloat16 and the scaled
dequant kernels' oracle), views, lifecycle errors, and axpyOntoResident
(runtime/axpy.go:44-93) with the reference's cases (runtime/axpy_test.go:14-68).
"""
import numpy as np
import pytest

import manifesto_amd as M
from manifesto_amd.backend import (Backend, ERR_LAYOUT_UNSUPPORTED, ERR_SHAPE_INVALID, ERR_TENSOR_CLOSED,
                                   STATE_CLOSED, STATE_PENDING, STATE_READY)
import oracle as O

from gpu_util import log

pytestmark = pytest.mark.gpu

CHUNK = 16 << 20  # the backend's staging chunk; sizes below cross several


@pytest.fixture(scope="module")
def backend():
    b = Backend(0)
    yield b
    b.release()


def code(err):
    return err.value.code


def test_backend_contract(backend):
    assert backend.location() == "hip"
    assert backend.supported_dtypes() == [O.FLOAT32, O.FLOAT16, O.BFLOAT16, O.F8E4M3, O.F8E5M2, O.INT4]
    assert backend.supported_layouts() == [0]
    caps = backend.capabilities()
    assert caps.max_bytes > (100 << 30) and caps.supports_async == 1 and caps.supports_sparse == 0
    assert caps.native_alignment == 256 and caps.numa_nodes == 1
    with pytest.raises(M.MFHError) as e:
        backend.upload_sparse()
    assert code(e) == ERR_LAYOUT_UNSUPPORTED


@pytest.mark.parametrize("dims", [[0], [], [3], [2, 3, 4], [4096, 4097]])
@pytest.mark.parametrize("dt, np_dt", [(O.FLOAT32, np.float32), (O.FLOAT16, np.uint16), (O.BFLOAT16, np.uint16)])
def test_upload_download_round_trip(backend, dims, dt, np_dt):
    n = int(np.prod(dims)) if dims else 1
    rng = np.random.default_rng(n)
    data = rng.integers(0, 2 ** 31, n, dtype=np.uint32).astype(np_dt) if np_dt != np.float32 else \
        rng.normal(0, 1, n).astype(np.float32)
    t = backend.upload(dims, dt, data.tobytes())
    assert t.shape() == dims and t.len() == n and t.dtype() == dt and t.location() == "hip"
    assert t.bytes() == data.nbytes and t.state() == STATE_READY
    got_dt, raw = backend.download(t)
    assert got_dt == dt and raw == data.tobytes()
    assert t.raw_bytes() == (dt, data.tobytes())
    t.release()


@pytest.mark.parametrize("fmt", [O.F8E4M3, O.F8E5M2])
def test_upload_fp8_is_stored_as_bfloat16(backend, fmt):
    # BytesToBFloat16 on the device (dtype/convert/convert.go:155-171)
    codes = np.tile(np.arange(256, dtype=np.uint8), 16)
    t = backend.upload([16, 256], fmt, codes)
    dt, raw = backend.download(t)
    assert dt == O.BFLOAT16 and t.dtype() == O.BFLOAT16 and t.shape() == [16, 256]
    assert np.frombuffer(raw, np.uint16).tolist() == O.bytes_to_bf16(fmt, codes).tolist()
    # large enough to cross staging chunks
    big = np.random.default_rng(fmt).integers(0, 256, 3 * CHUNK + 12345, dtype=np.uint8)
    t = backend.upload([big.size], fmt, big)
    dt, raw = backend.download(t)
    np.testing.assert_array_equal(np.frombuffer(raw, np.uint16), O.bytes_to_bf16(fmt, big))


def test_upload_int4_is_stored_as_bfloat16(backend):
    packed = np.arange(256, dtype=np.uint8)
    t = backend.upload([511], O.INT4, packed)  # odd count: the last byte's low nibble only
    dt, raw = backend.download(t)
    assert dt == O.BFLOAT16 and t.len() == 511
    np.testing.assert_array_equal(np.frombuffer(raw, np.uint16), O.bytes_to_bf16(O.INT4, packed)[:511])
    big = np.random.default_rng(5).integers(0, 256, 2 * CHUNK + 999, dtype=np.uint8)
    t = backend.upload([big.size * 2], O.INT4, big)
    dt, raw = backend.download(t)
    np.testing.assert_array_equal(np.frombuffer(raw, np.uint16), O.bytes_to_bf16(O.INT4, big))


@pytest.mark.parametrize("out_dt", [O.BFLOAT16, O.FLOAT16, O.FLOAT32])
def test_scaled_fp8_upload(backend, out_dt):
    codes = np.random.default_rng(2).integers(0, 256, 2 * CHUNK + 77, dtype=np.uint8)
    t = backend.upload_fp8([codes.size], O.F8E4M3, codes, 0.0125, out_dt)
    dt, raw = backend.download(t)
    want = O.dequant_fp8(codes, O.F8E4M3, 0.0125, out_dt)
    assert dt == out_dt
    np.testing.assert_array_equal(np.frombuffer(raw, want.dtype).view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("group, scale_dt", [(128, O.FLOAT16), (64, O.BFLOAT16), (4096, O.FLOAT32)])
def test_scaled_int4_upload(backend, group, scale_dt):
    rows, cols = 2048, 8192 * 2  # 33.5M nibbles: more than one staging chunk
    n = rows * cols
    rng = np.random.default_rng(group)
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    s32 = rng.uniform(0.005, 0.02, n // group).astype(np.float32)
    scales = O.encode(s32, scale_dt) if scale_dt != O.FLOAT32 else s32
    t = backend.upload_int4([rows, cols], packed, scales, scale_dt, group, O.BFLOAT16)
    dt, raw = backend.download(t)
    want = O.dequant_int4(packed, n, scales, scale_dt, group, O.BFLOAT16)
    assert dt == O.BFLOAT16
    np.testing.assert_array_equal(np.frombuffer(raw, np.uint16), want)
    log(f"int4 group {group}: {n} nibbles ok")


def test_upload_errors(backend):
    with pytest.raises(M.MFHError) as e:
        backend.upload([3], O.FLOAT32, b"\0" * 11)
    assert code(e) == -3
    with pytest.raises(M.MFHError) as e:
        backend.upload([2, -1], O.FLOAT32, b"")
    assert code(e) == ERR_SHAPE_INVALID
    with pytest.raises(M.MFHError) as e:
        backend.upload([2], O.FLOAT64, b"\0" * 16)
    assert code(e) == -2
    with pytest.raises(M.MFHError) as e:
        backend.upload([3], O.INT4, b"\0" * 1)  # 3 nibbles need 2 bytes
    assert code(e) == -3


def test_async_upload_and_sync(backend):
    data = np.random.default_rng(9).normal(0, 1, 5 * CHUNK // 4 + 3).astype(np.float32)
    src = data.copy()
    t = backend.upload_async([data.size], O.FLOAT32, src)
    src[:] = 0  # the source may be reused as soon as the call returns
    assert t.state() in (STATE_PENDING, STATE_READY)
    t.sync()
    assert t.state() == STATE_READY
    assert backend.download(t)[1] == data.tobytes()


def test_queued_scaled_uploads_back_to_back(backend):
    # Scaled FP8 and grouped Int4 uploads queued without a wait (tensors of
    # 1 to 3 staging chunks, so each starts on either ring slot), their host
    # buffers overwritten as soon as each call returns: every tensor matches
    # the oracle.
    rng = np.random.default_rng(11)
    rows, cols, group = 1024, 8192, 128
    cases = []
    for k, n_codes in enumerate([2 * CHUNK + 77, CHUNK // 3, CHUNK + 5]):
        codes = rng.integers(0, 256, n_codes, dtype=np.uint8)
        cases.append(("fp8", codes.copy(), O.dequant_fp8(codes, O.F8E5M2 if k % 2 else O.F8E4M3, -0.75,
                                                           O.BFLOAT16), k % 2))
        packed = rng.integers(0, 256, rows * cols // 2 * (k + 1), dtype=np.uint8)
        s16 = O.f32_to_f16(rng.uniform(0.005, 0.02, rows * cols * (k + 1) // group).astype(np.float32))
        cases.append(("int4", (packed.copy(), s16.copy()),
                      O.dequant_int4(packed, rows * cols * (k + 1), s16, O.FLOAT16, group, O.BFLOAT16), k))
    tensors = []
    for kind, src, want, k in cases:
        if kind == "fp8":
            t = backend.upload_fp8([src.size], O.F8E5M2 if k else O.F8E4M3, src, -0.75, O.BFLOAT16, queued=True)
            src[:] = 0
        else:
            packed, s16 = src
            t = backend.upload_int4([rows * (k + 1), cols], packed, s16, O.FLOAT16, group, O.BFLOAT16, queued=True)
            packed[:] = 0
            s16[:] = 0
        assert t.state() in (STATE_PENDING, STATE_READY)
        tensors.append((t, want))
    for t, want in tensors:
        t.sync()
        assert t.state() == STATE_READY
        np.testing.assert_array_equal(np.frombuffer(backend.download(t)[1], np.uint16), want)
        t.release()
    log("queued scaled uploads match the oracle")


def test_views_and_lifecycle(backend):
    data = np.arange(24, dtype=np.float32)
    t = backend.upload([2, 3, 4], O.FLOAT32, data)
    s = t.slice(5, 10)
    assert s.shape() == [10] and backend.download(s)[1] == data[5:15].tobytes()
    assert s.dispatch_pointer() == t.dispatch_pointer() + 20
    r = t.reshape([6, 4])
    assert r.shape() == [6, 4] and backend.download(r)[1] == data.tobytes()
    with pytest.raises(M.MFHError) as e:
        t.slice(20, 5)
    assert code(e) == ERR_SHAPE_INVALID
    with pytest.raises(M.MFHError) as e:
        t.reshape([5, 5])
    assert code(e) == -3
    s.close()
    s.close()  # idempotent
    assert s.state() == STATE_CLOSED and backend.download(t)[1] == data.tobytes()  # a view's close frees nothing
    t.close()
    assert t.state() == STATE_CLOSED and r.state() == STATE_CLOSED and t.dispatch_pointer() == 0
    with pytest.raises(M.MFHError) as e:
        backend.download(r)  # closing the parent invalidates its views
    assert code(e) == ERR_TENSOR_CLOSED


def test_axpy_onto_resident(backend):
    # runtime/axpy_test.go:26-52: bf16 y = [1,2,3], x = [4,5,6], alpha 0.5 -> [3,4.5,6]
    y = backend.upload([3], O.BFLOAT16, O.f32_to_bf16(np.array([1, 2, 3], np.float32)))
    x = backend.upload([3], O.BFLOAT16, O.f32_to_bf16(np.array([4, 5, 6], np.float32)))
    assert backend.axpy_onto_resident(y, x, 0.5) is y
    dt, raw = backend.download(y)
    assert dt == O.BFLOAT16 and O.bytes_to_f32(O.BFLOAT16, np.frombuffer(raw, np.uint8)).tolist() == [3, 4.5, 6]
    # f32 at size, against the oracle's unfused axpy
    rng = np.random.default_rng(1)
    yv, xv = rng.uniform(-1, 1, 1 << 22).astype(np.float32), rng.uniform(-1, 1, 1 << 22).astype(np.float32)
    y = backend.upload([yv.size], O.FLOAT32, yv)
    x = backend.upload([xv.size], O.FLOAT32, xv)
    backend.axpy_onto_resident(y, x, -0.25)
    y.sync()
    np.testing.assert_array_equal(np.frombuffer(backend.download(y)[1], np.float32), O.axpy_f32(yv, xv, -0.25))
    # the reference's checks and messages (runtime/axpy.go:72-82)
    z = backend.upload([3], O.FLOAT32, np.zeros(3, np.float32))
    with pytest.raises(M.MFHError, match="math.axpy: y dtype F32 does not match x dtype BF16"):
        backend.axpy_onto_resident(z, backend.upload([3], O.BFLOAT16, np.zeros(3, np.uint16)), 1.0)
    with pytest.raises(M.MFHError, match="math.axpy: y length 3 does not match x length 4"):
        backend.axpy_onto_resident(z, backend.upload([4], O.FLOAT32, np.zeros(4, np.float32)), 1.0)


def test_axpy_through_another_backend():
    # y and x held by backend A, the axpy queued through backend B: A's
    # download, sync and close are ordered after B's launch.
    a, b = Backend(0), Backend(0)
    try:
        rng = np.random.default_rng(2)
        n = (48 << 20) // 4 + 7  # larger than the staging ring, so the launch is still running at download
        yv, xv = rng.uniform(-1, 1, n).astype(np.float32), rng.uniform(-1, 1, n).astype(np.float32)
        y = a.upload([n], O.FLOAT32, yv)
        x = a.upload_async([n], O.FLOAT32, xv)
        for k in range(3):
            b.axpy_onto_resident(y, x, 0.5 + k)
        assert y.state() in (STATE_PENDING, STATE_READY)
        want = O.axpy_f32(O.axpy_f32(O.axpy_f32(yv, xv, 0.5), xv, 1.5), xv, 2.5)
        got = np.frombuffer(a.download(y)[1], np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        # bf16: the reference's golden case through the second backend, then
        # the tensors close through their owner right after the launch
        yb = a.upload([3], O.BFLOAT16, O.f32_to_bf16(np.array([1, 2, 3], np.float32)))
        xb = a.upload([3], O.BFLOAT16, O.f32_to_bf16(np.array([4, 5, 6], np.float32)))
        b.axpy_onto_resident(yb, xb, 0.5)
        yb.sync()
        assert O.bytes_to_f32(O.BFLOAT16, np.frombuffer(a.download(yb)[1], np.uint8)).tolist() == [3, 4.5, 6]
        b.axpy_onto_resident(y, x, 1.0)
        x.close()
        y.close()
    finally:
        b.release()
        a.release()


def test_closed_blocks_are_reused_for_the_same_size():
    # a closed tensor's block returns to its backend's cache and the next
    # tensor of the same byte size gets it, with its own contents
    b = Backend(0)
    try:
        rng = np.random.default_rng(41)
        n = 3 * CHUNK // 4 + 5  # f32: several staging chunks
        first = rng.normal(0, 1, n).astype(np.float32)
        t = b.upload([n], O.FLOAT32, first)
        p = t.dispatch_pointer()
        t.release()
        second = rng.normal(0, 1, n).astype(np.float32)
        u = b.upload([n], O.FLOAT32, second)  # same bytes: the cached block
        assert u.dispatch_pointer() == p
        v = b.upload([n + 1], O.FLOAT32, np.ones(n + 1, np.float32))  # another size: a new block
        assert v.dispatch_pointer() != p
        assert b.download(u)[1] == second.tobytes()
        # an FP8 upload stored as bf16 takes a block of its stored size
        codes = rng.integers(0, 256, 2 * n, dtype=np.uint8)
        u.release()
        w = b.upload([2 * n], O.F8E4M3, codes)  # 2n bf16 = the f32 block's bytes
        assert w.dispatch_pointer() == p
        assert b.download(w)[1] == O.bytes_to_bf16(O.F8E4M3, codes).tobytes()
        v.release()
        w.release()
    finally:
        b.release()


def test_backend_close_invalidates_tensors():
    b = Backend(0)
    t = b.upload([4], O.FLOAT32, np.ones(4, np.float32))
    b.close()
    b.close()  # idempotent
    assert t.state() == STATE_CLOSED
    with pytest.raises(M.MFHError) as e:
        t.sync()
    assert code(e) == ERR_TENSOR_CLOSED
    with pytest.raises(M.MFHError) as e:
        b.upload([1], O.FLOAT32, np.ones(1, np.float32))
    assert code(e) == -7
    t.release()
    b.release()


def _affine_graph():
    # a = x + bias (also an output, so it stays its own node); y = a * 1.1 + residual, fused
    from manifesto_amd.graph import Graph, GraphNode
    f16 = O.FLOAT16
    return Graph(inputs=["x", "bias", "residual"], outputs={"out": "y", "pre": "a"}, execution_dtype=f16, nodes=[
        GraphNode("s", "math.constant", [], attributes={"value": 1.1}),
        GraphNode("a", "math.add", ["x", "bias"], input_types=[f16, f16], output_type=f16),
        GraphNode("m", "math.mul", ["a", "s"], input_types=[f16, O.FLOAT32], output_type=f16),
        GraphNode("y", "math.add", ["m", "residual"], input_types=[f16, f16], output_type=f16),
    ])


def _affine_want(xs, bs, rs):
    f = lambda h: O.bytes_to_f32(O.FLOAT16, h.view(np.uint8))  # noqa: E731
    rows = xs.size // bs.size
    a = O.f32_to_f16(f(xs) + np.tile(f(bs), rows))
    y = O.f32_to_f16(f(a) * np.float32(1.1) + f(rs))
    return a, y


def test_graph_call_over_resident_tensors():
    # runtime.Backend.CallGraph (runtime/executor.go:22-27): inputs are tensors
    # of two backends, some still pending; outputs are allocated by the call.
    from manifesto_amd import graph as G
    a, b = Backend(0), Backend(0)
    try:
        graph = _affine_graph()
        G.run(graph)
        assert [n.op for n in graph.nodes] == ["math.constant", "math.add", G.FUSE_OP]
        G.attach_kernels(graph)
        rng = np.random.default_rng(3)
        n, period = 4096 * 1031, 4096
        xs = O.f32_to_f16(rng.standard_normal(n).astype(np.float32))
        bs = O.f32_to_f16((rng.standard_normal(period) * 0.02).astype(np.float32))
        rs = O.f32_to_f16(rng.standard_normal(n).astype(np.float32))
        tx = a.upload_async([n], O.FLOAT16, xs)
        tb = a.upload([period], O.FLOAT16, bs)
        tr = b.upload_async([n], O.FLOAT16, rs)  # another backend's tensor
        outs = a.graph_call(graph, {"x": tx, "bias": tb, "residual": tr}, ["out", "pre", "out"])
        assert sorted(outs) == ["out", "pre"]
        out, pre = outs["out"], outs["pre"]
        assert out.dtype() == O.FLOAT16 and out.len() == n and out.shape() == [n]
        assert out.state() in (STATE_PENDING, STATE_READY)
        want_a, want_y = _affine_want(xs, bs, rs)
        out.sync()
        assert out.state() == STATE_READY
        np.testing.assert_array_equal(np.frombuffer(a.download(out)[1], np.uint16), want_y)
        np.testing.assert_array_equal(np.frombuffer(a.download(pre)[1], np.uint16), want_a)
        log(f"graph call over resident tensors: {n} elements bit-exact, inputs from two backends")
        # a second call reads the first one's output (ordered on the stream)
        outs2 = b.graph_call(graph, {"x": out, "bias": tb, "residual": tr}, ["out"])
        _, want2 = _affine_want(want_y, bs, rs)
        np.testing.assert_array_equal(np.frombuffer(b.download(outs2["out"])[1], np.uint16), want2)
        # errors come back before anything is queued, with no outputs
        with pytest.raises(M.MFHError) as e:
            a.graph_call(graph, {"x": tx, "bias": tx.slice(0, 4095), "residual": tr}, ["out"])
        assert code(e) == -3 and "operand \"bias\" has 4095 elements" in str(e.value)
        with pytest.raises(M.MFHError, match="unknown output \"nope\""):
            a.graph_call(graph, {"x": tx, "bias": tb, "residual": tr}, ["nope"])
        for t in (out, pre, outs2["out"]):
            t.release()
        tr.close()
        b.close()
        with pytest.raises(M.MFHError) as e:
            a.graph_call(graph, {"x": tx, "bias": tb, "residual": tr}, ["out"])
        assert code(e) == ERR_TENSOR_CLOSED
        a.close()
        with pytest.raises(M.MFHError) as e:
            a.graph_call(graph, {"x": tx, "bias": tb}, ["out"])
        assert code(e) == -7
    finally:
        b.release()
        a.release()


def test_close_waits_for_its_own_work_not_the_device():
    # tensor.Tensor.Close drains the tensor's own in-flight work
    # (tensor/tensor.go:66-70) and nothing else: with a long run of resident
    # axpys queued on backend B, closing an idle tensor of backend A returns
    # while they still run; closing a tensor that they read waits for its last
    # use; a tensor whose device address was handed out (the caller may have
    # launched on it anywhere) waits for the whole device.
    import torch
    a, b = Backend(0), Backend(0)
    try:
        n = 1 << 26  # 256 MiB of f32: one axpy streams 768 MiB, about 0.13 ms
        ones = np.ones(n, np.float32)
        y = b.upload([n], O.FLOAT32, np.zeros(n, np.float32))
        xb = b.upload([n], O.FLOAT32, ones)
        xa = a.upload([n], O.FLOAT32, ones)
        idle = a.upload([1024], O.FLOAT32, np.arange(1024, dtype=np.float32))
        log("close: queueing 400 axpys on backend B")
        for _ in range(400):  # about 50 ms of device work
            b.axpy_onto_resident(y, xb, 1.0)
        for _ in range(8):  # the last reads of xa
            b.axpy_onto_resident(y, xa, 1.0)
        assert y.state() == STATE_PENDING
        idle.close()
        assert y.state() == STATE_PENDING, "closing an unrelated tensor waited for another backend's work"
        xa.close()
        assert y.state() == STATE_READY, "closing a tensor returned before the work that reads it"
        # a handed-out address: the caller's own launch on another stream
        xe = a.upload([n], O.FLOAT32, ones)
        s = torch.cuda.current_stream()
        for _ in range(100):
            M.axpy(y.dispatch_pointer(), xe.dispatch_pointer(), n, 1.0, M.FLOAT32, s.cuda_stream)
        done = torch.cuda.Event()
        done.record(s)
        xe.close()
        assert done.query(), "closing a tensor with a handed-out address returned before the device was idle"
        got = np.frombuffer(b.download(y)[1], np.float32)
        assert np.all(got == 508.0)
        xb.close()
        y.close()
    finally:
        b.release()
        a.release()
