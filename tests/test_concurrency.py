"""The C ABI called from several threads at once, as cgo calls arrive on any
OS thread (ctypes releases the GIL around each foreign call, so these calls
really overlap inside libmfh).

CPU: generated kernels compiled concurrently (the hiprtc cache is shared and
keyed by source text) come out identical to serial compiles, and each
thread's mfh_last_error holds its own failure.  GPU: dequant, axpy and
fused launches from eight threads, each on its own stream and buffers,
match the oracle, and so do eight threads uploading, dequantising, running
resident axpy and downloading through one shared backend.
"""
import threading

import numpy as np
import pytest

import manifesto_amd as M
import oracle as O

THREADS = 8


def run_threads(fn, n=THREADS):
    errors = []
    barrier = threading.Barrier(n)

    def body(k):
        try:
            barrier.wait()
            fn(k)
        except BaseException as e:  # noqa: BLE001 - reported below
            errors.append((k, repr(e)))

    ts = [threading.Thread(target=body, args=(k,)) for k in range(n)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors


def chain(k):
    # a different chain per k % 4, the same chain for k and k + 4
    leaf = ("in", 0)
    body = [(O.N_MUL, (O.N_SILU, leaf), ("in", 1)), (O.N_ADD, (O.N_GELU, leaf), ("in", 1)),
            (O.N_SUB, (O.N_RELU, leaf), ("in", 1)), (O.N_MAX, (O.N_SIGMOID, leaf), ("in", 1))][k % 4]
    return O.flatten(body)


def test_concurrent_compiles_match_serial_ones():
    sources = {}

    def compile_k(k):
        kern = M.FusedKernel(chain(k), [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, f"conc_{k % 4}")
        sources[k] = kern.source

    run_threads(compile_k)
    for k in range(THREADS):
        serial = M.FusedKernel(chain(k), [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, f"conc_{k % 4}")
        assert sources[k] == serial.source
        assert sources[k] == sources[k % 4]


def test_last_error_is_per_thread():
    seen = {}
    barrier = threading.Barrier(THREADS)

    def fail_k(k):
        with pytest.raises(M.MFHError):
            M.set_launch_config(f"family{k}", 1, 1)
        barrier.wait()  # every thread has failed before any reads its message
        seen[k] = M.last_error()

    run_threads(fail_k)
    for k in range(THREADS):
        assert f'"family{k}"' in seen[k], seen[k]


def test_sticky_errors_are_per_stream():
    # The odd threads' axpys fail (the library has no device here), each on
    # its own stream handle; every odd thread then finds its failure on its
    # stream, once, and no even thread finds one on its own, although all the
    # failures were recorded before anyone collected.  The handles are never
    # dereferenced: the calls fail before any device work.
    if M.lib().mfh_capabilities(None, None, None) == 0:
        pytest.skip("library already initialised on a device")
    barrier = threading.Barrier(THREADS)
    seen = {}

    def fail_k(k):
        handle = 0x1000 * (k + 1)
        if k % 2:
            M.axpy(1, 1, 4, 1.0, M.FLOAT32, handle)
        barrier.wait()  # every failure is recorded before any thread collects
        try:
            M.take_sticky_error(handle)
            seen[k] = "ok"
        except M.MFHError as e:
            seen[k] = str(e)
        M.take_sticky_error(handle)  # collected once

    run_threads(fail_k)
    for k in range(THREADS):
        if k % 2:
            assert "mfh_axpy: mfh_init has not been called" in seen[k], (k, seen[k])
        else:
            assert seen[k] == "ok", (k, seen[k])


@pytest.mark.gpu
def test_sticky_error_reaches_only_its_streams_owner():
    import torch
    M.init(0)
    y = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    x = torch.ones(1 << 16, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    barrier = threading.Barrier(2)
    outcome = {}

    def work(k):
        s = streams[k].cuda_stream
        if k == 0:
            M.axpy(y.data_ptr(), x.data_ptr(), y.numel(), 1.0, M.INT32, s)  # unsupported: sticky on s
        barrier.wait()
        if k == 1:
            M.axpy(y.data_ptr(), x.data_ptr(), y.numel(), 2.0, M.FLOAT32, s)
        try:
            M.stream_sync(s)
            outcome[k] = "ok"
        except M.MFHError as e:
            outcome[k] = str(e)

    run_threads(work, 2)
    assert "is not f32/bf16/f16" in outcome[0], outcome
    assert outcome[1] == "ok", outcome
    M.stream_sync(streams[0].cuda_stream)  # consumed
    assert float(y.cpu()[0]) == 2.0


@pytest.mark.gpu
def test_concurrent_launches_on_separate_streams():
    import torch
    M.init(0)
    rng = np.random.default_rng(11)
    n = (1 << 20) + 5
    codes = rng.integers(0, 256, n, dtype=np.uint8)
    packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    scales = O.f32_to_f16(rng.uniform(0.005, 0.02, -(-n // 128)).astype(np.float32))
    x = rng.uniform(-1, 1, n).astype(np.float32)
    y = rng.uniform(-1, 1, n).astype(np.float32)
    g = O.f32_to_bf16(rng.normal(0, 1, n).astype(np.float32))
    u = O.f32_to_bf16(rng.normal(0, 1, n).astype(np.float32))
    want_fp8 = O.dequant_fp8(codes, O.F8E4M3, 0.0125, O.BFLOAT16)
    want_int4 = O.dequant_int4(packed, n, scales, O.FLOAT16, 128, O.BFLOAT16)
    want_axpy = O.axpy_f32(y, x, 0.75)
    nodes = O.flatten((O.N_ADD, (O.N_MUL, ("in", 0), ("in", 1)), ("in", 1)))
    want_chain = O.f32_to_bf16(O.run(nodes, [O.decode(g, O.BFLOAT16), O.decode(u, O.BFLOAT16)], n))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).copy()).cuda()  # noqa: E731
    d_codes, d_packed, d_scales, d_x, d_g, d_u = map(dev, (codes, packed, scales, x, g, u))
    torch.cuda.synchronize()
    results = {}

    def work(k):
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            o8 = torch.empty(n * 2, dtype=torch.uint8, device="cuda")
            o4 = torch.empty(n * 2, dtype=torch.uint8, device="cuda")
            oy = dev(y)
            oc = torch.empty(n * 2, dtype=torch.uint8, device="cuda")
        kern = M.FusedKernel(nodes, [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, "conc_chain")
        for _ in range(3 if k % 2 else 1):  # repeated launches rewrite the same outputs
            M.dequant_fp8(o8.data_ptr(), M.BFLOAT16, d_codes.data_ptr(), M.F8E4M3, n, 0.0125, s.cuda_stream)
            M.dequant_int4(o4.data_ptr(), M.BFLOAT16, d_packed.data_ptr(), n, d_scales.data_ptr(), M.FLOAT16, 128,
                           s.cuda_stream)
            kern.launch([d_g.data_ptr(), d_u.data_ptr()], oc.data_ptr(), n, s.cuda_stream)
        M.axpy(oy.data_ptr(), d_x.data_ptr(), n, 0.75, M.FLOAT32, s.cuda_stream)
        M.stream_sync(s.cuda_stream)
        results[k] = tuple(t.cpu().numpy() for t in (o8, o4, oy, oc))

    run_threads(work)
    for k in range(THREADS):
        o8, o4, oy, oc = results[k]
        assert np.array_equal(o8.view(np.uint16), want_fp8), f"thread {k}: fp8"
        assert np.array_equal(o4.view(np.uint16), want_int4), f"thread {k}: int4"
        assert np.array_equal(oy.view(np.uint32), want_axpy.view(np.uint32)), f"thread {k}: axpy"
        assert np.array_equal(oc.view(np.uint16), want_chain), f"thread {k}: chain"


@pytest.mark.gpu
def test_one_backend_from_many_threads():
    # tensor.Backend shared by goroutines: uploads through the one staging
    # ring (f32 as is, FP8 and Int4 dequantised on the device), resident axpy
    # and downloads interleave across threads; every tensor keeps its bytes
    from manifesto_amd.backend import Backend
    M.init(0)
    b = Backend(0)
    rng = np.random.default_rng(12)
    n = (20 << 20) + 3  # more than one 16 MiB staging chunk for the f32 upload
    x = rng.uniform(-1, 1, n).astype(np.float32)
    codes = rng.integers(0, 256, n, dtype=np.uint8)
    m = (1 << 21) + 4  # Int4 nibbles, groups of 64
    packed = rng.integers(0, 256, m // 2, dtype=np.uint8)
    scales = O.f32_to_f16(rng.uniform(0.005, 0.02, m // 64).astype(np.float32))
    want_fp8 = O.dequant_fp8(codes, O.F8E4M3, 0.5, O.BFLOAT16).tobytes()
    want_int4 = O.dequant_int4(packed, m, scales, O.FLOAT16, 64, O.BFLOAT16).tobytes()
    results = {}
    try:
        def work(k):
            y0 = np.random.default_rng(100 + k).uniform(-1, 1, n).astype(np.float32)
            ty = b.upload([n], O.FLOAT32, y0)
            tx = b.upload([n], O.FLOAT32, x)
            t8 = b.upload_fp8([n], O.F8E4M3, codes, 0.5)
            t4 = b.upload_int4([m], packed, scales, O.FLOAT16, 64)
            b.axpy_onto_resident(ty, tx, 0.25 * (k + 1))
            results[k] = (bytes(b.download(ty)[1]), bytes(b.download(t8)[1]), bytes(b.download(t4)[1]),
                          O.axpy_f32(y0, x, 0.25 * (k + 1)).tobytes())
            for t in (ty, tx, t8, t4):
                t.close()

        run_threads(work)
    finally:
        b.release()
    for k in range(THREADS):
        got_y, got_8, got_4, want_y = results[k]
        assert got_y == want_y, f"thread {k}: axpy"
        assert got_8 == want_fp8, f"thread {k}: fp8 upload"
        assert got_4 == want_int4, f"thread {k}: int4 upload"


@pytest.mark.gpu
def test_backend_per_thread_uploads_and_downloads():
    # One backend per thread (one stream and staging ring each); every
    # staging copy goes through the library's shared pool of host copy
    # threads, so uploads and downloads of different backends interleave
    # there.  Every tensor keeps its bytes, and a SafeTensors-sized FP8 load
    # crosses several staging chunks per thread.
    from manifesto_amd.backend import Backend
    M.init(0)
    n = (36 << 20) + 5
    codes = np.random.default_rng(31).integers(0, 256, n, dtype=np.uint8)
    want_fp8 = O.dequant_fp8(codes, O.F8E5M2, 2.0, O.FLOAT16).tobytes()
    results = {}

    def work(k):
        b = Backend(0)
        try:
            f = np.random.default_rng(200 + k).standard_normal(n // 4).astype(np.float32)
            tf = b.upload_async([f.size], O.FLOAT32, f)
            t8 = b.upload_fp8([n], O.F8E5M2, codes, 2.0, O.FLOAT16)
            results[k] = (bytes(b.download(tf)[1]) == f.tobytes(), bytes(b.download(t8)[1]) == want_fp8)
            for t in (tf, t8):
                t.release()
        finally:
            b.release()

    run_threads(work)
    for k in range(THREADS):
        assert results[k] == (True, True), f"thread {k}: {results[k]}"
