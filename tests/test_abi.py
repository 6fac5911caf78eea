"""CPU tests of the C ABI library: symbols, JIT codegen and error paths.

No kernel is launched here; launches are the GPU tests.
"""
import os
import re
import subprocess

import pytest

import manifesto_amd as M
from oracle import (N_ADD, N_GELU, N_INPUT, N_MUL, N_RELU, N_SILU, N_SIGMOID, N_SUB, N_CONSTANT,
                    N_EXP, N_LEAKY_RELU, flatten)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_symbols():
    """Every function declared by the headers under include/."""
    names = set()
    for header in sorted(os.listdir(INCLUDE)):
        if header.endswith(".h"):
            text = open(os.path.join(INCLUDE, header)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(mfh_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", M.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_library_exports_every_declared_symbol():
    declared = declared_symbols()
    assert len(declared) >= 50
    missing = [s for s in declared if s not in exported_symbols()]
    assert not missing, missing
    for s in declared:
        getattr(M.lib(), s)  # resolvable through ctypes too
    assert M.lib().mfh_version() == 100


def declared_prototypes():
    """(return type, name, parameter list) of every function the headers declare."""
    text = ""
    for header in sorted(os.listdir(INCLUDE)):
        if header.endswith(".h"):
            t = open(os.path.join(INCLUDE, header)).read()
            t = re.sub(r"/\*.*?\*/", "", t, flags=re.S)
            text += re.sub(r"//[^\n]*", "", t)
    return re.findall(r"([A-Za-z_][\w \*]*?[\s\*])(mfh_\w+)\s*\(([^;{]*?)\)\s*;", text)


# (kind, bytes) of a C type as the ABI passes it: pointers, integers, floats.
_C_KINDS = {"int": ("i", 4), "int32_t": ("i", 4), "int64_t": ("i", 8), "uint8_t": ("i", 1),
            "uint32_t": ("i", 4), "size_t": ("i", 8), "float": ("f", 4), "double": ("f", 8), "void": ("v", 0)}


def c_kind(decl):
    decl = " ".join(decl.replace("const", "").split())
    if "*" in decl or decl == "hipStream_t":
        return ("p", 8)
    return _C_KINDS.get(decl, ("?", decl))


def ctypes_kind(t):
    import ctypes
    if t is None:
        return ("v", 0)
    if t in (ctypes.c_void_p, ctypes.c_char_p) or (isinstance(t, type) and issubclass(t, ctypes._Pointer)):
        return ("p", 8)
    if t in (ctypes.c_float, ctypes.c_double):
        return ("f", ctypes.sizeof(t))
    return ("i", ctypes.sizeof(t))


def test_ctypes_bindings_match_the_header_prototypes():
    # Every function of include/*.h is declared to ctypes by the package, with
    # the header's arity and, per argument and result, the same kind (pointer,
    # integer, float) and width: a 64-bit count bound as a 32-bit one would be
    # truncated without an error.
    from manifesto_amd import backend, graph, plan, safetensors
    L = M.lib()
    for module in (backend, graph, plan, safetensors):
        module._L()
    protos = declared_prototypes()
    assert len(protos) == len(declared_symbols())
    undeclared, mismatched = [], []
    for ret, name, params in protos:
        fn = getattr(L, name)
        if fn.argtypes is None:
            undeclared.append(name)
            continue
        want = [c_kind(ret)]
        for p in (p.strip() for p in params.split(",")):
            if p and p != "void":
                m = re.match(r"(.*?[\s\*])\w+$", p)
                want.append(c_kind(m.group(1) if m else p))
        got = [ctypes_kind(fn.restype)] + [ctypes_kind(a) for a in fn.argtypes]
        if want != got:
            mismatched.append((name, want, got))
    assert not undeclared, undeclared
    assert not mismatched, mismatched


def swiglu_nodes():
    # Mul(Silu(In0), In1): what Fuse builds from swish -> mul (optimizer/fuse.go:199-265).
    return flatten((N_MUL, (N_SILU, ("in", 0)), ("in", 1)))


def test_emit_hip_swiglu_source_shape():
    k = M.FusedKernel(swiglu_nodes(), [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, "mlp.swiglu-out")
    src = k.source
    assert k.kernel_name == "fused_mlp_swiglu_out"  # like metalKernelName (codegen/metal.go:281-290)
    assert k.identifier == "mlp.swiglu-out"  # Identifier() is the output port (codegen/metal.go:143)
    assert f'void {k.kernel_name}(' in src
    # reads 4 B per element, writes 2: streamed (non-temporal) loads
    assert "mfh_ld8_bf16<1>(p0, e0, a0[u])" in src and "mfh_ld8_bf16<1>(p1, e0, a1[u])" in src
    assert "streamed loads" in src
    assert "mfh_st8_bf16(pout, it * 8, r)" in src
    assert src.count("for (mfh_i64 i = nvec * 8 + tid; i < n; i += stride)") == 1
    # every element runs the branch-free fast form, which sets the element's
    # flag; flagged elements (vector loop and scalar tail) are recomputed with
    # the reference form as a real call.  No Add/Sub follows the activation:
    # no cancellation guard.
    assert src.count("mfh_silu_fast(x0, qe)") == 2 and "if (qany) {" in src and "if (qe) {" in src
    assert src.count("mfh_silu_rare(x0)") == 2 and "qe |=" not in src
    assert "8 elements per item, 1 item(s) per thread" in src  # f32-only math: one item per thread


def test_emit_hip_broadcast_operands():
    # Add(Gelu(Mul(Add(x, bias), s)), residual), bias periodic over 4096, s scalar.
    nodes = flatten((N_ADD, (N_GELU, (N_MUL, (N_ADD, ("in", 0), ("in", 1)), ("in", 2))), ("in", 3)))
    ops = [(M.FLOAT16, M.OPERAND_FULL, 0), (M.FLOAT16, M.OPERAND_PERIODIC, 4096),
           (M.FLOAT32, M.OPERAND_SCALAR, 0), (M.FLOAT16, M.OPERAND_FULL, 0)]
    k = M.FusedKernel(nodes, ops, M.FLOAT16, "chain")
    src = k.source
    # f16 operands stay packed in the vector loop; adds take them directly
    # the periodic bias is re-read across the grid: a cached load; x streams
    assert "mfh_ldw8_f16(p1, (e0 % 4096LL), w1[u])" in src and "mfh_ldw8_f16<1>(p0, e0, w0[u])" in src
    assert "mfh_add_hh(w0[u][j >> 1], j & 1, w1[u][j >> 1], j & 1)" in src
    assert "mfh_add_fh(t2, w3[u][j >> 1], j & 1)" in src
    assert "const float x1 = mfh_ld1_f16(p1, (i % 4096LL));" in src  # element loop decodes
    assert "const float s2 = mfh_ld1_f32(p2, 0);" in src
    assert "mfh_gelu_fast(t1, qe)" in src and "mfh_gelu_rare(f1)" in src
    # gelu + residual can cancel: f16 output, so the guard's factor is 0.7 * 2^12 / 2
    assert src.count("qe |= !(mfh_absf(t3) * 1433.0f >= mfh_absf(t2));") == 2
    # one item per thread; only a Sigmoid (mostly f64 work) takes two by default
    assert "8 elements per item, 1 item(s) per thread" in src
    sig = M.FusedKernel(flatten((N_SIGMOID, ("in", 0))), [(M.FLOAT16, M.OPERAND_FULL, 0)], M.FLOAT16, "sig")
    assert "8 elements per item, 2 item(s) per thread" in sig.source
    # precise: the rounding-tested form, the reference form for the elements it
    # flags, and no cancellation guard (its results are the reference's)
    precise = M.FusedKernel(nodes, ops, M.FLOAT16, "chain", flags=M.FUSION_PRECISE)
    body = precise.source.split("EmitHIP")[1]
    assert body.count("mfh_gelu_cr(t1, qe)") == 2 and body.count("mfh_gelu_rare(f1)") == 2
    assert "_fast(" not in body and "qe |=" not in body and "2 item(s) per thread" in precise.source
    plain = M.FusedKernel(nodes, ops, M.FLOAT16, "chain", flags=M.FUSION_PRECISE | M.FUSION_NO_ROUNDING_TEST)
    body = plain.source.split("EmitHIP")[1]
    assert "mfh_gelu_ref(t1)" in body and "_cr(" not in body and "qe" not in body
    assert "1 item(s) per thread" in plain.source


def guard_lines(src):
    return [l.strip() for l in src.splitlines() if l.strip().startswith("qe |=")]


@pytest.mark.parametrize("out_dt, threshold", [(M.FLOAT16, 1433), (M.BFLOAT16, 11468), (M.FLOAT32, None)])
def test_cancellation_guard_threshold_follows_the_output(out_dt, threshold):
    # Sub(Gelu(x), y): the activation's 2-ulp error, amplified by the
    # cancellation, must stay below 0.7 of a storage ulp: factor
    # 0.7 * 2^(22 - mantissa bits) / 2, i.e. 1433 for f16 and 11468 for bf16;
    # f32 outputs keep the node-envelope contract and take no guard.
    nodes = flatten((N_SUB, (N_GELU, ("in", 0)), ("in", 1)))
    k = M.FusedKernel(nodes, [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, out_dt, "g")
    lines = guard_lines(k.source)
    if threshold is None:
        assert lines == []
    else:
        assert lines == [f"qe |= !(mfh_absf(t1) * {threshold}.0f >= mfh_absf(t0));"] * 2


def test_cancellation_guard_counts_the_error_on_its_operands():
    bf = [(M.BFLOAT16, M.OPERAND_FULL, 0)]
    # one rounding op between the activation and the add: 3 ulps
    k = M.FusedKernel(flatten((N_ADD, (N_MUL, (N_SILU, ("in", 0)), ("in", 1)), ("in", 2))), bf * 3, M.FLOAT16, "m")
    assert guard_lines(k.source)[0] == "qe |= !(mfh_absf(t2) * 955.0f >= mfh_absf(t1));"
    # activations on both operands: compared with the larger, 2 + 2 ulps
    k = M.FusedKernel(flatten((N_SUB, (N_SILU, ("in", 0)), (N_GELU, ("in", 1)))), bf * 2, M.FLOAT16, "b")
    assert guard_lines(k.source)[0] == "qe |= !(mfh_absf(t2) * 716.0f >= mfh_maxf(mfh_absf(t0), mfh_absf(t1)));"
    # a second add on the path, or a transcendental above: no guarantee, no guard
    k = M.FusedKernel(flatten((N_ADD, (N_ADD, (N_GELU, ("in", 0)), ("in", 1)), ("in", 2))), bf * 3, M.FLOAT16, "a2")
    assert guard_lines(k.source) == []
    k = M.FusedKernel(flatten((N_EXP, (N_ADD, (N_GELU, ("in", 0)), ("in", 1)))), bf * 2, M.FLOAT16, "e")
    assert guard_lines(k.source) == []
    # no activation, no guard; precise forms, no guard
    k = M.FusedKernel(flatten((N_ADD, (N_RELU, ("in", 0)), ("in", 1))), bf * 2, M.FLOAT16, "r")
    assert guard_lines(k.source) == [] and "qe" not in k.source
    k = M.FusedKernel(flatten((N_ADD, (N_GELU, ("in", 0)), ("in", 1))), bf * 2, M.FLOAT16, "p",
                      flags=M.FUSION_PRECISE)
    assert guard_lines(k.source) == []


def test_chains_that_stream_f32_take_the_rounding_tested_forms():
    # An f32 output or a full or periodic f32 operand: every activation ulp
    # shows, so Sigmoid, Silu and Gelu take the rounding-tested forms (the
    # reference's values), with no cancellation guard and two items per thread.
    silu = flatten((N_MUL, (N_SILU, ("in", 0)), ("in", 1)))
    gelu = flatten((N_GELU, ("in", 0)))
    bf, f32 = (M.BFLOAT16, M.OPERAND_FULL, 0), (M.FLOAT32, M.OPERAND_FULL, 0)
    assert "mfh_silu_fast(x0, qe)" in M.FusedKernel(silu, [bf, bf], M.BFLOAT16, "s16").source
    assert "mfh_silu_cr(x0, qe)" in M.FusedKernel(silu, [bf, bf], M.FLOAT32, "s32").source
    assert "mfh_silu_cr(x0, qe)" in M.FusedKernel(silu, [f32, bf], M.BFLOAT16, "s32i").source
    # a scalar f32 operand does not make the chain stream f32
    assert "mfh_silu_fast(x0, qe)" in M.FusedKernel(silu, [bf, (M.FLOAT32, M.OPERAND_SCALAR, 0)],
                                                    M.BFLOAT16, "ss").source
    assert "mfh_gelu_cr(x0, qe)" in M.FusedKernel(gelu, [f32], M.FLOAT32, "g32").source
    short = M.FusedKernel(gelu, [f32], M.FLOAT32, "g32s", flags=M.FUSION_SHORT_QUOTIENT)
    assert "mfh_gelu_fast(x0, qe)" in short.source
    sig = M.FusedKernel(flatten((N_SIGMOID, ("in", 0))), [f32], M.FLOAT32, "sg")
    assert "mfh_sigmoid_cr(x0, qe)" in sig.source and "2 item(s) per thread" in sig.source
    assert "2 item(s) per thread" in M.FusedKernel(gelu, [f32], M.FLOAT32, "g32u").source
    assert "1 item(s) per thread" in short.source
    # f32 operand, bf16 output: exact activations need no guard; the 16-bit
    # chain's fast form does
    add = flatten((N_ADD, (N_GELU, ("in", 0)), ("in", 1)))
    assert guard_lines(M.FusedKernel(add, [f32, bf], M.BFLOAT16, "ga32").source) == []
    assert guard_lines(M.FusedKernel(add, [bf, bf], M.BFLOAT16, "ga16").source) != []


def test_emit_hip_item_width_follows_the_widest_operand():
    relu_add = flatten((N_RELU, (N_ADD, ("in", 0), ("in", 1))))
    k16 = M.FusedKernel(relu_add, [(M.BFLOAT16, M.OPERAND_FULL, 0), (M.FLOAT16, M.OPERAND_FULL, 0)], M.BFLOAT16, "a")
    assert "mfh_ld8_bf16<1>(p0" in k16.source and "8 elements per item, 1 item(s)" in k16.source
    k32 = M.FusedKernel(relu_add, [(M.BFLOAT16, M.OPERAND_FULL, 0), (M.FLOAT32, M.OPERAND_FULL, 0)], M.BFLOAT16, "b")
    assert "mfh_ld4_bf16<1>(p0" in k32.source and "mfh_ld4_f32<1>(p1" in k32.source and "mfh_st4_bf16(pout" in k32.source
    # a scalar f32 operand does not narrow the item
    ks = M.FusedKernel(relu_add, [(M.BFLOAT16, M.OPERAND_FULL, 0), (M.FLOAT32, M.OPERAND_SCALAR, 0)], M.BFLOAT16, "c")
    assert "mfh_ld8_bf16<1>(p0" in ks.source
    # a kernel that writes more than it reads keeps cached loads
    widen = M.FusedKernel(flatten((N_RELU, ("in", 0))), [(M.BFLOAT16, M.OPERAND_FULL, 0)], M.FLOAT32, "w")
    assert "mfh_ld4_bf16(p0" in widen.source and "streamed loads" not in widen.source


def test_emit_hip_constants_are_rounded_to_f32():
    nodes = flatten((N_MUL, ("in", 0), ("const", 0.1)))
    k = M.FusedKernel(nodes, [(M.FLOAT32, M.OPERAND_FULL, 0)], M.FLOAT32, "c")
    assert "mfh_fromfbits(0x3dcccccdu)" in k.source  # float32(0.1)


@pytest.mark.parametrize("nodes, n_in, msg", [
    ([], 1, "fusion root is required"),
    ([(N_ADD, 0, 0.0), (N_INPUT, 0, 0.0)], 1, "not one pre-order tree"),
    ([(N_RELU, 0, 0.0), (N_INPUT, 3, 0.0)], 2, "input index 3 out of range"),
    ([(42, 0, 0.0)], 1, "unsupported node type 42"),
    ([(N_RELU, 0, 0.0), (N_INPUT, 0, 0.0), (N_INPUT, 0, 0.0)], 1, "not one pre-order tree"),
])
def test_emit_hip_rejects_malformed_trees(nodes, n_in, msg):
    with pytest.raises(M.MFHError, match=msg):
        M.FusedKernel(nodes, [(M.FLOAT32, M.OPERAND_FULL, 0)] * n_in, M.FLOAT32, "bad")


def test_emit_hip_rejects_bad_dtypes_and_periods():
    relu = flatten((N_RELU, ("in", 0)))
    with pytest.raises(M.MFHError, match="output dtype"):
        M.FusedKernel(relu, [(M.FLOAT32, M.OPERAND_FULL, 0)], M.F8E4M3, "x")
    with pytest.raises(M.MFHError, match="input 0 dtype"):
        M.FusedKernel(relu, [(M.INT32, M.OPERAND_FULL, 0)], M.FLOAT32, "x")
    with pytest.raises(M.MFHError, match="period must be positive"):
        M.FusedKernel(relu, [(M.FLOAT32, M.OPERAND_PERIODIC, 0)], M.FLOAT32, "x")


def test_launch_rejects_input_count_like_the_cpu_kernel():
    # codegen/codegen_test.go:52-56: "expects 2 inputs".
    k = M.FusedKernel(flatten((N_RELU, (N_ADD, ("in", 0), ("in", 1)))),
                      [(M.FLOAT32, M.OPERAND_FULL, 0)] * 2, M.FLOAT32, "result")
    with pytest.raises(M.MFHError, match='kernel "result" expects 2 inputs, got 1'):
        k.launch([1], 2, 2)


def test_entry_points_require_init():
    # Without mfh_init every device entry point fails cleanly.
    if M.lib().mfh_capabilities(None, None, None) == 0:
        pytest.skip("library already initialised on a device")
    with pytest.raises(M.MFHError, match="mfh_init has not been called"):
        M.dequant_fp8(1, M.BFLOAT16, 1, M.F8E4M3, 16, 1.0)
    M.axpy(1, 1, 4, 1.0, M.FLOAT32)  # no error channel: the failure is sticky
    with pytest.raises(M.MFHError, match="mfh_init has not been called"):
        M.take_sticky_error()
    M.take_sticky_error()  # cleared


def _device_asm(source: str, tmp_path) -> str:
    src = tmp_path / "k.hip"
    src.write_text("#include <hip/hip_runtime.h>\n" + source)  # hiprtc pre-includes it
    asm = tmp_path / "k.s"
    cmd = ["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
           "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(src), "-o", str(asm)]
    subprocess.run(cmd, check=True, capture_output=True)
    return asm.read_text()


def test_generated_arithmetic_is_not_contracted(tmp_path):
    # Sub(Mul(x, y), z): Go rounds the product before the subtraction.
    nodes = flatten((N_SUB, (N_MUL, ("in", 0), ("in", 1)), ("in", 2)))
    k = M.FusedKernel(nodes, [(M.FLOAT32, M.OPERAND_FULL, 0)] * 3, M.FLOAT32, "fms")
    asm = _device_asm(k.source, tmp_path)
    body = asm[asm.index("fused_fms:"):]
    assert "v_mul_f32" in body and "v_sub_f32" in body
    assert not re.search(r"v_fma_f32|v_fmac_f32|v_mad_f32|v_pk_(fma|mul|add)_f32", body)


def test_generated_activation_chain_uses_no_packed_fp32(tmp_path):
    nodes = flatten((N_LEAKY_RELU, (N_ADD, (N_SIGMOID, ("in", 0)), (N_EXP, ("in", 1)))))
    k = M.FusedKernel(nodes, [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, "act")
    asm = _device_asm(k.source, tmp_path)
    assert not re.search(r"v_pk_(fma|mul|add)_f32", asm)


def test_backend_open_without_a_device_fails_loudly():
    from manifesto_amd.backend import Backend
    if M.lib().mfh_init(0) == 0:
        pytest.skip("a GPU is present; the backend is covered by the GPU tests")
    with pytest.raises(M.MFHError):
        Backend(0)


def test_launch_config_set_keep_and_restore():
    default = M.get_launch_config("fp8")
    M.set_launch_config("fp8", 7, 4)
    assert M.get_launch_config("fp8") == (7, 4)
    M.set_launch_config("fp8", 0, 0)  # 0 keeps
    assert M.get_launch_config("fp8") == (7, 4)
    M.set_launch_config("fp8", -1, -1)  # -1 restores the default
    assert M.get_launch_config("fp8") == default
    with pytest.raises(M.MFHError):
        M.set_launch_config("fp8", -2, 0)
    with pytest.raises(M.MFHError):
        M.set_launch_config("fp8", 0, 3)
    with pytest.raises(M.MFHError):
        M.set_launch_config("nope", 1, 1)
    # the casts pick their items per thread themselves unless one is set
    assert M.get_launch_config("convert")[1] == 0
    M.set_launch_config("convert", 0, 2)
    assert M.get_launch_config("convert")[1] == 2
    M.set_launch_config("convert", 0, -1)
    assert M.get_launch_config("convert")[1] == 0


def test_launch_threads_set_keep_restore_and_limits():
    # defaults: the measured workgroup size of each family
    assert [M.get_launch_threads(f) for f in ("fp8", "int4", "axpy", "axpy16", "convert")] == [128, 512, 64, 64, 0]
    assert M.get_launch_threads("fused") == 0  # each generated kernel's default
    k = M.FusedKernel(swiglu_nodes(), [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, "threads_default")
    assert "__launch_bounds__(64)" in k.source and "gridDim.x * 64;" in k.source
    try:
        M.set_launch_threads("fused", 256)
        assert M.get_launch_threads("fused") == 256
        M.set_launch_threads("fused", 0)  # 0 keeps
        assert M.get_launch_threads("fused") == 256
        k = M.FusedKernel(swiglu_nodes(), [(M.BFLOAT16, M.OPERAND_FULL, 0)] * 2, M.BFLOAT16, "threads_256")
        assert "__launch_bounds__(256)" in k.source and "blockIdx.x * 256 + threadIdx.x" in k.source
        for bad in (32, 96, 2048):
            with pytest.raises(M.MFHError, match=f"workgroups of 64, 128, 256, 512, 1024 threads, not {bad}"):
                M.set_launch_threads("fused", bad)
        assert M.get_launch_threads("fused") == 256
    finally:
        M.set_launch_threads("fused", -1)
    assert M.get_launch_threads("fused") == 0
    try:
        for t in (64, 128, 256):
            M.set_launch_threads("fp8", t)
            assert M.get_launch_threads("fp8") == t
        with pytest.raises(M.MFHError, match="workgroups of 64, 128, 256 threads, not 512"):
            M.set_launch_threads("axpy", 512)
        with pytest.raises(M.MFHError, match="workgroups of 64, 128, 256, 512 threads, not 1024"):
            M.set_launch_threads("int4", 1024)
        M.set_launch_threads("int4", 512)
        assert M.get_launch_threads("int4") == 512
        M.set_launch_threads("int4", 128)
        assert M.get_launch_threads("int4") == 128
    finally:
        M.set_launch_threads("fp8", -1)
        M.set_launch_threads("int4", -1)
    assert M.get_launch_threads("fp8") == 128
    with pytest.raises(M.MFHError, match="unknown kernel family"):
        M.set_launch_threads("nope", 64)


HEADERS = sorted(h for h in os.listdir(INCLUDE) if h.endswith(".h"))


@pytest.mark.parametrize("std, compiler", [("c99", "gcc"), ("c11", "gcc"), ("c++17", "g++")])
def test_headers_compile_as_strict_c_and_cxx(tmp_path, std, compiler):
    # each header alone (twice, for its include guard), then all together in
    # both orders, as a cgo or C host would include them
    orders = [[h, h] for h in HEADERS] + [HEADERS, HEADERS[::-1]]
    for k, order in enumerate(orders):
        src = tmp_path / f"h{k}.{'cc' if compiler == 'g++' else 'c'}"
        src.write_text("".join(f'#include "{h}"\n' for h in order) + "int main(void) { return 0; }\n")
        r = subprocess.run([compiler, f"-std={std}", "-pedantic-errors", "-Wall", "-Wextra", "-Werror",
                            "-fsyntax-only", "-I", INCLUDE, str(src)], capture_output=True, text=True)
        assert r.returncode == 0, (order, r.stderr)


def test_c99_program_links_every_declared_function(tmp_path):
    # a C99 caller that takes the address of every function the headers
    # declare links against the library and loads it
    names = declared_symbols()
    src = tmp_path / "link.c"
    src.write_text("".join(f'#include "{h}"\n' for h in HEADERS) + "#include <stdio.h>\n"
                   "typedef void (*fn)(void);\n"
                   "int main(void)\n{\n    int n = 0;\n"
                   + "".join(f"    n += (fn)&{s} != 0;\n" for s in names)
                   + '    printf("%d\\n", n);\n    return 0;\n}\n')
    exe = tmp_path / "link"
    lib_dir = os.path.dirname(M.LIB_PATH)
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-Wno-pedantic", "-I", INCLUDE, str(src), "-o", str(exe),
                        "-L", lib_dir, "-l:" + os.path.basename(M.LIB_PATH), f"-Wl,-rpath,{lib_dir}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and out.stdout.strip() == str(len(names)), (out.stdout, out.stderr)
