"""C-ABI and host-logic tests (no GPU needed).

- libmxrt.so loads and exports every function include/mxrt.h declares;
- graph building on a host_only backend: shape inference and the validation errors of
  FusedQuantizedDense (quantizeddense.go:92-130) and DotGeneral (dotgeneral.go:16-152), value
  ownership across builders, NotImplemented for unsupported configurations, and that every
  device operation fails loudly (no host fallback).
"""
import ctypes
import os
import re

import numpy as np
import pytest

import compute_amd as ca
from compute_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    text = open(os.path.join(ROOT, "include", "mxrt.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    names = _declared_functions()
    assert len(names) >= 50
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares a signature for each of them
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_backend_identity(host_backend):
    b = host_backend
    assert b.Name() == "mi355x"
    assert "MI355X" in b.Description()
    assert b.NumDevices() == 0
    assert not b.HasSharedBuffers()
    caps = b.Capabilities()
    assert caps.Operations.get(ca.OpType.FusedQuantizedDense)
    assert caps.Operations.get(ca.OpType.DotGeneral)
    assert not caps.Operations.get(ca.OpType.FusedScaledDotProductAttention, False)
    assert caps.DTypes.get(ca.BFloat16) and caps.DTypes.get(ca.Int4)


def test_bad_config_rejected():
    with pytest.raises(ca.ComputeError):
        ca.New("mi355x:frobnicate")


def test_device_operations_fail_loudly_host_only(host_backend):
    with pytest.raises(ca.ErrNoDevice):
        host_backend.BufferFromFlatData(0, np.zeros(4, np.float32), ca.Shape(ca.Float32, 4))
    with pytest.raises(ca.ErrNoDevice):
        host_backend.Synchronize()
    with pytest.raises(ca.ErrNoDevice):
        host_backend.DebugStreamRead([], 1)


def _qd_builder(b, xs, ws, ss, bias_shape=None):
    bld = b.Builder("qd")
    f = bld.Main()
    x = f.Parameter("x", xs)
    w = f.Parameter("w", ws)
    s = f.Parameter("s", ss)
    bias = f.Parameter("bias", bias_shape) if bias_shape else None
    return bld, f, x, w, s, bias


def test_qdense_shape_inference(host_backend):
    bld, f, x, w, s, bias = _qd_builder(host_backend, ca.Shape(ca.BFloat16, 2, 3, 64), ca.Shape(ca.Int4, 64, 40),
                                        ca.Shape(ca.BFloat16, 2, 40), ca.Shape(ca.BFloat16, 40))
    y = f.FusedQuantizedDense(x, w, bias, ca.Quantization(ca.QuantLinear, s, None, 0, 32), ca.ActivationSilu)
    assert f.Shape(y) == ca.Shape(ca.BFloat16, 2, 3, 40)
    assert bld.OpShape(y) == ca.Shape(ca.BFloat16, 2, 3, 40)
    f.Return([y])
    exe = bld.Compile()
    names, shapes = exe.Inputs()
    assert names == ["x", "w", "s", "bias"]
    assert exe.Outputs() == [ca.Shape(ca.BFloat16, 2, 3, 40)]


def test_qdense_reference_layout_and_per_channel_vector(host_backend):
    # Reference layout: BlockAxis=1, scale [K, ceil(N/B)] with a ragged last block.
    _, f, x, w, s, _ = _qd_builder(host_backend, ca.Shape(ca.Float32, 4, 16), ca.Shape(ca.Int8, 16, 10),
                                   ca.Shape(ca.Float32, 16, 3))
    y = f.FusedQuantizedDense(x, w, None, ca.Quantization(ca.QuantLinear, s, None, 1, 4), ca.ActivationNone)
    assert f.Shape(y) == ca.Shape(ca.Float32, 4, 10)
    # Per-output-channel scale given as [N].
    _, f, x, w, s, _ = _qd_builder(host_backend, ca.Shape(ca.Float32, 4, 16), ca.Shape(ca.Int8, 16, 10),
                                   ca.Shape(ca.Float32, 10))
    y = f.FusedQuantizedDense(x, w, None, ca.Quantization(ca.QuantLinear, s, None, 0, 16), ca.ActivationGelu)
    assert f.Shape(y) == ca.Shape(ca.Float32, 4, 10)


@pytest.mark.parametrize("case", ["wrongK", "scales", "bias", "axis", "nf4zp", "xint", "wfloat", "blocksize"])
def test_qdense_validation_errors(host_backend, case):
    b = host_backend
    bld = b.Builder("bad")
    f = bld.Main()
    x = f.Parameter("x", ca.Shape(ca.Int32 if case == "xint" else ca.Float32, 2, 16))
    w = f.Parameter("w", ca.Shape(ca.Float32 if case == "wfloat" else ca.Int8, 8 if case == "wrongK" else 16, 12))
    s = f.Parameter("s", ca.Shape(ca.Float32, 16, 5 if case == "scales" else 3))
    zp = f.Parameter("zp", ca.Shape(ca.Float32, 16, 3))
    bias = f.Parameter("b", ca.Shape(ca.Float32, 11 if case == "bias" else 12))
    q = ca.Quantization(ca.QuantNF4 if case == "nf4zp" else ca.QuantLinear, s, zp if case == "nf4zp" else None,
                        2 if case == "axis" else 1, 0 if case == "blocksize" else 4)
    expect = ca.ErrNotImplemented if case in ("xint", "wfloat") else ca.ComputeError
    with pytest.raises(expect) as ei:
        f.FusedQuantizedDense(x, w, bias, q, ca.ActivationNone)
    if expect is ca.ComputeError:
        assert not ca.IsNotImplemented(ei.value)


def _ggml_q(t):
    return ca.Quantization(ca.QuantGGML, None, None, 1, 1, int(t))


def test_qdense_ggml_shape_and_validation(host_backend):
    """FusedQuantizedDenseGGML's rules (quantizeddense.go:145-248)."""
    b = host_backend
    f = b.Builder("g").Main()
    x = f.Parameter("x", ca.Shape(ca.Float32, 2, 3, 512))
    w = f.Parameter("w", ca.Shape(ca.Uint8, 40, 512 // 32 * 18))
    bias = f.Parameter("b", ca.Shape(ca.Float32, 40))
    y = f.FusedQuantizedDense(x, w, bias, _ggml_q(ca.GGMLQ4_0), ca.ActivationGelu)
    assert f.Shape(y) == ca.Shape(ca.Float32, 2, 3, 40)
    wk = f.Parameter("wk", ca.Shape(ca.Uint8, 40, 2 * 210))
    assert f.Shape(f.FusedQuantizedDense(x, wk, None, _ggml_q(ca.GGMLQ6_K), ca.ActivationNone)) == \
        ca.Shape(ca.Float32, 2, 3, 40)
    # unsupported block formats are NotImplemented (validateGGMLTypeSupported)
    wq2 = f.Parameter("wq2", ca.Shape(ca.Uint8, 40, 2 * 84))
    with pytest.raises(ca.ErrNotImplemented):
        f.FusedQuantizedDense(x, wq2, None, _ggml_q(ca.GGMLQ2_K), ca.ActivationNone)
    bad = []
    # bytesPerRow not a multiple of the block size, x not f32, K mismatch, zero point, bad bias
    wodd = f.Parameter("wodd", ca.Shape(ca.Uint8, 40, 17))
    bad.append(lambda: f.FusedQuantizedDense(x, wodd, None, _ggml_q(ca.GGMLQ4_0), ca.ActivationNone))
    xb = f.Parameter("xb", ca.Shape(ca.BFloat16, 2, 512))
    bad.append(lambda: f.FusedQuantizedDense(xb, w, None, _ggml_q(ca.GGMLQ4_0), ca.ActivationNone))
    x2 = f.Parameter("x2", ca.Shape(ca.Float32, 2, 256))
    bad.append(lambda: f.FusedQuantizedDense(x2, w, None, _ggml_q(ca.GGMLQ4_0), ca.ActivationNone))
    zp = f.Parameter("zp", ca.Shape(ca.Float32, 40))
    bad.append(lambda: f.FusedQuantizedDense(x, w, None, ca.Quantization(ca.QuantGGML, None, zp, 1, 1, 0),
                                             ca.ActivationNone))
    b2 = f.Parameter("b2", ca.Shape(ca.Float32, 41))
    bad.append(lambda: f.FusedQuantizedDense(x, w, b2, _ggml_q(ca.GGMLQ4_0), ca.ActivationNone))
    wi = f.Parameter("wi", ca.Shape(ca.Int8, 40, 288))
    bad.append(lambda: f.FusedQuantizedDense(x, wi, None, _ggml_q(ca.GGMLQ4_0), ca.ActivationNone))
    for call in bad:
        with pytest.raises(ca.ComputeError) as ei:
            call()
        assert not ca.IsNotImplemented(ei.value)


def test_quantized_embedding_lookup_shape_and_validation(host_backend):
    """QuantizedEmbeddingLookup's rules (quantizeddense.go:266-321)."""
    f = host_backend.Builder("e").Main()
    data = f.Parameter("d", ca.Shape(ca.Uint8, 100, 2 * 34))
    idx = f.Parameter("i", ca.Shape(ca.Int32, 2, 3, 1))
    y = f.QuantizedEmbeddingLookup(data, idx, _ggml_q(ca.GGMLQ8_0))
    assert f.Shape(y) == ca.Shape(ca.Float32, 2, 3, 64)
    s = f.Parameter("s", ca.Shape(ca.Float32, 1))
    with pytest.raises(ca.ErrNotImplemented):
        f.QuantizedEmbeddingLookup(data, idx, ca.Quantization(ca.QuantLinear, s, None, 1, 1))
    with pytest.raises(ca.ErrNotImplemented):
        f.QuantizedEmbeddingLookup(data, idx, _ggml_q(ca.GGMLQ5_K))
    i2 = f.Parameter("i2", ca.Shape(ca.Int32, 2, 3))
    fi = f.Parameter("fi", ca.Shape(ca.Float32, 2, 1))
    d3 = f.Parameter("d3", ca.Shape(ca.Uint8, 100, 2, 34))
    for call in (lambda: f.QuantizedEmbeddingLookup(data, i2, _ggml_q(ca.GGMLQ8_0)),
                 lambda: f.QuantizedEmbeddingLookup(data, fi, _ggml_q(ca.GGMLQ8_0)),
                 lambda: f.QuantizedEmbeddingLookup(d3, idx, _ggml_q(ca.GGMLQ8_0)),
                 lambda: f.QuantizedEmbeddingLookup(data, idx, _ggml_q(ca.GGMLQ4_0))):  # 68 % 18 != 0
        with pytest.raises(ca.ComputeError) as ei:
            call()
        assert not ca.IsNotImplemented(ei.value)


def test_values_from_other_builder_rejected(host_backend):
    b1 = host_backend.Builder("one")
    b2 = host_backend.Builder("two")
    x1 = b1.Main().Parameter("x", ca.Shape(ca.Float32, 3))
    f2 = b2.Main()
    x2 = f2.Parameter("x", ca.Shape(ca.Float32, 3))
    with pytest.raises(ca.ComputeError, match="different builder"):
        f2.Add(x1, x2)


def test_return_then_modify_and_compile_rules(host_backend):
    bld = host_backend.Builder("r")
    f = bld.Main()
    x = f.Parameter("x", ca.Shape(ca.Float32, 3))
    f.Return([x])
    with pytest.raises(ca.ComputeError):
        f.Neg(x)
    bld.Compile()
    bld2 = host_backend.Builder("no-return")
    bld2.Main().Parameter("x", ca.Shape(ca.Float32, 3))
    with pytest.raises(ca.ComputeError, match="Return"):
        bld2.Compile()


def test_dot_general_shape_kat(host_backend):
    # support/backendtest/dotgeneral.go:26-81
    bld = host_backend.Builder("DotGeneral Test")
    f = bld.Main()
    lhs = f.Parameter("lhs", ca.Shape(ca.Float32, 2, 3, 4, 5))
    rhs = f.Parameter("rhs", ca.Shape(ca.Float32, 5, 1, 2, 3))
    y = f.DotGeneral(lhs, [1], [3, 0], rhs, [3], [0, 2])
    assert f.Shape(y) == ca.Shape(ca.Float32, 5, 2, 4, 1)
    y2 = f.DotGeneral(lhs, [1], [3, 0], rhs, [3], [0, 2], ca.DotGeneralConfig(OutputDType=ca.Float64))
    assert f.Shape(y2) == ca.Shape(ca.Float64, 5, 2, 4, 1)


def test_fused_dense_layout_shapes(host_backend):
    # fusedops/dense.go:59-80: InputOutputs contracts the weight's first axis, OutputsInput its last;
    # the output is x's leading dims followed by the weight's output dims.
    f = host_backend.Builder("dense").Main()
    x = f.Parameter("x", ca.Shape(ca.Float32, 2, 5, 3))
    w_io = f.Parameter("w_io", ca.Shape(ca.Float32, 3, 4, 6))
    w_oi = f.Parameter("w_oi", ca.Shape(ca.Float32, 4, 6, 3))
    b = f.Parameter("b", ca.Shape(ca.Float32, 4, 6))
    y = f.FusedDense(x, w_io, b, ca.DenseConfig(ca.ActivationRelu))
    assert f.Shape(y) == ca.Shape(ca.Float32, 2, 5, 4, 6)
    y = f.FusedDense(x, w_oi, b, ca.DenseConfig(ca.ActivationGelu, ca.DenseLayoutOutputsInput))
    assert f.Shape(y) == ca.Shape(ca.Float32, 2, 5, 4, 6)
    y = f.FusedDense(x, w_oi, None, ca.DenseConfig(WeightLayout=ca.DenseLayoutOutputsInput))
    assert f.Shape(y) == ca.Shape(ca.Float32, 2, 5, 4, 6)
    assert f.Shape(f.FusedDense(x, w_io, None)) == ca.Shape(ca.Float32, 2, 5, 4, 6)


@pytest.mark.parametrize("case", ["io_dim", "oi_dim", "layout", "rank"])
def test_fused_dense_layout_errors(host_backend, case):
    f = host_backend.Builder("dense").Main()
    x = f.Parameter("x", ca.Shape(ca.Float32, 2, 3))
    w = f.Parameter("w", ca.Shape(ca.Float32, 4, 3))  # [out, in]: wrong for InputOutputs
    w1 = f.Parameter("w1", ca.Shape(ca.Float32, 3))
    # The reference's messages (dense.go:52-53, 62-63, 71-72, 80).
    want, call = {
        "io_dim": (r"x's last dim \(3\) must match weight's first dim \(4\) for DenseLayoutInputOutputs",
                   lambda: f.FusedDense(x, w, None, ca.DenseConfig())),
        "oi_dim": (r"x's last dim \(3\) must match weight's last dim \(2\) for DenseLayoutOutputsInput",
                   lambda: f.FusedDense(x, f.Parameter("w2", ca.Shape(ca.Float32, 3, 2)), None,
                                        ca.DenseConfig(WeightLayout=ca.DenseLayoutOutputsInput))),
        "layout": ("unknown WeightLayout", lambda: f.FusedDense(x, w, None, ca.DenseConfig(WeightLayout=7))),
        "rank": (r"x must have rank >= 1 \(got 2\), weight must have rank >= 2 \(got 1\)",
                 lambda: f.FusedDense(x, w1, None)),
    }[case]
    with pytest.raises(ca.ComputeError, match="FusedDense: " + want):
        call()


@pytest.mark.parametrize("case", ["dtype", "ncontract", "dim", "reuse", "range"])
def test_dot_general_errors(host_backend, case):
    f = host_backend.Builder("e").Main()
    lhs = f.Parameter("l", ca.Shape(ca.Float32, 2, 3))
    rhs = f.Parameter("r", ca.Shape(ca.Float64 if case == "dtype" else ca.Float32, 4 if case == "dim" else 3, 5))
    args = {
        "dtype": ([1], [], [0], []), "ncontract": ([1], [], [0, 1], []), "dim": ([1], [], [0], []),
        "reuse": ([1, 1], [], [0, 1], []), "range": ([2], [], [0], []),
    }[case]
    with pytest.raises(ca.ComputeError):
        f.DotGeneral(lhs, args[0], args[1], rhs, args[2], args[3])


def test_binary_broadcast_rules(host_backend):
    f = host_backend.Builder("bin").Main()
    a = f.Parameter("a", ca.Shape(ca.BFloat16, 8, 1))
    b = f.Parameter("b", ca.Shape(ca.BFloat16, 8, 4096))
    s = f.Parameter("s", ca.Shape(ca.BFloat16))
    assert f.Shape(f.Mul(a, b)) == ca.Shape(ca.BFloat16, 8, 4096)
    assert f.Shape(f.Add(s, b)) == ca.Shape(ca.BFloat16, 8, 4096)
    c = f.Parameter("c", ca.Shape(ca.BFloat16, 4096))
    with pytest.raises(ca.ComputeError):
        f.Add(b, c)  # different rank, neither scalar
    d = f.Parameter("d", ca.Shape(ca.Float32, 8, 4096))
    with pytest.raises(ca.ComputeError):
        f.Add(b, d)  # dtype mismatch


def test_shape_ops_inference(host_backend):
    f = host_backend.Builder("shapes").Main()
    x = f.Parameter("x", ca.Shape(ca.Uint8, 6, 4))
    assert f.Shape(f.Bitcast(x, ca.Int4)) == ca.Shape(ca.Int4, 6, 4, 2)
    assert f.Shape(f.Reshape(f.Bitcast(x, ca.Int4), 6, 8)) == ca.Shape(ca.Int4, 6, 8)
    y = f.Parameter("y", ca.Shape(ca.Float32, 2, 3, 4))
    assert f.Shape(f.Transpose(y, 2, 0, 1)) == ca.Shape(ca.Float32, 4, 2, 3)
    assert f.Shape(f.ReduceSum(y, 1)) == ca.Shape(ca.Float32, 2, 4)
    assert f.Shape(f.ReduceSum(y)) == ca.Shape(ca.Float32)
    assert f.Shape(f.Slice(y, [0, 1, 0], [2, 3, 4], [1, 1, 2])) == ca.Shape(ca.Float32, 2, 2, 2)
    v = f.Parameter("v", ca.Shape(ca.Float32, 3))
    assert f.Shape(f.BroadcastInDim(v, ca.Shape(ca.Float32, 2, 3), [1])) == ca.Shape(ca.Float32, 2, 3)
    assert f.Shape(f.Iota(ca.Shape(ca.Float32, 16), 0)) == ca.Shape(ca.Float32, 16)
    with pytest.raises(ca.ComputeError):
        f.Reshape(y, 5, 5)


def test_fault_injection_flag_is_host_side(host_backend):
    # The knob is set on the host; the allocation it fails happens only on a device backend.
    host_backend.DebugFailAllocAfter(1)
    host_backend.DebugFailAllocAfter(0)


def _plan(backend, M, K, N, *, x_dtype, w_dtype, s_dtype, block_axis, block_size, zp=False, scheme=0, act=0):
    """Kernel choice for a problem; the pointers are aligned placeholders (planning reads no data)."""
    a = ca._lib.mx_qdense_args()
    a.x, a.w, a.scale, a.out = 0x10000, 0x20000, 0x30000, 0x40000
    if zp:
        a.zero_point = 0x50000
        a.zero_point_dtype = s_dtype
    a.M, a.K, a.N = M, K, N
    a.x_dtype, a.w_dtype, a.scale_dtype = int(x_dtype), int(w_dtype), int(s_dtype)
    a.scheme, a.block_axis, a.block_size, a.activation = scheme, block_axis, block_size, act
    return backend.QDensePlan(a)


def test_qdense_plan_selection():
    """Which kernel each regime takes (host-only planning): the MFMA decode kernel for bf16 x with
    K-blocked scales, the GEMV for the reference's own layout / f32 x / zero points / NF4 up to
    64 rows, the MFMA GEMM at prefill, the f32 dequantise-and-contract path for the reference
    layout past 64 rows, the reference-order kernel for small problems and for everything with
    the "exact" option."""
    F32, BF16 = ca.Float32, ca.BFloat16
    for opts, exact in (("host_only", False), ("host_only,exact", True)):
        b = ca.New(opts)
        try:
            def want(name):
                return "qdense_exact" if exact else name
            assert _plan(b, 1, 4096, 11008, x_dtype=BF16, w_dtype=ca.Int4, s_dtype=BF16, block_axis=0,
                         block_size=128) == want("qdense_skinny_mfma_i4")
            assert _plan(b, 1, 4096, 11008, x_dtype=F32, w_dtype=ca.Int4, s_dtype=F32, block_axis=1,
                         block_size=128) == want("qdense_gemv_i4")
            assert _plan(b, 3, 4096, 11008, x_dtype=F32, w_dtype=ca.Int8, s_dtype=F32, block_axis=1,
                         block_size=64, zp=True) == want("qdense_gemv_i8_zp")
            assert _plan(b, 1, 4096, 4096, x_dtype=F32, w_dtype=ca.Uint8, s_dtype=F32, block_axis=1,
                         block_size=128, scheme=1) == want("qdense_gemv_nf4_8bit")
            assert _plan(b, 2, 4096, 4096, x_dtype=BF16, w_dtype=ca.Uint4, s_dtype=BF16, block_axis=0,
                         block_size=64, zp=True) == want("qdense_gemv_u4_zp")
            assert _plan(b, 1, 4096, 4096, x_dtype=F32, w_dtype=ca.Int4, s_dtype=F32, block_axis=0,
                         block_size=4096) == want("qdense_gemv_i4")
            assert _plan(b, 2048, 4096, 4096, x_dtype=BF16, w_dtype=ca.Int8, s_dtype=F32, block_axis=0,
                         block_size=4096) == want("qdense_gemm_mfma_i8")
            # Past the skinny kernel's 16 rows, bf16 x runs the skinny kernel once per group of 16
            # rows up to 48 rows (per-channel scales) or 64 (scale groups), then the GEMM (weights
            # read once); never the GEMV (weights re-read for every 4 rows).
            for M, per_channel, grouped in ((17, "skinny_rows16", "skinny_rows16"), (48, "skinny_rows16", "skinny_rows16"),
                                            (49, "gemm_mfma", "skinny_rows16"), (64, "gemm_mfma", "skinny_rows16"),
                                            (65, "gemm_mfma", "gemm_mfma")):
                assert _plan(b, M, 4096, 11008, x_dtype=BF16, w_dtype=ca.Int8, s_dtype=F32, block_axis=0,
                             block_size=4096) == want(f"qdense_{per_channel}_i8")
                assert _plan(b, M, 4096, 11008, x_dtype=BF16, w_dtype=ca.Uint8, s_dtype=BF16, block_axis=0,
                             block_size=4096) == want(f"qdense_{per_channel}_u8")
                sfx = "_grouped" if grouped == "gemm_mfma" else ""
                assert _plan(b, M, 4096, 14336, x_dtype=BF16, w_dtype=ca.Int4, s_dtype=BF16, block_axis=0,
                             block_size=128) == want(f"qdense_{grouped}_i4{sfx}")
            # Rows that start mid-word (odd N): the GEMV's two-word loads (the MFMA kernels need
            # aligned rows).
            assert _plan(b, 1, 4096, 32001, x_dtype=BF16, w_dtype=ca.Int4, s_dtype=BF16, block_axis=0,
                         block_size=128) == want("qdense_gemv_i4")
            assert _plan(b, 4, 4096, 32001, x_dtype=F32, w_dtype=ca.Int8, s_dtype=F32, block_axis=1,
                         block_size=128) == want("qdense_gemv_i8")
            # ... past 64 rows as well, once the weights reach 2^24 (the GEMV per four rows beats
            # the exact kernel there); smaller weights keep the exact kernel.
            assert _plan(b, 512, 4096, 32001, x_dtype=F32, w_dtype=ca.Int4, s_dtype=F32, block_axis=1,
                         block_size=128) == want("qdense_gemv_i4")
            assert _plan(b, 512, 1024, 1031, x_dtype=F32, w_dtype=ca.Int4, s_dtype=F32, block_axis=1,
                         block_size=64) == want("qdense_exact")
            # Where the GEMM does not fit (f32 x here), rows up to 64 stay on the GEMV.
            assert _plan(b, 32, 4096, 11008, x_dtype=F32, w_dtype=ca.Int8, s_dtype=F32, block_axis=0,
                         block_size=64) == want("qdense_gemv_i8")
            # Prefill with 4-bit weights and K-grouped scales: the GEMM with a scale-group fold.
            assert _plan(b, 2048, 4096, 14336, x_dtype=BF16, w_dtype=ca.Int4, s_dtype=BF16, block_axis=0,
                         block_size=128) == want("qdense_gemm_mfma_i4_grouped")
            assert _plan(b, 512, 4096, 4096, x_dtype=BF16, w_dtype=ca.Uint4, s_dtype=F32, block_axis=0,
                         block_size=4096) == want("qdense_gemm_mfma_u4")
            assert _plan(b, 2048, 4096, 14336, x_dtype=BF16, w_dtype=ca.Int8, s_dtype=BF16, block_axis=0,
                         block_size=64) == want("qdense_gemm_mfma_i8_grouped")
            # Groups that do not tile K in 64-row blocks take the f32 dequantise-and-contract path,
            # except groups of 32 rows (two per block, each step folded).
            assert _plan(b, 2048, 4096, 4096, x_dtype=BF16, w_dtype=ca.Int4, s_dtype=BF16, block_axis=0,
                         block_size=96) == want("qdense_refgemm_f32_mfma")
            for s_dt in (BF16, F32):
                assert _plan(b, 2048, 4096, 4096, x_dtype=BF16, w_dtype=ca.Int4, s_dtype=s_dt, block_axis=0,
                             block_size=32) == want("qdense_gemm_mfma_i4_grouped")
            # Small problems, M > 64 with the reference layout, unsupported block sizes: reference order.
            assert _plan(b, 1, 512, 1024, x_dtype=F32, w_dtype=ca.Int8, s_dtype=F32, block_axis=1,
                         block_size=64) == "qdense_exact"
            assert _plan(b, 8, 4096, 4096, x_dtype=F32, w_dtype=ca.Int8, s_dtype=F32, block_axis=1,
                         block_size=64) == want("qdense_gemv_i8")
            # Past the GEMV's 64 rows, the reference layout dequantises into f32 for the matrix cores.
            assert _plan(b, 65, 4096, 4096, x_dtype=F32, w_dtype=ca.Int8, s_dtype=F32, block_axis=1,
                         block_size=64) == want("qdense_refgemm_f32_mfma")
            assert _plan(b, 512, 4096, 4096, x_dtype=BF16, w_dtype=ca.Uint4, s_dtype=F32, block_axis=1,
                         block_size=128, scheme=1) == want("qdense_refgemm_f32_mfma")
            assert _plan(b, 1, 4096, 4096, x_dtype=F32, w_dtype=ca.Int8, s_dtype=F32, block_axis=1,
                         block_size=16) == "qdense_exact"
            # The reference's BenchmarkQuantizedDense shapes (at most 2^24 multiply-adds) keep the
            # exact kernel; one row more takes the dequantise-and-contract path.
            for scheme, w_dt in ((0, ca.Int8), (1, ca.Uint8)):
                assert _plan(b, 32, 512, 1024, x_dtype=F32, w_dtype=w_dt, s_dtype=F32, block_axis=1,
                             block_size=128, scheme=scheme) == "qdense_exact"
                assert _plan(b, 33, 512, 1024, x_dtype=F32, w_dtype=w_dt, s_dtype=F32, block_axis=1,
                             block_size=128, scheme=scheme) == want("qdense_refgemm_f32_mfma")
        finally:
            b.Finalize()
    b = ca.New("host_only,gemv_over_gemm")
    try:
        assert _plan(b, 32, 4096, 11008, x_dtype=BF16, w_dtype=ca.Int8, s_dtype=F32, block_axis=0,
                     block_size=4096) == "qdense_gemv_i8"
        assert _plan(b, 2048, 4096, 4096, x_dtype=BF16, w_dtype=ca.Int8, s_dtype=F32, block_axis=0,
                     block_size=4096) == "qdense_gemm_mfma_i8"
    finally:
        b.Finalize()
