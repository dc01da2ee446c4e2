"""GPU mirror of the reference's backend compliance suite (support/backendtest) for every op the
backend declares in Capabilities: the suite's literal inputs and expected values
(tests/golden/backendtest_cases.json, each case citing its source lines), run through Builder ->
Compile -> Execute on the device and compared the way testutil compares them (IsEqual: integers
exactly, floats by value; IsInDelta / IsInRelativeDelta with the suite's tolerances).  Exec's
error cases (support/backendtest/exec.go:72-111) and FusedGelu's exact/approximate check
(fusedops.go:89-124) are written out below; DotGeneral, FusedDense, FusedQuantizedDense and
QuantizedEmbeddingLookup have their own GPU suites (test_gpu_dot, test_gpu_qdense, test_gpu_ggml).
A test also checks that every declared op has a case here or in those suites.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from compute_amd import backend as B
from compute_amd.dtypes import DType, Shape
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = json.loads((GOLDEN / "backendtest_cases.json").read_text())["cases"]
KATS = json.loads((GOLDEN / "reference_kats.json").read_text())

# Ops whose compliance cases live in other GPU test modules.
COVERED_ELSEWHERE = {
    B.OpType.DotGeneral: "test_gpu_dot.py (dotgeneral.go KATs)",
    B.OpType.FusedDense: "test_gpu_dot.py (fusedops.go FusedDense KATs)",
    B.OpType.FusedQuantizedDense: "test_gpu_qdense.py / test_gpu_skinny.py / test_gpu_gemm.py / test_gpu_gemv.py",
    B.OpType.QuantizedEmbeddingLookup: "test_gpu_ggml.py",
    B.OpType.Parameter: "every case below",
    B.OpType.Constant: "test_exec_compile_and_execute",
    B.OpType.FusedGelu: "test_fused_gelu_exact_and_approximate",
}


def host_array(spec) -> np.ndarray:
    """A fixture tensor as flat host storage of its dtype."""
    dt = DType[spec["dtype"]]
    shape = spec["shape"]
    n = int(np.prod(shape)) if shape else 1
    if spec.get("iota"):
        vals = np.arange(n, dtype=np.float64)
    elif "rows" in spec:
        vals = np.repeat(np.asarray(spec["rows"], np.float64), shape[1])
    else:
        vals = np.asarray(spec["data"], dtype=np.float64 if dt.is_float() else object)
    if dt == DType.BFloat16:
        return O.bf16_round(vals.astype(np.float32)).ravel()
    if dt == DType.Float16:
        return vals.astype(np.float16).ravel()
    if dt == DType.Bool:
        return vals.astype(np.int64).astype(np.bool_).ravel()
    return np.asarray([int(v) for v in vals] if not dt.is_float() else vals, dtype=dt.numpy_storage()).ravel()


def as_values(arr: np.ndarray, dt: DType) -> np.ndarray:
    """Stored values as numbers: half types widened to f64, the rest as stored."""
    if dt == DType.BFloat16:
        return O.bf16_to_f32(arr).astype(np.float64)
    if dt in (DType.Float16, DType.Float32, DType.Float64):
        return arr.astype(np.float64)
    if dt == DType.Bool:
        return arr.astype(np.int64)
    return arr


def build_op(f, case, params):
    op, at = case["op"], case.get("attrs", {})
    if op == "ConvertDType":
        return f.ConvertDType(params[0], DType[at["dtype"]])
    if op == "Bitcast":
        return f.Bitcast(params[0], DType[at["dtype"]])
    if op == "Reshape":
        return f.Reshape(params[0], *at["dims"])
    if op in ("ReduceMax", "ReduceSum"):
        return getattr(f, op)(params[0], *at["axes"])
    if op == "Transpose":
        return f.Transpose(params[0], *at["perm"])
    if op == "Iota":
        return f.Iota(Shape(DType[at["dtype"]], *at["shape"]), at["axis"])
    if op == "BroadcastInDim":
        return f.BroadcastInDim(params[0], Shape(DType[at["dtype"]], *at["shape"]), at["axes"])
    if op == "Slice":
        return f.Slice(params[0], at["starts"], at["limits"], at["strides"])
    if op == "FusedGelu":
        return f.FusedGelu(params[0], at["exact"])
    return getattr(f, op)(*params)


def exec1(backend, case):
    """testutil.Exec1: parameters from the inputs, one op, one output."""
    bld = backend.Builder(case["name"])
    f = bld.Main()
    shapes = [Shape(DType[s["dtype"]], *s["shape"]) for s in case["inputs"]]
    params = [f.Parameter(f"p{i}", sh) for i, sh in enumerate(shapes)]
    f.Return([build_op(f, case, params)])
    exe = bld.Compile()
    bufs = [backend.BufferFromFlatData(0, host_array(s), sh) for s, sh in zip(case["inputs"], shapes)]
    return exe.Execute(bufs)[0]


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_backendtest_case(backend, case):
    out = exec1(backend, case)
    want = case["want"]
    wdt = DType[want["dtype"]]
    shape = out.Shape()
    assert shape.dtype == wdt, f"{case['name']}: dtype {shape.dtype}"
    assert list(shape.dimensions) == want["shape"], f"{case['name']}: shape {shape.dimensions}"
    got = as_values(out.ToFlatData(), wdt)
    exp = as_values(host_array(want), wdt)
    if case["cmp"] == "equal":
        assert np.array_equal(got.ravel(), np.asarray(exp).ravel()), f"{case['name']}: {got} != {exp}"
    elif case["cmp"] == "delta":
        assert np.all(np.abs(got.astype(np.float64).ravel() - np.asarray(exp, np.float64).ravel()) <= case["tol"]), \
            f"{case['name']}: {got} vs {exp}"
    else:  # relative
        e = np.asarray(exp, np.float64).ravel()
        assert np.all(np.abs(got.astype(np.float64).ravel() - e) <= case["tol"] * np.abs(e)), f"{case['name']}"


def test_every_declared_op_has_a_case(backend):
    declared = set(backend.Capabilities().Operations)
    ops_here = {B.OpType[c["op"]] for c in CASES}
    missing = [op.name for op in declared if op not in ops_here and op not in COVERED_ELSEWHERE]
    assert not missing, f"declared ops without a compliance case: {missing}"


# ---------------------------------------------------------------------------------------------
# Exec (support/backendtest/exec.go:16-111).
# ---------------------------------------------------------------------------------------------
def test_exec_compile_and_execute(backend):
    """exec.go:16-69: Neg of a parameter and an int64 constant, two outputs."""
    bld = backend.Builder("test")
    f = bld.Main()
    x = f.Parameter("x", Shape(DType.Float32, 3))
    f.Return([f.Neg(x), f.Constant(np.array([1, 2, 3], np.int64), 3)])
    exe = bld.Compile()
    outs = exe.Execute([backend.BufferFromFlatData(0, np.array([3, 5, 7], np.float32), Shape(DType.Float32, 3))],
                       [False])
    assert len(outs) == 2
    assert np.array_equal(outs[0].ToFlatData(), np.array([-3, -5, -7], np.float32))
    assert outs[1].Shape().dtype == DType.Int64
    assert np.array_equal(outs[1].ToFlatData(), np.array([1, 2, 3], np.int64))


def _identity_exec(backend):
    bld = backend.Builder("test_err")
    f = bld.Main()
    f.Return([f.Parameter("x", Shape(DType.Float32, 3))])
    return bld.Compile()


def test_exec_wrong_number_of_parameters(backend):
    """exec.go:72-85: two buffers for a one-parameter function is an error."""
    exe = _identity_exec(backend)
    bufs = [backend.BufferFromFlatData(0, np.array([1, 2, 3], np.float32), Shape(DType.Float32, 3)) for _ in range(2)]
    with pytest.raises(B.ComputeError):
        exe.Execute(bufs, [True, True])


def test_exec_incompatible_parameters(backend):
    """exec.go:87-111: a buffer of another size, or of another dtype, is an error."""
    exe = _identity_exec(backend)
    with pytest.raises(B.ComputeError):
        exe.Execute([backend.BufferFromFlatData(0, np.array([1, 2, 3, 4], np.float32), Shape(DType.Float32, 4))], [True])
    with pytest.raises(B.ComputeError):
        exe.Execute([backend.BufferFromFlatData(0, np.array([1, 2, 3], np.uint32), Shape(DType.Uint32, 3))], [True])


# ---------------------------------------------------------------------------------------------
# FusedGelu (support/backendtest/fusedops.go:89-124).
# ---------------------------------------------------------------------------------------------
def test_fused_gelu_exact_and_approximate(backend):
    case = next(c for c in CASES if c["name"] == "FusedGelu/Exact")
    exact = exec1(backend, case).ToFlatData()
    assert np.all(np.abs(exact - np.asarray(case["want"]["data"], np.float32)) <= 1e-6)
    approx_case = dict(case, name="FusedGelu/Approximate", attrs={"exact": False})
    approx = exec1(backend, approx_case).ToFlatData()
    assert np.any(np.abs(approx - exact) > 1e-7), "approximate and exact GELU should differ for non-zero inputs"


# ---------------------------------------------------------------------------------------------
# Bitcast Uint8 -> Int4 (internal/gobackend/ops/bitcast_test.go:51-118): a pure reinterpretation,
# donated or not.  Through the builder the narrower target appends a trailing axis of
# srcBits / dstBits (shapeinference/shapeinference.go:1604), so uint8[2] becomes Int4[2, 2]; a
# Reshape gives the KAT's Int4[4].  The raw bytes stay the source's, and the packed nibbles read
# as the reference's Int4 values (low nibble first).
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("key,donate", [("bytes", False), ("owned_bytes", True)])
def test_bitcast_uint8_to_int4_kat(backend, key, donate):
    kat = KATS["bitcast_uint8_to_int4"]
    src = np.asarray(kat[key], np.uint8)
    bld = backend.Builder("bitcast_int4")
    f = bld.Main()
    x = f.Parameter("x", Shape(DType.Uint8, len(src)))
    y = f.Bitcast(x, DType.Int4)
    assert list(f.Shape(y).dimensions) == [len(src), 2]
    f.Return([y, f.Reshape(y, *kat["int4_shape"])])
    exe = bld.Compile()
    outs = exe.Execute([backend.BufferFromFlatData(0, src, Shape(DType.Uint8, len(src)))], [donate])
    assert list(outs[1].Shape().dimensions) == kat["int4_shape"] and outs[1].Shape().dtype == DType.Int4
    for o in outs:
        assert np.array_equal(o.ToFlatData(), src)
    assert np.array_equal(O.unpack_int4(outs[1].ToFlatData(), signed=True),
                          [((b >> s & 15) ^ 8) - 8 for b in src.tolist() for s in (0, 4)])


# ---------------------------------------------------------------------------------------------
# Measurement hooks of the benchmark (no reference counterpart): the streaming-floor pass rotates
# over its buffers, writes nothing, shows in the per-kernel profile and in a timed region, and
# rejects finalized buffers.
# ---------------------------------------------------------------------------------------------
def test_stream_read_measurement_hook(backend):
    rng = np.random.default_rng(3)
    data = [rng.integers(0, 256, (1 << 20) + 40, dtype=np.uint8) for _ in range(2)]
    bufs = [backend.BufferFromFlatData(0, d, Shape(DType.Uint8, d.size)) for d in data]
    backend.SetProfiling(True)
    backend.ProfileReset()
    try:
        backend.RegionBegin()
        backend.DebugStreamRead(bufs, 3, 64)
        backend.DebugStreamRead(bufs, 2)
        assert backend.RegionEnd() > 0
        prof = backend.Profile()
    finally:
        backend.SetProfiling(False)
    assert prof["stream_read"][0] == 5
    for b, d in zip(bufs, data):
        assert np.array_equal(b.ToFlatData(), d)
    backend.DebugStreamRead(bufs, 0)
    bufs[1].Finalize()
    with pytest.raises(B.ErrFinalized):
        backend.DebugStreamRead(bufs, 1)
    with pytest.raises(B.ComputeError):
        backend.DebugStreamRead([bufs[0]], -1)
