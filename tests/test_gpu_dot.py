"""DotGeneral and FusedDense on the GPU (the contraction FusedQuantizedDense lowers onto),
mirroring the reference's compliance cases (support/backendtest/dotgeneral.go, fusedops.go):
known answers from tests/golden/reference_kats.json, the dtype matrix, the TransposedLarge
brute force with the reference's own tolerance (abs 0.5 or rel 3%), and seeded random batched /
transposed layouts against the f64 restatement (oracle.dot_general)."""
import json
import os

import numpy as np
import pytest

import compute_amd as ca
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def run(backend, inputs, build):
    """inputs: [(numpy storage array, DType)]; build(f, params) -> Value.  Returns the output."""
    bld = backend.Builder("dot")
    f = bld.Main()
    params = [f.Parameter(f"p{i}", ca.Shape(dt, *a.shape)) for i, (a, dt) in enumerate(inputs)]
    f.Return([build(f, params)])
    exe = bld.Compile()
    bufs = [backend.BufferFromFlatData(0, a.ravel(), ca.Shape(dt, *a.shape)) for a, dt in inputs]
    out = exe.Execute(bufs)[0]
    sh = out.Shape()
    return out.ToFlatData().reshape(sh.dimensions), sh.dtype


def test_shuffled_axes_kat(backend):
    k = GOLDEN["dot_general_shuffled_axes"]
    lhs = np.arange(1, 1 + np.prod(k["lhs_iota_from_1_shape"]), dtype=np.float32).reshape(k["lhs_iota_from_1_shape"])
    rhs = np.arange(1, 1 + np.prod(k["rhs_iota_from_1_shape"]), dtype=np.float32).reshape(k["rhs_iota_from_1_shape"])
    y, _ = run(backend, [(lhs, ca.Float32), (rhs, ca.Float32)],
               lambda f, p: f.DotGeneral(p[0], k["lhs_contracting"], k["lhs_batch"], p[1], k["rhs_contracting"],
                                         k["rhs_batch"]))
    assert np.array_equal(y, np.array(k["want"], np.float32))


def test_axis_transposition_kat(backend):
    k = GOLDEN["dot_general_axis_transposition"]
    y, _ = run(backend, [(np.array(k["lhs"], np.float32), ca.Float32), (np.array(k["rhs"], np.float32), ca.Float32)],
               lambda f, p: f.DotGeneral(p[0], k["lhs_contracting"], k["lhs_batch"], p[1], k["rhs_contracting"],
                                         k["rhs_batch"]))
    assert np.array_equal(y, np.array(k["want"], np.float32))


def test_f64_very_large_kat(backend):
    k = GOLDEN["dot_general_f64_very_large"]
    lhs = ((np.arange(np.prod(k["lhs_shape"])) + 1.0) * 1e-5).reshape(k["lhs_shape"])
    rhs = np.ones(k["rhs_shape"])
    y, dt = run(backend, [(lhs, ca.Float64), (rhs, ca.Float64)], lambda f, p: f.DotGeneral(p[0], [2], [], p[1], [0], []))
    assert dt == ca.Float64 and abs(y[0, 0, 0] - k["want_out_0_0_0"]) < k["tolerance"]
    assert np.allclose(y, O.dot_general(lhs, [2], [], rhs, [0], []), rtol=1e-12, atol=0)


def test_bf16_f32_accumulation_kat(backend):
    k = GOLDEN["dot_general_bf16_f32_acc"]
    lhs = O.bf16_round(np.array(k["lhs"], np.float32))
    rhs = O.bf16_round(np.array(k["rhs"], np.float32))
    y, dt = run(backend, [(lhs, ca.BFloat16), (rhs, ca.BFloat16)],
                lambda f, p: f.DotGeneral(p[0], [1], [], p[1], [0], [], ca.DotGeneralConfig(AccumulatorDType=ca.Float32)))
    assert dt == ca.BFloat16 and O.bf16_to_f32(y)[0, 0] == k["want"]


def test_small_matmul_kats(backend):
    k = GOLDEN["dot_general_small_matmul"]
    a, b = np.array(k["a"], np.float32), np.array(k["b"], np.float32)
    for rc, want in (([0], k["non_transposed"]), ([1], k["transposed"])):
        y, _ = run(backend, [(a, ca.Float32), (b, ca.Float32)], lambda f, p: f.DotGeneral(p[0], [1], [], p[1], rc, []))
        assert np.array_equal(y, np.array(want, np.float32))
    vec, mat, mat2 = (np.array(k[n], np.float32) for n in ("vec", "mat", "mat2"))
    y, _ = run(backend, [(vec, ca.Float32), (mat, ca.Float32)], lambda f, p: f.DotGeneral(p[0], [0], [], p[1], [0], []))
    assert np.array_equal(y, np.array(k["vec_mat"], np.float32))
    y, _ = run(backend, [(mat2, ca.Float32), (vec, ca.Float32)], lambda f, p: f.DotGeneral(p[0], [1], [], p[1], [0], []))
    assert np.array_equal(y, np.array(k["mat_vec"], np.float32))


def test_dot_product_kats(backend):
    k = GOLDEN["dot_general_dot"]
    x, yv, x2 = (np.array(k[n], np.float32) for n in ("x", "y", "x2"))
    y, _ = run(backend, [(x, ca.Float32), (yv, ca.Float32)], lambda f, p: f.DotGeneral(p[0], [0], [], p[1], [0], []))
    assert float(y) == k["want"]
    y, _ = run(backend, [(x2, ca.Float32), (yv, ca.Float32)], lambda f, p: f.DotGeneral(p[0], [1], [], p[1], [0], []))
    assert np.array_equal(y, np.array(k["want2"], np.float32))


FLOATS = [ca.Float16, ca.BFloat16, ca.Float32, ca.Float64]


@pytest.mark.parametrize("in_dt", FLOATS)
@pytest.mark.parametrize("acc_dt", [ca.InvalidDType] + FLOATS)
@pytest.mark.parametrize("out_dt", [ca.InvalidDType] + FLOATS)
def test_dtype_matrix(backend, in_dt, acc_dt, out_dt):
    """dotgeneral.go:444-497: iota(16) . iota(16) = 1240 for every input/accumulator/output dtype;
    the output dtype is OutputDType, or the input dtype when unset."""
    def build(f, _):
        lhs = f.Iota(ca.Shape(in_dt, 16), 0)
        rhs = f.Iota(ca.Shape(in_dt, 16), 0)
        return f.DotGeneral(lhs, [0], [], rhs, [0], [], ca.DotGeneralConfig(AccumulatorDType=acc_dt, OutputDType=out_dt))

    try:
        y, dt = run(backend, [], build)
    except ca.ErrNotImplemented as e:
        pytest.skip(f"combination not implemented: {e}")
    want_dt = out_dt if out_dt != ca.InvalidDType else in_dt
    assert dt == want_dt
    v = float(O.bf16_to_f32(y)) if dt == ca.BFloat16 else float(y)
    assert v == 1240.0


def test_transposed_large(backend):
    """dotgeneral.go:499-599, same data and tolerance (abs 0.5 or rel 3%)."""
    lhs = (np.arange(4 * 32 * 8 * 2, dtype=np.float64) * 1e-4).astype(np.float32)
    lhs = np.repeat(lhs, 256).reshape(4, 32, 8, 2, 256)
    rhs = (np.arange(4 * 32 * 8 * 256, dtype=np.float64) * 1e-4).astype(np.float32).reshape(4, 32, 8, 256)
    y, _ = run(backend, [(lhs, ca.Float32), (rhs, ca.Float32)],
               lambda f, p: f.DotGeneral(p[0], [4], [0, 2], p[1], [3], [0, 2]))
    want = O.dot_general(lhs.astype(np.float64), [4], [0, 2], rhs.astype(np.float64), [3], [0, 2]).astype(np.float32)
    assert y.shape == want.shape == (4, 8, 32, 2, 32)
    diff = np.abs(y - want)
    assert np.all((diff <= 0.5) | (diff / np.maximum(np.abs(want), 1e-30) < 0.03))


@pytest.mark.parametrize("dt", [ca.Float32, ca.BFloat16, ca.Float16])
@pytest.mark.parametrize("transposed", [False, True])
def test_random_batched(backend, dt, transposed):
    """[B, M, K] x [B, K, N] (or [B, N, K]) with random data vs the f64 restatement: f32 within
    1e-5 of sum|terms|; half precision (f32 accumulation, rounded output) within rel 1e-2 /
    abs 1e-3 of the f64 value."""
    rng = np.random.default_rng(int(dt) + 7 * transposed)
    B, M, K, N = 3, 70, 130, 90
    lf = rng.standard_normal((B, M, K)).astype(np.float32)
    rf = rng.standard_normal((B, N, K) if transposed else (B, K, N)).astype(np.float32)
    if dt == ca.BFloat16:
        lhs, rhs = O.bf16_round(lf), O.bf16_round(rf)
        lv, rv = O.bf16_to_f32(lhs), O.bf16_to_f32(rhs)
    elif dt == ca.Float16:
        lhs, rhs = lf.astype(np.float16), rf.astype(np.float16)
        lv, rv = lhs.astype(np.float32), rhs.astype(np.float32)
    else:
        lhs, rhs, lv, rv = lf, rf, lf, rf
    rc = [2] if transposed else [1]
    y, odt = run(backend, [(lhs, dt), (rhs, dt)], lambda f, p: f.DotGeneral(p[0], [2], [0], p[1], rc, [0]))
    assert odt == dt
    truth = O.dot_general(lv.astype(np.float64), [2], [0], rv.astype(np.float64), rc, [0])
    got = O.bf16_to_f32(y) if dt == ca.BFloat16 else y.astype(np.float32)
    if dt == ca.Float32:
        scale = O.dot_general(np.abs(lv).astype(np.float64), [2], [0], np.abs(rv).astype(np.float64), rc, [0])
        assert np.all(np.abs(got - truth) <= 1e-5 * scale)
    else:
        assert np.all(np.abs(got - truth) <= 1e-3 + 1e-2 * np.abs(truth))


@pytest.mark.parametrize("layout", [ca.DenseLayoutInputOutputs, ca.DenseLayoutOutputsInput])
@pytest.mark.parametrize("case", ["fused_dense_none", "fused_dense_relu"])
def test_fused_dense_kats(backend, case, layout):
    # support/backendtest/fusedops.go:178-212; with DenseLayoutOutputsInput the same weights are
    # given transposed ([out, in]) and the expected values are the same.
    k = GOLDEN[case]
    act = ca.ActivationNone if case.endswith("none") else ca.ActivationRelu
    x, w, b = (np.array(k[n], np.float32) for n in ("x", "w", "bias"))
    if layout == ca.DenseLayoutOutputsInput:
        w = np.ascontiguousarray(w.T)
    y, _ = run(backend, [(x, ca.Float32), (w, ca.Float32), (b, ca.Float32)],
               lambda f, p: f.FusedDense(p[0], p[1], p[2], ca.DenseConfig(act, layout)))
    assert np.array_equal(y, np.array(k["want"], np.float32))


@pytest.mark.parametrize("layout", [ca.DenseLayoutInputOutputs, ca.DenseLayoutOutputsInput])
@pytest.mark.parametrize("act", range(6))
def test_fused_dense_random(backend, act, layout):
    rng = np.random.default_rng(act + 10 * int(layout))
    x = rng.standard_normal((33, 100)).astype(np.float32)
    w = (rng.standard_normal((100, 50)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(50) * 0.1).astype(np.float32)
    wg = w if layout == ca.DenseLayoutInputOutputs else np.ascontiguousarray(w.T)
    y, _ = run(backend, [(x, ca.Float32), (wg, ca.Float32), (b, ca.Float32)],
               lambda f, p: f.FusedDense(p[0], p[1], p[2], ca.DenseConfig(ca.ActivationType(act), layout)))
    rc = 0 if layout == ca.DenseLayoutInputOutputs else 1
    pre = O.dot_general(x.astype(np.float64), [1], [], wg.astype(np.float64), [rc], []) + b
    want = O.act(pre.astype(np.float32), act)
    scale = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64) + np.abs(b)
    assert np.all(np.abs(y - want) <= 1e-5 * scale + 1e-6)


@pytest.mark.parametrize("dt", [ca.Float32, ca.BFloat16])
@pytest.mark.parametrize("shape", [((2, 7, 64), (3, 5, 64)), ((300, 512), (1024, 512))])
def test_fused_dense_outputs_input_shapes(backend, dt, shape):
    """DenseLayoutOutputsInput with several output axes ([out..., in]) and at a matrix-core size:
    output dims are x's leading dims then the weight's leading dims (dense.go:69-77)."""
    xs, ws = shape
    rng = np.random.default_rng(len(xs) + len(ws))
    x = rng.standard_normal(xs).astype(np.float32)
    w = (rng.standard_normal(ws) * 0.1).astype(np.float32)
    b = (rng.standard_normal(ws[:-1]) * 0.1).astype(np.float32)
    if dt == ca.BFloat16:
        x, w, b = (O.bf16_to_f32(O.bf16_round(a)) for a in (x, w, b))
        ins = [(O.bf16_round(a), dt) for a in (x, w, b)]
    else:
        ins = [(a, dt) for a in (x, w, b)]
    y, odt = run(backend, ins, lambda f, p: f.FusedDense(p[0], p[1], p[2],
                                                       ca.DenseConfig(ca.ActivationSilu, ca.DenseLayoutOutputsInput)))
    assert odt == dt and y.shape == xs[:-1] + ws[:-1]
    got = O.bf16_to_f32(y) if dt == ca.BFloat16 else y
    pre = O.dot_general(x.astype(np.float64), [len(xs) - 1], [], w.astype(np.float64), [len(ws) - 1], []) + b
    want = O.act(pre.astype(np.float32), ca.ActivationSilu)
    if dt == ca.Float32:
        scale = O.dot_general(np.abs(x).astype(np.float64), [len(xs) - 1], [], np.abs(w).astype(np.float64),
                              [len(ws) - 1], []) + np.abs(b)
        assert np.all(np.abs(got - want) <= 1e-5 * scale + 1e-6)
    else:
        assert np.all(np.abs(got - want) <= 1e-3 + 1e-2 * np.abs(want))


# ---------------------------------------------------------------------------------------------
# Half-precision DotGeneral on the matrix cores (qdense_gemm.hip, dot_mfma_*): large enough
# contractions with K % 64 == 0 and N % 16 == 0 take it; its f32 sums differ from a sequential
# sum only in order (every half product is exact in f32).
# ---------------------------------------------------------------------------------------------
def _half(rng, shape, dt):
    f = rng.standard_normal(shape).astype(np.float32)
    if dt == ca.BFloat16:
        h = O.bf16_round(f)
        return h, O.bf16_to_f32(h)
    h = f.astype(np.float16)
    return h, h.astype(np.float32)


def _half_kernel(dt, shape):
    """The half-precision kernel dot.hip picks: qdense_gemm.hip's 256x128 tiles when K % 64 == 0,
    N % 16 == 0, M >= 256 and they give >= 64 workgroups, else the small-tile kernel."""
    B, M, K, N = shape
    name = "dot_mfma_bf16" if dt == ca.BFloat16 else "dot_mfma_f16"
    big = K % 64 == 0 and N % 16 == 0 and M >= 256 and B * -(-M // 256) * -(-N // 128) >= 64
    return name if big else name + "_tile"


@pytest.mark.parametrize("dt", [ca.BFloat16, ca.Float16])
@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("shape", [(2, 300, 512, 272), (1, 1024, 1024, 1024), (3, 17, 4096, 256),
                                   (1, 2048, 256, 4096), (2, 300, 1000, 270)])
def test_mfma_dot_f32_accumulation(backend, dt, transposed, shape):
    """OutputDType f32: the matrix-core sums within 1e-5 of sum|terms| of the f64 value; the
    kernel that ran is the expected matrix-core one (large tiles or small tiles)."""
    B, M, K, N = shape
    rng = np.random.default_rng(B * 1000 + M + int(dt) + 3 * transposed)
    lhs, lv = _half(rng, (B, M, K), dt)
    rhs, rv = _half(rng, (B, N, K) if transposed else (B, K, N), dt)
    rc = [2] if transposed else [1]
    backend.ProfileReset()
    backend.SetProfiling(True)
    try:
        y, odt = run(backend, [(lhs, dt), (rhs, dt)],
                     lambda f, p: f.DotGeneral(p[0], [2], [0], p[1], rc, [0], ca.DotGeneralConfig(OutputDType=ca.Float32)))
        prof = backend.Profile()
    finally:
        backend.SetProfiling(False)
    assert odt == ca.Float32
    assert _half_kernel(dt, shape) in prof, prof
    truth = O.dot_general(lv.astype(np.float64), [2], [0], rv.astype(np.float64), rc, [0])
    scale = O.dot_general(np.abs(lv).astype(np.float64), [2], [0], np.abs(rv).astype(np.float64), rc, [0])
    assert np.all(np.abs(y.astype(np.float64) - truth) <= 1e-5 * scale)


@pytest.mark.parametrize("dt", [ca.BFloat16, ca.Float16])
def test_mfma_dot_half_output_and_prefill_shape(backend, dt):
    """The prefill-shaped contraction x [2048, 4096] . W [4096, 4096] in half precision with the
    lowering's f32 accumulator and half output (rounded once), rel 1e-2 / abs 1e-3 of the f64
    value, on 256 sampled rows."""
    rng = np.random.default_rng(11 + int(dt))
    M, K, N = 2048, 4096, 4096
    lhs, lv = _half(rng, (M, K), dt)
    rhs, rv = _half(rng, (K, N), dt)
    y, odt = run(backend, [(lhs, dt), (rhs, dt)], lambda f, p: f.DotGeneral(p[0], [1], [], p[1], [0], []))
    assert odt == dt
    rows = rng.choice(M, 256, replace=False)
    truth = lv[rows].astype(np.float64) @ rv.astype(np.float64)
    got = O.bf16_to_f32(y[rows]) if dt == ca.BFloat16 else y[rows].astype(np.float32)
    assert np.all(np.abs(got - truth) <= 1e-3 + 1e-2 * np.abs(truth))


# ---------------------------------------------------------------------------------------------
# f32 DotGeneral on the matrix cores (dot.hip, dot_mfma_f32: v_mfma_f32_16x16x4_f32, fp32
# products and sums): contractions of >= 2^20 multiply-adds with K % 4 == 0.  The shapes reach
# every tile configuration (64x64, 32x32 with K split over the waves, 16x32, 32x32 for short K;
# transposed: the LDS-staged 64x64 tiles, 4 waves or 8 waves splitting K), ragged M and N, K
# tails inside a 32-deep step and an odd number of steps, M below one 16-row tile, and the
# reference's MiniLM and bge-small projection shapes (bench_dotgeneral.go).
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("shape", [(1, 416, 1536, 384), (2, 300, 1000, 272), (1, 1024, 1024, 1024),
                                   (2, 130, 64, 70), (1, 2048, 512, 1024), (192, 128, 32, 128), (1, 5, 4096, 520),
                                   (3, 777, 36, 1030), (1, 1920, 1536, 384), (1, 640, 1028, 1500)])
def test_mfma_dot_f32(backend, transposed, shape):
    """Within 1e-5 of sum|terms| of the f64 value (only the summation order differs from a
    sequential f32 sum), and the kernel that ran is the matrix-core one."""
    B, M, K, N = shape
    rng = np.random.default_rng(B * 7919 + M * 31 + K + 5 * transposed)
    lhs = rng.standard_normal((B, M, K)).astype(np.float32)
    rhs = rng.standard_normal((B, N, K) if transposed else (B, K, N)).astype(np.float32)
    rc = [2] if transposed else [1]
    backend.ProfileReset()
    backend.SetProfiling(True)
    try:
        y, odt = run(backend, [(lhs, ca.Float32), (rhs, ca.Float32)],
                     lambda f, p: f.DotGeneral(p[0], [2], [0], p[1], rc, [0]))
        prof = backend.Profile()
    finally:
        backend.SetProfiling(False)
    assert odt == ca.Float32 and y.shape == (B, M, N)
    assert "dot_mfma_f32" in prof, prof
    truth = O.dot_general(lhs.astype(np.float64), [2], [0], rhs.astype(np.float64), rc, [0])
    scale = O.dot_general(np.abs(lhs).astype(np.float64), [2], [0], np.abs(rhs).astype(np.float64), rc, [0])
    assert np.all(np.abs(y.astype(np.float64) - truth) <= 1e-5 * scale)


def test_mfma_dot_f32_special_values_and_repeat(backend):
    """Inf in a row of lhs reaches only that row's outputs (the zero padding of K tails and
    clamped columns never multiplies it), and repeated calls give the same bits."""
    rng = np.random.default_rng(4242)
    M, K, N = 300, 1028, 200
    lhs = rng.standard_normal((M, K)).astype(np.float32)
    rhs = np.abs(rng.standard_normal((K, N))).astype(np.float32)
    lhs[7, K - 1] = np.inf
    f = lambda f, p: f.DotGeneral(p[0], [1], [], p[1], [0], [])
    y1, _ = run(backend, [(lhs, ca.Float32), (rhs, ca.Float32)], f)
    y2, _ = run(backend, [(lhs, ca.Float32), (rhs, ca.Float32)], f)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    assert np.all(np.isposinf(y1[7]))
    others = np.delete(np.arange(M), 7)
    assert np.all(np.isfinite(y1[others]))
    truth = lhs[others].astype(np.float64) @ rhs.astype(np.float64)
    scale = np.abs(lhs[others]).astype(np.float64) @ rhs.astype(np.float64)
    assert np.all(np.abs(y1[others] - truth) <= 1e-5 * scale)


@pytest.mark.parametrize("dt", [ca.BFloat16, ca.Float16])
@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("shape", [(1, 2048, 1536, 384), (192, 128, 32, 128), (3, 77, 520, 130), (4, 130, 64, 70)])
def test_mfma_dot_half_output_small_tiles(backend, dt, transposed, shape):
    """Half inputs and output on the small-tile kernel (the bge-small projection and attention
    shapes, and a ragged one with a K tail): f32 sums rounded once, rel 1e-2 / abs 1e-3 of the
    f64 value; the bf16 result equals the f32-output result rounded to nearest even."""
    B, M, K, N = shape
    rng = np.random.default_rng(M * 13 + K + int(dt) + 3 * transposed)
    lhs, lv = _half(rng, (B, M, K), dt)
    rhs, rv = _half(rng, (B, N, K) if transposed else (B, K, N), dt)
    rc = [2] if transposed else [1]
    backend.ProfileReset()
    backend.SetProfiling(True)
    try:
        y, odt = run(backend, [(lhs, dt), (rhs, dt)], lambda f, p: f.DotGeneral(p[0], [2], [0], p[1], rc, [0]))
        prof = backend.Profile()
    finally:
        backend.SetProfiling(False)
    assert odt == dt and _half_kernel(dt, shape) in prof, prof
    truth = O.dot_general(lv.astype(np.float64), [2], [0], rv.astype(np.float64), rc, [0])
    got = O.bf16_to_f32(y) if dt == ca.BFloat16 else y.astype(np.float32)
    assert np.all(np.abs(got - truth) <= 1e-3 + 1e-2 * np.abs(truth))
    y32, _ = run(backend, [(lhs, dt), (rhs, dt)],
                 lambda f, p: f.DotGeneral(p[0], [2], [0], p[1], rc, [0], ca.DotGeneralConfig(OutputDType=ca.Float32)))
    want = O.bf16_round(y32.astype(np.float32)) if dt == ca.BFloat16 else y32.astype(np.float32).astype(np.float16)
    assert np.array_equal(y.view(np.uint16), want.view(np.uint16))


# ---------------------------------------------------------------------------------------------
# Data movement behind DotGeneral's axis normalization (elementwise.hip): a gather whose
# innermost output axis reads contiguous input of 64..4096 elements copies whole rows
# (gather_rows), any other one indexes element by element.  Both are exact copies.
# ---------------------------------------------------------------------------------------------
_MOVE_DTYPES = [(ca.Float32, np.float32), (ca.BFloat16, np.uint16), (ca.Float64, np.float64), (ca.Int8, np.int8)]


@pytest.mark.parametrize("dt,npt", _MOVE_DTYPES)
@pytest.mark.parametrize("perm", [(0, 2, 1, 3), (2, 0, 1, 3), (0, 1, 3, 2), (3, 2, 1, 0)])
def test_transpose_exact(backend, dt, npt, perm):
    rng = np.random.default_rng(sum(perm) * 31 + int(dt))
    x = (rng.standard_normal((5, 37, 6, 72)) * 50).astype(npt) if npt != np.uint16 else \
        rng.integers(0, 1 << 16, (5, 37, 6, 72), dtype=np.uint16)
    backend.ProfileReset()
    backend.SetProfiling(True)
    try:
        y, odt = run(backend, [(x, dt)], lambda f, p: f.Transpose(p[0], *perm))
        prof = backend.Profile()
    finally:
        backend.SetProfiling(False)
    assert odt == dt
    assert np.array_equal(y.view(np.uint8), np.ascontiguousarray(np.transpose(x, perm)).view(np.uint8))
    assert ("gather_rows" in prof) == (perm[-1] == 3), prof


@pytest.mark.parametrize("strides", [None, [1, 2, 1, 1], [1, 1, 1, 2]])
def test_slice_exact(backend, strides):
    """Slices with an offset: unit inner stride takes the row copy, a strided inner axis not."""
    x = np.arange(5 * 37 * 6 * 100, dtype=np.float32).reshape(5, 37, 6, 100)
    starts, limits = [1, 2, 0, 5], [4, 30, 6, 90]
    y, _ = run(backend, [(x, ca.Float32)], lambda f, p: f.Slice(p[0], starts, limits, strides))
    st = strides or [1, 1, 1, 1]
    want = x[tuple(slice(a, b, c) for a, b, c in zip(starts, limits, st))]
    assert np.array_equal(y, want)


# ---------------------------------------------------------------------------------------------
# Integer DotGeneral (the reference's noSIMD integer kernels, internal/gobackend/dot/matmul/
# nosimd.go:66-75, after convertToAccumulatorDType, dot/dot.go:340-372): exact, with the sums
# wrapping in the accumulator dtype, against the brute-force restatement oracle.dot_general_int.
# ---------------------------------------------------------------------------------------------
INT_CASES = [
    # (input dtype, numpy dtype, accumulator, output, value range)
    (ca.Int8, np.int8, None, None, (-128, 128)),          # wraps in int8
    (ca.Int8, np.int8, ca.Int32, ca.Int32, (-128, 128)),
    (ca.Int8, np.int8, ca.Int32, None, (-128, 128)),      # int32 sums converted back to int8
    (ca.Int16, np.int16, None, None, (-30000, 30000)),
    (ca.Int32, np.int32, None, None, (-(1 << 31), 1 << 31)),  # wraps in int32
    (ca.Int64, np.int64, None, None, (-(1 << 62), 1 << 62)),  # wraps in int64
    (ca.Uint8, np.uint8, None, None, (0, 256)),
    (ca.Uint8, np.uint8, ca.Uint32, ca.Uint32, (0, 256)),
    (ca.Uint32, np.uint32, None, None, (0, 1 << 32)),
    (ca.Uint64, np.uint64, None, None, (0, 1 << 63)),
]
NP_OF = {ca.Int8: np.int8, ca.Int16: np.int16, ca.Int32: np.int32, ca.Int64: np.int64, ca.Uint8: np.uint8,
         ca.Uint16: np.uint16, ca.Uint32: np.uint32, ca.Uint64: np.uint64}


@pytest.mark.parametrize("case", INT_CASES, ids=lambda c: f"{c[0].name}-acc{c[2].name if c[2] else 'none'}-out{c[3].name if c[3] else 'none'}")
@pytest.mark.parametrize("layout", ["plain", "transposed", "batched"])
def test_integer_dot_general_exact(backend, case, layout):
    dt, npdt, acc, out_dt, (lo, hi) = case
    rng = np.random.default_rng(abs(hash((dt.name, layout))) % 1000)
    if layout == "plain":      # [M, K] x [K, N]
        ls, rs, lc, lb, rc, rb = (5, 7), (7, 3), [1], [], [0], []
    elif layout == "transposed":  # [M, K] x [N, K]
        ls, rs, lc, lb, rc, rb = (4, 9), (6, 9), [1], [], [1], []
    else:                      # [K, B, M] x [B, N, K]
        ls, rs, lc, lb, rc, rb = (6, 2, 3), (2, 4, 6), [0], [1], [2], [0]
    l = rng.integers(lo, hi, ls, dtype=np.int64 if npdt != np.uint64 else np.uint64).astype(npdt)
    r = rng.integers(lo, hi, rs, dtype=np.int64 if npdt != np.uint64 else np.uint64).astype(npdt)
    got, gdt = run(backend, [(l, dt), (r, dt)],
                   lambda f, p: f.DotGeneral(p[0], lc, lb, p[1], rc, rb,
                                             ca.DotGeneralConfig(AccumulatorDType=acc or ca.InvalidDType,
                                                                 OutputDType=out_dt or ca.InvalidDType)))
    acc_np = NP_OF[acc] if acc is not None else None
    want = O.dot_general_int(l, lc, lb, r, rc, rb, acc_dtype=acc_np)
    final = out_dt if out_dt is not None else dt
    assert gdt == final
    assert np.array_equal(got, want.astype(NP_OF[final])), f"{case} {layout}"


def test_integer_dot_general_large_int32(backend):
    """A larger int32 contraction with no overflow: equal to the float64 matmul."""
    rng = np.random.default_rng(11)
    l = rng.integers(-100, 100, (2, 64, 128)).astype(np.int32)
    r = rng.integers(-100, 100, (2, 128, 96)).astype(np.int32)
    got, gdt = run(backend, [(l, ca.Int32), (r, ca.Int32)], lambda f, p: f.DotGeneral(p[0], [2], [0], p[1], [1], [0]))
    assert gdt == ca.Int32
    assert np.array_equal(got, np.matmul(l.astype(np.float64), r.astype(np.float64)).astype(np.int32))
