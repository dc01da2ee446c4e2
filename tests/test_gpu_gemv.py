"""Decode GEMV over the reference's own layouts (qdense_gemv.hip) vs the CPU oracle.

The reference's FusedQuantizedDense takes f32 x and scales in its own layout, scale[k, n/B]
(BlockAxis = 1, quantizeddense.go:111-123), with Linear (optionally with a zero point) or NF4
dequantisation.  Small problems keep the reference-order kernel (bit-identical); at decode sizes
(K*N >= 2^20, M <= 64, four rows per launch) the GEMV kernel runs, whose results differ from the reference loop only by
summation order and the folding of the scale into x:
  - f32 outputs: within 1e-5 of sum|terms| of the f64 value (the north star's fp32 bar);
  - bf16 outputs: within rel 1e-2 / abs 1e-3 of the oracle's f32 result, and the same
    accumulation bound plus half a bf16 ulp.
"""
import numpy as np
import pytest

import compute_amd as ca
from oracle import oracle as O
from tests.qd_helpers import QDenseRun, assert_bf16_close

pytestmark = pytest.mark.gpu

W_DTYPES = [O.DT_INT8, O.DT_UINT8, O.DT_INT4, O.DT_UINT4]


def _check(p, y, act_slack=1.0):
    truth = O.qdense_f64(p)
    scale = O.qdense_f64(p, absolute=True)
    ref = O.qdense_f32(p)
    if p.x_dtype == O.DT_FLOAT32:
        if p.act == O.ACT_NONE:
            assert np.all(np.abs(y.astype(np.float64) - truth) <= 1e-5 * scale + 1e-30), "f32 accumulation bound"
        else:
            err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
            assert np.all(err <= act_slack * 1e-5 * scale + 1e-6 * np.abs(ref)), "f32 bound through the activation"
    else:
        assert_bf16_close(y, ref)
        if p.act == O.ACT_NONE:
            got = O.bf16_to_f32(y).astype(np.float64)
            assert np.all(np.abs(got - truth) <= 2.0 ** -8 * np.abs(truth) + 1e-5 * scale)


def _run(backend, p, expect="qdense_gemv"):
    r = QDenseRun(backend, p)
    assert r.plan().startswith(expect), r.plan()
    return r, r.run()


@pytest.mark.parametrize("w_dtype", W_DTYPES)
@pytest.mark.parametrize("zp", [False, True])
@pytest.mark.parametrize("M", [1, 3])
def test_gemv_linear_f32(backend, w_dtype, zp, M):
    p = O.make_problem(M, 1024, 1024, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=64, bias=True, zp=zp, seed=100 + M * 10 + w_dtype)
    r, y = _run(backend, p)
    assert r.plan().endswith("_zp") == zp
    _check(p, y)


@pytest.mark.parametrize("w_dtype", [O.DT_UINT8, O.DT_INT8, O.DT_INT4, O.DT_UINT4])
@pytest.mark.parametrize("M", [1, 4])
def test_gemv_nf4(backend, w_dtype, M):
    p = O.make_problem(M, 1024, 1536, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=128, bias=M == 1, scheme=O.QUANT_NF4, seed=200 + M + w_dtype)
    r, y = _run(backend, p, "qdense_gemv_nf4")
    _check(p, y)


@pytest.mark.parametrize("w_dtype", W_DTYPES)
@pytest.mark.parametrize("scale_dtype", [O.DT_BFLOAT16, O.DT_FLOAT32])
def test_gemv_bf16_x(backend, w_dtype, scale_dtype):
    """bf16 activations with reference-layout scales (the MFMA decode kernel takes K-blocked ones)."""
    p = O.make_problem(2, 2048, 1024, w_dtype=w_dtype, x_dtype=O.DT_BFLOAT16, scale_dtype=scale_dtype,
                       block_axis=1, block_size=256, bias=True, seed=300 + w_dtype)
    r, y = _run(backend, p)
    _check(p, y)


@pytest.mark.parametrize("act", range(6))
def test_gemv_activations(backend, act):
    p = O.make_problem(1, 1024, 1024, w_dtype=O.DT_INT8, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=32, bias=True, act=act, scale_range=(0.01, 0.05), seed=400 + act)
    r, y = _run(backend, p)
    _check(p, y, act_slack=2.0)


@pytest.mark.parametrize("shape", [(1, 1100, 1032, 96), (4, 1300, 1032, 1032), (2, 257, 4104, 40),
                                   (3, 4096, 264, 33 * 8)])
@pytest.mark.parametrize("w_dtype", [O.DT_INT8, O.DT_INT4])
def test_gemv_ragged(backend, shape, w_dtype):
    """K not a multiple of the slice, N not a multiple of the column block, blocks straddling
    column blocks, a block size >= N (one scale per row)."""
    M, K, N, B = shape
    p = O.make_problem(M, K, N, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32, block_axis=1,
                       block_size=B, bias=True, zp=True, seed=500 + K + w_dtype)
    r, y = _run(backend, p)
    _check(p, y)


def test_gemv_deterministic_and_exact_option(backend):
    """Repeated calls give the same bits (split-K partials summed in a fixed order, counters
    reset); the "exact" option runs the reference-order kernel, bit-identical to the oracle."""
    p = O.make_problem(1, 4096, 2048, w_dtype=O.DT_INT4, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=128, bias=True, seed=600)
    r, y1 = _run(backend, p)
    assert np.array_equal(y1, r.run())
    _check(p, y1)
    ex = ca.New("exact")
    try:
        r2 = QDenseRun(ex, p)
        assert r2.plan() == "qdense_exact"
        y2 = r2.run()
    finally:
        ex.Finalize()
    assert np.array_equal(y2.view(np.uint32), O.qdense_f32(p).view(np.uint32))


@pytest.mark.parametrize("name,M,K,N,G", [("1x64x64_g64", 1, 64, 64, 64), ("8x128x256_g128", 8, 128, 256, 128),
                                         ("32x512x1024_g128", 32, 512, 1024, 128)])
@pytest.mark.parametrize("scheme", [O.QUANT_NF4, O.QUANT_LINEAR])
def test_reference_benchmark_shapes_bit_exact(backend, name, M, K, N, G, scheme):
    """The reference's BenchmarkQuantizedDense problems (support/backendtest/benchmarks.go:435-470:
    f32 x, Uint8 NF4 codes or Int8 weights, scales [K, ceil(N/G)] BlockAxis 1, bias): small enough
    for the reference-order kernel, so bit-identical to the oracle."""
    w_dtype = O.DT_UINT8 if scheme == O.QUANT_NF4 else O.DT_INT8
    p = O.make_problem(M, K, N, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32, block_axis=1,
                       block_size=G, bias=True, scheme=scheme, x_dist="uniform", seed=700 + M)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_exact"
    assert np.array_equal(r.run().view(np.uint32), O.qdense_f32(p).view(np.uint32))


# ---------------------------------------------------------------------------------------------
# K-blocked scales (BlockAxis = 0, [ceil(K/B), N]) at decode: f32 x, zero points and NF4 (the
# MFMA decode kernel takes bf16 x with plain Linear scales).
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("w_dtype", W_DTYPES)
@pytest.mark.parametrize("B,zp", [(128, False), (32, True), (None, True)])
@pytest.mark.parametrize("M", [1, 4])
def test_gemv_kblocked_f32(backend, w_dtype, B, zp, M):
    K = 2048
    p = O.make_problem(M, K, 768, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32, block_axis=0,
                       block_size=B if B else K, per_channel_1d=B is None, bias=True, zp=zp,
                       seed=800 + M * 7 + w_dtype + (B or 0))
    r, y = _run(backend, p)
    assert r.plan().endswith("_zp") == zp
    _check(p, y)


@pytest.mark.parametrize("w_dtype,scheme,zp", [(O.DT_INT4, O.QUANT_NF4, False), (O.DT_UINT8, O.QUANT_NF4, False),
                                               (O.DT_INT8, O.QUANT_LINEAR, True), (O.DT_UINT4, O.QUANT_LINEAR, True)])
def test_gemv_kblocked_bf16_nf4_zp(backend, w_dtype, scheme, zp):
    p = O.make_problem(2, 4096, 512, w_dtype=w_dtype, x_dtype=O.DT_BFLOAT16, scale_dtype=O.DT_BFLOAT16,
                       block_axis=0, block_size=64, bias=False, zp=zp, scheme=scheme, seed=900 + w_dtype)
    r, y = _run(backend, p)
    _check(p, y)


def test_gemv_kblocked_plain_bf16_stays_on_mfma(backend):
    p = O.make_problem(1, 2048, 1024, w_dtype=O.DT_INT4, x_dtype=O.DT_BFLOAT16, scale_dtype=O.DT_BFLOAT16,
                       block_axis=0, block_size=128, bias=False, seed=901)
    assert QDenseRun(backend, p).plan().startswith("qdense_skinny_mfma")


@pytest.mark.parametrize("shape", [(3, 1100, 1032, 96), (1, 4000, 264, 4000), (2, 257 * 4, 4104, 64)])
def test_gemv_kblocked_ragged(backend, shape):
    """K not a multiple of the slice (a group straddles slices), N not a multiple of the column
    block, per-channel scales."""
    M, K, N, B = shape
    p = O.make_problem(M, K, N, w_dtype=O.DT_INT4, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32, block_axis=0,
                       block_size=B, bias=True, zp=True, seed=950 + K)
    r, y = _run(backend, p)
    _check(p, y)


@pytest.mark.parametrize("M", [5, 8, 13, 16])
@pytest.mark.parametrize("w_dtype,scheme,zp", [(O.DT_INT4, O.QUANT_LINEAR, True), (O.DT_UINT8, O.QUANT_NF4, False)])
def test_gemv_row_groups(backend, M, w_dtype, scheme, zp):
    """M > 4: one launch per group of four rows (x and output offsets per group)."""
    p = O.make_problem(M, 1024, 1536, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=128, bias=True, zp=zp, scheme=scheme, seed=990 + M)
    r, y = _run(backend, p)
    _check(p, y)


@pytest.mark.parametrize("w_dtype", W_DTYPES)
@pytest.mark.parametrize("M,K,N,axis,B", [(1, 1024, 1031, 1, 64), (3, 1040, 1235, 0, 64), (1, 4096, 32001, 1, 128),
                                          (2, 4096, 32001, 0, 128)])
def test_gemv_rows_starting_mid_word(backend, w_dtype, M, K, N, axis, B):
    """N not a multiple of 8 (4-bit) or 4 (8-bit): row k of the packed weights starts mid-word
    (mid-byte for odd N and 4-bit weights); each lane's word is read as two aligned words and a
    funnel shift.  f32 x in both scale layouts, zero points, bias; split K on the larger ones."""
    if w_dtype in (O.DT_INT8, O.DT_UINT8) and N % 4 == 0:
        pytest.skip("aligned rows")
    p = O.make_problem(M, K, N, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=axis, block_size=B, bias=True, zp=True, seed=1300 + N + w_dtype)
    r, y = _run(backend, p)
    _check(p, y)
    assert np.array_equal(y.view(np.uint32), r.run().view(np.uint32))


@pytest.mark.parametrize("w_dtype,x_dtype,axis", [(O.DT_INT4, O.DT_FLOAT32, 1), (O.DT_UINT8, O.DT_FLOAT32, 0),
                                                  (O.DT_INT4, O.DT_BFLOAT16, 0)])
def test_gemv_rows_starting_mid_word_past_64_rows(backend, w_dtype, x_dtype, axis):
    """Odd N past 64 rows with 2^24 weights: no MFMA kernel takes rows that start mid-word, and
    the GEMV once per group of four rows replaces the exact kernel (17 groups here, the last of
    two rows); zero points and bias with f32 x."""
    f32 = x_dtype == O.DT_FLOAT32
    p = O.make_problem(66, 4096, 4097, w_dtype=w_dtype, x_dtype=x_dtype, scale_dtype=x_dtype, block_axis=axis,
                       block_size=128, bias=True, zp=f32, scale_range=(0.002, 0.02), seed=1500 + w_dtype + axis)
    r, y = _run(backend, p)  # asserts the GEMV plan
    _check(p, y)


@pytest.mark.parametrize("w_dtype,scheme", [(O.DT_INT4, O.QUANT_LINEAR), (O.DT_UINT4, O.QUANT_NF4),
                                            (O.DT_INT8, O.QUANT_LINEAR)])
@pytest.mark.parametrize("M", [1, 6])
def test_gemv_rows_starting_mid_word_bf16(backend, w_dtype, scheme, M):
    """bf16 x with K-blocked bf16 scales at an odd width (the MFMA decode kernel needs aligned
    rows): the GEMV with two-word loads; NF4 codes and row groups past four rows."""
    p = O.make_problem(M, 2048, 4097, w_dtype=w_dtype, x_dtype=O.DT_BFLOAT16, scale_dtype=O.DT_BFLOAT16,
                       block_axis=0, block_size=128, bias=True, scheme=scheme, scale_range=(0.002, 0.02),
                       seed=1400 + M + w_dtype)
    r, y = _run(backend, p)
    _check(p, y)
