"""Prefill FusedQuantizedDense (bf16 rows past the skinny kernel's row groups: M > 48 with one
scale per output column, M > 64 with scale groups): the dequantise-into-MFMA GEMM on the GPU vs
the CPU oracle.

The kernel factors the per-channel scale out of the K sum and accumulates in f32 on the matrix
cores in another order than the reference loop, so: bf16 outputs within rel 1e-2 / abs 1e-3 of
the oracle's f32 result, and (without activation) within 2^-8 relative (bf16 rounding) plus
1e-5 of sum|terms| of the exact f64 value.  Large cases check a seeded sample of rows (the
oracle computes rows independently).
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.qd_helpers import QDenseRun, assert_bf16_close

pytestmark = pytest.mark.gpu


def check_rows(r: QDenseRun, rows=None, threads=1, what=""):
    p = r.p
    y = r.run()
    sel = slice(None) if rows is None else rows
    assert_bf16_close(y[sel], O.qdense_f32(p, rows=rows, threads=threads), what=what)
    if p.act == O.ACT_NONE:
        truth = O.qdense_f64(p, rows)
        scale = O.qdense_f64(p, rows, absolute=True)
        got = O.bf16_to_f32(y[sel]).astype(np.float64)
        assert np.all(np.abs(got - truth) <= 2.0 ** -8 * np.abs(truth) + 1e-5 * scale), what
    return y


@pytest.mark.parametrize("shape", [(49, 64, 16), (300, 128, 272), (512, 256, 384), (256, 640, 128), (1000, 64, 4112)])
@pytest.mark.parametrize("w_dtype", [O.DT_INT8, O.DT_UINT8])
def test_gemm_shapes(backend, shape, w_dtype):
    M, K, N = shape
    p = O.make_problem(M, K, N, w_dtype=w_dtype, block_axis=0, block_size=K, per_channel_1d=True,
                       scale_dtype=O.DT_FLOAT32, bias=True, seed=M + K + N)
    r = QDenseRun(backend, p)
    assert r.plan().startswith("qdense_gemm_mfma")
    check_rows(r, what=f"{shape}")


@pytest.mark.parametrize("act", range(6))
def test_gemm_activations(backend, act):
    p = O.make_problem(64, 128, 256, w_dtype=O.DT_INT8, block_axis=0, block_size=128, per_channel_1d=True,
                       scale_dtype=O.DT_BFLOAT16, bias=True, act=act, scale_range=(0.01, 0.05), seed=act)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_gemm_mfma_i8"
    check_rows(r, what=f"act {act}")


def test_gemm_c4_config_full_size(backend):
    """x bf16 [2048,4096], int8 [4096,4096] per-channel f32 scales, bias,
    exact GELU.  128 seeded rows are checked against the oracle; two calls must agree bitwise."""
    p = O.baseline_config(3)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_gemm_mfma_i8"
    rows = np.sort(np.random.default_rng(4).choice(p.M, 128, replace=False))
    y = check_rows(r, rows=rows, threads=8, what="C4")
    assert np.array_equal(y, r.run())


@pytest.mark.parametrize("M", [49, 64])
def test_gemm_small_batch_rows(backend, M):
    """49..64 bf16 rows with per-channel int8 (past the skinny kernel's row groups, within the
    GEMV's row range): the GEMM takes them, at the C2 matrix size, with the same bounds."""
    p = O.make_problem(M, 4096, 11008, w_dtype=O.DT_INT8, block_axis=0, block_size=4096, per_channel_1d=True,
                       scale_dtype=O.DT_FLOAT32, bias=False, seed=M)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_gemm_mfma_i8"
    check_rows(r, threads=8, what=f"M={M}")


# ---------------------------------------------------------------------------------------------
# 4-bit weights and K-grouped scales (scale [K/G, N], G a multiple of 64, or 32 with bf16
# scales): the same GEMM with the nibbles converted into the LDS tile and a per-group accumulator
# folded with the group's scales (twice per 64-row block for G = 32).
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("w_dtype", [O.DT_INT4, O.DT_UINT4, O.DT_INT8, O.DT_UINT8])
@pytest.mark.parametrize("G", [None, 32, 64, 128, 256])
def test_gemm_4bit_and_groups(backend, w_dtype, G):
    M, K, N = 300, 512, 272
    p = O.make_problem(M, K, N, w_dtype=w_dtype, block_axis=0, block_size=G if G else K, per_channel_1d=G is None,
                       scale_dtype=O.DT_BFLOAT16 if G else O.DT_FLOAT32, bias=True, seed=7 + (G or 0))
    r = QDenseRun(backend, p)
    want = "qdense_gemm_mfma_" + {O.DT_INT4: "i4", O.DT_UINT4: "u4", O.DT_INT8: "i8", O.DT_UINT8: "u8"}[w_dtype]
    assert r.plan() == want + ("_grouped" if G else "")
    check_rows(r, what=f"{w_dtype} G={G}")
    assert np.array_equal(r.run(), r.run())


@pytest.mark.parametrize("shape", [(17, 128, 16, 64), (1000, 1024, 4112, 128), (513, 2048, 1040, 512), (300, 512, 272, 32)])
def test_gemm_grouped_shapes(backend, shape):
    M, K, N, G = shape
    p = O.make_problem(M, K, N, w_dtype=O.DT_INT4, block_axis=0, block_size=G, scale_dtype=O.DT_FLOAT32,
                       bias=False, act=O.ACT_NONE, scale_range=(0.002, 0.02), seed=M)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_gemm_mfma_i4_grouped"
    check_rows(r, threads=8, what=f"{shape}")


@pytest.mark.parametrize("act", [O.ACT_SILU, O.ACT_GELU])
def test_gemm_grouped_activations(backend, act):
    p = O.make_problem(65, 256, 256, w_dtype=O.DT_UINT4, block_axis=0, block_size=64, bias=True, act=act,
                       scale_range=(0.01, 0.05), seed=act)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_gemm_mfma_u4_grouped"  # past the skinny row groups (64 rows)
    check_rows(r, what=f"act {act}")


@pytest.mark.parametrize("w_dtype,G", [(O.DT_INT4, 128), (O.DT_INT8, 64), (O.DT_INT4, 32)])
def test_gemm_grouped_prefill_full_size(backend, w_dtype, G):
    """x bf16 [2048,4096] x Int4 [4096,14336] g128 (the MLP's gate/up weights at prefill) and the
    int8 g64 layout of BASELINE configs[2] at the same size: 128 seeded rows against the oracle,
    two calls bit-equal."""
    p = O.make_problem(2048, 4096, 14336, w_dtype=w_dtype, block_axis=0, block_size=G, bias=False,
                       scale_range=(0.002, 0.02), seed=G)
    r = QDenseRun(backend, p)
    assert r.plan().endswith("_grouped")
    rows = np.sort(np.random.default_rng(5).choice(p.M, 128, replace=False))
    y = check_rows(r, rows=rows, threads=8, what=f"{w_dtype} g{G}")
    assert np.array_equal(y, r.run())


@pytest.mark.parametrize("w_dtype,G,s_dtype,act", [(O.DT_INT8, None, O.DT_FLOAT32, O.ACT_GELU),
                                                    (O.DT_INT4, 128, O.DT_FLOAT32, O.ACT_NONE),
                                                    (O.DT_UINT4, 64, O.DT_BFLOAT16, O.ACT_SILU),
                                                    (O.DT_INT4, 32, O.DT_BFLOAT16, O.ACT_NONE),
                                                    (O.DT_UINT8, 32, O.DT_FLOAT32, O.ACT_GELU)])
def test_gemm_split_tail(backend, w_dtype, G, s_dtype, act):
    """272 tiles of 256 x 128 (x [512, 1024], N = 17408): the 16 tiles past the last whole round of
    256 are computed as two halves of K whose partial tiles the second half adds (per-channel
    scales with bias and GELU, f32 and bf16 group scales).  All rows of a sample against the
    oracle, including the tail tiles' columns; two calls bit-equal (the halves' arrival counters
    are back at zero)."""
    M, K, N = 512, 1024, 17408
    p = O.make_problem(M, K, N, w_dtype=w_dtype, block_axis=0, block_size=G if G else K, per_channel_1d=G is None,
                       scale_dtype=s_dtype, bias=True, act=act, scale_range=(0.002, 0.02), seed=11 + (G or 0))
    r = QDenseRun(backend, p)
    assert r.plan().startswith("qdense_gemm_mfma")
    rows = np.sort(np.concatenate([np.arange(0, 8), np.arange(256, 264), np.arange(504, 512)]))
    y = check_rows(r, rows=rows, threads=8, what=f"{w_dtype} G={G}")
    assert np.array_equal(y, r.run())
