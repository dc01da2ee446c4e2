"""Skinny-M FusedQuantizedDense (decode and small batches, M <= 16 bf16 rows, and once per group
of 16 rows up to 48 rows with per-channel scales or 64 with scale groups) on the GPU vs the CPU
oracle.

The kernel sums in another order than the reference loop (per-group partial sums on the matrix
cores, the group scale applied once per group, split-K partials added in slice order), so:
  - bf16 outputs must be within rel 1e-2 / abs 1e-3 of the oracle's f32 result;
  - the pre-rounding f32 accumulation must be within 1e-5 of sum|terms| of the exact (f64)
    value, checked through the bf16 output (half an ulp of bf16, 2^-9 relative, is allowed on
    top);
  - two calls on the same inputs must return identical bits (deterministic reduction).
"""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from tests.qd_helpers import QDenseRun, assert_bf16_close

pytestmark = pytest.mark.gpu

W_DTYPES = [O.DT_INT8, O.DT_UINT8, O.DT_INT4, O.DT_UINT4]


def check(r: QDenseRun, threads: int = 1, what: str = ""):
    p = r.p
    y = r.run()
    assert_bf16_close(y, O.qdense_f32(p, threads=threads), what=what)
    if p.act == O.ACT_NONE:
        truth = O.qdense_f64(p)
        scale = O.qdense_f64(p, absolute=True)
        got = O.bf16_to_f32(y).astype(np.float64)
        assert np.all(np.abs(got - truth) <= 2.0 ** -8 * np.abs(truth) + 1e-5 * scale), what
    y2 = r.run()
    assert np.array_equal(y, y2), f"{what}: not deterministic"
    return y


@pytest.mark.parametrize("M", [1, 2, 5, 8, 16])
@pytest.mark.parametrize("w_dtype", W_DTYPES)
def test_skinny_rows_and_dtypes(backend, M, w_dtype):
    p = O.make_problem(M, 512, 768, w_dtype=w_dtype, block_axis=0, block_size=64, bias=True,
                       act=O.ACT_NONE, seed=100 + M)
    r = QDenseRun(backend, p)
    assert r.plan().startswith("qdense_skinny_mfma")
    check(r, what=f"M={M} w={w_dtype}")


@pytest.mark.parametrize("scale_dtype", [O.DT_BFLOAT16, O.DT_FLOAT32])
@pytest.mark.parametrize("act", range(6))
def test_skinny_activations_scales(backend, scale_dtype, act):
    p = O.make_problem(4, 256, 512, w_dtype=O.DT_INT4, scale_dtype=scale_dtype, block_axis=0, block_size=128,
                       bias=True, act=act, scale_range=(0.01, 0.05), seed=7 * act + scale_dtype)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_skinny_mfma_i4"
    check(r, what=f"act {act}")


@pytest.mark.parametrize("shape", [(3, 352, 272, 64), (16, 96, 16, 32), (7, 128, 4112, 128), (1, 32, 48, 32),
                                   (2, 64, 4128, 64)])
def test_skinny_ragged(backend, shape):
    """K not a multiple of the group, N not a multiple of 256 columns, single-step K, S = 1.
    (Packed 4-bit rows are read 32 columns at a time, so N is rounded up to a multiple of 32.)"""
    M, K, N, G = shape
    for w_dtype in (O.DT_INT8, O.DT_INT4):
        if w_dtype == O.DT_INT4:
            N = (N + 31) // 32 * 32
        p = O.make_problem(M, K, N, w_dtype=w_dtype, block_axis=0, block_size=G, bias=True, seed=K + N)
        r = QDenseRun(backend, p)
        assert r.plan().startswith("qdense_skinny_mfma")
        check(r, what=f"{shape} {w_dtype}")


@pytest.mark.parametrize("w_dtype", [O.DT_INT8, O.DT_INT4])
def test_skinny_per_channel(backend, w_dtype):
    """One scale per output column, given as shape [N] (block size = K)."""
    p = O.make_problem(6, 1024, 512, w_dtype=w_dtype, scale_dtype=O.DT_FLOAT32, block_axis=0, block_size=1024,
                       per_channel_1d=True, bias=False, seed=3)
    r = QDenseRun(backend, p)
    assert r.plan().startswith("qdense_skinny_mfma")
    check(r, what="per-channel")


def test_skinny_c3_config_full_size(backend):
    """x bf16 [16,4096], int8 [4096,14336] g64 bf16 scales, bias, SiLU."""
    p = O.baseline_config(2)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_skinny_mfma_i8"
    check(r, threads=8, what="C3")


def test_skinny_mlp_gate_shape(backend):
    """The MLP's gate/up projection: x bf16 [8,4096], Int4 [4096,14336] g128 (no activation),
    and its down projection Int4 [14336,4096] g128."""
    for K, N in ((4096, 14336), (14336, 4096)):
        p = O.make_problem(8, K, N, w_dtype=O.DT_INT4, block_axis=0, block_size=128, bias=False,
                           scale_range=(0.002, 0.02), seed=K)
        r = QDenseRun(backend, p)
        assert r.plan() == "qdense_skinny_mfma_i4"
        check(r, threads=8, what=f"MLP {K}x{N}")


# Shapes around the split-K decomposition: one or many column blocks, K from one step to deep
# slices, a partial last column block, and the headline C2 / MLP shapes.
PARTITION_SHAPES = [
    (1, 64, 256, 32),
    (2, 1024, 512, 128),
    (1, 8192, 256, 128),
    (3, 2080, 1024, 32),
    (1, 4096, 11008, 128),
    (8, 14336, 4096, 128),
]


@pytest.mark.parametrize("shape", PARTITION_SHAPES)
@pytest.mark.parametrize("w_dtype", [O.DT_INT4, O.DT_UINT8])
def test_skinny_partitions(backend, shape, w_dtype):
    M, K, N, G = shape
    p = O.make_problem(M, K, N, w_dtype=w_dtype, block_axis=0, block_size=G, bias=True, act=O.ACT_NONE,
                       scale_range=(0.002, 0.02), seed=K + N + M)
    r = QDenseRun(backend, p)
    assert r.plan().startswith("qdense_skinny_mfma")
    check(r, threads=8, what=f"{shape} {w_dtype}")


SUFFIX = {O.DT_INT8: "i8", O.DT_UINT8: "u8", O.DT_INT4: "i4", O.DT_UINT4: "u4"}


@pytest.mark.parametrize("M,w_dtype,G", [(17, O.DT_INT8, None), (33, O.DT_UINT8, None), (48, O.DT_INT8, None),
                                         (40, O.DT_INT4, 128), (64, O.DT_INT8, 64), (23, O.DT_UINT4, 64)])
def test_skinny_row_groups(backend, M, w_dtype, G):
    """Past 16 rows: one launch per group of 16 rows, each launch the one a problem of just those
    rows makes (the split and summation order depend on K and N only), so the rows of a group are
    bit-identical to that problem's output."""
    K, N = 1024, 2048
    p = O.make_problem(M, K, N, w_dtype=w_dtype, block_axis=0, block_size=G if G else K, per_channel_1d=G is None,
                       scale_dtype=O.DT_BFLOAT16 if G else O.DT_FLOAT32, bias=True, act=O.ACT_NONE,
                       scale_range=(0.002, 0.02), seed=M)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_skinny_rows16_" + SUFFIX[w_dtype]
    y = check(r, threads=8, what=f"M={M} w={w_dtype} G={G}")
    hi = min(32, M)  # the second group of rows
    sub = dataclasses.replace(p, M=hi - 16, x=np.ascontiguousarray(p.x[16:hi]))
    r16 = QDenseRun(backend, sub)
    assert r16.plan() == "qdense_skinny_mfma_" + SUFFIX[w_dtype]
    assert np.array_equal(r16.run(), y[16:hi])


def test_skinny_shape_sequence(backend):
    """Calls of different shapes share the backend's split-K scratch (arrival counters and partial
    tiles): alternating shapes, each call checked, each repeated call equal."""
    probs = [O.make_problem(M, K, N, w_dtype=O.DT_INT4, block_axis=0, block_size=128, bias=False, seed=s)
             for s, (M, K, N) in enumerate([(1, 4096, 2048), (16, 1024, 4096), (4, 8192, 512)])]
    runs = [QDenseRun(backend, p) for p in probs]
    first = [r.run() for r in runs]
    for r, y in zip(runs, first):
        assert_bf16_close(y, O.qdense_f32(r.p, threads=8), what=f"{r.p.M}x{r.p.K}x{r.p.N}")
    for _ in range(2):
        for r, y in zip(runs[::-1], first[::-1]):
            assert np.array_equal(r.run(), y)
