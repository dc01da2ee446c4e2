"""The reference's own quantization layouts at prefill size on the GPU: scale [K, ceil(N/B)] with
BlockAxis = 1 (fused_ops.go:208-229), f32 or bf16 x, zero points (quantizeddense.go:630-638) and
NF4 (quantizeddense.go:586-609), past the GEMV's 64 rows.  The fused kernel dequantises each K
block of the weights into LDS the way the reference forms each term's weight factor and contracts
on the f32 matrix cores, so only rounding order differs from the reference loop: every output
must be within
2^-22 |y| + 1e-5 * sum_k |term_k| of the exact (f64) value; with bf16 x the output is bf16, and
the relative part of the bound is one bf16 ulp, 2^-8 |y|, instead.  Rows are sampled at the largest size (the oracle computes rows
independently)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.qd_helpers import QDenseRun

pytestmark = pytest.mark.gpu


def check(r: QDenseRun, rows=None):
    p = r.p
    y = r.run()
    sel = slice(None) if rows is None else rows
    truth = O.qdense_f64(p, rows)
    scale = O.qdense_f64(p, rows, absolute=True)
    got = (O.bf16_to_f32(y[sel]) if p.x_dtype == O.DT_BFLOAT16 else y[sel]).astype(np.float64)
    rel = 2.0 ** -8 if p.x_dtype == O.DT_BFLOAT16 else 2.0 ** -22
    bad = np.abs(got - truth) > rel * np.abs(truth) + 1e-5 * scale
    assert not bad.any(), f"{bad.sum()} outputs outside the bound; worst at {np.argwhere(bad)[0]}"
    assert np.array_equal(y, r.run()), "not deterministic"


@pytest.mark.parametrize("w_dtype", [O.DT_INT8, O.DT_UINT8, O.DT_INT4, O.DT_UINT4])
@pytest.mark.parametrize("zp", [False, True])
def test_reference_layout_prefill(backend, w_dtype, zp):
    """BlockAxis = 1 scales [K, ceil(N/B)], f32 x, M = 512."""
    p = O.make_problem(512, 1024, 1040, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=64, zp=zp, bias=True, seed=31 + w_dtype + zp)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_refgemm_f32_mfma"
    check(r)


@pytest.mark.parametrize("w_dtype", [O.DT_UINT4, O.DT_UINT8])
def test_nf4_prefill(backend, w_dtype):
    p = O.make_problem(512, 1024, 768, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=128, scheme=O.QUANT_NF4, bias=False, seed=7)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_refgemm_f32_mfma"
    check(r)


@pytest.mark.parametrize("act", range(6))
def test_reference_layout_prefill_activations_bf16_x(backend, act):
    """bf16 x and bias with the reference layout, every activation (the reference's formulas)."""
    p = O.make_problem(300, 512, 272, w_dtype=O.DT_INT8, x_dtype=O.DT_BFLOAT16, scale_dtype=O.DT_BFLOAT16,
                       block_axis=1, block_size=32, bias=True, act=act, scale_range=(0.01, 0.05), seed=act)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_refgemm_f32_mfma"
    y = r.run()
    from tests.qd_helpers import assert_bf16_close
    assert_bf16_close(y, O.qdense_f32(p, threads=8), what=f"act {act}")


def test_reference_layout_full_size(backend):
    """x f32 [2048,4096] x Int4 [4096,11008], scale [4096, 86] (B = 128), zero points: 64 sampled rows."""
    p = O.make_problem(2048, 4096, 11008, w_dtype=O.DT_INT4, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=128, zp=True, bias=True, seed=5)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_refgemm_f32_mfma"
    rows = np.sort(np.random.default_rng(6).choice(p.M, 64, replace=False))
    check(r, rows)


@pytest.mark.parametrize("block_axis,block_size", [(1, 64), (1, 8), (0, 96)])
def test_reference_layout_prefill_allocates_nothing(backend, block_axis, block_size):
    """The call makes no device allocation (the next one is made to fail): no f32 copy of the
    weights, no workspace.  Its result equals the compiled graph's, bit for bit."""
    p = O.make_problem(512, 1024, 1040, w_dtype=O.DT_INT4, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=block_axis, block_size=block_size, zp=True, bias=True, seed=77 + block_size)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_refgemm_f32_mfma"
    import compute_amd as ca
    out = backend.BufferFromFlatData(0, np.zeros(p.M * p.N, np.float32), ca.Shape(ca.Float32, p.M, p.N))
    backend.Synchronize()
    backend.DebugFailAllocAfter(1)
    try:
        r.run_direct(out)
    finally:
        backend.DebugFailAllocAfter(0)
    got = out.ToFlatData().reshape(p.M, p.N)
    assert np.array_equal(got.view(np.uint32), r.run().view(np.uint32))
    truth = O.qdense_f64(p)
    scale = O.qdense_f64(p, absolute=True)
    assert np.all(np.abs(got.astype(np.float64) - truth) <= 2.0 ** -22 * np.abs(truth) + 1e-5 * scale)
