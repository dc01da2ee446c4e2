"""FusedQuantizedDense on the GPU vs the CPU oracle (the reference's arithmetic restated).

Bars (from the task's north star):
  - f32 activations: the exact kernel reproduces the reference loop order, so results must be
    bit-identical to the oracle's f32 result;
  - bf16 activations through the exact kernel: bit-identical to RNE(oracle f32);
  - bf16 activations through the fast kernels (other summation order): within rel 1e-2 /
    abs 1e-3 of the oracle's f32 result, and the kernel's f32 accumulation (checked with the
    identity activation on a f32 output) within 1e-5 of sum|terms| of the f64 value.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.qd_helpers import QDenseRun, assert_bf16_close, run_qdense

pytestmark = pytest.mark.gpu

W_DTYPES = [O.DT_INT8, O.DT_UINT8, O.DT_INT4, O.DT_UINT4]
FAST_DECODE = "qdense_skinny_mfma"


# ---------------------------------------------------------------------------------------------
# Exact kernel: bit-exact vs the reference loop.
# ---------------------------------------------------------------------------------------------
def test_c1_config_bit_exact(backend):
    """int8 per-channel, x f32 [4,512], bias, no activation."""
    p = O.baseline_config(0)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_exact"
    y = r.run()
    assert np.array_equal(y.view(np.uint32), O.qdense_f32(p).view(np.uint32))


@pytest.mark.parametrize("w_dtype", W_DTYPES)
@pytest.mark.parametrize("block_axis", [0, 1])
@pytest.mark.parametrize("zp", [False, True])
def test_exact_f32_variants(backend, w_dtype, block_axis, zp):
    p = O.make_problem(5, 37, 29, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=block_axis, block_size=8, bias=True, zp=zp, act=O.ACT_GELU, seed=11)
    y = run_qdense(backend, p)
    assert np.array_equal(y.view(np.uint32), O.qdense_f32(p).view(np.uint32))


@pytest.mark.parametrize("act", range(6))
def test_exact_activations(backend, act):
    p = O.make_problem(3, 64, 48, w_dtype=O.DT_INT8, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=16, bias=True, act=act, scale_range=(0.05, 0.2), seed=act)
    y = run_qdense(backend, p)
    assert np.array_equal(y.view(np.uint32), O.qdense_f32(p).view(np.uint32))


@pytest.mark.parametrize("w_dtype", [O.DT_INT4, O.DT_UINT8])
def test_exact_nf4(backend, w_dtype):
    p = O.make_problem(4, 40, 33, w_dtype=w_dtype, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32, block_axis=1,
                       block_size=11, bias=True, scheme=O.QUANT_NF4, seed=5)
    y = run_qdense(backend, p)
    assert np.array_equal(y.view(np.uint32), O.qdense_f32(p).view(np.uint32))


@pytest.mark.parametrize("shape", [(1, 33, 17), (9, 7, 3), (2, 1, 1), (17, 130, 65)])
def test_exact_bf16_ragged_shapes(backend, shape):
    M, K, N = shape
    p = O.make_problem(M, K, N, w_dtype=O.DT_INT4, block_axis=0, block_size=4, bias=True, act=O.ACT_SILU, seed=M)
    r = QDenseRun(backend, p)
    assert r.plan() == "qdense_exact"
    assert np.array_equal(r.run(), O.expected_output(p))


# The reference-order kernel's own paths, forced with the exact option: rows longer than one LDS
# chunk of x (512 values, the last batch partial), odd N with 4-bit storage (the nibble of
# element k*N + n alternates with k), bf16 scales / zero points stepped along K (their position
# in the 32-bit word alternates too), and the 8-rows-per-thread variant taken by grids with many
# rows.
EXACT_CASES = [
    # M, K, N, w_dtype, x_dtype, scale_dtype, block_axis, block_size, zp, scheme
    (3, 1100, 67, O.DT_INT4, O.DT_FLOAT32, O.DT_FLOAT32, 0, None, False, O.QUANT_LINEAR),   # one scale per column
    (3, 1100, 67, O.DT_INT4, O.DT_FLOAT32, O.DT_BFLOAT16, 0, 48, False, O.QUANT_LINEAR),    # groups across batches
    (2, 700, 45, O.DT_UINT4, O.DT_FLOAT32, O.DT_BFLOAT16, 1, 16, True, O.QUANT_LINEAR),     # reference layout, zp
    (2, 530, 31, O.DT_UINT4, O.DT_BFLOAT16, O.DT_FLOAT32, 1, 7, False, O.QUANT_NF4),        # NF4, odd N
    (600, 40, 256, O.DT_INT8, O.DT_FLOAT32, O.DT_FLOAT32, 0, None, False, O.QUANT_LINEAR),  # 8 rows per thread
    (600, 40, 130, O.DT_INT4, O.DT_FLOAT32, O.DT_BFLOAT16, 0, 16, True, O.QUANT_LINEAR),    # 8 rows, zp, groups
]


@pytest.mark.parametrize("case", EXACT_CASES, ids=lambda c: f"M{c[0]}K{c[1]}N{c[2]}_w{c[3]}_ax{c[6]}_B{c[7]}_zp{int(c[8])}_s{c[9]}")
def test_exact_kernel_paths(case):
    import compute_amd as ca
    M, K, N, w_dtype, x_dtype, s_dtype, axis, B, zp, scheme = case
    p = O.make_problem(M, K, N, w_dtype=w_dtype, x_dtype=x_dtype, scale_dtype=s_dtype, block_axis=axis,
                       block_size=B, bias=True, zp=zp, scheme=scheme, act=O.ACT_SILU, seed=M + K + N)
    ex = ca.New("exact")
    try:
        r = QDenseRun(ex, p)
        assert r.plan() == "qdense_exact"
        y = r.run()
    finally:
        ex.Finalize()
    want = O.expected_output(p)
    assert np.array_equal(y.view(np.uint16 if x_dtype == O.DT_BFLOAT16 else np.uint32),
                          want.view(np.uint16 if x_dtype == O.DT_BFLOAT16 else np.uint32))


def test_empty_and_zero_k(backend):
    p = O.make_problem(0, 16, 8, w_dtype=O.DT_INT8, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=8)
    assert run_qdense(backend, p).shape == (0, 8)
    # K = 0: the output is act(bias) (reference loop adds no terms).
    p = O.make_problem(3, 0, 8, w_dtype=O.DT_INT8, x_dtype=O.DT_FLOAT32, scale_dtype=O.DT_FLOAT32,
                       block_axis=1, block_size=8, bias=True, act=O.ACT_TANH)
    y = run_qdense(backend, p)
    assert np.array_equal(y, np.broadcast_to(O.act(p.bias, O.ACT_TANH), (3, 8)))


# ---------------------------------------------------------------------------------------------
# Decode (M = 1, bf16): the skinny MFMA kernel.
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("w_dtype", W_DTYPES)
@pytest.mark.parametrize("scale_dtype", [O.DT_BFLOAT16, O.DT_FLOAT32])
def test_gemv_small(backend, w_dtype, scale_dtype):
    p = O.make_problem(1, 512, 768, w_dtype=w_dtype, scale_dtype=scale_dtype, block_axis=0, block_size=128,
                       bias=True, act=O.ACT_SILU, seed=7)
    r = QDenseRun(backend, p)
    assert r.plan().startswith(FAST_DECODE)
    assert_bf16_close(r.run(), O.qdense_f32(p), what=f"gemv {w_dtype}")


@pytest.mark.parametrize("act", range(6))
def test_gemv_activations_and_per_channel(backend, act):
    p = O.make_problem(1, 1024, 512, w_dtype=O.DT_INT4, block_axis=0, block_size=1024, per_channel_1d=True,
                       bias=act % 2 == 0, act=act, scale_range=(0.01, 0.05), seed=20 + act)
    r = QDenseRun(backend, p)
    assert r.plan().startswith(FAST_DECODE)
    assert_bf16_close(r.run(), O.qdense_f32(p), what=f"act {act}")


def test_gemv_c2_config_full_size(backend):
    """x bf16 [1,4096], Int4 [4096,11008] g128, bf16 scales, no bias."""
    p = O.baseline_config(1)
    r = QDenseRun(backend, p)
    assert r.plan().startswith(FAST_DECODE) and r.plan().endswith("_i4")
    y1 = r.run()
    assert_bf16_close(y1, O.qdense_f32(p, threads=8), what="C2")
    # Deterministic across calls (split-K partials are summed in a fixed order; the arrival
    # counters are reset by the last workgroup).
    y2 = r.run()
    assert np.array_equal(y1, y2)


def test_gemv_accumulation_f32_bound(backend):
    """The fast kernel's f32 accumulation, before bf16 rounding, measured through a bf16 output
    of a problem whose result magnitude is dominated by one exactly-representable term."""
    p = O.make_problem(1, 2048, 1024, w_dtype=O.DT_INT4, block_axis=0, block_size=128, bias=False, seed=9)
    y = QDenseRun(backend, p).run()
    ref = O.qdense_f32(p)
    # bf16 rounding is at most half an ulp (2^-9 relative); allow that plus the accumulation term.
    truth = O.qdense_f64(p)
    scale = O.qdense_f64(p, absolute=True)
    got = O.bf16_to_f32(y).astype(np.float64)
    assert np.all(np.abs(got - truth) <= 2.0 ** -8 * np.abs(truth) + 1e-5 * scale)
    assert_bf16_close(y, ref)
