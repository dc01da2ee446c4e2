"""Pins the CPU oracle (oracle/qdense_ref.c) before it is trusted as the parity checker.

Every oracle function is checked against the reference's own known-answer vectors
(tests/golden/reference_kats.json) and/or against what the mathematics fixes: closed forms,
exhaustive tables, exact-integer special cases and invariants.  Each check is chosen so that a
plausible slip (a dropped term, a wrong scale index, a swapped nibble, a missing rounding) fails.

  oracle function            pinned by
  -------------------------  ------------------------------------------------------------------
  oracle_unpack_int4/uint4   reference KAT {0xF0,0x87}; exhaustive 256-byte closed form
  oracle_f32_to_bf16         nearest-even by brute force over both neighbours; ties; NaN/Inf
  oracle_act                 reference GELU KAT (tol 1e-6); closed forms in float64 for the rest
  oracle_nf4                 reference table literal
  oracle_qdense (Linear)     identity weights (exact), one-hot scale blocks/groups (exact closed
                             form), 2^p scale invariance (exact), zero x -> act(bias) (exact),
                             int4 == int8 with the same values (exact), f64 brute force bound
  oracle_qdense (zero point) w = 0 -> x . zp closed form
  oracle_qdense (NF4)        one-hot x selects NF4[w] exactly
  dot_general (numpy)        reference DotGeneral KATs
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


# ---------------------------------------------------------------------------------------------
# Int4 unpacking.
# ---------------------------------------------------------------------------------------------
def test_int4_unpack_reference_kat():
    k = GOLDEN["int4_unpack"]
    assert O.unpack_int4(np.array(k["packed"], np.uint8)).tolist() == k["int4"]
    assert O.unpack_int4(np.array(k["packed"], np.uint8), signed=False).tolist() == k["uint4"]


def test_int4_unpack_exhaustive_closed_form():
    b = np.arange(256, dtype=np.uint8)
    got = O.unpack_int4(b).astype(np.int64)
    lo, hi = (b & 15).astype(np.int64), (b >> 4).astype(np.int64)
    # two's complement of a 4-bit field: v - 16 when the sign bit (8) is set
    assert np.array_equal(got[0::2], lo - 16 * (lo >= 8))
    assert np.array_equal(got[1::2], hi - 16 * (hi >= 8))
    gotu = O.unpack_int4(b, signed=False).astype(np.int64)
    assert np.array_equal(gotu[0::2], lo) and np.array_equal(gotu[1::2], hi)
    # pack is the inverse on the whole signed range
    vals = np.tile(np.arange(-8, 8), 3)
    assert np.array_equal(O.unpack_int4(O.pack_int4(vals))[: vals.size], vals)


# ---------------------------------------------------------------------------------------------
# bf16 rounding.
# ---------------------------------------------------------------------------------------------
def _bf16_nearest_even(x: float) -> int:
    """Independent formulation: pick the nearer of the two bf16 neighbours, ties to even."""
    bits = int(np.float32(x).view(np.uint32))
    lo = bits >> 16          # truncated magnitude
    hi = lo + 1              # next magnitude away from zero (same sign)
    val = lambda h: float(np.array([h << 16], np.uint32).view(np.float32)[0])
    xd = float(np.float32(x))
    dlo, dhi = abs(xd - val(lo)), abs(val(hi) - xd)
    if dlo != dhi:
        return lo if dlo < dhi else hi
    return lo if lo % 2 == 0 else hi


def test_bf16_round_nearest_even_brute_force():
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.standard_normal(2000).astype(np.float32),
                         (rng.standard_normal(500) * 1e-30).astype(np.float32),
                         (rng.standard_normal(500) * 1e30).astype(np.float32)])
    got = O.bf16_round(xs)
    for x, g in zip(xs, got):
        assert int(g) == _bf16_nearest_even(float(x)), x


def test_bf16_round_ties_and_specials():
    f = lambda bits: np.array([bits], np.uint32).view(np.float32)
    assert O.bf16_round(f(0x3F800000))[0] == 0x3F80          # 1.0
    assert O.bf16_round(f(0x3F808000))[0] == 0x3F80          # tie, even stays
    assert O.bf16_round(f(0x3F818000))[0] == 0x3F82          # tie, odd rounds up
    assert O.bf16_round(f(0x3F808001))[0] == 0x3F81          # above tie
    assert O.bf16_round(f(0xBF808001))[0] == 0xBF81          # sign symmetric
    assert O.bf16_round(f(0x7F800000))[0] == 0x7F80          # +Inf
    assert O.bf16_round(f(0x7FC00001))[0] == 0x7FC0          # NaN keeps its top bits
    assert O.bf16_round(f(0x7F7FFFFF))[0] == 0x7F80          # max float rounds to Inf


# ---------------------------------------------------------------------------------------------
# Activations.
# ---------------------------------------------------------------------------------------------
def test_gelu_reference_kat():
    k = GOLDEN["gelu_exact"]
    got = O.act(np.array(k["input"], np.float32), O.ACT_GELU)
    assert np.allclose(got, k["want"], atol=k["tolerance"], rtol=0)


@pytest.mark.parametrize("a", [O.ACT_GELU, O.ACT_SILU, O.ACT_TANH, O.ACT_RELU, O.ACT_HARDSWISH, O.ACT_NONE])
def test_activation_closed_forms(a):
    rng = np.random.default_rng(a)
    x = (rng.standard_normal(4000) * 4).astype(np.float32)
    xd = x.astype(np.float64)
    want = {
        O.ACT_GELU: xd * 0.5 * (1 + np.vectorize(math.erf)(xd / math.sqrt(2))),
        O.ACT_SILU: xd / (1 + np.exp(-xd)),
        O.ACT_TANH: np.tanh(xd),
        O.ACT_RELU: np.maximum(xd, 0),
        O.ACT_HARDSWISH: xd * np.clip(xd / 6 + 0.5, 0, 1),
        O.ACT_NONE: xd,
    }[a]
    got = O.act(x, a).astype(np.float64)
    assert np.allclose(got, want, rtol=4e-7, atol=1e-7)
    # special values
    assert O.act(np.array([0.0], np.float32), a)[0] == 0.0
    if a != O.ACT_NONE:
        assert np.isnan(O.act(np.array([np.nan], np.float32), a)[0])


def test_nf4_table_literal():
    vals = [O.lib().oracle_nf4(i) for i in range(16)]
    assert np.array_equal(np.float32(vals), np.float32(GOLDEN["nf4_table"]["values"]))


# ---------------------------------------------------------------------------------------------
# QuantizedDense.
# ---------------------------------------------------------------------------------------------
def _prob(M, K, N, **kw):
    kw.setdefault("x_dtype", O.DT_FLOAT32)
    kw.setdefault("scale_dtype", O.DT_FLOAT32)
    return O.make_problem(M, K, N, **kw)


def test_qdense_identity_weights_exact():
    K = N = 24
    p = _prob(3, K, N, w_dtype=O.DT_INT8, block_axis=1, block_size=N, bias=True)
    p.w = np.eye(K, dtype=np.int8)
    p.scale = np.ones(p.scale_shape, np.float32)
    y = O.qdense_f32(p)
    x = p.x.reshape(3, K)
    assert np.array_equal(y, (x + p.bias[None, :]).astype(np.float32))


@pytest.mark.parametrize("w_dtype", [O.DT_INT8, O.DT_UINT8, O.DT_INT4, O.DT_UINT4])
def test_qdense_one_hot_block_axis1_exact(w_dtype):
    # scales [K, ceil(N/B)] with a ragged last block: only block (k0, j0) is non-zero.
    M, K, N, B = 2, 10, 13, 4
    p = _prob(M, K, N, w_dtype=w_dtype, block_axis=1, block_size=B, bias=False)
    p.x = np.round(p.x * 4).astype(np.float32)  # small integers: every product/sum exact
    wv = O.unpack_int4(p.w, signed=w_dtype == O.DT_INT4)[: K * N] if w_dtype in (O.DT_INT4, O.DT_UINT4) \
        else p.w.ravel().astype(np.int64)
    wv = np.asarray(wv, np.int64).reshape(K, N)
    for k0, j0 in [(0, 0), (7, 3), (9, 2)]:
        p.scale = np.zeros((K, (N + B - 1) // B), np.float32)
        p.scale[k0, j0] = 1.0
        y = O.qdense_f32(p)
        want = np.zeros((M, N))
        cols = slice(j0 * B, min(N, (j0 + 1) * B))
        want[:, cols] = p.x.reshape(M, K)[:, k0:k0 + 1] * wv[k0, cols][None, :]
        assert np.array_equal(y, want.astype(np.float32)), (k0, j0)


@pytest.mark.parametrize("w_dtype", [O.DT_INT8, O.DT_INT4])
def test_qdense_one_hot_group_block_axis0_exact(w_dtype):
    # scales [ceil(K/G), N] with a ragged last group.
    M, K, N, G = 3, 22, 6, 8
    p = _prob(M, K, N, w_dtype=w_dtype, block_axis=0, block_size=G, bias=False)
    p.x = np.round(p.x * 4).astype(np.float32)
    wv = (O.unpack_int4(p.w)[: K * N] if w_dtype == O.DT_INT4 else p.w.ravel()).astype(np.int64).reshape(K, N)
    for g0, n0 in [(0, 0), (2, 5), (1, 3)]:
        p.scale = np.zeros(((K + G - 1) // G, N), np.float32)
        p.scale[g0, n0] = 2.0
        y = O.qdense_f32(p)
        ks = slice(g0 * G, min(K, (g0 + 1) * G))
        want = np.zeros((M, N))
        want[:, n0] = 2.0 * (p.x.reshape(M, K)[:, ks] @ wv[ks, n0])
        assert np.array_equal(y, want.astype(np.float32)), (g0, n0)


def test_qdense_power_of_two_scale_invariance_exact():
    p = _prob(4, 64, 48, w_dtype=O.DT_INT8, block_axis=1, block_size=16, bias=False)
    y1 = O.qdense_f32(p)
    p.scale = (p.scale * np.float32(8.0)).astype(np.float32)
    y2 = O.qdense_f32(p)
    assert np.array_equal(y2, y1 * np.float32(8.0))


@pytest.mark.parametrize("a", [O.ACT_NONE, O.ACT_GELU, O.ACT_SILU, O.ACT_TANH])
def test_qdense_zero_x_gives_act_bias(a):
    p = _prob(2, 32, 40, w_dtype=O.DT_INT4, block_axis=0, block_size=16, bias=True, act=a)
    p.x = np.zeros_like(p.x)
    y = O.qdense_f32(p)
    assert np.array_equal(y, np.broadcast_to(O.act(p.bias, a), y.shape))


def test_qdense_int4_equals_int8_same_values():
    K, N = 32, 40
    p4 = _prob(3, K, N, w_dtype=O.DT_INT4, block_axis=1, block_size=8, bias=True, act=O.ACT_SILU)
    vals = O.unpack_int4(p4.w)[: K * N].reshape(K, N)
    p8 = O.QDenseProblem(**{**p4.__dict__, "w": vals.astype(np.int8), "w_dtype": O.DT_INT8})
    assert np.array_equal(O.qdense_f32(p4), O.qdense_f32(p8))


@pytest.mark.parametrize("block_axis", [0, 1])
def test_qdense_brute_force_f64_bound(block_axis):
    M, K, N = 3, 50, 21
    p = _prob(M, K, N, w_dtype=O.DT_INT8, block_axis=block_axis, block_size=7, bias=True)
    x = p.x.reshape(M, K).astype(np.float64)
    w = p.w.astype(np.float64)
    s = p.scale.astype(np.float64)
    want = np.zeros((M, N))
    absum = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = float(p.bias[n])
            ab = abs(float(p.bias[n]))
            for k in range(K):
                sv = s[k, n // 7] if block_axis == 1 else s[k // 7, n]
                t = x[m, k] * w[k, n] * sv
                acc += t
                ab += abs(t)
            want[m, n] = acc
            absum[m, n] = ab
    y = O.qdense_f32(p).astype(np.float64)
    eps = np.finfo(np.float32).eps
    assert np.all(np.abs(y - want) <= 3 * K * eps * absum + 1e-30)
    assert np.allclose(O.qdense_f64(p), want, rtol=1e-12, atol=1e-12)
    assert np.allclose(O.qdense_f64(p, absolute=True), absum, rtol=1e-12, atol=1e-12)


def test_qdense_zero_point_closed_form():
    M, K, N = 2, 12, 10
    p = _prob(M, K, N, w_dtype=O.DT_INT8, block_axis=1, block_size=5, bias=False, zp=True)
    p.w = np.zeros((K, N), np.int8)
    p.x = np.round(p.x * 4).astype(np.float32)
    p.zp = np.round(p.zp * 64).astype(np.float32) / 64  # dyadic: exact sums
    y = O.qdense_f32(p)
    zexp = np.repeat(p.zp, 5, axis=1)[:, :N]
    assert np.array_equal(y, (p.x.reshape(M, K) @ zexp).astype(np.float32))


def test_qdense_nf4_one_hot_x():
    K, N = 6, 16
    p = _prob(K, K, N, w_dtype=O.DT_UINT8, block_axis=1, block_size=N, bias=False, scheme=O.QUANT_NF4)
    p.x = np.eye(K, dtype=np.float32)
    p.w = (np.arange(K * N) % 16).astype(np.uint8).reshape(K, N)
    p.scale = np.ones(p.scale_shape, np.float32)
    y = O.qdense_f32(p)
    table = np.float32(GOLDEN["nf4_table"]["values"])
    assert np.array_equal(y, table[p.w.astype(np.int64)])


# Order of operations of the reference loop (quantizeddense.go:616-650): the output starts at the
# bias, the terms are added in increasing k, and each term is ((x * w) * s), or x * (w * s + zp)
# with zero points, (x * nf4[w]) * s for NF4, every operation rounded to f32.  Each case below has
# an expected result that any other order or grouping changes.
def _one_term(x_bits, w, s_bits, w_dtype=O.DT_INT8, zp_bits=None, scheme=O.QUANT_LINEAR):
    p = _prob(1, 1, 1, w_dtype=w_dtype, block_axis=1, block_size=1, bias=False, zp=zp_bits is not None,
              scheme=scheme)
    p.x = np.array([[x_bits]], np.uint32).view(np.float32)
    p.w = np.array([[w]], np.int8 if w_dtype == O.DT_INT8 else np.uint8)
    p.scale = np.array([[s_bits]], np.uint32).view(np.float32)
    if zp_bits is not None:
        p.zp = np.array([[zp_bits]], np.uint32).view(np.float32)
    return int(O.qdense_f32(p).view(np.uint32)[0, 0])


def test_qdense_bias_is_added_first():
    # bias 2^24, then eight terms of 1: each 2^24 + 1 rounds back to 2^24 (ties to even), so the
    # result stays 2^24; summing the terms first would give 2^24 + 8.
    K = 8
    p = _prob(1, K, 1, w_dtype=O.DT_INT8, block_axis=1, block_size=1, bias=True)
    p.x = np.ones((1, K), np.float32)
    p.w = np.ones((K, 1), np.int8)
    p.scale = np.ones((K, 1), np.float32)
    p.bias = np.array([2.0 ** 24], np.float32)
    assert O.qdense_f32(p)[0, 0] == np.float32(2.0 ** 24)


def test_qdense_terms_in_increasing_k():
    # x = [2^24, 1 (six times), -2^24]: in increasing k the six ones are lost against 2^24 and the
    # result is 0; decreasing k gives 6, and pairwise or blocked sums give other values.
    K = 8
    p = _prob(1, K, 1, w_dtype=O.DT_INT8, block_axis=1, block_size=1, bias=False)
    p.x = np.array([[2.0 ** 24] + [1.0] * 6 + [-(2.0 ** 24)]], np.float32)
    p.w = np.ones((K, 1), np.int8)
    p.scale = np.ones((K, 1), np.float32)
    assert O.qdense_f32(p)[0, 0] == np.float32(0.0)


def test_qdense_term_is_x_times_w_then_scale():
    # x = -0.96694475 (bits 3212282289), w = -59, s = 0.008319432 (bits 1007177274):
    # (x * w) * s rounds to bits 1056113044; x * (w * s) would round to 1056113045.
    assert _one_term(3212282289, -59, 1007177274) == 1056113044


def test_qdense_zero_point_term_grouping():
    # x * (w * s + zp) with x bits 1063174608, w = 27, s bits 1007202239, zp bits 3175853478 rounds
    # to bits 1042048540; (x * w) * s + x * zp gives 1042048542 and x * (w * s) + x * zp gives
    # 1042048541.
    assert _one_term(1063174608, 27, 1007202239, zp_bits=3175853478) == 1042048540


def test_qdense_nf4_term_is_x_times_value_then_scale():
    # NF4 code 12, x bits 1019326333, s bits 991334551: (x * nf4[12]) * s rounds to bits 935907406;
    # x * (nf4[12] * s) would round to 935907407.
    assert _one_term(1019326333, 12, 991334551, w_dtype=O.DT_UINT8, scheme=O.QUANT_NF4) == 935907406


def test_qdense_threads_do_not_change_result():
    p = O.make_problem(1, 256, 300, w_dtype=O.DT_INT4, block_axis=0, block_size=64, seed=3)
    assert np.array_equal(O.qdense_f32(p, threads=1), O.qdense_f32(p, threads=4))
    p = O.make_problem(5, 128, 64, w_dtype=O.DT_INT8, block_axis=0, block_size=32, seed=4)
    assert np.array_equal(O.qdense_f32(p, threads=1), O.qdense_f32(p, threads=3))


def test_baseline_config_shapes():
    c1 = O.baseline_config(0)
    assert (c1.M, c1.K, c1.N, c1.scale.shape, c1.x.dtype) == (4, 512, 512, (512,), np.float32)
    c2 = O.baseline_config(1)
    assert c2.w.nbytes == 4096 * 11008 // 2 and c2.scale.shape == (32, 11008)
    assert O.algorithmic_bytes(c2) == 23_279_104
    assert O.algorithmic_bytes(c1) == 282_624


# ---------------------------------------------------------------------------------------------
# DotGeneral restatement vs the reference KATs.
# ---------------------------------------------------------------------------------------------
def test_dot_general_kats():
    k = GOLDEN["dot_general_shuffled_axes"]
    lhs = np.arange(1, 1 + np.prod(k["lhs_iota_from_1_shape"]), dtype=np.float64).reshape(k["lhs_iota_from_1_shape"])
    rhs = np.arange(1, 1 + np.prod(k["rhs_iota_from_1_shape"]), dtype=np.float64).reshape(k["rhs_iota_from_1_shape"])
    got = O.dot_general(lhs, k["lhs_contracting"], k["lhs_batch"], rhs, k["rhs_contracting"], k["rhs_batch"])
    assert np.array_equal(got, np.array(k["want"], np.float64))
    k = GOLDEN["dot_general_axis_transposition"]
    got = O.dot_general(np.array(k["lhs"]), k["lhs_contracting"], k["lhs_batch"], np.array(k["rhs"]),
                        k["rhs_contracting"], k["rhs_batch"])
    assert np.array_equal(got, np.array(k["want"]))
    k = GOLDEN["dot_general_small_matmul"]
    a, b = np.array(k["a"]), np.array(k["b"])
    assert np.array_equal(O.dot_general(a, [1], [], b, [0], []), k["non_transposed"])
    assert np.array_equal(O.dot_general(a, [1], [], b, [1], []), k["transposed"])
    assert np.array_equal(O.dot_general(np.array(k["vec"]), [0], [], np.array(k["mat"]), [0], []), k["vec_mat"])
    assert np.array_equal(O.dot_general(np.array(k["mat2"]), [1], [], np.array(k["vec"]), [0], []), k["mat_vec"])
    k = GOLDEN["dot_general_shape"]
    got = O.dot_general(np.zeros(k["lhs_shape"]), k["lhs_contracting"], k["lhs_batch"], np.zeros(k["rhs_shape"]),
                        k["rhs_contracting"], k["rhs_batch"])
    assert list(got.shape) == k["want_shape"]
    k = GOLDEN["dot_general_f64_very_large"]
    lhs = ((np.arange(np.prod(k["lhs_shape"])) + 1.0) * 1e-5).reshape(k["lhs_shape"])
    got = O.dot_general(lhs, [2], [], np.ones(k["rhs_shape"]), [0], [])
    assert abs(got[0, 0, 0] - k["want_out_0_0_0"]) < k["tolerance"]


def test_rmsnorm_chain_closed_forms():
    """Constant rows c: the sequential f32 sum of D squares is D c^2 exactly (multiples of c^2 with
    few significant bits), so h = bf16(c / sqrt(c^2 + eps)); with eps = 0 that is exactly +-1.
    Alternating signs give the same magnitudes; a row scaled by 2^k normalises to the same h."""
    D = 4096
    for c in (0.75, -1.5, 3.0):
        x = O.bf16_round(np.full((2, D), c, np.float32))
        h = O.rmsnorm_chain(x, 0.0)
        assert np.all(O.bf16_to_f32(h) == np.sign(c)), c
        alt = O.bf16_round(np.tile(np.array([c, -c], np.float32), (1, D // 2)))
        assert np.array_equal(np.abs(O.bf16_to_f32(O.rmsnorm_chain(alt, 0.0))), np.ones((1, D), np.float32))
        h_eps = O.bf16_to_f32(O.rmsnorm_chain(x, 1e-6))
        want = np.float32(c) / np.sqrt(np.float64(c) ** 2 + np.float64(np.float32(1e-6)))
        assert np.all(np.abs(h_eps - want) <= 2.0 ** -8 * abs(want)), c
    rng = np.random.default_rng(3)
    xf = rng.standard_normal((3, 512)).astype(np.float32)
    a = O.rmsnorm_chain(O.bf16_round(xf), 0.0)
    b = O.rmsnorm_chain(O.bf16_round(xf * 8.0), 0.0)
    assert np.array_equal(a, b)


def test_rmsnorm_chain_sum_is_sequential():
    """A row whose in-order f32 sum differs from the exact sum: 4096^2 = 2^24 first, then 63 ones,
    each of which is lost in f32 (2^24 + 1 rounds to 2^24).  In order the mean square is exactly
    2^24 / 64 = 2^18 and Rsqrt is 2^-9; any order that adds the ones first gives another f32."""
    D = 64
    x = np.ones((1, D), np.float32)
    x[0, 0] = 4096.0
    _, inv = O.rmsnorm_chain(O.bf16_round(x), 0.0, return_inv=True)
    assert inv[0] == np.float32(2.0 ** -9)
    exact = 1.0 / np.sqrt((2.0 ** 24 + 63) / 64)
    assert np.float32(exact) != np.float32(2.0 ** -9)


def test_dot_general_int_closed_forms():
    """Integer DotGeneral restatement: identity contraction, the int8 wrap (100 * 2 + 100 * 2 =
    400 = -112 mod 256), int32 overflow (2^30 * 4 = 0 mod 2^32), an accumulator dtype that
    avoids the wrap, unsigned wrap, and agreement with float64 matmul where nothing wraps."""
    eye = np.eye(3, dtype=np.int32)
    x = np.arange(6, dtype=np.int32).reshape(2, 3)
    assert np.array_equal(O.dot_general_int(x, [1], [], eye, [0], []), x)
    a = np.array([[100, 100]], np.int8)
    b = np.array([[2], [2]], np.int8)
    assert O.dot_general_int(a, [1], [], b, [0], [])[0, 0] == np.int8(-112)
    assert O.dot_general_int(a, [1], [], b, [0], [], acc_dtype=np.int32)[0, 0] == 400
    big = np.array([[1 << 30]], np.int32)
    assert O.dot_general_int(big, [1], [], np.array([[4]], np.int32), [0], [])[0, 0] == 0
    u = np.array([[255, 255]], np.uint8)
    assert O.dot_general_int(u, [1], [], np.array([[255], [1]], np.uint8), [0], [])[0, 0] == (255 * 255 + 255) % 256
    rng = np.random.default_rng(0)
    l = rng.integers(-50, 50, (2, 3, 4)).astype(np.int32)
    r = rng.integers(-50, 50, (2, 4, 5)).astype(np.int32)
    assert np.array_equal(O.dot_general_int(l, [2], [0], r, [1], [0]), O.dot_general(l, [2], [0], r, [1], [0]).astype(np.int32))
