"""Pins the GGML part of the CPU oracle (oracle/ggml_ref.c) before it is trusted as the checker.

The reference has no test of its own for the GGML formats (the formats are pinned only by their
definitions), so each function is checked against something independent of its code:
  oracle_f16_to_f32          every one of the 65536 half bit patterns against numpy's IEEE
                             conversion (bit-exact, NaN payloads included)
  block geometry             the literals of fused_ops.go:148-177
  Q8_0 / Q4_0 / IQ4_NL       blocks built so that each output position has a distinct, known
                             value: the nibble order (low nibbles first, then high) and the
                             offsets / table entries are fixed by closed forms; the IQ4_NL table is
                             the literal of fused_ops.go:127-130
  Q4_K / Q6_K                blocks produced by encoders written here from the block layout (the
                             inverse direction of the decoder), with d = dmin = 1 so every value is
                             an exact small integer sc*q - m / sc*(q - 32); then general scales
                             against the f64 product within one f32 rounding per operation
  dense product              one-hot x (exact), the bias added after the sum (a case where the
                             order changes the f32 result), brute-force f64 within the f32
                             accumulation bound
  embedding lookup           rows equal the dequantised rows; an out-of-range index is an error
"""
import numpy as np
import pytest

from oracle import oracle as O

RNG = np.random.default_rng(20260514)


def f16_bits(v) -> int:
    return int(np.array(v, dtype=np.float16).view(np.uint16))


def test_f16_to_f32_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32(h).view(np.uint32)
    want = h.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got, want)


def test_block_geometry_literals():
    assert O.ggml_block(O.GGML_Q4_0) == (32, 18)
    assert O.ggml_block(O.GGML_Q8_0) == (32, 34)
    assert O.ggml_block(O.GGML_IQ4_NL) == (32, 18)
    assert O.ggml_block(O.GGML_Q4_K) == (256, 144)
    assert O.ggml_block(O.GGML_Q6_K) == (256, 210)


def test_q8_0_closed_form():
    d = 0.375
    q = np.arange(-128, 128, dtype=np.int8)  # 256 values = 8 blocks
    blocks = []
    for b in range(8):
        blk = np.zeros(34, dtype=np.uint8)
        blk[0:2] = np.array([f16_bits(d)], dtype=np.uint16).view(np.uint8)
        blk[2:] = q[32 * b:32 * b + 32].view(np.uint8)
        blocks.append(blk)
    row = np.concatenate(blocks)[None, :]
    got = O.ggml_dequant(O.GGML_Q8_0, row)[0]
    assert np.array_equal(got, (d * q.astype(np.float64)).astype(np.float32))


def _nibble_block(d, lo, hi):
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = np.array([f16_bits(d)], dtype=np.uint16).view(np.uint8)
    blk[2:] = (np.asarray(lo) & 15) | ((np.asarray(hi) & 15) << 4)
    return blk


def test_q4_0_layout_and_offset():
    lo = np.arange(16)
    hi = 15 - np.arange(16)
    d = -0.25
    got = O.ggml_dequant(O.GGML_Q4_0, _nibble_block(d, lo, hi)[None, :])[0]
    want = np.concatenate([d * (lo - 8.0), d * (hi - 8.0)]).astype(np.float32)
    assert np.array_equal(got, want)


def test_iq4_nl_table_and_layout():
    table = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.float64)
    lo = np.arange(16)
    hi = (np.arange(16) * 7 + 3) % 16
    d = 0.5
    got = O.ggml_dequant(O.GGML_IQ4_NL, _nibble_block(d, lo, hi)[None, :])[0]
    want = np.concatenate([d * table[lo], d * table[hi]]).astype(np.float32)
    assert np.array_equal(got, want)


def encode_q4_k(d, dmin, sc, m, q):
    """One Q4_K block from 8 six-bit scales sc, 8 six-bit mins m and 256 nibbles q (0..15)."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.array([f16_bits(d)], dtype=np.uint16).view(np.uint8)
    blk[2:4] = np.array([f16_bits(dmin)], dtype=np.uint16).view(np.uint8)
    s = np.zeros(12, dtype=np.int64)
    for j in range(4):  # sub-blocks 0-3: 6 bits each in bytes j (scale) and j + 4 (min)
        s[j] |= sc[j] & 63
        s[j + 4] |= m[j] & 63
    for j in range(4, 8):  # sub-blocks 4-7: low 4 bits in byte j + 4, high 2 bits on top of j-4 / j
        s[j + 4] |= (sc[j] & 15) | ((m[j] & 15) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (m[j] >> 4) << 6
    blk[4:16] = s.astype(np.uint8)
    # 4 chunks of 64 values: 32 bytes, values 0-31 of a chunk in the low nibbles, 32-63 high.
    q = np.asarray(q).reshape(4, 2, 32)
    blk[16:] = (q[:, 0, :] | (q[:, 1, :] << 4)).astype(np.uint8).ravel()
    return blk


def test_q4_k_exact_integers_from_encoder():
    for _ in range(20):
        sc = RNG.integers(0, 64, 8)
        m = RNG.integers(0, 64, 8)
        q = RNG.integers(0, 16, 256)
        got = O.ggml_dequant(O.GGML_Q4_K, encode_q4_k(1.0, 1.0, sc, m, q)[None, :])[0]
        want = (np.repeat(sc, 32) * q - np.repeat(m, 32)).astype(np.float32)
        assert np.array_equal(got, want)


def test_q4_k_general_scales_one_rounding():
    sc = RNG.integers(0, 64, 8)
    m = RNG.integers(0, 64, 8)
    q = RNG.integers(0, 16, 256)
    d, dmin = 0.0123, 0.00456
    blk = encode_q4_k(d, dmin, sc, m, q)
    d16, dm16 = float(np.float16(d)), float(np.float16(dmin))
    got = O.ggml_dequant(O.GGML_Q4_K, blk[None, :])[0].astype(np.float64)
    exact = d16 * np.repeat(sc, 32) * q - dm16 * np.repeat(m, 32)
    # d*sc, d*sc*q and dmin*m are exact in f32 (<= 24 significant bits); only the subtraction rounds.
    assert np.all(np.abs(got - exact) <= np.abs(exact) * 2.0 ** -24 + 1e-30)


def encode_q6_k(d, sc, q):
    """One Q6_K block from 16 int8 scales and 256 six-bit values q (0..63; value = q - 32)."""
    q = np.asarray(q).reshape(2, 4, 32)  # [half][quarter][l]
    ql = np.zeros((2, 64), dtype=np.int64)
    qh = np.zeros((2, 32), dtype=np.int64)
    for h in range(2):
        q1, q2, q3, q4 = q[h]
        ql[h, :32] = (q1 & 15) | ((q3 & 15) << 4)
        ql[h, 32:] = (q2 & 15) | ((q4 & 15) << 4)
        qh[h] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    blk = np.zeros(210, dtype=np.uint8)
    blk[0:128] = ql.ravel().astype(np.uint8)
    blk[128:192] = qh.ravel().astype(np.uint8)
    blk[192:208] = np.asarray(sc, dtype=np.int8).view(np.uint8)
    blk[208:210] = np.array([f16_bits(d)], dtype=np.uint16).view(np.uint8)
    return blk


def q6_k_scale_of_position():
    """Scale index of each of the 256 positions: half h, quarter j, l -> 8h + 2j + l // 16."""
    idx = np.empty(256, dtype=np.int64)
    for h in range(2):
        for j in range(4):
            for l in range(32):
                idx[128 * h + 32 * j + l] = 8 * h + 2 * j + l // 16
    return idx


def test_q6_k_exact_integers_from_encoder():
    pos = q6_k_scale_of_position()
    for _ in range(20):
        sc = RNG.integers(-128, 128, 16)
        q = RNG.integers(0, 64, 256)
        got = O.ggml_dequant(O.GGML_Q6_K, encode_q6_k(1.0, sc, q)[None, :])[0]
        want = (sc[pos] * (q - 32)).astype(np.float32)
        assert np.array_equal(got, want)


def test_q6_k_general_scale_rounding():
    pos = q6_k_scale_of_position()
    sc = RNG.integers(-128, 128, 16)
    q = RNG.integers(0, 64, 256)
    d = 0.000731
    got = O.ggml_dequant(O.GGML_Q6_K, encode_q6_k(d, sc, q)[None, :])[0].astype(np.float64)
    exact = float(np.float16(d)) * sc[pos] * (q - 32)
    # d*sc is exact; the product with q rounds once.
    assert np.all(np.abs(got - exact) <= np.abs(exact) * 2.0 ** -24)


def random_rows(t, n, k, rng=RNG):
    """Random GGML rows with finite, moderate block scales."""
    vpb, bpb = O.ggml_block(t)
    nb = k // vpb
    rows = rng.integers(0, 256, (n, nb, bpb), dtype=np.uint8)
    scale_at = {O.GGML_Q4_0: [0], O.GGML_Q8_0: [0], O.GGML_IQ4_NL: [0], O.GGML_Q4_K: [0, 2], O.GGML_Q6_K: [208]}[t]
    for off in scale_at:
        d = rng.uniform(0.001, 0.02, (n, nb)).astype(np.float16).view(np.uint16)
        rows[:, :, off] = d & 0xFF
        rows[:, :, off + 1] = d >> 8
    return rows.reshape(n, nb * bpb)


@pytest.mark.parametrize("t", O.GGML_TYPES)
def test_dense_one_hot_is_exact(t):
    K, N = 512, 24
    w = random_rows(t, N, K)
    deq = O.ggml_dequant(t, w)
    ks = [0, 1, 31, 32, 255, 256, 511]
    x = np.zeros((len(ks), K), dtype=np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    got = O.ggml_dense(x, w, t)
    assert np.array_equal(got, deq[:, ks].T)


def test_dense_bias_is_added_after_the_sum():
    # Two terms that cancel exactly, then the bias: bias-last gives 1, bias-first loses it.
    t = O.GGML_Q8_0
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = np.array([f16_bits(1.0)], dtype=np.uint16).view(np.uint8)
    blk[2] = 1
    blk[3] = 0xFF  # -1
    x = np.zeros((1, 32), dtype=np.float32)
    x[0, 0] = 1.0e8
    x[0, 1] = 1.0e8
    got = O.ggml_dense(x, blk[None, :], t, bias=np.array([1.0], dtype=np.float32))
    assert got[0, 0] == 1.0


@pytest.mark.parametrize("t", O.GGML_TYPES)
def test_dense_matches_f64_within_accumulation_bound(t):
    M, K, N = 3, 1024, 40
    w = random_rows(t, N, K)
    x = RNG.standard_normal((M, K)).astype(np.float32)
    b = RNG.standard_normal(N).astype(np.float32)
    got = O.ggml_dense(x, w, t, bias=b)
    exact, ab = O.ggml_dense_f64(x, w, t, bias=b)
    # K + 1 roundings of at most 2^-24 relative each on partial sums bounded by sum |terms|.
    assert np.all(np.abs(got - exact) <= (K + 2) * 2.0 ** -24 * ab + 1e-30)
    # and the bound is not vacuous: the values differ from a sloppy computation that drops the bias.
    assert not np.allclose(got, exact - b, rtol=0, atol=1e-6)


@pytest.mark.parametrize("t", O.GGML_TYPES)
def test_embedding_rows_are_dequantised_rows(t):
    V, K = 37, 512
    data = random_rows(t, V, K)
    idx = np.array([[3], [0], [36], [3]])
    got = O.ggml_embedding(data, t, idx)
    assert np.array_equal(got, O.ggml_dequant(t, data)[idx.ravel()])
    with pytest.raises(IndexError):
        O.ggml_embedding(data, t, np.array([[5], [37]]))
