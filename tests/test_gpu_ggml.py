"""GPU parity of the GGML block formats (compute_amd/csrc/ggml.hip) against the CPU oracle.

- ggml_dense_exact (problems of at most 2^24 multiply-adds past 4 rows, anything the GEMV does
  not take, and every size under the exact backend option): bit-identical f32 output, bias and
  activation included (the reference's order: dot, then bias, then activation).
- ggml_gemv (M <= 4, and M <= 20 as one launch per group of four rows; rows too long for one
  launch in K segments added in order): f32 accumulation bar —
  |y - exact| <= 1e-5 * sum|x*w| per output (the kernel sums in another order), identical bits
  on repeated calls, rows whose byte length is not a multiple of 16 (staging skew), the decode
  shape [1, 4096] x 11008 rows, ragged last groups (M = 5, 15).
- ggml_dequant_f32_mfma (M > 20): rows dequantised to f32, contracted on the matrix cores, bias
  and activation after the sum; the same accumulation bar, activation within float tolerance.
- QuantizedEmbeddingLookup: bit-identical rows for every index dtype; an index outside
  [0, vocab) fails the Execute call, as the reference's executor does.
"""
import numpy as np
import pytest
from scipy.special import erf, expit

import compute_amd as ca
from compute_amd import _lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TYPES = [ca.GGMLQ4_0, ca.GGMLQ8_0, ca.GGMLIQ4NL, ca.GGMLQ4_K, ca.GGMLQ6_K]
RNG = np.random.default_rng(7)


class GgmlRun:
    def __init__(self, backend, t, x, w, bias=None, act=ca.ActivationNone):
        self.backend, self.t, self.act = backend, int(t), int(act)
        self.M, self.K = x.shape
        self.N, self.bpr = w.shape
        bld = backend.Builder("ggml")
        f = bld.Main()
        shapes = [ca.Shape(ca.Float32, self.M, self.K), ca.Shape(ca.Uint8, self.N, self.bpr)]
        datas = [x.astype(np.float32), w.astype(np.uint8)]
        px = f.Parameter("x", shapes[0])
        pw = f.Parameter("w", shapes[1])
        pb = None
        if bias is not None:
            shapes.append(ca.Shape(ca.Float32, self.N))
            datas.append(bias.astype(np.float32))
            pb = f.Parameter("b", shapes[-1])
        y = f.FusedQuantizedDense(px, pw, pb, ca.Quantization(ca.QuantGGML, None, None, 1, 1, self.t), act)
        f.Return([y])
        self.exe = bld.Compile()
        self.inputs = [backend.BufferFromFlatData(0, d.ravel(), sh) for d, sh in zip(datas, shapes)]
        self.has_bias = bias is not None

    def plan(self):
        a = _lib.mx_qdense_args()
        a.x, a.w = self.inputs[0].DevicePtr(), self.inputs[1].DevicePtr()
        a.out = self.inputs[0].DevicePtr()
        if self.has_bias:
            a.bias, a.bias_dtype = self.inputs[2].DevicePtr(), O.DT_FLOAT32
        a.M, a.K, a.N = self.M, self.K, self.N
        a.x_dtype, a.scheme, a.ggml_type, a.activation = O.DT_FLOAT32, int(ca.QuantGGML), self.t, self.act
        return self.backend.QDensePlan(a)

    def run(self):
        out = self.exe.Execute(self.inputs)[0]
        y = out.ToFlatData()
        out.Finalize()
        return y.reshape(self.M, self.N)


def problem(t, M, K, N, bias=True):
    w = O.ggml_random_rows(int(t), N, K, RNG)
    x = RNG.standard_normal((M, K)).astype(np.float32)
    b = RNG.standard_normal(N).astype(np.float32) if bias else None
    return x, w, b


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("act", [ca.ActivationNone, ca.ActivationGelu, ca.ActivationSilu])
def test_exact_kernel_bit_identical(backend, t, act):
    x, w, b = problem(t, 6, 512, 72)
    r = GgmlRun(backend, t, x, w, b, act)
    assert r.plan() == "ggml_dense_exact"
    got = r.run()
    want = O.ggml_dense(x, w, int(t), b, int(act))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def accumulation_check(got, x, w, t, b, rel=1e-5):
    exact, ab = O.ggml_dense_f64(x, w, int(t), b)
    err = np.abs(got.astype(np.float64) - exact)
    bound = rel * ab + 1e-30
    assert (err <= bound).all(), f"worst {np.max(err / bound)} x the bound"


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_accumulation_bound(backend, t, M):
    x, w, b = problem(t, M, 1024, 301)
    r = GgmlRun(backend, t, x, w, b)
    assert r.plan() == "ggml_gemv"
    got = r.run()
    accumulation_check(got, x, w, t, b)
    assert np.array_equal(got.view(np.uint32), r.run().view(np.uint32))


@pytest.mark.parametrize("t,K", [(ca.GGMLQ6_K, 256), (ca.GGMLQ8_0, 32), (ca.GGMLQ4_0, 96), (ca.GGMLQ4_K, 768)])
def test_gemv_rows_not_16_byte_aligned(backend, t, K):
    x, w, b = problem(t, 2, K, 37)
    r = GgmlRun(backend, t, x, w, b)
    assert r.plan() == "ggml_gemv"
    accumulation_check(r.run(), x, w, t, b)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("M,N", [(5, 3400), (8, 2100), (15, 1200)])
def test_gemv_row_groups_accumulation_bound(backend, t, M, N):
    # Past 2^24 multiply-adds and up to 20 rows: the GEMV once per group of four rows.
    assert M * 1024 * N > 1 << 24
    x, w, b = problem(t, M, 1024, N)
    r = GgmlRun(backend, t, x, w, b)
    assert r.plan() == "ggml_gemv"
    got = r.run()
    accumulation_check(got, x, w, t, b)
    assert np.array_equal(got.view(np.uint32), r.run().view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("M", [21, 65, 200])
def test_dequant_mfma_accumulation_bound(backend, t, M):
    N = 264 if M > 64 else 1300
    assert M * 1024 * N > 1 << 24
    x, w, b = problem(t, M, 1024, N)
    r = GgmlRun(backend, t, x, w, b)
    assert r.plan() == "ggml_dequant_f32_mfma"
    got = r.run()
    accumulation_check(got, x, w, t, b)
    assert np.array_equal(got.view(np.uint32), r.run().view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
def test_dequant_mfma_values_exact(backend, t):
    # x = identity: every sum has one nonzero term, so the output is the dequantised matrix
    # transposed, each value as the reference forms it (compared with ==, so +0 equals -0).
    K, N = 512, 128
    w = O.ggml_random_rows(int(t), N, K, RNG)
    x = np.eye(K, dtype=np.float32)
    r = GgmlRun(backend, t, x, w)
    assert r.plan() == "ggml_dequant_f32_mfma"
    deq = O.ggml_embedding(w, int(t), np.arange(N))
    assert (r.run() == deq.T).all()


@pytest.mark.parametrize("t", [ca.GGMLQ4_0, ca.GGMLQ6_K])
@pytest.mark.parametrize("act", [ca.ActivationGelu, ca.ActivationSilu])
def test_dequant_mfma_activation(backend, t, act):
    x, w, b = problem(t, 96, 512, 400)
    r = GgmlRun(backend, t, x, w, b, act)
    assert r.plan() == "ggml_dequant_f32_mfma"
    # The accumulation bar carried through the activation: GELU's and SiLU's slopes stay below
    # 1.2, and the activation's own f32 rounding adds a few ulps of the result.
    exact, ab = O.ggml_dense_f64(x, w, int(t), b)
    if act == ca.ActivationGelu:
        want = 0.5 * exact * (1.0 + erf(exact / np.sqrt(2.0)))
    else:
        want = exact * expit(exact)
    err = np.abs(r.run().astype(np.float64) - want)
    bound = 1.2 * 1e-5 * ab + 4 * np.finfo(np.float32).eps * np.abs(want) + 1e-30
    assert (err <= bound).all(), f"worst {np.max(err / bound)} x the bound"


@pytest.mark.parametrize("t", [ca.GGMLQ4_0, ca.GGMLQ4_K])
@pytest.mark.parametrize("M", [8, 96])
def test_exact_option_keeps_reference_order(t, M):
    # The exact backend option selects the reference-order kernel at sizes that otherwise take
    # the GEMV row groups or the dequantised matrix-core path.
    x, w, b = problem(t, M, 1024, 2100 if M < 16 else 300)
    assert M * 1024 * (2100 if M < 16 else 300) > 1 << 24
    ex = ca.New("exact")
    try:
        r = GgmlRun(ex, t, x, w, b, ca.ActivationSilu)
        assert r.plan() == "ggml_dense_exact"
        got = r.run()
    finally:
        ex.Finalize()
    want = O.ggml_dense(x, w, int(t), b, int(ca.ActivationSilu))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", [ca.GGMLQ4_0, ca.GGMLQ4_K])
def test_gemv_activation(backend, t):
    x, w, b = problem(t, 1, 512, 64)
    got = GgmlRun(backend, t, x, w, b, ca.ActivationGelu).run()
    want = O.ggml_dense(x, w, int(t), b, int(ca.ActivationGelu))
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("t", [ca.GGMLQ4_0, ca.GGMLQ8_0, ca.GGMLQ4_K])
def test_gemv_decode_shape(backend, t):
    x, w, b = problem(t, 1, 4096, 11008, bias=False)
    r = GgmlRun(backend, t, x, w, b)
    assert r.plan() == "ggml_gemv"
    accumulation_check(r.run(), x, w, t, b)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("M,K,N", [(1, 14336, 1200), (2, 14336, 600), (3, 14336, 420), (7, 8192, 300)])
def test_gemv_long_rows_in_k_segments(backend, t, M, K, N):
    """Rows longer than the GEMV holds at once (row bytes past 8 per lane, or rows of x past the
    LDS) run as K segments whose sums are added to the output in order; bias once, at the end."""
    assert M * K * N > 1 << 24
    x, w, b = problem(t, M, K, N)
    r = GgmlRun(backend, t, x, w, b)
    assert r.plan() == "ggml_gemv"
    got = r.run()
    accumulation_check(got, x, w, t, b)
    assert np.array_equal(got.view(np.uint32), r.run().view(np.uint32))


@pytest.mark.parametrize("t", [ca.GGMLQ4_0, ca.GGMLQ6_K])
def test_gemv_k_segments_activation_after_the_last(backend, t):
    # The activation of the whole sum: applied once, by the last segment's launch.
    x, w, b = problem(t, 2, 14336, 640)
    r = GgmlRun(backend, t, x, w, b, ca.ActivationSilu)
    assert r.plan() == "ggml_gemv"
    exact, ab = O.ggml_dense_f64(x, w, int(t), b)
    want = exact * expit(exact)
    err = np.abs(r.run().astype(np.float64) - want)
    bound = 1.2 * 1e-5 * ab + 4 * np.finfo(np.float32).eps * np.abs(want) + 1e-30
    assert (err <= bound).all(), f"worst {np.max(err / bound)} x the bound"


def test_gemv_k_segments_noalloc(backend):
    # The allocation-free entry point takes the same segments (the output is their accumulator).
    t = ca.GGMLQ6_K
    x, w, b = problem(t, 1, 14336, 1200)
    r = GgmlRun(backend, t, x, w, b)
    out = backend.BufferFromFlatData(0, np.full(1200, np.nan, np.float32), ca.Shape(ca.Float32, 1, 1200))
    a = _lib.mx_qdense_args()
    a.x, a.w, a.out = r.inputs[0].DevicePtr(), r.inputs[1].DevicePtr(), out.DevicePtr()
    a.bias, a.bias_dtype = r.inputs[2].DevicePtr(), O.DT_FLOAT32
    a.M, a.K, a.N = 1, 14336, 1200
    a.x_dtype, a.scheme, a.ggml_type, a.activation = O.DT_FLOAT32, int(ca.QuantGGML), int(t), 0
    assert backend.QDensePlan(a) == "ggml_gemv"
    backend.QDenseNoAlloc(a)
    got = out.ToFlatData().reshape(1, 1200)
    assert np.array_equal(got.view(np.uint32), r.run().view(np.uint32))


def embed_graph(backend, t, data, idx, idx_dtype):
    bld = backend.Builder("emb")
    f = bld.Main()
    ds = ca.Shape(ca.Uint8, *data.shape)
    is_ = ca.Shape(idx_dtype, *idx.shape)
    pd = f.Parameter("d", ds)
    pi = f.Parameter("i", is_)
    f.Return([f.QuantizedEmbeddingLookup(pd, pi, ca.Quantization(ca.QuantGGML, None, None, 1, 1, int(t)))])
    exe = bld.Compile()
    np_dt = {ca.Int32: np.int32, ca.Int64: np.int64, ca.Uint16: np.uint16, ca.Int8: np.int8}[idx_dtype]
    ins = [backend.BufferFromFlatData(0, data.ravel(), ds),
           backend.BufferFromFlatData(0, idx.astype(np_dt).ravel(), is_)]
    return exe, ins


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("idx_dtype", [ca.Int32, ca.Int64, ca.Uint16, ca.Int8])
def test_embedding_bit_identical(backend, t, idx_dtype):
    V, K = 97, 512
    data = O.ggml_random_rows(int(t), V, K, RNG)
    idx = RNG.integers(0, V, (2, 3, 1))
    idx[0, 0, 0] = V - 1
    exe, ins = embed_graph(backend, t, data, idx, idx_dtype)
    out = exe.Execute(ins)[0]
    got = out.ToFlatData().reshape(2, 3, K)
    out.Finalize()
    want = O.ggml_embedding(data, int(t), idx).reshape(2, 3, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_embedding_out_of_range_fails_the_call(backend):
    t, V, K = ca.GGMLQ8_0, 10, 64
    data = O.ggml_random_rows(int(t), V, K, RNG)
    for bad in (10, -1):
        idx = np.array([[1], [bad], [2]])
        exe, ins = embed_graph(backend, t, data, idx, ca.Int64)
        with pytest.raises(ca.ComputeError, match=f"index {bad} out of range"):
            exe.Execute(ins)


def test_embedding_direct_entry_point(backend):
    t, V, K = ca.GGMLQ4_K, 33, 1024
    data = O.ggml_random_rows(int(t), V, K, RNG)
    idx = RNG.integers(0, V, 17).astype(np.int32)
    bd = backend.BufferFromFlatData(0, data.ravel(), ca.Shape(ca.Uint8, *data.shape))
    bi = backend.BufferFromFlatData(0, idx, ca.Shape(ca.Int32, 17))
    bo = backend.BufferFromFlatData(0, np.zeros(17 * K, np.float32), ca.Shape(ca.Float32, 17, K))
    a = _lib.mx_qembed_args()
    a.data, a.indices, a.out = bd.DevicePtr(), bi.DevicePtr(), bo.DevicePtr()
    a.vocab, a.bytes_per_row, a.n = V, data.shape[1], 17
    a.index_dtype, a.ggml_type = 4, int(t)  # Int32
    backend.QEmbed(a)
    got = bo.ToFlatData().reshape(17, K)
    assert np.array_equal(got.view(np.uint32), O.ggml_embedding(data, int(t), idx).view(np.uint32))
