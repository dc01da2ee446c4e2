"""mx_qdense_noalloc (FusedQuantizedDense without device allocation) through the C ABI, against
mx_qdense on the same device buffers.

The allocation-free entry point runs mx_qdense's kernels with their split-K scratch taken from a
static per-GPU array, so on the skinny, GEMV, GEMM and fused reference-layout paths its result
must be bit-identical to mx_qdense's, and within the oracle bars of those paths (bf16 outputs rel
1e-2 / abs 1e-3 of the reference's f32 result, f32 outputs the f32 accumulation bound).  GGML rows
past 20 rows, which mx_qdense dequantises into an f32 copy, take the GEMV once per group of four
rows on the allocation-free call, within the same bound, and a GEMM tail that mx_qdense splits
into two K halves is computed whole (another summation order for those tiles only).  Each case makes two
calls in a row, the second on a smaller problem, as a caller reusing the shared array would.
"""
import ctypes as C

import numpy as np
import pytest

import compute_amd as ca
from compute_amd import _lib
from oracle import oracle as O
from tests.qd_helpers import DT, assert_bf16_close, assert_f32_accumulation_close

pytestmark = pytest.mark.gpu


class Direct:
    """A FusedQuantizedDense problem on device buffers, with one output buffer per entry point."""

    def __init__(self, backend, p: O.QDenseProblem):
        self.backend, self.p = backend, p
        up = lambda a, sh: backend.BufferFromFlatData(0, np.ascontiguousarray(a).ravel(), sh)
        self.x = up(p.x, ca.Shape(DT[p.x_dtype], p.M, p.K))
        self.w = up(p.w, ca.Shape(DT[p.w_dtype], p.K, p.N))
        self.s = up(p.scale, ca.Shape(DT[p.scale_dtype], *p.scale_shape))
        self.zp = up(p.zp, ca.Shape(DT[p.zp_dtype], *p.scale_shape)) if p.zp is not None else None
        self.bias = up(p.bias, ca.Shape(DT[p.bias_dtype], p.N)) if p.bias is not None else None
        out_shape = ca.Shape(DT[p.x_dtype], p.M, p.N)
        zeros = np.zeros(p.M * p.N, dtype=out_shape.dtype.numpy_storage())
        self.outs = [up(zeros, out_shape) for _ in range(2)]

    def args(self, out) -> _lib.mx_qdense_args:
        p = self.p
        a = _lib.mx_qdense_args()
        a.x, a.w, a.scale = self.x.DevicePtr(), self.w.DevicePtr(), self.s.DevicePtr()
        if self.zp is not None:
            a.zero_point, a.zero_point_dtype = self.zp.DevicePtr(), p.zp_dtype
        if self.bias is not None:
            a.bias, a.bias_dtype = self.bias.DevicePtr(), p.bias_dtype
        a.out = out.DevicePtr()
        a.M, a.K, a.N = p.M, p.K, p.N
        a.x_dtype, a.w_dtype, a.scale_dtype = p.x_dtype, p.w_dtype, p.scale_dtype
        a.scheme, a.block_axis, a.block_size, a.activation = p.scheme, p.block_axis, p.block_size, p.act
        return a

    def call(self, entry: str, out) -> int:
        lib = self.backend._lib
        return getattr(lib, entry)(self.backend._h, C.byref(self.args(out)))

    def run_both(self):
        """(mx_qdense result, mx_qdense_noalloc result), each read back after the stream drains."""
        for entry, out in zip(("mx_qdense", "mx_qdense_noalloc"), self.outs):
            rc = self.call(entry, out)
            assert rc == _lib.MX_OK, f"{entry}: {self.backend._lib.mx_last_error().decode()}"
        shape = (self.p.M, self.p.N)
        return tuple(o.ToFlatData().reshape(shape) for o in self.outs)


def problem(M, K, N, seed, **kw):
    kw.setdefault("bias", True)
    kw.setdefault("scale_range", (0.002, 0.02))
    return O.make_problem(M, K, N, seed=seed, **kw)


# (first call, second smaller call) per kernel family; the plan of mx_qdense is asserted so each
# pair exercises the path it names.
SKINNY = [problem(4, 4096, 4096, 1, w_dtype=O.DT_INT4, block_axis=0, block_size=128),
          problem(2, 2048, 1024, 2, w_dtype=O.DT_INT4, block_axis=0, block_size=128)]
SKINNY_I8 = [problem(16, 4096, 14336, 3, w_dtype=O.DT_INT8, block_axis=0, block_size=64, act=O.ACT_SILU),
             problem(1, 4096, 11008, 4, w_dtype=O.DT_INT8, block_axis=0, block_size=4096, per_channel_1d=True,
                     scale_dtype=O.DT_FLOAT32)]
GEMV = [problem(3, 4096, 2048, 5, w_dtype=O.DT_INT8, x_dtype=O.DT_FLOAT32, block_axis=0, block_size=64),
        problem(2, 1024, 1024, 6, w_dtype=O.DT_INT8, x_dtype=O.DT_FLOAT32, block_axis=0, block_size=64)]
GEMM = [problem(64, 1024, 2048, 7, w_dtype=O.DT_INT8, block_axis=0, block_size=1024, per_channel_1d=True,
                scale_dtype=O.DT_FLOAT32),
        problem(49, 512, 1024, 8, w_dtype=O.DT_INT8, block_axis=0, block_size=512, per_channel_1d=True,
                scale_dtype=O.DT_FLOAT32)]
SKINNY_ROWS = [problem(40, 4096, 2048, 12, w_dtype=O.DT_INT4, block_axis=0, block_size=128),
               problem(20, 2048, 1024, 13, w_dtype=O.DT_INT4, block_axis=0, block_size=128)]


@pytest.mark.parametrize("pair,plan", [(SKINNY, "qdense_skinny_mfma_i4"), (SKINNY_I8, "qdense_skinny_mfma_i8"),
                                       (SKINNY_ROWS, "qdense_skinny_rows16_i4"), (GEMV, "qdense_gemv_i8"),
                                       (GEMM, "qdense_gemm_mfma_i8")],
                         ids=["skinny_i4", "skinny_i8", "skinny_rows", "gemv", "gemm"])
def test_noalloc_matches_qdense(backend, pair, plan):
    for p in pair:
        d = Direct(backend, p)
        assert backend.QDensePlan(d.args(d.outs[0])) == plan
        ref, got = d.run_both()
        assert np.array_equal(got, ref), f"{p.M}x{p.K}x{p.N}: mx_qdense_noalloc differs from mx_qdense"
        want = O.qdense_f32(p, threads=8)
        if p.x_dtype == O.DT_BFLOAT16:
            assert_bf16_close(got, want, what=f"{p.M}x{p.K}x{p.N}")
        else:
            assert_f32_accumulation_close(got, p, what=f"{p.M}x{p.K}x{p.N}")


def test_noalloc_gemm_split_tail_whole(backend):
    """272 GEMM tiles (x [512, 1024], N = 17408): mx_qdense splits the 16 tiles past the first 256
    into two K halves that exchange partial tiles through its scratch; the allocation-free call
    computes them whole.  Outside those tiles (rows 256..511, columns 15360..17407) the results are
    bit-identical, inside they are another summation order, and both meet the oracle's bars."""
    pair = [problem(512, 1024, 17408, 14, w_dtype=O.DT_INT8, block_axis=0, block_size=1024, per_channel_1d=True,
                    scale_dtype=O.DT_FLOAT32, act=O.ACT_GELU),
            GEMM[1]]
    for i, p in enumerate(pair):
        d = Direct(backend, p)
        assert backend.QDensePlan(d.args(d.outs[0])) == "qdense_gemm_mfma_i8"
        ref, got = d.run_both()
        rows = (np.sort(np.concatenate([np.arange(0, 8), np.arange(256, 264), np.arange(p.M - 8, p.M)]))
                if i == 0 else np.arange(p.M))
        want = O.qdense_f32(p, rows=rows, threads=8)
        assert_bf16_close(got[rows], want, what="noalloc")
        assert_bf16_close(ref[rows], want, what="mx_qdense")
        if i == 0:
            tail = np.zeros(got.shape, bool)
            tail[256:512, 15360:17408] = True
            assert np.array_equal(got[~tail], ref[~tail]), "tiles outside the split tail differ"
        else:
            assert np.array_equal(got, ref)


def test_noalloc_reference_layout_fused(backend):
    """Reference layout at prefill size: both entry points run the fused kernel, which dequantises
    each K block into LDS and needs no workspace, so the results are bit-identical."""
    pair = [problem(96, 512, 1024, 9, w_dtype=O.DT_INT4, x_dtype=O.DT_FLOAT32, block_axis=1, block_size=64),
            problem(64, 512, 768, 10, w_dtype=O.DT_UINT8, x_dtype=O.DT_FLOAT32, block_axis=1, block_size=32,
                    zp=True)]
    for p in pair:
        d = Direct(backend, p)
        assert backend.QDensePlan(d.args(d.outs[0])) == "qdense_refgemm_f32_mfma"
        ref, got = d.run_both()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "mx_qdense_noalloc differs from mx_qdense"
        assert_f32_accumulation_close(got, p, what="fused reference layout")


def test_noalloc_rejects_oversized_scratch(backend):
    """A GEMV problem whose split-K tiles exceed the static array is refused before any launch;
    the backend then keeps working on both entry points."""
    M, K, N = 4, 32768, 8192  # 128 slices of [4, 8192] f32 partial tiles: 16 MiB + counters
    p = O.QDenseProblem(M=M, K=K, N=N, x=np.zeros((M, K), np.float32), w=np.zeros(K * N // 2, np.uint8),
                        scale=np.zeros((K // 128, N), np.float32), x_dtype=O.DT_FLOAT32, w_dtype=O.DT_INT4,
                        scale_dtype=O.DT_FLOAT32, scale_shape=(K // 128, N), block_axis=0, block_size=128)
    d = Direct(backend, p)
    assert backend.QDensePlan(d.args(d.outs[0])).startswith("qdense_gemv")
    rc = d.call("mx_qdense_noalloc", d.outs[1])
    assert rc == _lib.MX_ERR_INVALID
    msg = backend._lib.mx_last_error().decode()
    assert "exceeds the static maximum" in msg and str(_lib.MX_QDENSE_NOALLOC_SCRATCH_BYTES) in msg
    small = Direct(backend, SKINNY[1])
    ref, got = small.run_both()
    assert np.array_equal(got, ref)


def test_noalloc_second_backend_shares_array(backend):
    """A second backend on the same GPU gets the same static array (set up once per device) and
    computes the same result."""
    b2 = ca.New("mi355x")
    try:
        assert backend.DebugNoAllocScratch() != 0
        assert b2.DebugNoAllocScratch() == backend.DebugNoAllocScratch()
        d = Direct(b2, SKINNY[0])
        ref, got = d.run_both()
        assert np.array_equal(got, ref)
        assert_bf16_close(got, O.qdense_f32(SKINNY[0], threads=8), what="second backend")
    finally:
        b2.Finalize()


def test_noalloc_calls_from_two_streams_are_ordered(backend):
    """Calls queued back to back on two backends' streams (no host synchronisation between them),
    alternating problems whose split-K slice counts and column blocks differ, each give
    mx_qdense's bits: every call's stream waits for the previous call on the GPU, so no two calls
    share the static array at once and the arrival counters stay consistent."""
    b2 = ca.New("mi355x")
    try:
        cases = [Direct(backend, SKINNY[0]), Direct(b2, SKINNY_I8[0]), Direct(b2, GEMV[0]),
                 Direct(backend, SKINNY[1])]
        refs = []
        for d in cases:
            assert d.call("mx_qdense", d.outs[0]) == _lib.MX_OK
            refs.append(d.outs[0].ToFlatData().reshape(d.p.M, d.p.N))
        outs = []
        for rnd in range(3):
            for d in cases:
                sh = ca.Shape(DT[d.p.x_dtype], d.p.M, d.p.N)
                o = d.backend.BufferFromFlatData(0, np.zeros(d.p.M * d.p.N, sh.dtype.numpy_storage()), sh)
                d.backend.Synchronize()  # the upload is done before any call is queued
                outs.append((d, o))
        for d, o in outs:
            rc = d.call("mx_qdense_noalloc", o)
            assert rc == _lib.MX_OK, d.backend._lib.mx_last_error().decode()
        for i, (d, o) in enumerate(outs):
            got = o.ToFlatData().reshape(d.p.M, d.p.N)
            assert np.array_equal(got, refs[i % len(cases)]), f"call {i} ({d.p.M}x{d.p.K}x{d.p.N}) differs"
    finally:
        b2.Finalize()


def test_noalloc_ggml_prefill_takes_gemv_groups(backend):
    """GGML rows past 20 rows: mx_qdense dequantises them into an f32 copy for the matrix cores;
    the allocation-free call runs the GEMV once per group of four rows instead, within the same
    f32 accumulation bound.  The second, smaller call (8 rows) takes the GEMV groups on both."""
    rng = np.random.default_rng(11)
    t = int(ca.GGMLQ4_K)
    for M, K, N, plan in ((32, 1024, 1536, "ggml_dequant_f32_mfma"), (8, 1024, 2400, "ggml_gemv")):
        w = O.ggml_random_rows(t, N, K, rng)
        x = rng.standard_normal((M, K)).astype(np.float32)
        bias = rng.standard_normal(N).astype(np.float32)
        up = lambda a, sh: backend.BufferFromFlatData(0, np.ascontiguousarray(a).ravel(), sh)
        bx, bw, bb = up(x, ca.Shape(ca.Float32, M, K)), up(w, ca.Shape(ca.Uint8, N, w.shape[1])), up(bias, ca.Shape(ca.Float32, N))
        outs = [up(np.zeros(M * N, np.float32), ca.Shape(ca.Float32, M, N)) for _ in range(2)]

        def args(out):
            a = _lib.mx_qdense_args()
            a.x, a.w, a.out = bx.DevicePtr(), bw.DevicePtr(), out.DevicePtr()
            a.bias, a.bias_dtype = bb.DevicePtr(), O.DT_FLOAT32
            a.M, a.K, a.N = M, K, N
            a.x_dtype, a.scheme, a.ggml_type = O.DT_FLOAT32, int(ca.QuantGGML), t
            return a

        assert backend.QDensePlan(args(outs[0])) == plan
        for entry, out in zip(("mx_qdense", "mx_qdense_noalloc"), outs):
            rc = getattr(backend._lib, entry)(backend._h, C.byref(args(out)))
            assert rc == _lib.MX_OK, f"{entry}: {backend._lib.mx_last_error().decode()}"
        ref, got = (o.ToFlatData().reshape(M, N) for o in outs)
        exact, ab = O.ggml_dense_f64(x, w, t, bias)
        for y in (ref, got):
            assert (np.abs(y.astype(np.float64) - exact) <= 1e-5 * ab + 1e-30).all()
        if plan == "ggml_gemv":
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
