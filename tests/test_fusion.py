"""Compile-time fusion of the graph compiler (CPU: what gets fused; GPU: fused == unfused bits).

Fusion must not change results: each fused kernel rounds every intermediate exactly as the
separate ops do, so a graph compiled with fusion and the same graph compiled op by op
("nofusion" backend option) return identical bits.
"""
import numpy as np
import pytest

import compute_amd as ca
from compute_amd import backend as B
from compute_amd import workloads
from compute_amd.dtypes import BFloat16, Float32, Int4, Int8, Shape, Uint4, Uint8, bf16_from_f32, pack_int4
from tests.qd_helpers import assert_bf16_close
from oracle import oracle as O

UNFUSED_MLP = ['ConvertDType', 'Binary', 'Reduce', 'Binary', 'Binary', 'Unary', 'Gather', 'Binary', 'ConvertDType',
               'FusedQuantizedDense', 'FusedQuantizedDense', 'Binary', 'FusedQuantizedDense', 'Binary']


@pytest.fixture(scope="module")
def host():
    b = ca.New("host_only")
    yield b
    b.Finalize()


def test_mlp_fused_ops(host):
    wl = workloads.make("C5")
    assert wl.compile(host).Describe() == ['RmsNorm', 'FusedQuantizedDense+Pair', 'FusedQuantizedDense+Add']


def test_nofusion_option():
    b = ca.New("host_only,nofusion")
    try:
        assert workloads.make("C5").compile(b).Describe() == UNFUSED_MLP
    finally:
        b.Finalize()


def _qd_graph(backend, extra_use: bool, op: str = "add", res_first: bool = False, x_dtype=BFloat16, M=2):
    bld = backend.Builder("qd_res")
    f = bld.Main()
    x = f.Parameter("x", Shape(x_dtype, M, 64))
    w = f.Parameter("w", Shape(Int8, 64, 32))
    s = f.Parameter("s", Shape(Float32, 32))
    r = f.Parameter("r", Shape(x_dtype, M, 32))
    y = f.FusedQuantizedDense(x, w, None, B.Quantization(B.QuantLinear, s, None, 0, 64), B.ActivationRelu)
    fn = f.Add if op == "add" else f.Mul
    z = fn(r, y) if res_first else fn(y, r)
    f.Return([z, y] if extra_use else [z])
    return bld.Compile()


def test_dense_epilogue_fusion_rules(host):
    assert _qd_graph(host, False).Describe() == ["FusedQuantizedDense+Add"]
    assert _qd_graph(host, False, "mul", res_first=True).Describe() == ["FusedQuantizedDense+Mul"]
    # The dense result is also an output: it must exist on its own, so nothing is folded.
    assert _qd_graph(host, True).Describe() == ["FusedQuantizedDense", "Binary"]


def test_rmsnorm_not_fused_when_intermediate_is_used(host):
    bld = host.Builder("rms_partial")
    f = bld.Main()
    M, D = 4, 256
    x = f.Parameter("x", Shape(BFloat16, M, D))
    xf = f.ConvertDType(x, Float32)
    ss = f.ReduceSum(f.Mul(xf, xf), 1)
    inv = f.Rsqrt(f.Add(f.Mul(ss, f.Constant(np.full(M, 1.0 / D, np.float32))),
                        f.Constant(np.full(M, 1e-6, np.float32))))
    h = f.ConvertDType(f.Mul(xf, f.BroadcastInDim(inv, Shape(Float32, M, D), [0])), BFloat16)
    f.Return([h, ss])  # the sum of squares is an output too
    assert "RmsNorm" not in bld.Compile().Describe()


@pytest.mark.gpu
def test_mlp_fused_equals_unfused_bits(backend):
    wl = workloads.make("C5")
    nf = ca.New("nofusion")
    try:
        y_fused = wl.compile(backend).Execute(wl.upload(backend))[0].ToFlatData()
        y_plain = wl.compile(nf).Execute(wl.upload(nf))[0].ToFlatData()
    finally:
        nf.Finalize()
    assert np.array_equal(y_fused, y_plain)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 3, 8])
def test_rmsnorm_small_rows_equal_unfused(backend, M):
    rng = np.random.default_rng(M)
    D = 512
    xb = bf16_from_f32(rng.standard_normal((M, D)).astype(np.float32) * 3)

    def build(b):
        bld = b.Builder("rms")
        f = bld.Main()
        x = f.Parameter("x", Shape(BFloat16, M, D))
        xf = f.ConvertDType(x, Float32)
        ms = f.Mul(f.Constant(np.full(M, 1.0 / D, np.float32)), f.ReduceSum(f.Mul(xf, xf), 1))
        inv = f.Rsqrt(f.Add(f.Constant(np.full(M, 1e-5, np.float32)), ms))
        h = f.ConvertDType(f.Mul(f.BroadcastInDim(inv, Shape(Float32, M, D), [0]), xf), BFloat16)
        f.Return([h])
        return bld.Compile()

    nf = ca.New("nofusion")
    try:
        e1 = build(backend)
        assert e1.Describe() == ["RmsNorm"]
        h1 = e1.Execute([backend.BufferFromFlatData(0, xb, Shape(BFloat16, M, D))])[0].ToFlatData()
        h2 = build(nf).Execute([nf.BufferFromFlatData(0, xb, Shape(BFloat16, M, D))])[0].ToFlatData()
    finally:
        nf.Finalize()
    assert np.array_equal(h1, h2)


@pytest.mark.gpu
@pytest.mark.parametrize("x_dtype,op,res_first,M", [(BFloat16, "add", False, 2), (BFloat16, "mul", True, 2),
                                                    (Float32, "add", True, 2), (Float32, "mul", False, 2),
                                                    (BFloat16, "add", True, 40), (BFloat16, "mul", False, 24)])
def test_dense_epilogue_equals_unfused(backend, x_dtype, op, res_first, M):
    """bf16 x takes the skinny kernel (epilogue in the kernel; past 16 rows once per group of 16
    rows, the operand's rows offset with the output's); f32 x the exact kernel (dense result to a
    temporary, then the elementwise kernel)."""
    rng = np.random.default_rng(7)
    xs = rng.standard_normal((M, 64)).astype(np.float32)
    rs = rng.standard_normal((M, 32)).astype(np.float32)
    x = bf16_from_f32(xs) if x_dtype == BFloat16 else xs
    r = bf16_from_f32(rs) if x_dtype == BFloat16 else rs
    w = rng.integers(-127, 128, (64, 32)).astype(np.int8)
    s = rng.uniform(0.01, 0.05, 32).astype(np.float32)
    shapes = [Shape(x_dtype, M, 64), Shape(Int8, 64, 32), Shape(Float32, 32), Shape(x_dtype, M, 32)]
    nf = ca.New("nofusion")
    try:
        outs = []
        for b in (backend, nf):
            e = _qd_graph(b, False, op, res_first, x_dtype, M)
            bufs = [b.BufferFromFlatData(0, d, sh) for d, sh in zip([x, w, s, r], shapes)]
            outs.append(e.Execute(bufs)[0].ToFlatData())
    finally:
        nf.Finalize()
    assert np.array_equal(outs[0], outs[1])


# ---------------------------------------------------------------------------------------------
# Pair fusion: Mul(dense(x, w_gate), dense(x, w_up)) over one x runs as one launch.
# ---------------------------------------------------------------------------------------------
def _pair_data(M, K, N, wdt, G, bias_g, bias_u, x_dtype, seed):
    rng = np.random.default_rng(seed)
    xs = rng.standard_normal((M, K)).astype(np.float32)
    x = bf16_from_f32(xs) if x_dtype == BFloat16 else xs
    packed = wdt in (Int4, Uint4)
    lo, hi = {Int4: (-8, 8), Uint4: (0, 16), Int8: (-127, 128), Uint8: (0, 256)}[wdt]
    ng = 1 if G >= K else K // G
    sdims = (N,) if G >= K else (ng, N)

    def weights():
        v = rng.integers(lo, hi, (K, N))
        return pack_int4(v) if packed else v.astype(np.int8 if wdt == Int8 else np.uint8)

    def scales():
        return bf16_from_f32(rng.uniform(0.002, 0.02, sdims).astype(np.float32))

    def bias():
        return bf16_from_f32((rng.standard_normal(N) * 0.05).astype(np.float32))

    data = {"x": x, "wg": weights(), "sg": scales(), "wu": weights(), "su": scales()}
    if bias_g:
        data["bg"] = bias()
    if bias_u:
        data["bu"] = bias()
    shapes = {"x": Shape(x_dtype, M, K), "wg": Shape(wdt, K, N), "sg": Shape(BFloat16, *sdims),
              "wu": Shape(wdt, K, N), "su": Shape(BFloat16, *sdims), "bg": Shape(BFloat16, N),
              "bu": Shape(BFloat16, N)}
    return data, shapes


def _pair_graph(backend, data, shapes, G, act_g, act_u, gate_first=True, gate_output=False, other_x=False):
    bld = backend.Builder("pair")
    f = bld.Main()
    p = {k: f.Parameter(k, shapes[k]) for k in data}
    xg = p["x"]
    if other_x:
        xg = f.ConvertDType(f.ConvertDType(p["x"], Float32), shapes["x"].dtype)

    def qd(x, w, s, b, act):
        return f.FusedQuantizedDense(x, p[w], p.get(b), B.Quantization(B.QuantLinear, p[s], None, 0, G),
                                     B.ActivationType(act))

    g = qd(xg, "wg", "sg", "bg", act_g)
    u = qd(p["x"], "wu", "su", "bu", act_u)
    y = f.Mul(g, u) if gate_first else f.Mul(u, g)
    f.Return([y, g] if gate_output else [y])
    return bld.Compile()


def test_pair_fusion_rules(host):
    data, shapes = _pair_data(2, 256, 64, Int8, 64, False, True, BFloat16, 0)
    silu, none = int(B.ActivationSilu), int(B.ActivationNone)
    assert _pair_graph(host, data, shapes, 64, silu, none).Describe() == ["FusedQuantizedDense+Pair"]
    assert _pair_graph(host, data, shapes, 64, silu, none, gate_first=False).Describe() == [
        "FusedQuantizedDense+Pair"]
    # The gate is also an output: it must exist on its own, so only the Mul is folded.
    assert _pair_graph(host, data, shapes, 64, silu, none, gate_output=True).Describe() == [
        "FusedQuantizedDense", "FusedQuantizedDense+Mul"]
    # Different x operands: no pair.
    assert "FusedQuantizedDense+Pair" not in _pair_graph(host, data, shapes, 64, silu, none, other_x=True).Describe()


PAIR_CASES = [
    # M, K, N, wdt, G, bias_g, bias_u, x_dtype
    (1, 4096, 512, Int4, 128, False, False, BFloat16),   # S = 4 slices per matrix
    (8, 4096, 768, Int4, 128, False, False, BFloat16),   # the C5 shape family (batch 8)
    (3, 1024, 256, Uint4, 1024, True, False, BFloat16),  # per-channel scales, S = 1
    (16, 2048, 384, Int8, 64, True, True, BFloat16),     # int8 g64, both biases
    (5, 512, 160, Uint8, 512, False, True, BFloat16),    # S = 1, ragged column block
    (4, 256, 64, Int8, 64, True, True, Float32),         # f32 x: exact kernels, pair fallback
    (40, 1024, 512, Int4, 128, True, False, BFloat16),   # 40 rows: one pair launch per 16 rows
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", PAIR_CASES, ids=lambda c: f"M{c[0]}K{c[1]}N{c[2]}_{c[3].name}_g{c[4]}")
def test_pair_equals_unfused(backend, case):
    M, K, N, wdt, G, bias_g, bias_u, x_dtype = case
    data, shapes = _pair_data(M, K, N, wdt, G, bias_g, bias_u, x_dtype, seed=M * 131 + K)
    nf = ca.New("nofusion")
    try:
        outs = []
        for b, gate_first in ((backend, True), (backend, False), (nf, True)):
            e = _pair_graph(b, data, shapes, G, int(B.ActivationSilu), int(B.ActivationNone), gate_first)
            if b is backend:
                assert e.Describe() == ["FusedQuantizedDense+Pair"]
            bufs = [b.BufferFromFlatData(0, data[k], shapes[k]) for k in data]
            outs.append(e.Execute(bufs)[0].ToFlatData())
            outs.append(e.Execute(bufs)[0].ToFlatData())  # a second launch reuses the counters
    finally:
        nf.Finalize()
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)


def _dot_graph(backend, M, K, N, dt, transposed=False, batch=1):
    bld = backend.Builder("dot_half")
    f = bld.Main()
    x = f.Parameter("x", Shape(dt, batch, M, K))
    w = f.Parameter("w", Shape(dt, batch, N, K) if transposed else Shape(dt, batch, K, N))
    f.Return([f.DotGeneral(x, [2], [0], w, [2] if transposed else [1], [0])])
    return bld.Compile()


def test_dot_convert_fusion_rules(host):
    """Half DotGeneral: the f32 sum's ConvertDType back to the input dtype folds into the
    contraction (dot.go:340-372); an explicit f32 output keeps no conversion at all."""
    assert _dot_graph(host, 4, 64, 32, BFloat16).Describe() == ["DotGeneral"]
    nf = ca.New("host_only,nofusion")
    try:
        assert _dot_graph(nf, 4, 64, 32, BFloat16).Describe() == ["DotGeneral", "ConvertDType"]
    finally:
        nf.Finalize()


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [BFloat16, ca.Float16])
@pytest.mark.parametrize("shape", [(256, 512, 512, False, 1), (300, 1024, 272, True, 2), (70, 130, 90, False, 3)])
def test_dot_half_output_equals_unfused(backend, dt, shape):
    """Matrix-core epilogue rounding (first two shapes) and the f32-temporary fallback (the last,
    K % 64 != 0) give the bits of the separate ConvertDType."""
    M, K, N, transposed, batch = shape
    rng = np.random.default_rng(M + K)
    xf = rng.standard_normal((batch, M, K)).astype(np.float32)
    wf = rng.standard_normal((batch, N, K) if transposed else (batch, K, N)).astype(np.float32)
    cast = bf16_from_f32 if dt == BFloat16 else (lambda a: a.astype(np.float16))
    x, w = cast(xf), cast(wf)
    nf = ca.New("nofusion")
    try:
        outs = []
        for b in (backend, nf):
            e = _dot_graph(b, M, K, N, dt, transposed, batch)
            bufs = [b.BufferFromFlatData(0, x.ravel(), Shape(dt, *x.shape)),
                    b.BufferFromFlatData(0, w.ravel(), Shape(dt, *w.shape))]
            outs.append(e.Execute(bufs)[0].ToFlatData())
    finally:
        nf.Finalize()
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
