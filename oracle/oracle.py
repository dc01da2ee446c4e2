"""TEST INFRASTRUCTURE ONLY — Python side of the CPU oracle.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker (or the timed CPU baseline), never as a product path.

It loads oracle/_build/liboracle.so (a plain-C restatement of the reference's arithmetic,
qdense_ref.c and ggml_ref.c) and provides numpy helpers: seeded generators for the BASELINE configurations, the
reference packing of 4-bit weights, bf16 rounding, and brute-force numpy restatements of the
DotGeneral output layout (shapeinference/dotgeneral.go:16-152) for small cases.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "qdense_ref.c"
SRC_GGML = HERE / "ggml_ref.c"
LIB = HERE / "_build" / "liboracle.so"

DT_INT8, DT_UINT8, DT_INT4, DT_UINT4 = 2, 6, 21, 22
DT_FLOAT32, DT_BFLOAT16 = 11, 13
ACT_NONE, ACT_GELU, ACT_RELU, ACT_SILU, ACT_HARDSWISH, ACT_TANH = range(6)
QUANT_LINEAR, QUANT_NF4 = 0, 1


def build() -> Path:
    """Compiles the C restatement (gcc, -ffp-contract=off, OpenMP for the timed baseline)."""
    LIB.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
           "-o", str(tmp), str(SRC), str(SRC_GGML), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    os.replace(tmp, LIB)
    return LIB


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        fp = C.POINTER(C.c_float)
        dp = C.POINTER(C.c_double)
        L.oracle_unpack_int4.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p]
        L.oracle_unpack_uint4.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p]
        L.oracle_f32_to_bf16.argtypes = [C.c_float]
        L.oracle_f32_to_bf16.restype = C.c_uint16
        L.oracle_f32_to_bf16_array.argtypes = [fp, C.c_size_t, C.c_void_p]
        L.oracle_act.argtypes = [C.c_float, C.c_int]
        L.oracle_act.restype = C.c_float
        L.oracle_act_array.argtypes = [fp, C.c_size_t, C.c_int]
        L.oracle_nf4.argtypes = [C.c_int]
        L.oracle_nf4.restype = C.c_float
        common = [fp, C.c_void_p, C.c_int, fp, fp, fp]
        L.oracle_qdense.argtypes = common + [fp] + [C.c_int64] * 3 + [C.c_int, C.c_int, C.c_int64, C.c_int,
                                                                       C.c_int64, C.c_int64, C.c_int]
        L.oracle_qdense_f64.argtypes = common + [dp] + [C.c_int64] * 3 + [C.c_int, C.c_int, C.c_int64,
                                                                          C.c_int64, C.c_int64]
        L.oracle_qdense_abs.argtypes = common + [dp] + [C.c_int64] * 3 + [C.c_int, C.c_int, C.c_int64,
                                                                          C.c_int64, C.c_int64]
        u8p = C.c_void_p
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_f16_to_f32.restype = C.c_float
        L.oracle_f16_to_f32_array.argtypes = [C.c_void_p, C.c_size_t, fp]
        L.oracle_ggml_values_per_block.argtypes = [C.c_int]
        L.oracle_ggml_bytes_per_block.argtypes = [C.c_int]
        L.oracle_ggml_dequant_row.argtypes = [C.c_int, u8p, C.c_int64, fp]
        L.oracle_ggml_dense.argtypes = [fp, u8p, C.c_int, fp, fp, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int]
        L.oracle_ggml_dense_f64.argtypes = [fp, u8p, C.c_int, fp, dp, dp, C.c_int64, C.c_int64, C.c_int64,
                                            C.c_int64]
        L.oracle_ggml_embedding.argtypes = [u8p, C.c_int64, C.c_int64, C.c_int, C.c_void_p, C.c_int64, fp]
        L.oracle_ggml_embedding.restype = C.c_int64
        _lib = L
    return _lib


# ---------------------------------------------------------------------------------------------
# bf16 / int4 helpers (numpy restatements of bfloat16.go:25-39 and convertdtype.go:202-222).
# ---------------------------------------------------------------------------------------------
def bf16_round(x) -> np.ndarray:
    """f32 -> bf16 bits via the C oracle (round to nearest even; NaN/Inf truncated)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16_array(a.ctypes.data_as(C.POINTER(C.c_float)), a.size, out.ctypes.data)
    return out


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rmsnorm_chain(x_bits: np.ndarray, eps: float, return_inv: bool = False):
    """The MLP's RMSNorm as the reference executes its graph, op by op in f32 (bf16 x in, bf16 out):
      xf = ConvertDType(x, F32); ms = ReduceSum(xf * xf, 1) * f32(1/D); inv = Rsqrt(ms + f32(eps));
      h = ConvertDType(xf * inv, BF16).
    ReduceSum adds the row's elements in order into an f32 accumulator starting at 0
    (execReduceSumGeneric, internal/gobackend/ops/reduce.go:403-414); Rsqrt is
    float32(1 / math.Sqrt(float64(v))) (execRsqrtGeneric, internal/gobackend/ops/unaryops.go:812-816);
    every other op rounds its f32 result once.  return_inv also returns the f32 Rsqrt per row."""
    xf = bf16_to_f32(x_bits).astype(np.float32)
    M, D = xf.shape
    sq = (xf * xf).astype(np.float32)
    acc = np.zeros(M, dtype=np.float32)
    for k in range(D):  # sequential over the row, vectorised over rows
        acc = (acc + sq[:, k]).astype(np.float32)
    ms = (acc * np.float32(1.0 / D)).astype(np.float32)
    v = (ms + np.float32(eps)).astype(np.float32)
    inv = (1.0 / np.sqrt(v.astype(np.float64))).astype(np.float32)
    h = bf16_round((xf * inv[:, None]).astype(np.float32))
    return (h, inv) if return_inv else h


def unpack_int4(packed, signed=True) -> np.ndarray:
    p = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    out = np.empty(p.size * 2, dtype=np.int8)
    fn = lib().oracle_unpack_int4 if signed else lib().oracle_unpack_uint4
    fn(p.ctypes.data, p.size, out.ctypes.data)
    return out


def pack_int4(values) -> np.ndarray:
    v = np.asarray(values).astype(np.int64).ravel() & 0xF
    if v.size % 2:
        v = np.concatenate([v, [0]])
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


def act(x, a: int) -> np.ndarray:
    arr = np.array(x, dtype=np.float32, copy=True).ravel()
    lib().oracle_act_array(arr.ctypes.data_as(C.POINTER(C.c_float)), arr.size, a)
    return arr.reshape(np.shape(x))


# ---------------------------------------------------------------------------------------------
# QuantizedDense problems.
# ---------------------------------------------------------------------------------------------
@dataclass
class QDenseProblem:
    """One FusedQuantizedDense call, with host data in the storage dtypes the backend takes."""

    M: int
    K: int
    N: int
    x: np.ndarray              # [M, K] float32 or bf16 bits (uint16)
    x_dtype: int
    w: np.ndarray              # [K, N] int8/uint8, or packed bytes for Int4/Uint4
    w_dtype: int
    scale: np.ndarray          # f32 or bf16 bits
    scale_dtype: int
    scale_shape: tuple
    block_axis: int
    block_size: int
    bias: Optional[np.ndarray] = None
    bias_dtype: int = DT_FLOAT32
    zp: Optional[np.ndarray] = None
    zp_dtype: int = DT_FLOAT32
    scheme: int = QUANT_LINEAR
    act: int = ACT_NONE
    name: str = ""
    extra: dict = field(default_factory=dict)

    def as_f32(self, a: Optional[np.ndarray], dt: int) -> Optional[np.ndarray]:
        if a is None:
            return None
        if dt == DT_BFLOAT16:
            return np.ascontiguousarray(bf16_to_f32(a))
        return np.ascontiguousarray(a, dtype=np.float32)

    def out_dtype(self) -> int:
        return self.x_dtype


def _fp(a):
    return None if a is None else a.ctypes.data_as(C.POINTER(C.c_float))


def qdense_f32(p: QDenseProblem, rows: Optional[np.ndarray] = None, threads: int = 1) -> np.ndarray:
    """Reference-order f32 result (with activation), before any output rounding.  `rows`
    selects a subset of x's rows (the oracle computes rows independently)."""
    x = p.as_f32(p.x, p.x_dtype).reshape(p.M, p.K)
    if rows is not None:
        x = np.ascontiguousarray(x[rows])
    m = x.shape[0]
    s, z, b = p.as_f32(p.scale, p.scale_dtype), p.as_f32(p.zp, p.zp_dtype), p.as_f32(p.bias, p.bias_dtype)
    w = np.ascontiguousarray(p.w)
    out = np.empty((m, p.N), dtype=np.float32)
    lib().oracle_qdense(_fp(x), w.ctypes.data, p.w_dtype, _fp(s), _fp(z), _fp(b), _fp(out), p.M, p.K, p.N,
                        p.scheme, p.block_axis, p.block_size, p.act, 0, m, threads)
    return out


def qdense_f64(p: QDenseProblem, rows: Optional[np.ndarray] = None, absolute: bool = False) -> np.ndarray:
    """Pre-activation sum in f64 (or the sum of |terms| with absolute=True)."""
    x = p.as_f32(p.x, p.x_dtype).reshape(p.M, p.K)
    if rows is not None:
        x = np.ascontiguousarray(x[rows])
    m = x.shape[0]
    s, z, b = p.as_f32(p.scale, p.scale_dtype), p.as_f32(p.zp, p.zp_dtype), p.as_f32(p.bias, p.bias_dtype)
    w = np.ascontiguousarray(p.w)
    out = np.empty((m, p.N), dtype=np.float64)
    fn = lib().oracle_qdense_abs if absolute else lib().oracle_qdense_f64
    fn(_fp(x), w.ctypes.data, p.w_dtype, _fp(s), _fp(z), _fp(b), out.ctypes.data_as(C.POINTER(C.c_double)),
       p.M, p.K, p.N, p.scheme, p.block_axis, p.block_size, 0, m)
    return out


def expected_output(p: QDenseProblem, rows=None, threads: int = 1) -> np.ndarray:
    """What the backend must return: the f32 result, rounded to bf16 bits when x is bf16."""
    y = qdense_f32(p, rows, threads)
    return bf16_round(y) if p.x_dtype == DT_BFLOAT16 else y


# ---------------------------------------------------------------------------------------------
# Seeded generators for BASELINE.json configs (and smaller variants of the same form).
# ---------------------------------------------------------------------------------------------
def _bf16(rng_vals) -> np.ndarray:
    return bf16_round(np.asarray(rng_vals, dtype=np.float32))


def make_problem(M, K, N, *, w_dtype=DT_INT8, x_dtype=DT_BFLOAT16, scale_dtype=DT_BFLOAT16, block_axis=0,
                 block_size=None, per_channel_1d=False, bias=True, bias_dtype=None, zp=False, scheme=QUANT_LINEAR,
                 act=ACT_NONE, scale_range=(0.001, 0.01), x_dist="normal", seed=0, name="") -> QDenseProblem:
    """Random problem: x ~ N(0,1) (or U(-1,1)), weights uniform over the full code range, scales
    U(scale_range), bias N(0, 0.02).  Seeds: one PCG64 stream per tensor, derived from `seed`."""
    ss = np.random.SeedSequence(seed)
    rx, rw, rs, rb, rz = [np.random.Generator(np.random.PCG64(s)) for s in ss.spawn(5)]
    if x_dist == "uniform":
        xf = rx.uniform(-1, 1, size=(M, K)).astype(np.float32)
    else:
        xf = rx.standard_normal(size=(M, K)).astype(np.float32)
    x = _bf16(xf) if x_dtype == DT_BFLOAT16 else xf
    if w_dtype == DT_INT8:
        w = rw.integers(-127, 128, size=(K, N), dtype=np.int64).astype(np.int8)
    elif w_dtype == DT_UINT8:
        w = rw.integers(0, 256, size=(K, N), dtype=np.int64).astype(np.uint8)
    elif w_dtype == DT_INT4:
        w = pack_int4(rw.integers(-8, 8, size=K * N))
    else:
        w = pack_int4(rw.integers(0, 16, size=K * N))
    B = block_size if block_size is not None else (K if block_axis == 0 else N)
    if block_axis == 0:
        kb = (K + B - 1) // B
        sshape = (N,) if (per_channel_1d and kb == 1) else (kb, N)
    else:
        sshape = (K, (N + B - 1) // B)
    sf = rs.uniform(scale_range[0], scale_range[1], size=sshape).astype(np.float32)
    scale = _bf16(sf) if scale_dtype == DT_BFLOAT16 else sf
    bdt = bias_dtype if bias_dtype is not None else (DT_BFLOAT16 if x_dtype == DT_BFLOAT16 else DT_FLOAT32)
    b = None
    if bias:
        bf = (rb.standard_normal(size=N) * 0.02).astype(np.float32)
        b = _bf16(bf) if bdt == DT_BFLOAT16 else bf
    z = None
    if zp:
        zf = rz.uniform(-0.05, 0.05, size=sshape).astype(np.float32)
        z = _bf16(zf) if scale_dtype == DT_BFLOAT16 else zf
    return QDenseProblem(M=M, K=K, N=N, x=x, x_dtype=x_dtype, w=w, w_dtype=w_dtype, scale=scale,
                         scale_dtype=scale_dtype, scale_shape=sshape, block_axis=block_axis, block_size=B, bias=b,
                         bias_dtype=bdt, zp=z, zp_dtype=scale_dtype, scheme=scheme, act=act, name=name)


def baseline_config(i: int, seed: int = 0) -> QDenseProblem:
    """BASELINE.json configs[i] as a QDenseProblem (i = 0..3; config 4 is the MLP graph)."""
    if i == 0:
        return make_problem(4, 512, 512, w_dtype=DT_INT8, x_dtype=DT_FLOAT32, scale_dtype=DT_FLOAT32, block_axis=0,
                            block_size=512, per_channel_1d=True, bias=True, bias_dtype=DT_FLOAT32,
                            x_dist="uniform", seed=seed, name="C1_int8_perchannel_f32")
    if i == 1:
        return make_problem(1, 4096, 11008, w_dtype=DT_INT4, block_axis=0, block_size=128, bias=False,
                            scale_range=(0.002, 0.02), seed=seed, name="C2_decode_int4_g128")
    if i == 2:
        return make_problem(16, 4096, 14336, w_dtype=DT_INT8, block_axis=0, block_size=64, bias=True,
                            act=ACT_SILU, seed=seed, name="C3_batched_decode_int8_g64_silu")
    if i == 3:
        return make_problem(2048, 4096, 4096, w_dtype=DT_INT8, block_axis=0, block_size=4096, per_channel_1d=True,
                            scale_dtype=DT_FLOAT32, bias=True, bias_dtype=DT_BFLOAT16, act=ACT_GELU, seed=seed,
                            name="C4_prefill_int8_perchannel_gelu")
    raise ValueError(i)


def algorithmic_bytes(p: QDenseProblem) -> int:
    """Each operand read once at its storage dtype, output written once."""
    nb = p.x.nbytes + p.w.nbytes + p.scale.nbytes
    nb += 0 if p.bias is None else p.bias.nbytes
    nb += 0 if p.zp is None else p.zp.nbytes
    nb += p.M * p.N * (2 if p.x_dtype == DT_BFLOAT16 else 4)
    return nb


# ---------------------------------------------------------------------------------------------
# DotGeneral restatement (output layout of shapeinference/dotgeneral.go:16-152), brute force in
# float64 for small tensors.
# ---------------------------------------------------------------------------------------------
def dot_general(lhs: np.ndarray, lc, lb, rhs: np.ndarray, rc, rb) -> np.ndarray:
    lc, lb, rc, rb = list(lc), list(lb), list(rc), list(rb)
    lcross = [a for a in range(lhs.ndim) if a not in lc and a not in lb]
    rcross = [a for a in range(rhs.ndim) if a not in rc and a not in rb]
    L = np.transpose(lhs.astype(np.float64), lb + lcross + lc)
    R = np.transpose(rhs.astype(np.float64), rb + rc + rcross)
    bshape = [lhs.shape[a] for a in lb]
    mshape = [lhs.shape[a] for a in lcross]
    nshape = [rhs.shape[a] for a in rcross]
    Bn = int(np.prod(bshape, dtype=np.int64))
    Mn = int(np.prod(mshape, dtype=np.int64))
    Nn = int(np.prod(nshape, dtype=np.int64))
    Kn = int(np.prod([lhs.shape[a] for a in lc], dtype=np.int64))
    L = L.reshape(Bn, Mn, Kn)
    R = R.reshape(Bn, Kn, Nn)
    out = np.matmul(L, R)  # float64
    return out.reshape(bshape + mshape + nshape)


def dot_general_int(lhs: np.ndarray, lc, lb, rhs: np.ndarray, rc, rb, acc_dtype=None) -> np.ndarray:
    """Integer DotGeneral as the reference computes it: inputs converted to the accumulator dtype
    when one is given (convertToAccumulatorDType, internal/gobackend/dot/dot.go:340-372), products
    and sums wrapping in that dtype (the noSIMD kernels' Go integer arithmetic,
    dot/matmul/nosimd.go:66-75).  Brute force, one output element at a time, for small cases:
    every product and partial sum is reduced modulo 2^bits and reinterpreted in the dtype."""
    dt = np.dtype(acc_dtype) if acc_dtype is not None else lhs.dtype
    bits = dt.itemsize * 8
    mod = 1 << bits

    def wrap(v: int) -> int:
        v %= mod
        return v - mod if (dt.kind == "i" and v >= mod // 2) else v

    lc, lb, rc, rb = list(lc), list(lb), list(rc), list(rb)
    lcross = [a for a in range(lhs.ndim) if a not in lc and a not in lb]
    rcross = [a for a in range(rhs.ndim) if a not in rc and a not in rb]
    L = np.transpose(lhs, lb + lcross + lc)
    R = np.transpose(rhs, rb + rc + rcross)
    bshape = [lhs.shape[a] for a in lb]
    mshape = [lhs.shape[a] for a in lcross]
    nshape = [rhs.shape[a] for a in rcross]
    Bn, Mn, Nn = (int(np.prod(x, dtype=np.int64)) for x in (bshape, mshape, nshape))
    Kn = int(np.prod([lhs.shape[a] for a in lc], dtype=np.int64))
    L = L.reshape(Bn, Mn, Kn)
    R = R.reshape(Bn, Kn, Nn)
    out = np.zeros((Bn, Mn, Nn), dtype=dt)
    for b in range(Bn):
        for m in range(Mn):
            for n in range(Nn):
                acc = 0
                for k in range(Kn):
                    acc = wrap(acc + wrap(wrap(int(L[b, m, k])) * wrap(int(R[b, k, n]))))
                out[b, m, n] = acc
    return out.reshape(bshape + mshape + nshape)


# ---------------------------------------------------------------------------------------------
# GGML block formats (quantizeddense_ggml.go, quantizeddense.go:455-499).
# ---------------------------------------------------------------------------------------------
GGML_Q4_0, GGML_Q8_0, GGML_IQ4_NL, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 5, 7
GGML_TYPES = (GGML_Q4_0, GGML_Q8_0, GGML_IQ4_NL, GGML_Q4_K, GGML_Q6_K)


def ggml_block(t: int):
    """(values per block, bytes per block) of a GGML type (fused_ops.go:148-177)."""
    return lib().oracle_ggml_values_per_block(t), lib().oracle_ggml_bytes_per_block(t)


def f16_to_f32(h) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(h, dtype=np.uint16))
    out = np.empty(a.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(a.ctypes.data, a.size, out.ctypes.data_as(C.POINTER(C.c_float)))
    return out


def ggml_dequant(t: int, rows) -> np.ndarray:
    """[R, bytesPerRow] uint8 -> [R, K] float32 (dequantXXXRow per row)."""
    r = np.ascontiguousarray(np.asarray(rows, dtype=np.uint8))
    R, bpr = r.shape
    vpb, bpb = ggml_block(t)
    K = bpr // bpb * vpb
    out = np.empty((R, K), dtype=np.float32)
    for i in range(R):
        rc = lib().oracle_ggml_dequant_row(t, r[i].ctypes.data, bpr,
                                           out[i].ctypes.data_as(C.POINTER(C.c_float)))
        if rc != 0:
            raise ValueError(f"unsupported GGML type {t}")
    return out


def ggml_dense(x, w, t: int, bias=None, act_: int = ACT_NONE) -> np.ndarray:
    """Reference-order f32 result of FusedQuantizedDense(GGML): x [M, K] f32, w [N, bytesPerRow]."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    w = np.ascontiguousarray(np.asarray(w, dtype=np.uint8))
    M, K = x.shape
    N, bpr = w.shape
    out = np.empty((M, N), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(np.asarray(bias, dtype=np.float32))
    fp = C.POINTER(C.c_float)
    rc = lib().oracle_ggml_dense(x.ctypes.data_as(fp), w.ctypes.data, t, None if b is None else b.ctypes.data_as(fp),
                                 out.ctypes.data_as(fp), M, K, N, bpr, act_)
    if rc != 0:
        raise ValueError(f"oracle_ggml_dense failed ({rc})")
    return out


def ggml_dense_f64(x, w, t: int, bias=None):
    """(exact f64 value, sum of |terms|) of x @ dequant(w)^T + bias."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    w = np.ascontiguousarray(np.asarray(w, dtype=np.uint8))
    M, K = x.shape
    N, bpr = w.shape
    out = np.empty((M, N), dtype=np.float64)
    ab = np.empty((M, N), dtype=np.float64)
    b = None if bias is None else np.ascontiguousarray(np.asarray(bias, dtype=np.float32))
    fp, dp = C.POINTER(C.c_float), C.POINTER(C.c_double)
    rc = lib().oracle_ggml_dense_f64(x.ctypes.data_as(fp), w.ctypes.data, t, None if b is None else b.ctypes.data_as(fp),
                                     out.ctypes.data_as(dp), ab.ctypes.data_as(dp), M, K, N, bpr)
    if rc != 0:
        raise ValueError(f"oracle_ggml_dense_f64 failed ({rc})")
    return out, ab


def ggml_embedding(data, t: int, idx) -> np.ndarray:
    """QuantizedEmbeddingLookup: data [vocab, bytesPerRow], idx int (any shape) -> [n, K] f32."""
    d = np.ascontiguousarray(np.asarray(data, dtype=np.uint8))
    i = np.ascontiguousarray(np.asarray(idx, dtype=np.int64).ravel())
    vpb, bpb = ggml_block(t)
    K = d.shape[1] // bpb * vpb
    out = np.empty((i.size, K), dtype=np.float32)
    rc = lib().oracle_ggml_embedding(d.ctypes.data, d.shape[0], d.shape[1], t, i.ctypes.data, i.size,
                                     out.ctypes.data_as(C.POINTER(C.c_float)))
    if rc != 0:
        raise IndexError(f"index {int(i[rc - 1])} out of range [0, {d.shape[0]})")
    return out


def ggml_random_rows(t: int, n: int, k: int, rng) -> np.ndarray:
    """Random GGML rows [n, bytesPerRow] with finite block scales in U(0.001, 0.02) (test data)."""
    vpb, bpb = ggml_block(t)
    nb = k // vpb
    rows = rng.integers(0, 256, (n, nb, bpb), dtype=np.uint8)
    scale_at = {GGML_Q4_0: [0], GGML_Q8_0: [0], GGML_IQ4_NL: [0], GGML_Q4_K: [0, 2], GGML_Q6_K: [208]}[t]
    for off in scale_at:
        d = rng.uniform(0.001, 0.02, (n, nb)).astype(np.float16).view(np.uint16)
        rows[:, :, off] = d & 0xFF
        rows[:, :, off + 1] = d >> 8
    return rows.reshape(n, nb * bpb)
