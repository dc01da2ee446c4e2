"""Synthetic workloads of the benchmark: the BASELINE.json configurations of FusedQuantizedDense.

Each workload builds seeded host data in the storage dtypes the backend takes (bf16 as uint16
bits, Int4 packed two per byte in the reference packing) and compiles the graph the reference's
callers would build: Parameter x, w, scale[, bias] -> FusedQuantizedDense -> Return.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import backend as B
from .dtypes import BFloat16, DType, Float32, Int4, Int8, Shape, Uint4, Uint8, bf16_from_f32, pack_int4


@dataclass
class QDWorkload:
    name: str
    M: int
    K: int
    N: int
    x_dtype: DType
    w_dtype: DType
    scale_dtype: DType
    scale_shape: tuple
    block_axis: int
    block_size: int
    bias_dtype: Optional[DType]
    act: int
    x: np.ndarray
    w: np.ndarray
    scale: np.ndarray
    bias: Optional[np.ndarray]
    scheme: int = int(B.QuantLinear)

    def shapes(self):
        s = [Shape(self.x_dtype, self.M, self.K), Shape(self.w_dtype, self.K, self.N),
             Shape(self.scale_dtype, *self.scale_shape)]
        if self.bias is not None:
            s.append(Shape(self.bias_dtype, self.N))
        return s

    def host_inputs(self):
        d = [self.x, self.w, self.scale]
        if self.bias is not None:
            d.append(self.bias)
        return d

    def compile(self, backend: B.Backend) -> B.Executable:
        bld = backend.Builder(self.name)
        f = bld.Main()
        params = [f.Parameter(n, s) for n, s in zip(["x", "w", "scale", "bias"], self.shapes())]
        bias = params[3] if self.bias is not None else None
        q = B.Quantization(B.QuantizationScheme(self.scheme), params[2], None, self.block_axis, self.block_size)
        y = f.FusedQuantizedDense(params[0], params[1], bias, q, B.ActivationType(self.act))
        f.Return([y])
        return bld.Compile()

    def upload(self, backend: B.Backend):
        return [backend.BufferFromFlatData(0, d.ravel(), s) for d, s in zip(self.host_inputs(), self.shapes())]

    def weight_bytes(self) -> int:
        return self.w.nbytes

    def algorithmic_bytes(self) -> int:
        """Every operand read once at its storage dtype, the output written once."""
        out = self.M * self.N * (2 if self.x_dtype == BFloat16 else 4)
        return sum(a.nbytes for a in self.host_inputs()) + out

    def flops(self) -> int:
        return 2 * self.M * self.K * self.N


@dataclass
class MLPWorkload:
    """the quantized MLP built through the Builder API, batch 8 x seq 1:
    RMSNorm (eps 1e-6, no gamma) over bf16 x [8,4096]; gate and up FusedQuantizedDense Int4 g128
    [4096 -> 14336] (SiLU fused into gate's epilogue); SiLU(gate) * up; down FusedQuantizedDense
    Int4 g128 [14336 -> 4096]; residual add.  RMSNorm runs in f32 (ConvertDType around it)."""

    name: str
    M: int
    D: int
    F: int
    G: int
    x: np.ndarray
    weights: list  # [(w packed, scale bf16 bits, K, N)] for gate, up, down
    eps: float = 1e-6

    def shapes(self):
        s = [Shape(BFloat16, self.M, self.D)]
        for w, sc, K, N in self.weights:
            s += [Shape(Int4, K, N), Shape(BFloat16, K // self.G, N)]
        return s

    def host_inputs(self):
        d = [self.x]
        for w, sc, _, _ in self.weights:
            d += [w, sc]
        return d

    def compile(self, backend: B.Backend) -> B.Executable:
        bld = backend.Builder(self.name)
        f = bld.Main()
        names = ["x", "w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down"]
        p = [f.Parameter(n, sh) for n, sh in zip(names, self.shapes())]
        x = p[0]
        xf = f.ConvertDType(x, Float32)
        ms = f.Mul(f.ReduceSum(f.Mul(xf, xf), 1), f.Constant(np.full(self.M, 1.0 / self.D, np.float32)))
        inv = f.Rsqrt(f.Add(ms, f.Constant(np.full(self.M, self.eps, np.float32))))
        h = f.ConvertDType(f.Mul(xf, f.BroadcastInDim(inv, Shape(Float32, self.M, self.D), [0])), BFloat16)

        def qd(v, w, sc, act):
            q = B.Quantization(B.QuantLinear, sc, None, 0, self.G)
            return f.FusedQuantizedDense(v, w, None, q, B.ActivationType(act))

        g = qd(h, p[1], p[2], B.ActivationSilu)
        u = qd(h, p[3], p[4], B.ActivationNone)
        d = qd(f.Mul(g, u), p[5], p[6], B.ActivationNone)
        f.Return([f.Add(d, x)])
        return bld.Compile()

    def upload(self, backend: B.Backend):
        return [backend.BufferFromFlatData(0, d.ravel(), s) for d, s in zip(self.host_inputs(), self.shapes())]

    def weight_bytes(self) -> int:
        return sum(w.nbytes for w, _, _, _ in self.weights)

    def algorithmic_bytes(self) -> int:
        """Weights and scales read once, x read once, the output written once."""
        return sum(a.nbytes for a in self.host_inputs()) + self.M * self.D * 2

    def flops(self) -> int:
        return sum(2 * self.M * K * N for _, _, K, N in self.weights)


@dataclass
class GGMLWorkload:
    """FusedQuantizedDense over GGML block rows (not a BASELINE config; the reference's GGML
    scheme, quantizeddense_ggml.go): f32 x [M, K], weights [N, bytesPerRow] Uint8 in one of the
    supported block formats."""

    name: str
    M: int
    K: int
    N: int
    ggml_type: int
    x: np.ndarray
    w: np.ndarray

    def shapes(self):
        return [Shape(Float32, self.M, self.K), Shape(Uint8, *self.w.shape)]

    def host_inputs(self):
        return [self.x, self.w]

    def compile(self, backend: B.Backend) -> B.Executable:
        bld = backend.Builder(self.name)
        f = bld.Main()
        x, w = (f.Parameter(n, s) for n, s in zip(["x", "w"], self.shapes()))
        q = B.Quantization(B.QuantGGML, None, None, 1, 1, self.ggml_type)
        f.Return([f.FusedQuantizedDense(x, w, None, q, B.ActivationNone)])
        return bld.Compile()

    def upload(self, backend: B.Backend):
        return [backend.BufferFromFlatData(0, d.ravel(), s) for d, s in zip(self.host_inputs(), self.shapes())]

    def weight_bytes(self) -> int:
        return self.w.nbytes

    def algorithmic_bytes(self) -> int:
        """Blocks read once (scales included), x read once, the f32 output written once."""
        return self.x.nbytes + self.w.nbytes + self.M * self.N * 4

    def flops(self) -> int:
        return 2 * self.M * self.K * self.N


@dataclass
class DotWorkload:
    """DotGeneral at the prefill shape (the contraction FusedQuantizedDense lowers onto,
    standard_ops.go:339-361): x [M, K] . w [K, N] in bf16, f32 accumulation, bf16 output."""

    name: str
    M: int
    K: int
    N: int
    x: np.ndarray
    w: np.ndarray

    def shapes(self):
        return [Shape(BFloat16, self.M, self.K), Shape(BFloat16, self.K, self.N)]

    def host_inputs(self):
        return [self.x, self.w]

    def compile(self, backend: B.Backend) -> B.Executable:
        bld = backend.Builder(self.name)
        f = bld.Main()
        x, w = (f.Parameter(n, s) for n, s in zip(["x", "w"], self.shapes()))
        f.Return([f.DotGeneral(x, [1], [], w, [0], [])])
        return bld.Compile()

    def upload(self, backend: B.Backend):
        return [backend.BufferFromFlatData(0, d.ravel(), s) for d, s in zip(self.host_inputs(), self.shapes())]

    def weight_bytes(self) -> int:
        return self.w.nbytes

    def algorithmic_bytes(self) -> int:
        return self.x.nbytes + self.w.nbytes + self.M * self.N * 2

    def flops(self) -> int:
        return 2 * self.M * self.K * self.N


# DotGeneral model shapes of the reference's BenchmarkDotGeneral
# (support/backendtest/bench_dotgeneral.go:20-482): the all-MiniLM-L6-v2 cases and the first
# bge-small-en-v1.5 batch configurations, as (name, lhs dims, rhs dims, lhs contracting,
# lhs batch, rhs contracting, rhs batch).  The reference runs them in float32.
DOT_MODEL_CASES = [
    ("MiniLM/32x12x13x13.32x12x13x32", (32, 12, 13, 13), (32, 12, 13, 32), [3], [0, 1], [2], [0, 1]),
    ("MiniLM/32x12x13x32.32x12x32x13", (32, 12, 13, 32), (32, 12, 32, 13), [3], [0, 1], [2], [0, 1]),
    ("MiniLM/32x13x1536.1536x384", (32, 13, 1536), (1536, 384), [2], [], [0], []),
    ("MiniLM/32x13x1536.384x1536(T)", (32, 13, 1536), (384, 1536), [2], [], [1], []),
    ("MiniLM/32x13x384.384x1152", (32, 13, 384), (384, 1152), [2], [], [0], []),
    ("MiniLM/32x13x384.384x1536", (32, 13, 384), (384, 1536), [2], [], [0], []),
    ("MiniLM/32x13x384.384x384", (32, 13, 384), (384, 384), [2], [], [0], []),
    ("MiniLM/416x384.384x1152", (416, 384), (384, 1152), [1], [], [0], []),
    ("bge/10x192x12x192.10x192x12x32", (10, 192, 12, 192), (10, 192, 12, 32), [3], [0, 2], [1], [0, 2]),
    ("bge/10x192x1536.384x1536(T)", (10, 192, 1536), (384, 1536), [2], [], [1], []),
    ("bge/10x192x384.1536x384(T)", (10, 192, 384), (1536, 384), [2], [], [1], []),
    ("bge/10x192x384.384x384(T)", (10, 192, 384), (384, 384), [2], [], [1], []),
    ("bge/16x128x12x128.16x128x12x32", (16, 128, 12, 128), (16, 128, 12, 32), [3], [0, 2], [1], [0, 2]),
    ("bge/16x128x12x32.16x128x12x32", (16, 128, 12, 32), (16, 128, 12, 32), [3], [0, 2], [3], [0, 2]),
    ("bge/16x128x1536.384x1536(T)", (16, 128, 1536), (384, 1536), [2], [], [1], []),
    ("bge/16x128x384.1536x384(T)", (16, 128, 384), (1536, 384), [2], [], [1], []),
    ("bge/16x128x384.384x384(T)", (16, 128, 384), (384, 384), [2], [], [1], []),
    ("bge/256x8x1536.384x1536(T)", (256, 8, 1536), (384, 1536), [2], [], [1], []),
    ("bge/256x8x384.1536x384(T)", (256, 8, 384), (1536, 384), [2], [], [1], []),
    ("bge/256x8x384.384x384(T)", (256, 8, 384), (384, 384), [2], [], [1], []),
]


def dot_case_flops(case) -> int:
    """2 x (product of the output dims) x (product of the contracting dims)."""
    _, ls, rs, lc, lb, rc, rb = case
    out = int(np.prod([ls[a] for a in lb])) * int(np.prod([d for a, d in enumerate(ls) if a not in lc + lb])) * \
        int(np.prod([d for a, d in enumerate(rs) if a not in rc + rb]))
    return 2 * out * int(np.prod([ls[a] for a in lc]))


@dataclass
class DotCaseWorkload:
    """One DOT_MODEL_CASES entry in a float dtype: DotGeneral(lhs, rhs) with seeded N(0,1) data."""

    case: tuple
    dtype: DType
    seed: int = 0

    @property
    def name(self) -> str:
        return f"{self.case[0]}[{self.dtype.name}]"

    def shapes(self):
        return [Shape(self.dtype, *self.case[1]), Shape(self.dtype, *self.case[2])]

    def host_inputs(self):
        rng = np.random.default_rng(self.seed)
        out = []
        for dims in (self.case[1], self.case[2]):
            f = rng.standard_normal(dims).astype(np.float32)
            out.append(bf16_from_f32(f) if self.dtype == BFloat16 else f)
        return out

    def compile(self, backend: B.Backend) -> B.Executable:
        _, _, _, lc, lb, rc, rb = self.case
        bld = backend.Builder("dot_case")
        f = bld.Main()
        lhs, rhs = (f.Parameter(n, s) for n, s in zip(["lhs", "rhs"], self.shapes()))
        f.Return([f.DotGeneral(lhs, lc, lb, rhs, rc, rb)])
        return bld.Compile()

    def upload(self, backend: B.Backend):
        return [backend.BufferFromFlatData(0, d.ravel(), s) for d, s in zip(self.host_inputs(), self.shapes())]

    def weight_bytes(self) -> int:
        return sum(a.nbytes for a in self.host_inputs())

    def flops(self) -> int:
        return dot_case_flops(self.case)


def ggml_rows(t: int, n: int, k: int, rng) -> np.ndarray:
    """Random GGML rows [n, bytesPerRow]: random codes, block scales (f16) in U(0.001, 0.02)."""
    vpb, bpb = B.ggml_values_per_block(t), B.ggml_bytes_per_block(t)
    nb = k // vpb
    rows = rng.integers(0, 256, (n, nb, bpb), dtype=np.uint8)
    offsets = {B.GGMLQ4_K: [0, 2], B.GGMLQ6_K: [208]}.get(t, [0])
    for off in offsets:
        d = rng.uniform(0.001, 0.02, (n, nb)).astype(np.float16).view(np.uint16)
        rows[:, :, off] = d & 0xFF
        rows[:, :, off + 1] = d >> 8
    return rows.reshape(n, nb * bpb)


def _rngs(seed: int, n: int):
    return [np.random.Generator(np.random.PCG64(s)) for s in np.random.SeedSequence(seed).spawn(n)]


def make(name: str, seed: int = 0) -> QDWorkload:
    """C1 .. C5."""
    rx, rw, rs, rb = _rngs(seed, 4)
    if name == "C1":  # int8 per-channel, x f32 [4,512] U(-1,1), bias f32, no activation
        M, K, N = 4, 512, 512
        x = rx.uniform(-1, 1, (M, K)).astype(np.float32)
        w = rw.integers(-127, 128, (K, N)).astype(np.int8)
        s = rs.uniform(0.001, 0.01, N).astype(np.float32)
        b = (rb.standard_normal(N) * 0.02).astype(np.float32)
        return QDWorkload("C1_int8_perchannel_f32", M, K, N, Float32, Int8, Float32, (N,), 0, K, Float32, 0,
                          x, w, s, b)
    if name == "C2":  # decode GEMV, Int4 g128 along K, bf16 x/scales, no bias
        M, K, N, G = 1, 4096, 11008, 128
        x = bf16_from_f32(rx.standard_normal((M, K)).astype(np.float32))
        w = pack_int4(rw.integers(-8, 8, K * N))
        s = bf16_from_f32(rs.uniform(0.002, 0.02, (K // G, N)).astype(np.float32))
        return QDWorkload("C2_decode_gemv_int4_g128", M, K, N, BFloat16, Int4, BFloat16, (K // G, N), 0, G, None, 0,
                          x, w, s, None)
    if name == "C3":  # batched decode, int8 g64 along K, bias bf16, SiLU
        M, K, N, G = 16, 4096, 14336, 64
        x = bf16_from_f32(rx.standard_normal((M, K)).astype(np.float32))
        w = rw.integers(-127, 128, (K, N)).astype(np.int8)
        s = bf16_from_f32(rs.uniform(0.001, 0.01, (K // G, N)).astype(np.float32))
        b = bf16_from_f32((rb.standard_normal(N) * 0.02).astype(np.float32))
        return QDWorkload("C3_batched_decode_int8_g64_silu", M, K, N, BFloat16, Int8, BFloat16, (K // G, N), 0, G,
                          BFloat16, B.ActivationSilu, x, w, s, b)
    if name == "C4":  # prefill, int8 per-channel f32 scales, bias bf16, GELU
        M, K, N = 2048, 4096, 4096
        x = bf16_from_f32(rx.standard_normal((M, K)).astype(np.float32))
        w = rw.integers(-127, 128, (K, N)).astype(np.int8)
        s = rs.uniform(0.001, 0.01, N).astype(np.float32)
        b = bf16_from_f32((rb.standard_normal(N) * 0.02).astype(np.float32))
        return QDWorkload("C4_prefill_int8_perchannel_gelu", M, K, N, BFloat16, Int8, Float32, (N,), 0, K, BFloat16,
                          B.ActivationGelu, x, w, s, b)
    if name == "C5":  # quantized MLP graph, batch 8, Int4 g128, scales U(0.002, 0.02)
        M, D, F, G = 8, 4096, 14336, 128
        x = bf16_from_f32(rx.standard_normal((M, D)).astype(np.float32))
        ws = []
        for K, N in ((D, F), (D, F), (F, D)):
            w = pack_int4(rw.integers(-8, 8, K * N))
            sc = bf16_from_f32(rs.uniform(0.002, 0.02, (K // G, N)).astype(np.float32))
            ws.append((w, sc, K, N))
        return MLPWorkload("C5_mlp_int4_g128_batch8", M, D, F, G, x, ws)
    if name in ("P32", "P64"):  # small-batch prefill: int8 per-channel, bf16 x, the C2 matrix size
        M, K, N = int(name[1:]), 4096, 11008
        x = bf16_from_f32(rx.standard_normal((M, K)).astype(np.float32))
        w = rw.integers(-127, 128, (K, N)).astype(np.int8)
        s = rs.uniform(0.001, 0.01, N).astype(np.float32)
        return QDWorkload(f"P{M}_int8_perchannel_bf16", M, K, N, BFloat16, Int8, Float32, (N,), 0, K, None, 0,
                          x, w, s, None)
    if name in ("Q1", "Q2"):  # prefill with K-grouped scales: Int4 g128 (the MLP's gate/up) / int8 g64
        M, K, N = 2048, 4096, 14336
        i4 = name == "Q1"
        G = 128 if i4 else 64
        x = bf16_from_f32(rx.standard_normal((M, K)).astype(np.float32))
        w = pack_int4(rw.integers(-8, 8, K * N)) if i4 else rw.integers(-127, 128, (K, N)).astype(np.int8)
        s = bf16_from_f32(rs.uniform(0.002, 0.02, (K // G, N)).astype(np.float32))
        label = "Q1_prefill_int4_g128" if i4 else "Q2_prefill_int8_g64"
        return QDWorkload(label, M, K, N, BFloat16, Int4 if i4 else Int8, BFloat16, (K // G, N), 0, G, None, 0,
                          x, w, s, None)
    if name == "D1":  # DotGeneral bf16 at the C4 (prefill) shape
        M, K, N = 2048, 4096, 4096
        x = bf16_from_f32(rx.standard_normal((M, K)).astype(np.float32))
        w = bf16_from_f32((rw.standard_normal((K, N)) * 0.02).astype(np.float32))
        return DotWorkload("D1_dotgeneral_bf16_prefill", M, K, N, x, w)
    if name == "R3":  # the reference's own layout at prefill: f32 x [2048,4096], Int4, scale [K, N/128]
        M, K, N, G = 2048, 4096, 11008, 128
        x = rx.standard_normal((M, K)).astype(np.float32)
        w = pack_int4(rw.integers(-8, 8, K * N))
        s = rs.uniform(0.002, 0.02, (K, (N + G - 1) // G)).astype(np.float32)
        return QDWorkload("R3_ref_layout_prefill_int4_f32", M, K, N, Float32, Int4, Float32, s.shape, 1, G, None, 0,
                          x, w, s, None)
    if name in ("R1", "R2"):  # the reference's own layout at the C2 shape: f32 x, scale [K, N/128]
        M, K, N, G = 1, 4096, 11008, 128
        nf4 = name == "R2"
        x = rx.standard_normal((M, K)).astype(np.float32)
        w = pack_int4(rw.integers(0, 16, K * N) if nf4 else rw.integers(-8, 8, K * N))
        s = rs.uniform(0.002, 0.02, (K, (N + G - 1) // G)).astype(np.float32)
        label = "R2_ref_layout_decode_nf4_f32" if nf4 else "R1_ref_layout_decode_int4_f32"
        return QDWorkload(label, M, K, N, Float32, Uint4 if nf4 else Int4, Float32, s.shape, 1, G, None, 0, x, w, s,
                          None, scheme=int(B.QuantNF4) if nf4 else int(B.QuantLinear))
    ggml = {"G1": ("G1_ggml_q4_0_decode", B.GGMLQ4_0), "G2": ("G2_ggml_q4_k_decode", B.GGMLQ4_K),
            "G3": ("G3_ggml_q8_0_decode", B.GGMLQ8_0), "G4": ("G4_ggml_q6_k_decode", B.GGMLQ6_K)}
    if name in ggml:  # GGML decode GEMV at the C2 shape: x f32 [1,4096], 11008 block rows
        label, t = ggml[name]
        M, K, N = 1, 4096, 11008
        x = rx.standard_normal((M, K)).astype(np.float32)
        return GGMLWorkload(label, M, K, N, int(t), x, ggml_rows(int(t), N, K, rw))
    raise ValueError(f"unknown workload {name}")
