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
from .dtypes import BFloat16, DType, Float32, Int4, Int8, Shape, bf16_from_f32, pack_int4


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
        q = B.Quantization(B.QuantLinear, params[2], None, self.block_axis, self.block_size)
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


def _rngs(seed: int, n: int):
    return [np.random.Generator(np.random.PCG64(s)) for s in np.random.SeedSequence(seed).spawn(n)]


def make(name: str, seed: int = 0) -> QDWorkload:
    """C1 .. C4."""
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
    raise ValueError(f"unknown workload {name}")
