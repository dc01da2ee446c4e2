"""Helpers shared by the GPU tests: run a FusedQuantizedDense problem through the backend's
public API (Builder -> Compile -> Execute on device-resident buffers) and compare results."""
from __future__ import annotations

import numpy as np

import compute_amd as ca
from oracle import oracle as O

DT = {O.DT_INT8: ca.Int8, O.DT_UINT8: ca.Uint8, O.DT_INT4: ca.Int4, O.DT_UINT4: ca.Uint4,
      O.DT_FLOAT32: ca.Float32, O.DT_BFLOAT16: ca.BFloat16}


class QDenseRun:
    """Compiled FusedQuantizedDense graph for one problem, with its input buffers resident."""

    def __init__(self, backend: ca.Backend, p: O.QDenseProblem):
        self.p = p
        self.backend = backend
        bld = backend.Builder(p.name or "qdense")
        f = bld.Main()
        shapes = [ca.Shape(DT[p.x_dtype], p.M, p.K), ca.Shape(DT[p.w_dtype], p.K, p.N),
                  ca.Shape(DT[p.scale_dtype], *p.scale_shape)]
        datas = [p.x, p.w, p.scale]
        x = f.Parameter("x", shapes[0])
        w = f.Parameter("w", shapes[1])
        s = f.Parameter("scale", shapes[2])
        zp = None
        if p.zp is not None:
            shapes.append(ca.Shape(DT[p.zp_dtype], *p.scale_shape))
            datas.append(p.zp)
            zp = f.Parameter("zp", shapes[-1])
        bias = None
        if p.bias is not None:
            shapes.append(ca.Shape(DT[p.bias_dtype], p.N))
            datas.append(p.bias)
            bias = f.Parameter("bias", shapes[-1])
        q = ca.Quantization(ca.QuantizationScheme(p.scheme), s, zp, p.block_axis, p.block_size)
        y = f.FusedQuantizedDense(x, w, bias, q, ca.ActivationType(p.act))
        f.Return([y])
        self.exe = bld.Compile()
        self.inputs = [backend.BufferFromFlatData(0, d.ravel(), sh) for d, sh in zip(datas, shapes)]

    def args(self, out=None):
        """mx_qdense_args over the resident inputs; out: the output buffer (planning: none)."""
        p = self.p
        a = ca._lib.mx_qdense_args()
        a.x, a.w, a.scale = (self.inputs[i].DevicePtr() for i in range(3))
        k = 3
        if p.zp is not None:
            a.zero_point = self.inputs[k].DevicePtr()
            a.zero_point_dtype = p.zp_dtype
            k += 1
        if p.bias is not None:
            a.bias = self.inputs[k].DevicePtr()
            a.bias_dtype = p.bias_dtype
        a.out = (out or self.inputs[0]).DevicePtr()  # planning writes nothing
        a.M, a.K, a.N = p.M, p.K, p.N
        a.x_dtype, a.w_dtype, a.scale_dtype = p.x_dtype, p.w_dtype, p.scale_dtype
        a.scheme, a.block_axis, a.block_size, a.activation = p.scheme, p.block_axis, p.block_size, p.act
        return a

    def plan(self) -> str:
        return self.backend.QDensePlan(self.args())

    def run_direct(self, out) -> None:
        """mx_qdense on the resident inputs into the caller's output buffer (no graph)."""
        self.backend.QDense(self.args(out))

    def run(self) -> np.ndarray:
        out = self.exe.Execute(self.inputs)[0]
        y = out.ToFlatData()
        out.Finalize()
        return y.reshape(self.p.M, self.p.N)


def run_qdense(backend, p: O.QDenseProblem) -> np.ndarray:
    return QDenseRun(backend, p).run()


def assert_bf16_close(got_bits: np.ndarray, ref_f32: np.ndarray, rtol=1e-2, atol=1e-3, what=""):
    """bf16 output vs the reference's f32 result: |got - ref| <= atol + rtol*|ref|."""
    got = O.bf16_to_f32(got_bits).astype(np.float64)
    ref = ref_f32.astype(np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside rel {rtol} / abs {atol}; worst at {i}: "
                             f"got {got[i]}, want {ref[i]}")


def assert_f32_accumulation_close(got_f32: np.ndarray, p: O.QDenseProblem, rows=None, rel=1e-5, what=""):
    """f32 accumulation check of a kernel that sums in another order: the error against the f64
    value is bounded by rel * (sum of |terms|), the scale of any f32 summation's error."""
    truth = O.qdense_f64(p, rows)
    scale = O.qdense_f64(p, rows, absolute=True)
    err = np.abs(got_f32.astype(np.float64) - truth)
    bound = rel * scale + 1e-30
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} outside rel {rel} of sum|terms|; worst at {i}: got {got_f32[i]}, "
                             f"want {truth[i]} (sum|terms| {scale[i]})")
