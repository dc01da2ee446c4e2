"""Host-side mirror of the reference's `compute` API over libmxrt.so.

Names, argument meanings and error behaviour follow the reference's Go interfaces so the tests
read like support/backendtest:
  Backend          compute.go:68-102           Buffer      buffer.go:12-61
  Builder          builder.go:29-82            Function    function.go:23-135, fused_ops.go:317-462
  Executable       executable.go:10-37         Quantization / ActivationType  fused_ops.go:81-289
Errors: every failing call raises ComputeError; "unsupported" raises ErrNotImplemented (the
counterpart of compute.ErrNotImplemented, compute.go:104-115).
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import Any, Optional, Sequence

import numpy as np

from . import _lib
from .dtypes import DType, Shape


# ---------------------------------------------------------------------------------------------
# Errors.
# ---------------------------------------------------------------------------------------------
class ComputeError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class ErrNotImplemented(ComputeError):
    """compute.ErrNotImplemented: the op/config is not supported; callers may fall back."""


class ErrFinalized(ComputeError):
    pass


class ErrNoDevice(ComputeError):
    pass


def IsNotImplemented(err: BaseException) -> bool:
    return isinstance(err, ErrNotImplemented)


def _check(rc: int) -> None:
    if rc == _lib.MX_OK:
        return
    msg = _lib.load().mx_last_error().decode(errors="replace")
    cls = {
        _lib.MX_ERR_NOT_IMPLEMENTED: ErrNotImplemented,
        _lib.MX_ERR_FINALIZED: ErrFinalized,
        _lib.MX_ERR_NO_DEVICE: ErrNoDevice,
    }.get(rc, ComputeError)
    raise cls(rc, msg)


# ---------------------------------------------------------------------------------------------
# Enums and configuration structs.
# ---------------------------------------------------------------------------------------------
class QuantizationScheme(enum.IntEnum):
    QuantLinear = 0
    QuantNF4 = 1
    QuantGGML = 2


QuantLinear, QuantNF4, QuantGGML = QuantizationScheme


class ActivationType(enum.IntEnum):
    ActivationNone = 0
    ActivationGelu = 1
    ActivationRelu = 2
    ActivationSilu = 3
    ActivationHardSwish = 4
    ActivationTanh = 5


(ActivationNone, ActivationGelu, ActivationRelu, ActivationSilu, ActivationHardSwish,
 ActivationTanh) = ActivationType


class OpType(enum.IntEnum):
    """Subset of compute.OpType (optype.go:13-162) this backend reports in Capabilities."""

    Parameter = 1
    Constant = 2
    Identity = 3
    Abs = 10
    Add = 11
    Bitcast = 14
    BroadcastInDim = 19
    ConvertDType = 28
    Div = 30
    DotGeneral = 32
    Erf = 39
    Exp = 40
    Iota = 50
    Logistic = 63
    Max = 64
    Min = 65
    Mul = 66
    Neg = 67
    ReduceMax = 79
    ReduceSum = 82
    Reshape = 84
    Rsqrt = 88
    Slice = 100
    Sqrt = 101
    Sub = 102
    Tanh = 103
    Transpose = 104
    FusedGelu = 118
    FusedDense = 119
    FusedScaledDotProductAttention = 120
    FusedQuantizedDense = 123
    QuantizedEmbeddingLookup = 124


NF4LookupTable = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
], dtype=np.float32)  # fused_ops.go:116-121


class GGMLQuantType(enum.IntEnum):
    """compute.GGMLQuantType (fused_ops.go:134-146)."""

    GGMLQ4_0 = 0
    GGMLQ8_0 = 1
    GGMLIQ4NL = 2
    GGMLQ2_K = 3
    GGMLQ3_K = 4
    GGMLQ4_K = 5
    GGMLQ5_K = 6
    GGMLQ6_K = 7


GGMLQ4_0, GGMLQ8_0, GGMLIQ4NL, GGMLQ2_K, GGMLQ3_K, GGMLQ4_K, GGMLQ5_K, GGMLQ6_K = GGMLQuantType

IQ4NLLookupTable = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                            dtype=np.float32)  # fused_ops.go:127-130


def ggml_values_per_block(t: int) -> int:
    """GGMLQuantType.ValuesPerBlock (fused_ops.go:148-156)."""
    return {GGMLQ4_0: 32, GGMLQ8_0: 32, GGMLIQ4NL: 32, GGMLQ2_K: 256, GGMLQ3_K: 256, GGMLQ4_K: 256,
            GGMLQ5_K: 256, GGMLQ6_K: 256}.get(int(t), 0)


def ggml_bytes_per_block(t: int) -> int:
    """GGMLQuantType.BytesPerBlock (fused_ops.go:158-177)."""
    return {GGMLQ4_0: 18, GGMLQ8_0: 34, GGMLIQ4NL: 18, GGMLQ2_K: 84, GGMLQ3_K: 110, GGMLQ4_K: 144,
            GGMLQ5_K: 176, GGMLQ6_K: 210}.get(int(t), 0)


@dataclass
class Quantization:
    """compute.Quantization (fused_ops.go:204-234).

    BlockAxis=1 is the reference layout (Scale [K, ceil(N/BlockSize)]).  This backend also takes
    BlockAxis=0: scale blocks along K, Scale [ceil(K/BlockSize), N] (or [N] per output channel).
    """

    Scheme: QuantizationScheme = QuantLinear
    Scale: Any = None
    ZeroPoint: Any = None
    BlockAxis: int = 1
    BlockSize: int = 1
    GGMLType: int = 0


class DenseLayout(enum.IntEnum):
    """compute.DenseLayout (fused_ops.go:51-57)."""

    DenseLayoutInputOutputs = 0
    DenseLayoutOutputsInput = 1


DenseLayoutInputOutputs, DenseLayoutOutputsInput = DenseLayout


@dataclass
class DenseConfig:
    """compute.DenseConfig (fused_ops.go:73-77)."""

    Activation: ActivationType = ActivationNone
    WeightLayout: DenseLayout = DenseLayoutInputOutputs


@dataclass
class DotGeneralConfig:
    """compute.DotGeneralConfig (standard_ops.go:91-111)."""

    AccumulatorDType: DType = DType.InvalidDType
    OutputDType: DType = DType.InvalidDType


@dataclass
class Capabilities:
    """compute.Capabilities (capabilities.go:12-39)."""

    Operations: dict
    DTypes: dict
    Functions: bool = False
    DynamicAxes: bool = False


# ---------------------------------------------------------------------------------------------
# Helpers.
# ---------------------------------------------------------------------------------------------
def _to_c_shape(shape: Shape) -> _lib.mx_shape:
    if shape.rank() > _lib.MX_MAX_RANK:
        raise ComputeError(_lib.MX_ERR_INVALID, f"rank {shape.rank()} > {_lib.MX_MAX_RANK}")
    s = _lib.mx_shape()
    s.dtype = int(shape.dtype)
    s.rank = shape.rank()
    for i, d in enumerate(shape.dimensions):
        s.dims[i] = d
    return s


def _from_c_shape(s: _lib.mx_shape) -> Shape:
    return Shape(DType(s.dtype), *[s.dims[i] for i in range(s.rank)])


def _i32(values: Sequence[int] | None):
    values = list(values or [])
    arr = (C.c_int32 * max(1, len(values)))(*values)
    return arr, len(values)


def _i64(values: Sequence[int] | None):
    values = list(values or [])
    return (C.c_int64 * max(1, len(values)))(*values), len(values)


def _host_bytes(flat: Any, shape: Shape) -> np.ndarray:
    """Flat host data as a contiguous array in the storage dtype of `shape`."""
    want = shape.dtype.numpy_storage()
    arr = np.ascontiguousarray(np.asarray(flat))
    if arr.dtype != want:
        if shape.dtype in (DType.BFloat16, DType.Int4, DType.Uint4) and arr.dtype.kind == "f":
            raise ComputeError(_lib.MX_ERR_INVALID,
                               f"{shape.dtype} data must be given as {want} storage, got {arr.dtype}")
        arr = arr.astype(want)
    if arr.nbytes != shape.byte_size():
        raise ComputeError(_lib.MX_ERR_INVALID,
                           f"flat data has {arr.nbytes} bytes, shape {shape} needs {shape.byte_size()}")
    return arr


# ---------------------------------------------------------------------------------------------
# Backend.
# ---------------------------------------------------------------------------------------------
class Backend:
    """compute.Backend for the "mi355x" backend."""

    def __init__(self, config: str = ""):
        self._lib = _lib.load()
        h = C.c_void_p()
        _check(self._lib.mx_backend_new(config.encode(), C.byref(h)))
        self._h = h

    # -- identity -------------------------------------------------------------------------
    def _str(self, fn, *args) -> str:
        buf = C.create_string_buffer(512)
        _check(fn(self._h, *args, buf, len(buf)))
        return buf.value.decode()

    def Name(self) -> str:
        return self._str(self._lib.mx_backend_name)

    def String(self) -> str:
        return self.Name()

    def Description(self) -> str:
        return self._str(self._lib.mx_backend_description)

    def NumDevices(self) -> int:
        n = C.c_int()
        _check(self._lib.mx_backend_num_devices(self._h, C.byref(n)))
        return n.value

    def DeviceDescription(self, device: int = 0) -> str:
        return self._str(self._lib.mx_backend_device_description, device)

    def Capabilities(self) -> Capabilities:
        ops, dts = {}, {}
        v = C.c_int()
        for op in OpType:
            _check(self._lib.mx_backend_supports_op(self._h, int(op), C.byref(v)))
            if v.value:
                ops[op] = True
        for dt in DType:
            _check(self._lib.mx_backend_supports_dtype(self._h, int(dt), C.byref(v)))
            if v.value:
                dts[dt] = True
        return Capabilities(Operations=ops, DTypes=dts)

    def HasSharedBuffers(self) -> bool:
        v = C.c_int()
        _check(self._lib.mx_backend_has_shared_buffers(self._h, C.byref(v)))
        return bool(v.value)

    # -- lifecycle ------------------------------------------------------------------------
    def Finalize(self) -> None:
        _check(self._lib.mx_backend_finalize(self._h))

    def IsFinalized(self) -> bool:
        return bool(self._lib.mx_backend_is_finalized(self._h))

    def Synchronize(self) -> None:
        _check(self._lib.mx_backend_synchronize(self._h))

    # -- data -----------------------------------------------------------------------------
    def BufferFromFlatData(self, device: int, flat: Any, shape: Shape) -> "Buffer":
        arr = _host_bytes(flat, shape)
        cs = _to_c_shape(shape)
        h = C.c_void_p()
        _check(self._lib.mx_buffer_from_flat(self._h, device, arr.ctypes.data_as(C.c_void_p), arr.nbytes,
                                             C.byref(cs), C.byref(h)))
        return Buffer(self, h)

    # -- graphs ---------------------------------------------------------------------------
    def Builder(self, name: str) -> "Builder":
        h = C.c_void_p()
        _check(self._lib.mx_builder_new(self._h, name.encode(), C.byref(h)))
        return Builder(self, h, name)

    # -- direct kernel entry point ----------------------------------------------------------
    def QDense(self, args: _lib.mx_qdense_args) -> None:
        _check(self._lib.mx_qdense(self._h, C.byref(args)))

    def QDenseNoAlloc(self, args: _lib.mx_qdense_args) -> None:
        """mx_qdense without device allocation (split-K scratch from a static per-GPU array)."""
        _check(self._lib.mx_qdense_noalloc(self._h, C.byref(args)))

    def QDensePlan(self, args: _lib.mx_qdense_args) -> str:
        buf = C.create_string_buffer(128)
        _check(self._lib.mx_qdense_plan(self._h, C.byref(args), buf, len(buf)))
        return buf.value.decode()

    def QEmbed(self, args: _lib.mx_qembed_args) -> None:
        _check(self._lib.mx_quantized_embedding_lookup(self._h, C.byref(args)))

    # -- profiling / debugging ------------------------------------------------------------
    def SetProfiling(self, enabled: bool) -> None:
        _check(self._lib.mx_backend_set_profiling(self._h, int(bool(enabled))))

    def Profile(self) -> dict:
        """{kernel name: (launches, total_ms)} of the launches timed since the last reset."""
        n = C.c_int()
        _check(self._lib.mx_backend_profile_count(self._h, C.byref(n)))
        out = {}
        name = C.create_string_buffer(256)
        launches = C.c_int64()
        total = C.c_double()
        for i in range(n.value):
            _check(self._lib.mx_backend_profile_entry(self._h, i, name, len(name), C.byref(launches), C.byref(total)))
            out[name.value.decode()] = (launches.value, total.value)
        return out

    def ProfileReset(self) -> None:
        _check(self._lib.mx_backend_profile_reset(self._h))

    def DebugFailAllocAfter(self, n: int) -> None:
        _check(self._lib.mx_backend_debug_fail_alloc_after(self._h, n))

    def RegionBegin(self) -> None:
        """Records the start event of a timed stretch of queued work on the backend's stream."""
        _check(self._lib.mx_backend_region_begin(self._h))

    def RegionEnd(self) -> float:
        """Records the end event, waits for it; returns the device milliseconds since RegionBegin."""
        ms = C.c_double()
        _check(self._lib.mx_backend_region_end(self._h, C.byref(ms)))
        return ms.value

    def DebugStreamRead(self, bufs, passes: int, workgroups: int = 0) -> None:
        """Queues `passes` read-only passes, pass i over bufs[i % len(bufs)] (HBM streaming floor)."""
        arr = (C.c_void_p * len(bufs))(*[b._h for b in bufs])
        _check(self._lib.mx_backend_debug_stream_read(self._h, arr, len(bufs), int(passes), int(workgroups)))

    def DebugNoAllocScratch(self) -> int:
        """Device address of the static array mx_qdense_noalloc uses on this backend's GPU."""
        p = C.c_void_p()
        _check(self._lib.mx_backend_debug_noalloc_scratch(self._h, C.byref(p)))
        return int(p.value or 0)

    def __repr__(self) -> str:
        return f"Backend({self.Name()!r})"


def New(config: str = "") -> Backend:
    """compute.NewWithConfig for this backend ("mi355x[:config]" or just the config)."""
    if config.startswith("mi355x"):
        config = config[len("mi355x"):].lstrip(":")
    return Backend(config)


# ---------------------------------------------------------------------------------------------
# Buffer.
# ---------------------------------------------------------------------------------------------
class Buffer:
    """compute.Buffer: device-resident storage."""

    def __init__(self, backend: Backend, handle: C.c_void_p):
        self._backend = backend
        self._lib = backend._lib
        self._h = handle

    def Backend(self) -> Backend:
        return self._backend

    def Shape(self) -> Shape:
        s = _lib.mx_shape()
        _check(self._lib.mx_buffer_shape(self._h, C.byref(s)))
        return _from_c_shape(s)

    def DeviceNum(self) -> int:
        v = C.c_int()
        _check(self._lib.mx_buffer_device(self._h, C.byref(v)))
        return v.value

    def ToFlatData(self, flat: Optional[np.ndarray] = None) -> np.ndarray:
        """Copies the buffer into `flat` (or a new array of the storage dtype) and returns it."""
        shape = self.Shape()
        if flat is None:
            n = shape.byte_size() // max(1, shape.dtype.numpy_storage().itemsize) if shape.dtype.is_packed() \
                else shape.size()
            flat = np.empty(n, dtype=shape.dtype.numpy_storage())
        if not flat.flags.c_contiguous:
            raise ComputeError(_lib.MX_ERR_INVALID, "ToFlatData: destination must be contiguous")
        _check(self._lib.mx_buffer_to_flat(self._h, flat.ctypes.data_as(C.c_void_p), flat.nbytes))
        return flat

    def DevicePtr(self) -> int:
        p = C.c_void_p()
        _check(self._lib.mx_buffer_device_ptr(self._h, C.byref(p)))
        return p.value or 0

    def Finalize(self) -> None:
        _check(self._lib.mx_buffer_finalize(self._h))

    def __del__(self):
        try:
            if self._h and not self._backend.IsFinalized():
                self._lib.mx_buffer_destroy(self._h)
            self._h = None
        except Exception:
            pass


# ---------------------------------------------------------------------------------------------
# Builder / Function.
# ---------------------------------------------------------------------------------------------
class Value(int):
    """compute.Value: opaque handle of a graph value."""


class Builder:
    def __init__(self, backend: Backend, handle: C.c_void_p, name: str):
        self._backend = backend
        self._lib = backend._lib
        self._h = handle
        self._name = name
        self._main: Optional[Function] = None
        self._compiled = False

    def Name(self) -> str:
        return self._name

    def Main(self) -> "Function":
        if self._main is None:
            h = C.c_void_p()
            _check(self._lib.mx_builder_main(self._h, C.byref(h)))
            self._main = Function(self, h)
        return self._main

    def NewFunction(self, name: str):
        raise ErrNotImplemented(_lib.MX_ERR_NOT_IMPLEMENTED, "NewFunction: sub-functions are not supported")

    def OpShape(self, v: Value) -> Shape:
        s = _lib.mx_shape()
        _check(self._lib.mx_builder_op_shape(self._h, int(v), C.byref(s)))
        return _from_c_shape(s)

    def Compile(self) -> "Executable":
        h = C.c_void_p()
        self._compiled = True
        _check(self._lib.mx_builder_compile(self._h, C.byref(h)))
        return Executable(self._backend, h)

    def __del__(self):
        try:
            if self._h is not None:
                self._lib.mx_builder_destroy(self._h)
                self._h = None
        except Exception:
            pass


class Function:
    """compute.Function: StandardOps subset + FusedOps used by the quantized-dense path."""

    def __init__(self, builder: Builder, handle: C.c_void_p):
        self._builder = builder
        self._lib = builder._lib
        self._h = handle

    def _out(self, fn, *args) -> Value:
        v = C.c_uint64()
        _check(fn(self._h, *args, C.byref(v)))
        return Value(v.value)

    def Name(self) -> str:
        return "main"

    def Builder(self) -> Builder:
        return self._builder

    def Parameter(self, name: str, shape: Shape, sharding=None) -> Value:
        if sharding is not None:
            raise ErrNotImplemented(_lib.MX_ERR_NOT_IMPLEMENTED, "Parameter: sharding is not supported")
        cs = _to_c_shape(shape)
        return self._out(self._lib.mx_fn_parameter, name.encode(), C.byref(cs))

    def Constant(self, flat: Any, *dims: int, dtype: Optional[DType] = None) -> Value:
        arr = np.asarray(flat)
        if dtype is None:
            dtype = _dtype_of_numpy(arr.dtype)
        if not dims:
            dims = arr.shape
        shape = Shape(dtype, *dims)
        data = _host_bytes(arr.ravel(), shape)
        cs = _to_c_shape(shape)
        return self._out(self._lib.mx_fn_constant, data.ctypes.data_as(C.c_void_p), data.nbytes, C.byref(cs))

    def Shape(self, v: Value) -> Shape:
        s = _lib.mx_shape()
        _check(self._lib.mx_fn_shape(self._h, int(v), C.byref(s)))
        return _from_c_shape(s)

    def Return(self, outputs: Sequence[Value], shardings=None) -> None:
        arr = (C.c_uint64 * len(outputs))(*[int(o) for o in outputs])
        _check(self._lib.mx_fn_return(self._h, arr, len(outputs)))

    def Closure(self):
        raise ErrNotImplemented(_lib.MX_ERR_NOT_IMPLEMENTED, "Closure: not supported")

    # -- fused ops ------------------------------------------------------------------------
    def FusedQuantizedDense(self, x: Value, weights: Value, bias: Optional[Value],
                            weightsQuantization: Quantization, activation: ActivationType) -> Value:
        q = weightsQuantization
        cq = _lib.mx_quantization(int(q.Scheme), int(q.Scale or 0), int(q.ZeroPoint or 0), int(q.BlockAxis),
                                  int(q.BlockSize), int(q.GGMLType))
        return self._out(self._lib.mx_fn_fused_quantized_dense, int(x), int(weights), int(bias or 0), C.byref(cq),
                         int(activation))

    def QuantizedEmbeddingLookup(self, data: Value, indices: Value, dataQuantization: Quantization) -> Value:
        q = dataQuantization
        if q is None:
            raise ComputeError(_lib.MX_ERR_INVALID, "QuantizedEmbeddingLookup: quantization is nil")
        cq = _lib.mx_quantization(int(q.Scheme), int(q.Scale or 0), int(q.ZeroPoint or 0), int(q.BlockAxis),
                                  int(q.BlockSize), int(q.GGMLType))
        return self._out(self._lib.mx_fn_quantized_embedding_lookup, int(data), int(indices), C.byref(cq))

    def FusedDense(self, x: Value, weight: Value, bias: Optional[Value], options: DenseConfig = None) -> Value:
        o = options if options is not None else DenseConfig()
        cfg = _lib.mx_dense_config(int(o.Activation), int(o.WeightLayout))
        return self._out(self._lib.mx_fn_fused_dense, int(x), int(weight), int(bias or 0), C.byref(cfg))

    def FusedGelu(self, x: Value, exact: bool) -> Value:
        return self._out(self._lib.mx_fn_fused_gelu, int(x), int(bool(exact)))

    # -- standard ops ---------------------------------------------------------------------
    def DotGeneral(self, lhs: Value, lhsContractingAxes, lhsBatchAxes, rhs: Value, rhsContractingAxes,
                   rhsBatchAxes, config: Optional[DotGeneralConfig] = None) -> Value:
        config = config or DotGeneralConfig()
        lc, nlc = _i32(lhsContractingAxes)
        lb, nlb = _i32(lhsBatchAxes)
        rc, nrc = _i32(rhsContractingAxes)
        rb, nrb = _i32(rhsBatchAxes)
        return self._out(self._lib.mx_fn_dot_general, int(lhs), lc, nlc, lb, nlb, int(rhs), rc, nrc, rb, nrb,
                         int(config.AccumulatorDType), int(config.OutputDType))

    def _unary(self, op: OpType, x: Value) -> Value:
        return self._out(self._lib.mx_fn_unary, int(op), int(x))

    def _binary(self, op: OpType, lhs: Value, rhs: Value) -> Value:
        return self._out(self._lib.mx_fn_binary, int(op), int(lhs), int(rhs))

    def Abs(self, x): return self._unary(OpType.Abs, x)
    def Neg(self, x): return self._unary(OpType.Neg, x)
    def Exp(self, x): return self._unary(OpType.Exp, x)
    def Erf(self, x): return self._unary(OpType.Erf, x)
    def Logistic(self, x): return self._unary(OpType.Logistic, x)
    def Rsqrt(self, x): return self._unary(OpType.Rsqrt, x)
    def Sqrt(self, x): return self._unary(OpType.Sqrt, x)
    def Tanh(self, x): return self._unary(OpType.Tanh, x)
    def Identity(self, x): return self._unary(OpType.Identity, x)
    def Add(self, lhs, rhs): return self._binary(OpType.Add, lhs, rhs)
    def Sub(self, lhs, rhs): return self._binary(OpType.Sub, lhs, rhs)
    def Mul(self, lhs, rhs): return self._binary(OpType.Mul, lhs, rhs)
    def Div(self, lhs, rhs): return self._binary(OpType.Div, lhs, rhs)
    def Max(self, lhs, rhs): return self._binary(OpType.Max, lhs, rhs)
    def Min(self, lhs, rhs): return self._binary(OpType.Min, lhs, rhs)

    def ConvertDType(self, x: Value, dtype: DType) -> Value:
        return self._out(self._lib.mx_fn_convert_dtype, int(x), int(dtype))

    def Reshape(self, x: Value, *dims: int) -> Value:
        d, n = _i64(dims)
        return self._out(self._lib.mx_fn_reshape, int(x), d, n)

    def Bitcast(self, x: Value, targetDType: DType) -> Value:
        return self._out(self._lib.mx_fn_bitcast, int(x), int(targetDType))

    def BroadcastInDim(self, x: Value, outputShape: Shape, broadcastAxes: Sequence[int]) -> Value:
        cs = _to_c_shape(outputShape)
        a, n = _i32(broadcastAxes)
        return self._out(self._lib.mx_fn_broadcast_in_dim, int(x), C.byref(cs), a, n)

    def ReduceSum(self, x: Value, *axes: int) -> Value:
        a, n = _i32(axes)
        return self._out(self._lib.mx_fn_reduce, int(OpType.ReduceSum), int(x), a, n)

    def ReduceMax(self, x: Value, *axes: int) -> Value:
        a, n = _i32(axes)
        return self._out(self._lib.mx_fn_reduce, int(OpType.ReduceMax), int(x), a, n)

    def Transpose(self, x: Value, *permutation: int) -> Value:
        p, n = _i32(permutation)
        return self._out(self._lib.mx_fn_transpose, int(x), p, n)

    def Iota(self, shape: Shape, iotaAxis: int) -> Value:
        cs = _to_c_shape(shape)
        return self._out(self._lib.mx_fn_iota, C.byref(cs), int(iotaAxis))

    def Slice(self, x: Value, starts: Sequence[int], limits: Sequence[int], strides: Optional[Sequence[int]] = None) -> Value:
        s, n = _i64(starts)
        lm, _ = _i64(limits)
        st = _i64(strides)[0] if strides else None
        return self._out(self._lib.mx_fn_slice, int(x), s, lm, st, n)


def _dtype_of_numpy(dt: np.dtype) -> DType:
    table = {
        np.dtype(np.float32): DType.Float32, np.dtype(np.float64): DType.Float64,
        np.dtype(np.float16): DType.Float16, np.dtype(np.int8): DType.Int8, np.dtype(np.int16): DType.Int16,
        np.dtype(np.int32): DType.Int32, np.dtype(np.int64): DType.Int64, np.dtype(np.uint8): DType.Uint8,
        np.dtype(np.uint16): DType.Uint16, np.dtype(np.uint32): DType.Uint32, np.dtype(np.uint64): DType.Uint64,
        np.dtype(np.bool_): DType.Bool,
    }
    if dt not in table:
        raise ComputeError(_lib.MX_ERR_INVALID, f"unsupported numpy dtype {dt}")
    return table[dt]


# ---------------------------------------------------------------------------------------------
# Executable.
# ---------------------------------------------------------------------------------------------
class Executable:
    def __init__(self, backend: Backend, handle: C.c_void_p):
        self._backend = backend
        self._lib = backend._lib
        self._h = handle
        n = C.c_int()
        _check(self._lib.mx_exec_num_outputs(self._h, C.byref(n)))
        self._nout = n.value
        _check(self._lib.mx_exec_num_inputs(self._h, C.byref(n)))
        self._nin = n.value

    def Inputs(self):
        names, shapes = [], []
        for i in range(self._nin):
            buf = C.create_string_buffer(256)
            s = _lib.mx_shape()
            _check(self._lib.mx_exec_input(self._h, i, buf, len(buf), C.byref(s)))
            names.append(buf.value.decode())
            shapes.append(_from_c_shape(s))
        return names, shapes

    def Outputs(self):
        out = []
        for i in range(self._nout):
            s = _lib.mx_shape()
            _check(self._lib.mx_exec_output(self._h, i, C.byref(s)))
            out.append(_from_c_shape(s))
        return out

    def Describe(self) -> list:
        """The operations Execute runs, in order, after compile-time fusion (mx_exec_describe)."""
        buf = C.create_string_buffer(1 << 16)
        _check(self._lib.mx_exec_describe(self._h, buf, len(buf)))
        return [l for l in buf.value.decode().split("\n") if l]

    def Execute(self, inputs: Sequence[Buffer], donate: Optional[Sequence[bool]] = None, defaultDevice: int = 0):
        n = len(inputs)
        arr = (C.c_void_p * max(1, n))(*[b._h.value if b is not None else None for b in inputs])
        don = None
        if donate:
            don = (C.c_uint8 * max(1, n))(*[1 if d else 0 for d in donate])
        outs = (C.c_void_p * max(1, self._nout))()
        _check(self._lib.mx_exec_execute(self._h, arr, don, n, outs, self._nout))
        return [Buffer(self._backend, C.c_void_p(outs[i])) for i in range(self._nout)]

    def LoopSets(self, input_sets: Sequence[Sequence[Buffer]]):
        """The input sets of ExecuteLoop marshalled once for the library call (a caller timing the
        loop prepares them outside its timed region)."""
        flat = [b._h.value for s in input_sets for b in s]
        return (C.c_void_p * max(1, len(flat)))(*flat), len(input_sets)

    def ExecuteLoop(self, input_sets, iters: int) -> None:
        """Runs Execute `iters` times over rotating input sets, discarding outputs, in one call
        into the library (no per-iteration foreign-call overhead).  input_sets: a sequence of input
        sets, or what LoopSets returned for them."""
        arr, n = input_sets if isinstance(input_sets, tuple) else self.LoopSets(input_sets)
        _check(self._lib.mx_exec_execute_loop(self._h, arr, n, self._nin, int(iters)))

    def Finalize(self) -> None:
        if self._h is not None:
            _check(self._lib.mx_exec_finalize(self._h))
            self._h = None

    def __del__(self):
        try:
            if self._h is not None and not self._backend.IsFinalized():
                self._lib.mx_exec_finalize(self._h)
            self._h = None
        except Exception:
            pass
