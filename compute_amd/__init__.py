"""compute_amd — the MI355X-native `compute.Backend` ("mi355x") for the quantized-dense path.

The product is libmxrt.so (C ABI in include/mxrt.h, HIP kernels for gfx950 in csrc/); this
package is its host-side mirror of the reference's Go API (github.com/gomlx/compute).
"""
from .dtypes import (  # noqa: F401
    BFloat16, Bool, DType, Float16, Float32, Float64, Int4, Int8, Int16, Int32, Int64, InvalidDType, Shape,
    Uint4, Uint8, Uint16, Uint32, Uint64, bf16_from_f32, bf16_to_f32, make, pack_int4, unpack_int4,
)
from .backend import (  # noqa: F401
    ActivationGelu, ActivationHardSwish, ActivationNone, ActivationRelu, ActivationSilu, ActivationTanh,
    ActivationType, Backend, Buffer, Builder, Capabilities, ComputeError, DenseConfig, DenseLayout,
    DenseLayoutInputOutputs, DenseLayoutOutputsInput, DotGeneralConfig, ErrFinalized,
    ErrNoDevice, ErrNotImplemented, Executable, Function, IsNotImplemented, NF4LookupTable, New, OpType,
    QuantGGML, QuantLinear, QuantNF4, Quantization, QuantizationScheme, Value,
    GGMLQuantType, GGMLQ4_0, GGMLQ8_0, GGMLIQ4NL, GGMLQ2_K, GGMLQ3_K, GGMLQ4_K, GGMLQ5_K, GGMLQ6_K,
    IQ4NLLookupTable, ggml_bytes_per_block, ggml_values_per_block,
)

BackendName = "mi355x"
