"""ctypes binding of libmxrt.so (declared in include/mxrt.h).

The library is the product: this module only declares its C signatures.  Importing it fails
loudly when the library has not been built; nothing here computes on the host.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libmxrt.so"

MX_OK = 0
MX_ERR_INVALID = -1
MX_ERR_NOT_IMPLEMENTED = -2
MX_ERR_HIP = -3
MX_ERR_OUT_OF_MEMORY = -4
MX_ERR_FINALIZED = -5
MX_ERR_NO_DEVICE = -6

MX_MAX_RANK = 8
MX_QDENSE_NOALLOC_SCRATCH_BYTES = 16 << 20  # mxrt.h: the static per-GPU scratch of mx_qdense_noalloc


class mx_shape(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("rank", C.c_int32), ("dims", C.c_int64 * MX_MAX_RANK)]


class mx_quantization(C.Structure):
    _fields_ = [
        ("scheme", C.c_int32),
        ("scale", C.c_uint64),
        ("zero_point", C.c_uint64),
        ("block_axis", C.c_int32),
        ("block_size", C.c_int32),
        ("ggml_type", C.c_int32),
    ]


class mx_dense_config(C.Structure):
    _fields_ = [("activation", C.c_int32), ("weight_layout", C.c_int32)]


class mx_qdense_args(C.Structure):
    _fields_ = [
        ("x", C.c_void_p),
        ("w", C.c_void_p),
        ("scale", C.c_void_p),
        ("zero_point", C.c_void_p),
        ("bias", C.c_void_p),
        ("out", C.c_void_p),
        ("M", C.c_int64),
        ("K", C.c_int64),
        ("N", C.c_int64),
        ("x_dtype", C.c_int32),
        ("w_dtype", C.c_int32),
        ("scale_dtype", C.c_int32),
        ("zero_point_dtype", C.c_int32),
        ("bias_dtype", C.c_int32),
        ("scheme", C.c_int32),
        ("block_axis", C.c_int32),
        ("block_size", C.c_int32),
        ("activation", C.c_int32),
        ("ggml_type", C.c_int32),
    ]


class mx_qembed_args(C.Structure):
    _fields_ = [
        ("data", C.c_void_p),
        ("indices", C.c_void_p),
        ("out", C.c_void_p),
        ("vocab", C.c_int64),
        ("bytes_per_row", C.c_int64),
        ("n", C.c_int64),
        ("index_dtype", C.c_int32),
        ("ggml_type", C.c_int32),
    ]


_P = C.c_void_p
_I = C.c_int
_I32P = C.POINTER(C.c_int32)
_I64P = C.POINTER(C.c_int64)
_VAL = C.c_uint64
_VALP = C.POINTER(C.c_uint64)
_SHP = C.POINTER(mx_shape)
_SZ = C.c_size_t

# name -> argtypes (every function returns int status unless listed in _RESTYPES).
SIGNATURES = {
    "mx_last_error": [],
    "mx_backend_new": [C.c_char_p, C.POINTER(_P)],
    "mx_backend_finalize": [_P],
    "mx_backend_is_finalized": [_P],
    "mx_backend_name": [_P, C.c_char_p, _SZ],
    "mx_backend_description": [_P, C.c_char_p, _SZ],
    "mx_backend_num_devices": [_P, C.POINTER(_I)],
    "mx_backend_device_description": [_P, _I, C.c_char_p, _SZ],
    "mx_backend_supports_op": [_P, _I, C.POINTER(_I)],
    "mx_backend_supports_dtype": [_P, _I, C.POINTER(_I)],
    "mx_backend_synchronize": [_P],
    "mx_backend_set_profiling": [_P, _I],
    "mx_backend_profile_count": [_P, C.POINTER(_I)],
    "mx_backend_profile_entry": [_P, _I, C.c_char_p, _SZ, _I64P, C.POINTER(C.c_double)],
    "mx_backend_profile_reset": [_P],
    "mx_backend_debug_fail_alloc_after": [_P, _I],
    "mx_backend_debug_noalloc_scratch": [_P, C.POINTER(_P)],
    "mx_backend_debug_stream_read": [_P, C.POINTER(_P), _I, _I, _I],
    "mx_backend_region_begin": [_P],
    "mx_backend_region_end": [_P, C.POINTER(C.c_double)],
    "mx_backend_has_shared_buffers": [_P, C.POINTER(_I)],
    "mx_buffer_from_flat": [_P, _I, _P, _SZ, _SHP, C.POINTER(_P)],
    "mx_buffer_to_flat": [_P, _P, _SZ],
    "mx_buffer_shape": [_P, _SHP],
    "mx_buffer_device": [_P, C.POINTER(_I)],
    "mx_buffer_nbytes": [_P, C.POINTER(_SZ)],
    "mx_buffer_device_ptr": [_P, C.POINTER(_P)],
    "mx_buffer_finalize": [_P],
    "mx_buffer_destroy": [_P],
    "mx_builder_new": [_P, C.c_char_p, C.POINTER(_P)],
    "mx_builder_destroy": [_P],
    "mx_builder_main": [_P, C.POINTER(_P)],
    "mx_builder_op_shape": [_P, _VAL, _SHP],
    "mx_builder_compile": [_P, C.POINTER(_P)],
    "mx_fn_parameter": [_P, C.c_char_p, _SHP, _VALP],
    "mx_fn_constant": [_P, _P, _SZ, _SHP, _VALP],
    "mx_fn_shape": [_P, _VAL, _SHP],
    "mx_fn_return": [_P, _VALP, _I],
    "mx_fn_fused_quantized_dense": [_P, _VAL, _VAL, _VAL, C.POINTER(mx_quantization), _I, _VALP],
    "mx_fn_quantized_embedding_lookup": [_P, _VAL, _VAL, C.POINTER(mx_quantization), _VALP],
    "mx_fn_dot_general": [_P, _VAL, _I32P, _I, _I32P, _I, _VAL, _I32P, _I, _I32P, _I, _I, _I, _VALP],
    "mx_fn_fused_dense": [_P, _VAL, _VAL, _VAL, C.POINTER(mx_dense_config), _VALP],
    "mx_fn_fused_gelu": [_P, _VAL, _I, _VALP],
    "mx_fn_unary": [_P, _I, _VAL, _VALP],
    "mx_fn_binary": [_P, _I, _VAL, _VAL, _VALP],
    "mx_fn_convert_dtype": [_P, _VAL, _I, _VALP],
    "mx_fn_reshape": [_P, _VAL, _I64P, _I, _VALP],
    "mx_fn_bitcast": [_P, _VAL, _I, _VALP],
    "mx_fn_broadcast_in_dim": [_P, _VAL, _SHP, _I32P, _I, _VALP],
    "mx_fn_reduce": [_P, _I, _VAL, _I32P, _I, _VALP],
    "mx_fn_transpose": [_P, _VAL, _I32P, _I, _VALP],
    "mx_fn_iota": [_P, _SHP, _I, _VALP],
    "mx_fn_slice": [_P, _VAL, _I64P, _I64P, _I64P, _I, _VALP],
    "mx_exec_num_inputs": [_P, C.POINTER(_I)],
    "mx_exec_input": [_P, _I, C.c_char_p, _SZ, _SHP],
    "mx_exec_num_outputs": [_P, C.POINTER(_I)],
    "mx_exec_output": [_P, _I, _SHP],
    "mx_exec_execute": [_P, C.POINTER(_P), C.POINTER(C.c_uint8), _I, C.POINTER(_P), _I],
    "mx_exec_finalize": [_P],
    "mx_exec_execute_loop": [_P, C.POINTER(_P), _I, _I, _I],
    "mx_exec_describe": [_P, C.c_char_p, _SZ],
    "mx_qdense": [_P, C.POINTER(mx_qdense_args)],
    "mx_qdense_plan": [_P, C.POINTER(mx_qdense_args), C.c_char_p, _SZ],
    "mx_qdense_noalloc": [_P, C.POINTER(mx_qdense_args)],
    "mx_quantized_embedding_lookup": [_P, C.POINTER(mx_qembed_args)],
}

_RESTYPES = {"mx_last_error": C.c_char_p}

_lib = None


def load() -> C.CDLL:
    """Loads libmxrt.so (once).  Raises if it was not built: there is no fallback."""
    global _lib
    if _lib is not None:
        return _lib
    path = os.environ.get("MXRT_LIB", str(LIB_PATH))
    if not Path(path).exists():
        raise RuntimeError(
            f"libmxrt.so not found at {path}: build it with `python -m compute_amd.build` "
            "(or __graft_entry__.build()); the MI355X backend has no host fallback")
    lib = C.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, C.c_int)
    _lib = lib
    return lib
