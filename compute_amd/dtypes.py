"""DTypes and shapes of the backend API.

DType values equal the reference's dtypes.DType enum (dtypes/dtype_enum.go:20-140) so they pass
through the C ABI unchanged.  Host data for BFloat16 is carried as numpy uint16 bit patterns;
packed Int4/Uint4 data as numpy uint8 bytes in the reference packing (two values per byte, low
nibble first: dtypes/dtypes.go:190-239).
"""
from __future__ import annotations

import enum
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np


class DType(enum.IntEnum):
    InvalidDType = 0
    Bool = 1
    Int8 = 2
    Int16 = 3
    Int32 = 4
    Int64 = 5
    Uint8 = 6
    Uint16 = 7
    Uint32 = 8
    Uint64 = 9
    Float16 = 10
    Float32 = 11
    Float64 = 12
    BFloat16 = 13
    Int4 = 21
    Uint4 = 22

    def __str__(self) -> str:  # matches the reference's enumer names
        return self.name

    @property
    def bits(self) -> int:
        """Bits per value (dtypes.go:175-189)."""
        return _BITS[self]

    def is_packed(self) -> bool:
        return self.bits < 8

    def is_float(self) -> bool:
        return self in (DType.Float16, DType.Float32, DType.Float64, DType.BFloat16)

    def is_half_precision(self) -> bool:
        return self in (DType.Float16, DType.BFloat16)

    def numpy_storage(self) -> np.dtype:
        """numpy dtype of the flat host storage for this DType."""
        return _NP[self]

    def size_for_dimensions(self, *dims: int) -> int:
        """Storage bytes (dtypes.go:221-239): packed types round up to whole bytes."""
        n = 1
        for d in dims:
            if d < 0:
                raise ValueError(f"dim cannot be negative, got {dims}")
            n *= d
        return (n * self.bits + 7) // 8


_BITS = {
    DType.InvalidDType: 0, DType.Bool: 8, DType.Int8: 8, DType.Int16: 16, DType.Int32: 32,
    DType.Int64: 64, DType.Uint8: 8, DType.Uint16: 16, DType.Uint32: 32, DType.Uint64: 64,
    DType.Float16: 16, DType.Float32: 32, DType.Float64: 64, DType.BFloat16: 16, DType.Int4: 4,
    DType.Uint4: 4,
}

_NP = {
    DType.Bool: np.dtype(np.bool_), DType.Int8: np.dtype(np.int8), DType.Int16: np.dtype(np.int16),
    DType.Int32: np.dtype(np.int32), DType.Int64: np.dtype(np.int64), DType.Uint8: np.dtype(np.uint8),
    DType.Uint16: np.dtype(np.uint16), DType.Uint32: np.dtype(np.uint32), DType.Uint64: np.dtype(np.uint64),
    DType.Float16: np.dtype(np.float16), DType.Float32: np.dtype(np.float32),
    DType.Float64: np.dtype(np.float64), DType.BFloat16: np.dtype(np.uint16),
    DType.Int4: np.dtype(np.uint8), DType.Uint4: np.dtype(np.uint8),
}

# Re-exported names, as the reference's `dtypes.X`.
InvalidDType, Bool, Int8, Int16, Int32, Int64 = (DType.InvalidDType, DType.Bool, DType.Int8, DType.Int16,
                                                 DType.Int32, DType.Int64)
Uint8, Uint16, Uint32, Uint64 = DType.Uint8, DType.Uint16, DType.Uint32, DType.Uint64
Float16, Float32, Float64, BFloat16, Int4, Uint4 = (DType.Float16, DType.Float32, DType.Float64, DType.BFloat16,
                                                    DType.Int4, DType.Uint4)


@dataclass(frozen=True)
class Shape:
    """shapes.Shape{DType, Dimensions} (shapes/shapes.go:68-84), static dimensions only."""

    dtype: DType
    dimensions: tuple = field(default_factory=tuple)

    def __init__(self, dtype: DType, *dims: int):
        if len(dims) == 1 and isinstance(dims[0], (list, tuple)):
            dims = tuple(dims[0])
        object.__setattr__(self, "dtype", DType(dtype))
        object.__setattr__(self, "dimensions", tuple(int(d) for d in dims))

    def rank(self) -> int:
        return len(self.dimensions)

    def size(self) -> int:
        n = 1
        for d in self.dimensions:
            n *= d
        return n

    def byte_size(self) -> int:
        return self.dtype.size_for_dimensions(*self.dimensions)

    def is_scalar(self) -> bool:
        return not self.dimensions

    def __repr__(self) -> str:
        if not self.dimensions:
            return f"({self.dtype})"
        return f"({self.dtype})[{' '.join(map(str, self.dimensions))}]"


def make(dtype: DType, *dims: int) -> Shape:
    """shapes.Make."""
    return Shape(dtype, *dims)


# ------------------------------------------------------------------------------------------
# bf16 host helpers (bit patterns in uint16).
# ------------------------------------------------------------------------------------------
def bf16_from_f32(x) -> np.ndarray:
    """float32 -> bfloat16 bits with round-to-nearest-even; NaN/Inf keep their top 16 bits
    (bfloat16.FromFloat32, dtypes/bfloat16/bfloat16.go:30-39)."""
    b = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    special = (b & 0x7F800000) == 0x7F800000
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    out = np.where(special, b >> 16, rounded) & 0xFFFF
    return out.astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    """bfloat16 bits -> float32 (exact)."""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_int4(values: Sequence[int] | np.ndarray) -> np.ndarray:
    """Packs signed/unsigned 4-bit values (flat) into bytes: element i goes to byte i//2, low
    nibble when i is even (the reference packing)."""
    v = np.asarray(values).astype(np.int64).ravel() & 0xF
    if v.size % 2:
        v = np.concatenate([v, np.zeros(1, np.int64)])
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray, n: int, signed: bool = True) -> np.ndarray:
    """Inverse of pack_int4 for the first n values."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.size * 2, dtype=np.int8)
    lo = (p & 0xF).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    if signed:
        lo = np.where(lo >= 8, lo - 16, lo).astype(np.int8)
        hi = np.where(hi >= 8, hi - 16, hi).astype(np.int8)
    out[0::2] = lo
    out[1::2] = hi
    return out[:n]
