"""Intent scalar element types (reference: `python/intent/language/dtypes.py`).

A dtype is a (name, category, bit width) triple; the names are the ABI names
used in public interfaces ("f32", "bf16", ...)."""
from __future__ import annotations

import builtins as _py
from dataclasses import dataclass
from enum import Enum


class DTypeCategory(Enum):
    BOOL = "bool"
    SIGNED_INTEGER = "signed_integer"
    UNSIGNED_INTEGER = "unsigned_integer"
    INDEX = "index"
    FLOAT = "float"
    BFLOAT = "bfloat"


@dataclass(frozen=True, slots=True)
class DType:
    name: str
    category: DTypeCategory
    bits: int | None

    def __post_init__(self) -> None:
        if not self.name:
            raise ValueError("dtype name must not be empty")
        if not isinstance(self.category, DTypeCategory):
            raise TypeError("dtype category must be a DTypeCategory")
        if isinstance(self.bits, _py.bool) or (self.bits is not None and not isinstance(self.bits, _py.int)):
            raise TypeError("dtype bit width must be an integer or None")
        if self.bits is not None and self.bits <= 0:
            raise ValueError("dtype bit width must be positive")
        if self.category is DTypeCategory.INDEX and self.bits != 64:
            raise ValueError("logical index dtype must be signed 64-bit")

    @property
    def itemsize(self) -> int:
        return max(1, (self.bits + 7) // 8)

    def __repr__(self) -> str:
        return f"I.{self.name}"


_C = DTypeCategory
bool = DType("bool", _C.BOOL, 1)
index = DType("index", _C.INDEX, 64)
i8, i16, i32, i64 = (DType(f"i{w}", _C.SIGNED_INTEGER, w) for w in (8, 16, 32, 64))
u8, u16, u32, u64 = (DType(f"u{w}", _C.UNSIGNED_INTEGER, w) for w in (8, 16, 32, 64))
f8e4m3fn = DType("f8e4m3fn", _C.FLOAT, 8)
f8e5m2 = DType("f8e5m2", _C.FLOAT, 8)
f16 = DType("f16", _C.FLOAT, 16)
bf16 = DType("bf16", _C.BFLOAT, 16)
f32 = DType("f32", _C.FLOAT, 32)
f64 = DType("f64", _C.FLOAT, 64)

DTYPES = {d.name: d for d in (bool, index, i8, i16, i32, i64, u8, u16, u32, u64,
                              f8e4m3fn, f8e5m2, f16, bf16, f32, f64)}


def dtype(name: str) -> DType:
    return DTYPES[name]
