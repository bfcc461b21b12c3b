"""`intent.language` as `I`: annotations, dtypes and intrinsic names."""
from .annotations import (Constexpr, ConstexprSpec, Enum, In, InOut, Out, ShapeDim, StrideDim,
                          ViewConstraints, ViewKind, ViewSpec, constraints)
from .builtins import *  # noqa: F401,F403
from .builtins import LOG2E, inf
from .dtypes import (DType, DTypeCategory, bf16, bool, dtype, f8e4m3fn, f8e5m2, f16, f32, f64,
                     i8, i16, i32, i64, index, u8, u16, u32, u64)
