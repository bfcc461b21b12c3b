"""View/scalar/constexpr annotations of kernel parameters.

Same surface and validation rules as the reference's
`python/intent/language/annotations.py`: `I.In/Out/InOut[dtype, shape, constraints]`,
`I.constraints(strides=, alias=, noalias=)`, `I.Constexpr[type]`, `I.Enum`.
Shapes mix static extents (non-negative ints) and symbolic names (identifiers);
one symbol names one logical dimension across all parameters of a kernel."""
from __future__ import annotations

import builtins as _py
from dataclasses import dataclass
from enum import Enum as _PyEnum
from enum import IntEnum
from typing import Any

from .dtypes import DType

ShapeDim = int | str
StrideDim = int | str | None


def _shape(shape: object) -> tuple[ShapeDim, ...]:
    if not isinstance(shape, (tuple, list)):
        raise TypeError("tensor shape annotation must be a tuple or list")
    out: list[ShapeDim] = []
    for dim in shape:
        if isinstance(dim, _py.bool):
            raise TypeError("boolean is not a tensor shape dimension")
        if isinstance(dim, int):
            if dim < 0:
                raise ValueError("static tensor dimensions must be non-negative")
        elif isinstance(dim, str):
            if not dim.isidentifier():
                raise ValueError(f"invalid symbolic dimension: {dim!r}")
        else:
            raise TypeError(f"unsupported tensor shape dimension: {dim!r}")
        out.append(dim)
    return tuple(out)


@dataclass(frozen=True, slots=True)
class ViewConstraints:
    strides: tuple[StrideDim, ...] | None = None
    alias: str | None = None
    noalias: bool = False

    def __post_init__(self) -> None:
        if self.strides is not None:
            strides = tuple(self.strides)
            for stride in strides:
                if stride is None or (isinstance(stride, int) and not isinstance(stride, _py.bool)):
                    continue
                if isinstance(stride, str) and stride.isidentifier():
                    continue
                raise TypeError(f"unsupported stride constraint: {stride!r}")
            object.__setattr__(self, "strides", strides)
        if self.alias is not None and not self.alias:
            raise ValueError("alias group must not be empty")
        if self.alias is not None and self.noalias:
            raise ValueError("alias and noalias cannot be specified together")


def constraints(*, strides=None, alias=None, noalias=False) -> ViewConstraints:
    return ViewConstraints(strides=strides, alias=alias, noalias=noalias)


class ViewKind(IntEnum):
    IN = 0
    OUT = 1
    INOUT = 2


@dataclass(frozen=True, slots=True)
class ViewSpec:
    kind: ViewKind
    dtype: DType
    shape: tuple[ShapeDim, ...]
    constraints: ViewConstraints

    def __post_init__(self) -> None:
        if not isinstance(self.kind, ViewKind):
            raise TypeError("view kind must be a ViewKind")
        if not isinstance(self.dtype, DType):
            raise TypeError("view element type must be an Intent dtype")
        if not isinstance(self.constraints, ViewConstraints):
            raise TypeError("view constraints must be a ViewConstraints")
        object.__setattr__(self, "shape", _shape(self.shape))
        if self.constraints.strides is not None and len(self.constraints.strides) != len(self.shape):
            raise ValueError("stride constraint rank must match tensor rank")


class _View:
    kind: ViewKind

    def __class_getitem__(cls, parameters: object) -> ViewSpec:
        if not isinstance(parameters, tuple) or len(parameters) not in (2, 3):
            raise TypeError("view annotation expects dtype, shape, and optional constraints")
        extra = parameters[2] if len(parameters) == 3 else ViewConstraints()
        if not isinstance(extra, ViewConstraints):
            raise TypeError("third view annotation argument must be I.constraints(...)")
        return ViewSpec(cls.kind, parameters[0], _shape(parameters[1]), extra)


class In(_View):
    kind = ViewKind.IN


class Out(_View):
    """Output view; its incoming elements are undefined."""
    kind = ViewKind.OUT


class InOut(_View):
    kind = ViewKind.INOUT


@dataclass(frozen=True, slots=True)
class ConstexprSpec:
    value_type: Any


class Constexpr:
    def __class_getitem__(cls, value_type: Any) -> ConstexprSpec:
        if value_type is None:
            raise TypeError("Constexpr requires a value type")
        return ConstexprSpec(value_type)


class Enum(_PyEnum):
    """Base class for author specialization enums (constexpr-only)."""
