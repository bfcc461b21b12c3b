"""Parameter annotations of kernel definitions.

A kernel parameter is annotated with one of:

* a view, `I.In[dtype, shape]`, `I.Out[...]` or `I.InOut[...]`, with an optional third item
  `I.constraints(strides=..., alias=..., noalias=...)`;
* a scalar, the bare dtype (`scale: I.f32`);
* a specialization value, `I.Constexpr[type]`, fixed when the kernel is jitted.

A shape lists extents: a non-negative int fixes an extent, and an identifier names a logical
dimension. Every view of a kernel that uses the same name shares that extent. A stride constraint
is an int, an identifier that names a stride shared by the views that use it, or None for an axis
left free. An Out view's incoming elements are undefined.

The public names and the error classes are the reference's
(`python/intent/language/annotations.py`). Malformed entries raise TypeError and out-of-range
values raise ValueError. `In`, `Out`, `InOut` and `Constexpr` are subscriptable annotation objects
here. Nothing but subscription is asked of them, and the runtime reads the resulting specs by
attribute.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import Any

from .dtypes import DType

ShapeDim = int | str
StrideDim = int | str | None


def _entry_class(entry: object) -> str:
    """Classify one shape or stride entry: "int", "name", "none", "bad name" or "other".

    bool counts as "other" although it is an int subclass: True is no extent."""
    if entry is None:
        return "none"
    if isinstance(entry, bool):
        return "other"
    if isinstance(entry, int):
        return "int"
    if isinstance(entry, str):
        return "name" if entry.isidentifier() else "bad name"
    return "other"


def _extent(entry: object) -> ShapeDim:
    kind = _entry_class(entry)
    if kind == "name":
        return entry
    if kind == "int":
        if entry < 0:
            raise ValueError(f"a static extent cannot be negative, got {entry}")
        return entry
    if kind == "bad name":
        raise ValueError(f"{entry!r} is not an identifier and cannot name a dimension")
    raise TypeError(f"a shape entry is an int extent or a dimension name, not {entry!r}")


def _stride(entry: object) -> StrideDim:
    if _entry_class(entry) in ("int", "name", "none"):
        return entry
    raise TypeError(f"a stride constraint is an int, a stride name or None, not {entry!r}")


def _shape(shape: object) -> tuple[ShapeDim, ...]:
    if not isinstance(shape, (tuple, list)):
        raise TypeError(f"a view shape is a tuple or list of extents, not {type(shape).__name__}")
    return tuple(_extent(entry) for entry in shape)


@dataclass(frozen=True, slots=True)
class ViewConstraints:
    """Layout and allocation relations of one view (strides, alias group, noalias)."""

    strides: tuple[StrideDim, ...] | None = None
    alias: str | None = None
    noalias: bool = False

    def __post_init__(self) -> None:
        if self.strides is not None:
            object.__setattr__(self, "strides", tuple(_stride(entry) for entry in self.strides))
        if self.alias is not None:
            if self.noalias:
                raise ValueError("a view cannot both join an alias group and be noalias")
            if not self.alias:
                raise ValueError("an alias group needs a non-empty name")


def constraints(*, strides: tuple[StrideDim, ...] | None = None, alias: str | None = None,
                noalias: bool = False) -> ViewConstraints:
    """The optional third item of a view annotation."""
    return ViewConstraints(strides, alias, noalias)


class ViewKind(enum.IntEnum):
    IN = 0
    OUT = 1
    INOUT = 2


@dataclass(frozen=True, slots=True)
class ViewSpec:
    """A view parameter: access kind, element dtype, shape and constraints."""

    kind: ViewKind
    dtype: DType
    shape: tuple[ShapeDim, ...]
    constraints: ViewConstraints

    def __post_init__(self) -> None:
        for value, expected, what in ((self.kind, ViewKind, "access kind"), (self.dtype, DType, "element dtype"),
                                      (self.constraints, ViewConstraints, "constraints")):
            if not isinstance(value, expected):
                raise TypeError(f"a view's {what} must be a {expected.__name__}, got {value!r}")
        shape = _shape(self.shape)
        object.__setattr__(self, "shape", shape)
        strides = self.constraints.strides
        if strides is not None and len(strides) != len(shape):
            raise ValueError(f"{len(strides)} stride constraints for a view of rank {len(shape)}")


class _ViewAnnotation:
    """`In`, `Out` and `InOut`: subscripting one with (dtype, shape[, constraints]) gives a ViewSpec."""

    def __init__(self, kind: ViewKind, name: str, doc: str) -> None:
        self.kind, self.__name__, self.__doc__ = kind, name, doc

    def __getitem__(self, items: object) -> ViewSpec:
        if not isinstance(items, tuple) or not 2 <= len(items) <= 3:
            raise TypeError(f"I.{self.__name__}[...] takes a dtype, a shape and optionally I.constraints(...)")
        dtype, shape, *rest = items
        extra = rest[0] if rest else ViewConstraints()
        if not isinstance(extra, ViewConstraints):
            raise TypeError(f"the third item of I.{self.__name__}[...] must come from I.constraints(...), "
                            f"got {extra!r}")
        return ViewSpec(self.kind, dtype, _shape(shape), extra)

    def __repr__(self) -> str:
        return f"I.{self.__name__}"


In = _ViewAnnotation(ViewKind.IN, "In", "A view the kernel reads.")
Out = _ViewAnnotation(ViewKind.OUT, "Out", "A view the kernel writes; its incoming elements are undefined.")
InOut = _ViewAnnotation(ViewKind.INOUT, "InOut", "A view the kernel reads and writes.")


@dataclass(frozen=True, slots=True)
class ConstexprSpec:
    """A specialization parameter of type `value_type`, bound at jit time."""

    value_type: Any


class _ConstexprAnnotation:
    def __getitem__(self, value_type: Any) -> ConstexprSpec:
        if value_type is None:
            raise TypeError("I.Constexpr[...] needs the type of the specialization value")
        return ConstexprSpec(value_type)

    def __repr__(self) -> str:
        return "I.Constexpr"


Constexpr = _ConstexprAnnotation()


class Enum(enum.Enum):
    """Base class of author enums used as specialization values."""
