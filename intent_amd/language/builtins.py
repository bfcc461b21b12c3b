"""Intrinsic stubs of the kernel language.

The hip provider never executes a kernel body: it recognises a definition and
runs a hand-written HIP kernel for it. These names exist so that definitions
written against the reference DSL import unchanged; calling one outside a
kernel raises `LanguageUseError`, as the reference's stubs do
(`python/intent/language/builtins.py`)."""
from __future__ import annotations

import math
from dataclasses import dataclass

from ..diagnostics import LanguageUseError


@dataclass(frozen=True, slots=True)
class Intrinsic:
    name: str

    def __call__(self, *args, **kwargs):
        raise LanguageUseError(f"I.{self.name} is only valid inside an @intent.kernel or @intent.fn body")

    def __getattr__(self, member: str):
        if member.startswith("__"):
            raise AttributeError(member)
        return Intrinsic(f"{self.name}.{member}")

    def __repr__(self) -> str:
        return f"I.{self.name}"


_NAMES = (
    "abs add assume_in_bounds arg_reduce atomic buffer bitcast cast contract cummax cumsum dot "
    "matmul matvec outer vecmat cos domain end exp exp2 fdiv floor full gather histogram indices "
    "join log log1p mask maximum maximum_num minimum minimum_num members parallel ragged random "
    "record reduce region_fold region_scan reshape rsqrt sqrt sigmoid tanh sin asin scan "
    "scatter_reduce scatter_unique select store transpose zeros erf erfc i0 lgamma"
).split()

globals().update({name: Intrinsic(name) for name in _NAMES})

inf = math.inf
LOG2E = 1.4426950408889634

__all__ = [*_NAMES, "inf", "LOG2E", "Intrinsic"]
