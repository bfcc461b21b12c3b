"""Target protocols a provider's targets satisfy (reference: `python/intent/targets/base.py:12-27`).

A *resolved* target is a local runtime binding: it carries the compiler facts it was resolved to
(`compilation`) and turns a generated program into an artifact (`materialize`). The reference's
JIT refuses a backend whose local target is not one (`python/intent/jit/kernel.py:55-57`), and
`GeneratedProgram.materialize` requires one (`python/intent/compiler/artifact.py:169-177`).
"""
from __future__ import annotations

from typing import Protocol, runtime_checkable


@runtime_checkable
class ResolvedTarget(Protocol):
    @property
    def compilation(self): ...

    def materialize(self, program): ...


class SourceTarget(Protocol):
    def resolve(self): ...


class Target(SourceTarget, Protocol):
    def resolve(self) -> ResolvedTarget: ...
