"""Compiler facts of a target, independent of a runtime device.

`CompilationTarget` is the protocol of `python/intent/targets/specification.py:56-67`: a provider
name, the options it would pass to a compiler and a role string. `read_compilation_target` reads
the facts saved in a program's `artifact.json` through the owning provider's `read_target`, after
checking that the saved execution family is that provider's (`specification.py:70-79`).
"""
from __future__ import annotations

from typing import Protocol, runtime_checkable


@runtime_checkable
class CompilationTarget(Protocol):
    @property
    def provider(self) -> str: ...

    @property
    def compiler_options(self) -> tuple[str, ...]: ...

    @property
    def compiler_role(self) -> str: ...


def read_compilation_target(provider_name: str, facts) -> CompilationTarget:
    from .provider import provider

    if not isinstance(facts, dict):
        raise TypeError("compiler target facts must be a JSON object")
    values = dict(facts)
    family = values.pop("family", None)
    adapter = provider(provider_name)
    if adapter.execution_model != family:
        raise ValueError(f"target family {family!r} does not belong to provider {provider_name!r} "
                         f"(expected {adapter.execution_model!r})")
    if adapter.read_target is None:
        raise NotImplementedError(f"provider {provider_name!r} cannot read saved target facts")
    return adapter.read_target(provider_name, values)


def require_matching_target(compiled, selected) -> None:
    if compiled != selected:
        raise ValueError(f"the program was generated for {compiled}, the selected runtime target is {selected}")
