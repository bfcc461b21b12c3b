"""Provider registry (reference: `python/intent/targets/provider.py:26-56`).

A provider is a module named in `components.json` that exports `PROVIDER`.
`Provider.generate` is this package's direct-generation hook: a provider that
maps definitions straight to native kernels (the hip provider) makes its
`GeneratedProgram` without the reference's KIR/MLIR compiler stage; the JIT then
materializes that program through the resolved target, as for any provider."""
from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from importlib import import_module
from typing import Any


@dataclass(frozen=True, slots=True)
class EnvironmentCheck:
    name: str
    category: str
    action: Callable[[], object]


def unspecialized_call(target, definition, arguments, outputs):
    """The native ABI keeps runtime shapes and strides: one artifact per device."""
    return target, ()


@dataclass(frozen=True, slots=True)
class LocalExecution:
    device_kind: str
    indexed: bool
    options: frozenset
    resolve: Callable[..., Any]
    execution_key: Callable[[Any], object]
    host_storage: Callable[[Any, dict], Any]
    specialize: Callable[..., tuple] = unspecialized_call


@dataclass(frozen=True, slots=True)
class Provider:
    family: str
    target: type
    read_facts: Callable | None
    bind: Callable | None
    environment_checks: Callable[[Any], tuple]
    local: LocalExecution
    execution_model: str
    read_target: Callable | None
    environment_scope: str | None = None
    generate: Callable | None = None


def provider(name: str) -> Provider:
    from .components import COMPONENTS

    if name not in COMPONENTS:
        raise ValueError(f"Unknown backend {name!r}; choose from {', '.join(COMPONENTS)}")
    return import_module(COMPONENTS[name]).PROVIDER
