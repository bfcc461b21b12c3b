"""Compiled artifact and prepared-call protocols.

Public behaviour mirrors the reference's `python/intent/runtime/artifact.py:23-218`:
`run` allocates declared Out buffers and returns None / the single Out / a tuple;
`prepare` binds without executing; `launch` (also `__call__`) takes every runtime
argument including explicit Out buffers; `as_torch_op` registers a PyTorch custom
operator. For the hip provider `source` names the hand-written kernel entry the
definition maps to and `mlir` is empty (no KIR stage exists on this path).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Protocol, runtime_checkable

from .interface import PublicInterface


@runtime_checkable
class PreparedCall(Protocol):
    """Invocation-owned arguments and outputs; `result()` does not synchronize."""

    def compile(self) -> None: ...

    def launch(self) -> None: ...

    def result(self) -> object: ...

    @property
    def observation(self): ...

    def inspect_configurations(self) -> tuple: ...


@runtime_checkable
class PreparedRuntime(Protocol):
    def prepare_call(self, arguments: tuple, *, outputs: tuple | None = None) -> PreparedCall: ...


@dataclass(slots=True)
class CompiledArtifact:
    source: str
    mlir: str
    device: int
    runtime: Any = field(repr=False)
    _backend_ir_collector: Any = field(default=None, repr=False)
    device_type: str = field(default="cuda", kw_only=True)
    cache_directory: Path | None = field(default=None, kw_only=True)
    backend_ir: dict = field(default_factory=dict, init=False)

    @property
    def observation(self):
        """Latest native invocation snapshot, or None before one is reported."""
        return getattr(self.runtime, "observation", None)

    @property
    def entry(self):
        return self.__call__

    @property
    def ir(self) -> dict[str, str]:
        return {"intent": self.mlir, **self.backend_ir}

    @property
    def interface(self) -> PublicInterface:
        if not hasattr(self.runtime, "interface"):
            raise NotImplementedError("this runtime does not expose a typed invocation interface")
        return self.runtime.interface

    def run(self, *arguments: Any) -> object:
        """Allocate declared Out buffers and execute with inputs in declaration order."""
        return self.runtime.run(*arguments)

    def prepare(self, *arguments: Any, outputs: tuple | None = None) -> PreparedCall:
        """Bind arguments and allocate outputs/workspace without executing.

        Keep the arguments alive while using the prepared call; prepare again when
        their shape/stride metadata change."""
        if not isinstance(self.runtime, PreparedRuntime):
            raise NotImplementedError("this runtime does not expose prepared calls")
        return self.runtime.prepare_call(arguments, outputs=outputs)

    def as_torch_op(self, name: str):
        """Register a PyTorch custom operator with the declared Out/InOut behaviour."""
        from ..integrations.torch import register_operator

        return register_operator(self, name)

    def tuning_configurations(self, *arguments: Any) -> tuple:
        if not hasattr(self.runtime, "tuning_configurations"):
            raise NotImplementedError("this provider does not export structured tuning configurations")
        return self.runtime.tuning_configurations(*arguments)

    def inspect_configurations(self, *arguments: Any, outputs: tuple | None = None) -> tuple:
        return self.prepare(*arguments, outputs=outputs).inspect_configurations()

    def launch(self, *arguments: Any) -> None:
        """Execute with every runtime argument, including explicit Out buffers."""
        self.runtime.launch(*arguments)

    __call__ = launch
