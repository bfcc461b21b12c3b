"""`intent.jit`: one definition, per-device artifacts and fresh call bindings.

Same surface and semantics as the reference's `python/intent/jit/kernel.py:14-133`
(artifact cache keyed by (execution key, specialization) under an RLock;
`prepare(..., outputs=tuple)`, `run`, `__call__` with explicit Out buffers,
`as_torch_op`, `empty_like`, `prepare_fill`, `close` and context manager).
The only difference is where an artifact comes from: a provider with a
`materialize` hook (the hip provider) builds it directly from the definition."""
from __future__ import annotations

from copy import deepcopy
from threading import RLock

from ..api import KernelDefinition
from ..diagnostics import CompilationStageError
from ..language.annotations import ViewKind
from ..targets.local import resolve_local, select_device
from ..targets.provider import provider


def _is_constexpr(annotation) -> bool:
    return hasattr(annotation, "value_type") and not hasattr(annotation, "kind")


class JITKernel:
    """One author definition, with device-specific artifacts and fresh call bindings."""

    def __init__(self, definition, *, backend, device=None, compiler=None, constexprs=None,
                 tuning_config=None, options=None, workers=None, backend_options=None):
        if not isinstance(definition, KernelDefinition) and not _looks_like_kernel(definition):
            raise TypeError("intent.jit requires an @intent.kernel definition")
        self._provider = provider(backend)
        self.definition, self.backend, self.device = definition, backend, device
        self.compiler, self.tuning_config, self.options = compiler, tuning_config, options
        self.constexprs = deepcopy(dict(constexprs or {}))
        self.workers, self.backend_options = workers, deepcopy(dict(backend_options or {}))
        self._targets, self._artifacts = {}, {}
        self._lock = RLock()
        self._closed = False
        self.__name__ = definition.__name__
        self.__doc__ = definition.__doc__

    @property
    def artifacts(self):
        """Artifacts produced so far; reading this never compiles."""
        with self._lock:
            return tuple(self._artifacts.values())

    @property
    def interface(self):
        artifacts = self.artifacts
        if len(artifacts) != 1:
            raise ValueError("prepare one local specialization before inspecting its interface")
        return artifacts[0].interface

    def _artifact(self, arguments, outputs):
        device = select_device(self.backend, (*arguments, *(outputs or ())), self.device)
        execution = self._provider.local.execution_key(device)
        with self._lock:
            if self._closed:
                raise RuntimeError("JIT kernel is closed")
            if execution not in self._targets:
                self._targets[execution] = resolve_local(self.backend, device, workers=self.workers,
                                                         backend_options=self.backend_options)
            target, specialization = self._provider.local.specialize(
                self._targets[execution], self.definition, arguments, outputs)
            key = execution, specialization
            if key not in self._artifacts:
                if self._provider.materialize is None:
                    raise CompilationStageError("provider_materialization",
                                                f"{self.backend} cannot materialize definitions directly")
                self._artifacts[key] = self._provider.materialize(
                    target, self.definition, constexprs=self.constexprs,
                    tuning_config=self.tuning_config, options=self.options)
            return self._artifacts[key]

    def prepare(self, *arguments, outputs=None):
        """Bind a local call without executing it."""
        if outputs is not None and not isinstance(outputs, tuple):
            raise TypeError("outputs must be a tuple in declared Out order")
        return self._artifact(arguments, outputs).prepare(*arguments, outputs=outputs)

    def run(self, *arguments):
        call = self.prepare(*arguments)
        call.launch()
        return call.result()

    def empty_like(self, reference, shape, *, dtype):
        device = select_device(self.backend, (reference,), self.device)
        return self._provider.local.host_storage(device, self.backend_options).allocate(shape, dtype)

    def prepare_fill(self, value, scalar):
        device = select_device(self.backend, (value,), self.device)
        return self._provider.local.host_storage(device, self.backend_options).prepare_fill(value, scalar)

    def as_torch_op(self, name):
        artifacts = self.artifacts
        if len(artifacts) != 1:
            raise ValueError("prepare one device specialization before registering its PyTorch operator")
        return artifacts[0].as_torch_op(name)

    def __call__(self, *arguments):
        parameters = [p for p in self.definition.signature.parameters.values()
                      if not _is_constexpr(p.annotation)]
        if len(parameters) != len(arguments):
            raise TypeError(f"expected {len(parameters)} runtime arguments, got {len(arguments)}")
        inputs, outputs = [], []
        for parameter, value in zip(parameters, arguments):
            kind = getattr(parameter.annotation, "kind", None)
            (outputs if kind is not None and int(kind) == int(ViewKind.OUT) else inputs).append(value)
        self.prepare(*inputs, outputs=tuple(outputs)).launch()

    def close(self):
        with self._lock:
            for artifact in self._artifacts.values():
                close = getattr(artifact.runtime, "close", None)
                if close is not None:
                    close()
            self._artifacts.clear()
            self._targets.clear()
            self._closed = True

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()


def _looks_like_kernel(definition) -> bool:
    """Accept the reference's own `KernelDefinition` objects (duck-typed)."""
    kind = getattr(definition, "kind", None)
    return getattr(kind, "value", None) == "kernel" and hasattr(definition, "signature")


def jit(definition, *, backend, device=None, compiler=None, constexprs=None, tuning_config=None,
        options=None, workers=None, backend_options=None):
    """Create a local JIT callable; the backend is explicit and hardware is discovered on use."""
    return JITKernel(definition, backend=backend, device=device, compiler=compiler, constexprs=constexprs,
                     tuning_config=tuning_config, options=options, workers=workers,
                     backend_options=backend_options)
