"""`intent.jit`: a kernel definition bound to a backend, compiled per device on first use.

Public surface and error classes follow the reference's `python/intent/jit/kernel.py:14-133`:
`jit(definition, *, backend, device, compiler, constexprs, tuning_config, options, workers,
backend_options)` returns a `JITKernel` with `prepare(*inputs, outputs=tuple)`, `run`, a call form
that takes the Out buffers in declaration order, `artifacts`, `interface`, `as_torch_op`,
`empty_like`, `prepare_fill`, `close` and context-manager use.

Design here: the hip provider binds runtime shapes and strides at every call, so an artifact
depends only on the device (and on the provider's specialization key, which is empty for hip).
A `JITKernel` therefore keeps one `_DeviceSlot` per execution key, holding the resolved target
and the artifacts made for it. The split of a positional call into inputs and Out buffers is
read from the signature once (`_CallRoles`), not on every call.

As in the reference (`jit/kernel.py:52-68`), the local target must satisfy `ResolvedTarget`
(else NotImplementedError), and an artifact is a generated program materialized through that
target. The program comes from the provider's `generate` hook (the hip provider has no compiler
stage); a provider without one cannot be jitted (CompilationStageError, stage
"provider_generation").
"""
from __future__ import annotations

from copy import deepcopy
from threading import RLock

from ..api import KernelDefinition
from ..diagnostics import CompilationStageError
from ..language.annotations import ViewKind
from ..targets.base import ResolvedTarget
from ..targets.local import resolve_local, select_device
from ..targets.provider import provider


def _is_kernel_definition(definition) -> bool:
    """This package's KernelDefinition, or a definition object of the reference's own package
    (`kind.value == "kernel"` with a signature)."""
    if isinstance(definition, KernelDefinition):
        return True
    return getattr(getattr(definition, "kind", None), "value", None) == "kernel" and hasattr(definition, "signature")


class _CallRoles:
    """Which positional runtime arguments of a call are inputs and which are Out buffers."""

    def __init__(self, definition):
        annotations = [p.annotation for p in definition.signature.parameters.values()]
        runtime = [a for a in annotations if not (hasattr(a, "value_type") and not hasattr(a, "kind"))]
        self.count = len(runtime)
        self.out_positions = tuple(i for i, a in enumerate(runtime)
                                   if getattr(a, "kind", None) is not None and int(a.kind) == int(ViewKind.OUT))

    def split(self, arguments: tuple) -> tuple[tuple, tuple]:
        if len(arguments) != self.count:
            raise TypeError(f"this kernel takes {self.count} runtime arguments (Out buffers included), "
                            f"got {len(arguments)}")
        outs = set(self.out_positions)
        inputs = tuple(value for i, value in enumerate(arguments) if i not in outs)
        return inputs, tuple(arguments[i] for i in self.out_positions)


class _DeviceSlot:
    """The resolved target of one execution key and the artifacts made for it."""

    __slots__ = ("target", "artifacts")

    def __init__(self, target):
        self.target, self.artifacts = target, {}


class JITKernel:
    """One definition, compiled lazily for each device it is called on."""

    def __init__(self, definition, *, backend, device=None, compiler=None, constexprs=None,
                 tuning_config=None, options=None, workers=None, backend_options=None):
        if not _is_kernel_definition(definition):
            raise TypeError(f"intent.jit takes an @intent.kernel definition, not {type(definition).__name__}")
        self._provider = provider(backend)
        self.definition, self.backend, self.device = definition, backend, device
        self.compiler, self.tuning_config, self.options, self.workers = compiler, tuning_config, options, workers
        # Private copies: a caller mutating its dicts after jit() changes nothing here.
        self.constexprs = deepcopy(dict(constexprs or {}))
        self.backend_options = deepcopy(dict(backend_options or {}))
        self._slots: dict[object, _DeviceSlot] = {}
        self._roles = None
        self._lock = RLock()
        self._closed = False
        self.__name__, self.__doc__ = definition.__name__, definition.__doc__

    # -- artifacts ----------------------------------------------------------------------------
    @property
    def artifacts(self) -> tuple:
        """The artifacts made so far, in the order they were made. Reading this compiles nothing."""
        with self._lock:
            return tuple(artifact for slot in self._slots.values() for artifact in slot.artifacts.values())

    def _single_artifact(self, purpose: str):
        made = self.artifacts
        if len(made) != 1:
            raise ValueError(f"{purpose} needs exactly one prepared specialization; this kernel has {len(made)}")
        return made[0]

    @property
    def interface(self):
        return self._single_artifact("the interface").interface

    def _artifact(self, arguments: tuple, outputs):
        local = self._provider.local
        device = select_device(self.backend, arguments + tuple(outputs or ()), self.device)
        key = local.execution_key(device)
        with self._lock:
            if self._closed:
                raise RuntimeError(f"JIT kernel {self.__name__} is closed")
            slot = self._slots.get(key)
            if slot is None:
                resolved = resolve_local(self.backend, device, workers=self.workers,
                                         backend_options=self.backend_options)
                if not isinstance(resolved, ResolvedTarget):
                    raise NotImplementedError(f"{self.backend} has no local executable target")
                slot = _DeviceSlot(resolved)
                self._slots[key] = slot
            target, specialization = local.specialize(slot.target, self.definition, arguments, outputs)
            artifact = slot.artifacts.get(specialization)
            if artifact is None:
                if self._provider.generate is None:
                    raise CompilationStageError("provider_generation",
                                                f"the {self.backend} provider cannot generate definitions directly")
                program = self._provider.generate(self.definition, target=target, compiler=self.compiler,
                                                  constexprs=self.constexprs, tuning_config=self.tuning_config,
                                                  options=self.options)
                artifact = program.materialize()
                slot.artifacts[specialization] = artifact
            return artifact

    # -- calls --------------------------------------------------------------------------------
    def prepare(self, *arguments, outputs=None):
        """Bind a call (allocating absent Out buffers) without launching it."""
        if outputs is not None and not isinstance(outputs, tuple):
            raise TypeError(f"outputs is a tuple of Out buffers in declaration order, not {type(outputs).__name__}")
        return self._artifact(arguments, outputs).prepare(*arguments, outputs=outputs)

    def run(self, *arguments):
        """Bind, launch and return the Out buffers (one value, a tuple, or None)."""
        call = self.prepare(*arguments)
        call.launch()
        return call.result()

    def __call__(self, *arguments):
        """Launch with every runtime argument given, Out buffers in their declared places."""
        if self._roles is None:
            self._roles = _CallRoles(self.definition)
        inputs, outputs = self._roles.split(arguments)
        self.prepare(*inputs, outputs=outputs).launch()

    def as_torch_op(self, name):
        return self._single_artifact("registering a PyTorch operator").as_torch_op(name)

    # -- author storage -------------------------------------------------------------------------
    def _storage(self, like):
        device = select_device(self.backend, (like,), self.device)
        return self._provider.local.host_storage(device, self.backend_options)

    def empty_like(self, reference, shape, *, dtype):
        """Uninitialised author storage on the kernel's device (the device of `reference`)."""
        return self._storage(reference).allocate(shape, dtype)

    def prepare_fill(self, value, scalar):
        """A bound fill of `value` with `scalar`; nothing is written until it is launched."""
        return self._storage(value).prepare_fill(value, scalar)

    # -- lifetime -----------------------------------------------------------------------------
    def close(self):
        with self._lock:
            slots, self._slots, self._closed = self._slots, {}, True
        for slot in slots.values():
            for artifact in slot.artifacts.values():
                close = getattr(artifact.runtime, "close", None)
                if close is not None:
                    close()

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()


def jit(definition, *, backend, device=None, compiler=None, constexprs=None, tuning_config=None,
        options=None, workers=None, backend_options=None):
    """A JIT callable of `definition` on `backend`; devices are discovered from the calls."""
    return JITKernel(definition, backend=backend, device=device, compiler=compiler, constexprs=constexprs,
                     tuning_config=tuning_config, options=options, workers=workers,
                     backend_options=backend_options)
