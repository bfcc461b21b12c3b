"""`@intent.kernel` and `@intent.fn`: mark a Python function as a kernel or a helper.

The names, the two kinds and the error classes are the reference's
(`python/intent/api/definitions.py`). Wrapping anything but a plain Python function raises
DefinitionError. Calling a definition from host code raises LanguageUseError: a kernel runs only
through `intent.jit` or a generated program, and a helper only inside a kernel body.

The hip provider reads a definition's name and signature and never executes its body (the body
states the semantics the hand-written kernel implements). The signature is therefore evaluated
once, on first use, and kept: the launch path reads it on every `JITKernel.__call__`.
"""
from __future__ import annotations

import enum
import functools
import inspect
import textwrap
from dataclasses import dataclass
from types import FunctionType

from ..diagnostics import DefinitionError, LanguageUseError


class DefinitionKind(enum.Enum):
    KERNEL = "kernel"
    HELPER = "helper"


@dataclass(frozen=True, slots=True)
class DefinitionSource:
    """Where a definition is written: file and first line (decorators included)."""

    filename: str
    first_line: int


class Definition:
    """A wrapped author function; `kind` says how it may be used."""

    kind: DefinitionKind

    def __init__(self, function, kind: DefinitionKind | None = None) -> None:
        if not isinstance(function, FunctionType):
            raise DefinitionError(f"@intent.kernel and @intent.fn wrap Python functions, not {type(function).__name__}")
        if kind is not None:
            self.kind = DefinitionKind(kind)
        elif not hasattr(type(self), "kind"):
            raise TypeError("a Definition needs a DefinitionKind")
        code = function.__code__
        self.python_function = function
        self.source = DefinitionSource(inspect.getsourcefile(function) or code.co_filename, code.co_firstlineno)
        self._signature = None
        functools.update_wrapper(self, function)

    @property
    def signature(self) -> inspect.Signature:
        """Parameters with their annotations evaluated (string annotations included)."""
        if self._signature is None:
            self._signature = inspect.signature(self.python_function, eval_str=True)
        return self._signature

    def source_text(self) -> str:
        return textwrap.dedent(inspect.getsource(self.python_function))

    def __call__(self, *args, **kwargs):
        where = ("is launched through intent.jit or a generated program" if self.kind is DefinitionKind.KERNEL
                 else "is called only from inside an @intent.kernel body")
        raise LanguageUseError(f"{self.kind.value} {self.__name__} {where}, not from host code")

    def __repr__(self) -> str:
        return f"<intent {self.kind.value} {self.__module__}.{self.__qualname__}>"


class KernelDefinition(Definition):
    kind = DefinitionKind.KERNEL


class HelperDefinition(Definition):
    kind = DefinitionKind.HELPER


def _decorator(cls):
    def decorate(function=None):
        # `@intent.kernel` and `@intent.kernel()` both work: without a function, return the wrapper.
        return cls if function is None else cls(function)

    decorate.__name__ = "kernel" if cls is KernelDefinition else "fn"
    decorate.__doc__ = f"Wrap a Python function as an Intent {cls.kind.value} definition."
    return decorate


kernel = _decorator(KernelDefinition)
fn = _decorator(HelperDefinition)
