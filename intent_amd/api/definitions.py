"""`@intent.kernel` / `@intent.fn` definitions (reference: `python/intent/api/definitions.py`)."""
from __future__ import annotations

import functools
import inspect
import textwrap
from dataclasses import dataclass
from enum import Enum
from types import FunctionType

from ..diagnostics import DefinitionError, LanguageUseError


class DefinitionKind(Enum):
    KERNEL = "kernel"
    HELPER = "helper"


@dataclass(frozen=True, slots=True)
class DefinitionSource:
    filename: str
    first_line: int


class Definition:
    def __init__(self, function, kind: DefinitionKind) -> None:
        if not isinstance(function, FunctionType):
            raise DefinitionError("Intent definitions must decorate a Python function")
        self.python_function = function
        self.kind = kind
        self.source = DefinitionSource(inspect.getsourcefile(function) or function.__code__.co_filename,
                                       function.__code__.co_firstlineno)
        functools.update_wrapper(self, function)

    @property
    def signature(self) -> inspect.Signature:
        return inspect.signature(self.python_function, eval_str=True)

    def source_text(self) -> str:
        return textwrap.dedent(inspect.getsource(self.python_function))

    def __call__(self, *args, **kwargs):
        if self.kind is DefinitionKind.KERNEL:
            raise LanguageUseError(f"kernel {self.__name__} must be compiled before runtime invocation")
        raise LanguageUseError(f"helper {self.__name__} is only callable inside an @intent.kernel body")

    def __repr__(self) -> str:
        return f"<intent {self.kind.value} {self.__module__}.{self.__qualname__}>"


class KernelDefinition(Definition):
    def __init__(self, function) -> None:
        super().__init__(function, DefinitionKind.KERNEL)


class HelperDefinition(Definition):
    def __init__(self, function) -> None:
        super().__init__(function, DefinitionKind.HELPER)


def kernel(function=None):
    return KernelDefinition if function is None else KernelDefinition(function)


def fn(function=None):
    return HelperDefinition if function is None else HelperDefinition(function)
