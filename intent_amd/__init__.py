"""intent_amd — an MI355X-native `hip` provider for the IntentDSL `intent.jit` call surface.

Same public surface as the reference package `intent` for the operators this
provider runs: `kernel`/`fn` definitions, `language` (as `I`), `jit`/`JITKernel`,
`CompiledArtifact`, `PreparedCall`, `PublicInterface`, `CompilationStageError`.
Use it as `import intent_amd as intent`.
"""
from . import language
from .api import Definition, DefinitionKind, HelperDefinition, KernelDefinition, fn, kernel
from .compiler import GeneratedProgram, generate
from .diagnostics import CompilationStageError, DefinitionError, IntentError, LanguageUseError
from .jit import JITKernel, jit
from .runtime import (CompiledArtifact, ConfigurationAssessment, NativeObservation, NativeResource,
                      PreparedCall, PublicInterface, ScalarParameter, ViewParameter)


class CompileOptions:
    """Numerics options accepted by `jit(options=...)`; the hip provider runs `numerics="source"`
    (reference: `python/intent/compiler/options.py:9-69`)."""

    def __init__(self, numerics: str = "source", **extra):
        if numerics not in ("source", "relaxed_normalization"):
            raise ValueError(f"unknown numerics mode {numerics!r}")
        self.numerics = numerics
        self.extra = dict(extra)


__all__ = ["language", "Definition", "DefinitionKind", "HelperDefinition", "KernelDefinition", "fn", "kernel",
           "CompilationStageError", "DefinitionError", "IntentError", "LanguageUseError", "JITKernel", "jit",
           "CompiledArtifact", "ConfigurationAssessment", "NativeObservation", "NativeResource",
           "PreparedCall", "PublicInterface", "ScalarParameter", "ViewParameter", "CompileOptions",
           "GeneratedProgram", "generate"]
