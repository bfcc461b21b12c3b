"""intent_amd — an MI355X-native `hip` provider for the IntentDSL `intent.jit` call surface.

Same public surface as the reference package `intent` for the operators this
provider runs: `kernel`/`fn` definitions, `language` (as `I`), `jit`/`JITKernel`,
`CompiledArtifact`, `PreparedCall`, `PublicInterface`, `CompilationStageError`.
Use it as `import intent_amd as intent`.
"""
from . import language
from .api import Definition, DefinitionKind, HelperDefinition, KernelDefinition, fn, kernel
from .compiler import CompileOptions, GeneratedProgram, generate
from .diagnostics import CompilationStageError, DefinitionError, IntentError, LanguageUseError
from .jit import JITKernel, jit
from .runtime import (CompiledArtifact, ConfigurationAssessment, NativeObservation, NativeResource,
                      PreparedCall, PublicInterface, ScalarParameter, ViewParameter)


__all__ = ["language", "Definition", "DefinitionKind", "HelperDefinition", "KernelDefinition", "fn", "kernel",
           "CompilationStageError", "DefinitionError", "IntentError", "LanguageUseError", "JITKernel", "jit",
           "CompiledArtifact", "ConfigurationAssessment", "NativeObservation", "NativeResource",
           "PreparedCall", "PublicInterface", "ScalarParameter", "ViewParameter", "CompileOptions",
           "GeneratedProgram", "generate"]
