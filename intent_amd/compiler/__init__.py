"""Generated programs of the hip provider: `generate` and `GeneratedProgram` (save/load/materialize),
with the reference's on-disk layout (`python/intent/compiler/artifact.py:105-157`), and the
`CompileOptions` numerics policy (`python/intent/compiler/options.py:9-69`)."""
from .artifact import GeneratedProgram, generate
from .options import CompileOptions

__all__ = ["CompileOptions", "GeneratedProgram", "generate"]
