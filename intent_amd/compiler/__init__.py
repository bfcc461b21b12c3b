"""Generated programs of the hip provider: `generate` and `GeneratedProgram` (save/load/materialize),
with the reference's on-disk layout (`python/intent/compiler/artifact.py:105-157`)."""
from .artifact import GeneratedProgram, generate

__all__ = ["GeneratedProgram", "generate"]
