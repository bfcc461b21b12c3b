"""Error classes shared by the definition surface and the hip provider.

Mirrors the reference's `python/intent/diagnostics/errors.py` hierarchy and
`python/intent/compiler/toolchain.py:17-27` (`CompilationStageError`), so that
callers catching those types keep working.
"""
from __future__ import annotations

from pathlib import Path


class IntentError(Exception):
    """Base class of every error raised by this package."""


class DefinitionError(IntentError):
    """An `@intent.kernel`/`@intent.fn` decoration or signature is malformed."""


class LanguageUseError(IntentError):
    """A DSL intrinsic or definition was called outside a kernel body."""


class CompilationStageError(RuntimeError):
    """A provider stage failed; `stage` names it (for example `provider_recognition`,
    `native_loading`, `provider_invocation`). A failure never falls back to
    another provider."""

    def __init__(self, stage: str, message: str, *, cache_directory: Path | None = None,
                 candidate: str | None = None, artifacts: dict | None = None,
                 observation=None) -> None:
        super().__init__(message)
        self.stage = stage
        self.cache_directory = cache_directory
        self.candidate = candidate
        self.artifacts = dict(artifacts or {})
        self.observation = observation
