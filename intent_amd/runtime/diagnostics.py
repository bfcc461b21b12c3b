"""Observation records of an invocation (reference: `python/intent/runtime/diagnostics.py:23-145`).

For the hip provider the resource facts come from `hipFuncGetAttributes` of the
kernel that the prepared call launches (registers, LDS bytes, scratch), read
through the C-ABI; nothing here is an estimate."""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True, slots=True)
class NativeResource:
    name: str
    value: int | None
    unit: str
    source: str
    stage: str
    unavailable_reason: str | None = None


@dataclass(frozen=True, slots=True)
class NativeObservation:
    provider: str
    entry: str
    kernel: str
    configuration: tuple[tuple[str, object], ...]
    resources: tuple[NativeResource, ...] = field(default_factory=tuple)


@dataclass(frozen=True, slots=True)
class ConfigurationAssessment:
    """One candidate configuration of a prepared call, with its eligibility and the reasons of an
    ineligible one (the hip provider lists the rows of the definition's tuning family)."""

    configuration: tuple[tuple[str, object], ...]
    eligible: bool
    reasons: tuple[str, ...] = ()
