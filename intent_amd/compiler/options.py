"""Numerical permissions of one compilation (reference: `python/intent/compiler/options.py:9-69`).

`numerics="source"` keeps the language contract: every low-precision cast sits where the
definition puts it. `"relaxed_normalization"` additionally permits the normalized-summary
rewrite (`doc/dsl/types-numerics-and-effects.en.md:142-152`): a streaming summary may rescale
against a reference other than its own chunk maximum, which moves where low-precision weights
are rounded. The saved form is the three-key object the reference compiler writes into
`artifact.json`, read back without defaults.
"""
from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass, field
from types import MappingProxyType

NUMERICS = ("source", "relaxed_normalization")


@dataclass(frozen=True, slots=True)
class CompileOptions:
    numerics: str = "source"
    optimizations: Mapping = field(default_factory=dict)
    optimization_remarks: bool = False

    def __post_init__(self) -> None:
        if self.numerics not in NUMERICS:
            raise ValueError(f"numerics must be one of {NUMERICS}, got {self.numerics!r}")
        if not isinstance(self.optimizations, Mapping) or any(
                not isinstance(name, str) or not name or type(enabled) is not bool
                for name, enabled in self.optimizations.items()):
            raise TypeError("optimizations maps component names to booleans")
        if type(self.optimization_remarks) is not bool:
            raise TypeError("optimization_remarks must be a boolean")
        object.__setattr__(self, "optimizations", MappingProxyType(dict(sorted(self.optimizations.items()))))

    @classmethod
    def read(cls, metadata) -> "CompileOptions":
        """The saved policy, with every field present and nothing defaulted."""
        if not isinstance(metadata, dict) or set(metadata) != {"numerics", "optimizations", "optimization_remarks"}:
            raise ValueError("compile options require exactly numerics, optimizations and optimization_remarks")
        return cls(**metadata)

    def metadata(self) -> dict:
        return {"numerics": self.numerics, "optimizations": dict(self.optimizations),
                "optimization_remarks": self.optimization_remarks}

    @property
    def compiler_arguments(self) -> tuple[str, ...]:
        return (f"--numerics={self.numerics}", f"--optimization-remarks={str(self.optimization_remarks).lower()}",
                *(f"--optimization={name}={str(on).lower()}" for name, on in self.optimizations.items()))


def read_options(options) -> CompileOptions:
    """`jit(options=...)` / `generate(options=...)`: None means the source contract. Any object
    with a `numerics` attribute (the reference's own CompileOptions included) is accepted."""
    if options is None:
        return CompileOptions()
    if isinstance(options, CompileOptions):
        return options
    numerics = getattr(options, "numerics", None)
    if numerics is None:
        raise TypeError(f"options must be a CompileOptions or None, not {type(options).__name__}")
    return CompileOptions(numerics, dict(getattr(options, "optimizations", {}) or {}),
                          bool(getattr(options, "optimization_remarks", False)))
