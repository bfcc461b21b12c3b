"""The hip provider's configuration table and `tuning_config` overrides.

A tuning configuration file has the reference's form (`doc/getting-started/configuration.en.md:13`,
table format of `lib/Target/Triton/Transforms/Configuration/TuningProfiles.json`):

    {"columns": ["split"], "families": {"hip.attention_backward": [[0]]}}

Each family's rows are the complete, ordered candidate list of the kernels it covers; a supplied
family replaces its default rows as a group and omitted families keep theirs. The file is read once,
when a program is generated; the program keeps its effective rows (`artifact.json["hip"]["tuning"]`),
so a saved program runs with the rows it was generated with.

The hip kernels are compiled ahead of time, so a row can only choose among what they implement.
Each family below lists exactly that; a row outside it is a `CompilationStageError` at generation.

  hip.attention_backward   attention_backward_dq / attention_backward_dkdv. split = 1: a grid too
                           small to fill the device divides its work over more workgroups and folds
                           their f32 partial sums (a workspace allocated at prepare); split = 0: the
                           unsplit kernels.
  hip.latent_prefill       mla_prefill. split = 1: a small grid splits each query block's keys over
                           workgroups and merges the split states; split = 0: unsplit.
  hip.attention_forward    flash_attention_fwd, flash_gqa_attention_fwd, flash_attention_bf16_fwd:
                           the same key split for the batched attention forward.

A prepared call takes the first row, in table order, that is eligible for its arguments (split = 1
is eligible when the grid is small enough to split and the workspace policy allows a workspace).
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from enum import IntEnum
from pathlib import Path

COLUMNS = ("split",)

DEFAULT_FAMILIES = {
    "hip.attention_backward": ((1,), (0,)),
    "hip.latent_prefill": ((1,), (0,)),
    "hip.attention_forward": ((1,), (0,)),
}
IMPLEMENTED = {family: frozenset(rows) for family, rows in DEFAULT_FAMILIES.items()}

# The family of each definition that has one (definitions without one run one fixed configuration).
FAMILY_OF = {
    "attention_backward_dq": "hip.attention_backward",
    "attention_backward_dkdv": "hip.attention_backward",
    "mla_prefill": "hip.latent_prefill",
    "flash_attention_fwd": "hip.attention_forward",
    "flash_gqa_attention_fwd": "hip.attention_forward",
    "flash_attention_bf16_fwd": "hip.attention_forward",
}


class ParameterRole(IntEnum):
    """Roles of tuning parameters (reference `python/intent/runtime/artifact.py:61-72`)."""

    OWNERSHIP_M = 0
    OWNERSHIP_N = 1
    REDUCTION = 2
    SCAN_CHUNK = 3
    PROVIDER_OPTION = 4
    TRAVERSAL_WORKERS = 8
    TRAVERSAL_GROUP = 9
    RESIDENT_WORKERS = 10
    FULL_COVERAGE = 11
    REDUCTION_OUTER = 12
    REDUCTION_INNER = 13


@dataclass(frozen=True, slots=True)
class TuningParameter:
    name: str
    role: ParameterRole
    category: int
    candidates: tuple[int, ...]
    dimension: int | None
    source: tuple[int, int, bool] | None
    view_axis: tuple[int, int] | None


@dataclass(frozen=True, slots=True)
class TuningConfiguration:
    parameters: tuple[TuningParameter, ...]
    values: tuple[int, ...]


SPLIT = TuningParameter("split", ParameterRole.PROVIDER_OPTION, 0, (0, 1), None, None, None)


def read_tuning_config(path) -> dict[str, tuple[tuple[int, ...], ...]]:
    """The effective table: the defaults with the file's families replacing theirs."""
    from ...diagnostics import CompilationStageError

    try:
        data = json.loads(Path(path).read_text(encoding="utf-8"))
    except (OSError, UnicodeError, ValueError) as error:
        raise CompilationStageError("provider_configuration", f"tuning_config {path}: {error}") from error
    if not isinstance(data, dict) or set(data) != {"columns", "families"}:
        raise CompilationStageError("provider_configuration",
                                    "a tuning configuration is an object with exactly 'columns' and 'families'")
    if tuple(data["columns"]) != COLUMNS:
        raise CompilationStageError("provider_configuration",
                                    f"hip tuning configurations have the columns {list(COLUMNS)}, got {data['columns']}")
    families = data["families"]
    if not isinstance(families, dict):
        raise CompilationStageError("provider_configuration", "'families' must map family names to row lists")
    table = dict(DEFAULT_FAMILIES)
    for family, rows in families.items():
        if family not in IMPLEMENTED:
            raise CompilationStageError("provider_configuration",
                                        f"unknown hip tuning family {family!r}; families: {', '.join(sorted(IMPLEMENTED))}")
        if not isinstance(rows, list) or not rows:
            raise CompilationStageError("provider_configuration", f"{family}: a family needs a nonempty row list")
        parsed = []
        for row in rows:
            if (not isinstance(row, list) or len(row) != len(COLUMNS)
                    or any(type(value) is not int for value in row)):
                raise CompilationStageError("provider_configuration",
                                            f"{family}: row {row!r} is not {len(COLUMNS)} integers")
            if tuple(row) not in IMPLEMENTED[family]:
                raise CompilationStageError("provider_configuration",
                                            f"{family}: row {row!r} is not a configuration the hip kernels implement "
                                            f"({sorted(list(r) for r in IMPLEMENTED[family])})")
            parsed.append(tuple(row))
        if len(set(parsed)) != len(parsed):
            raise CompilationStageError("provider_configuration", f"{family}: duplicate rows")
        table[family] = tuple(parsed)
    return table


def table_metadata(table: dict) -> dict:
    return {"columns": list(COLUMNS), "families": {name: [list(row) for row in rows] for name, rows in table.items()}}


def table_from_metadata(metadata) -> dict:
    if metadata is None:
        return dict(DEFAULT_FAMILIES)
    if not isinstance(metadata, dict) or tuple(metadata.get("columns", ())) != COLUMNS:
        raise ValueError("saved hip tuning table has unknown columns")
    table = dict(DEFAULT_FAMILIES)
    for family, rows in metadata["families"].items():
        if family not in IMPLEMENTED or any(tuple(row) not in IMPLEMENTED[family] for row in rows) or not rows:
            raise ValueError(f"saved hip tuning family {family!r} holds rows the kernels do not implement")
        table[family] = tuple(tuple(row) for row in rows)
    return table
