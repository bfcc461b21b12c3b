"""The `hip` provider: hand-written gfx950 kernels behind the `intent.jit` surface.

Registered in `components.json` as `"hip"`. Device kind is "cuda" because
PyTorch-ROCm exposes HIP devices as `torch.device("cuda", i)`, so
`select_device` and `register_operator`'s {"cpu","cuda"} check apply unchanged
(reference contract: `python/intent/targets/provider.py:26-48`, example provider
`python/intent/targets/triton.py:10-51`).

Targets follow the reference's split between compiler facts and a runtime binding
(`python/intent/targets/base.py:12-27`):

  HipTarget             what a caller names: a device ordinal and the workspace policy.
  HipCompilationTarget  the facts a program is generated for: architecture, wavefront size and
                        LDS per workgroup. These are what the ahead-of-time code objects depend on;
                        grid sizes follow the device's compute units at launch, so a program saved
                        on one gfx950 device binds to any other.
  ResolvedHipTarget     a resolved local device: `compilation` gives its facts and
                        `materialize(program)` binds a generated program to it (the
                        `ResolvedTarget` protocol the reference's JIT and
                        `GeneratedProgram.materialize` require).

Generation has no compiler stage: `PROVIDER.generate` maps the definition to its kernel and
returns a `GeneratedProgram`, which `materialize()` binds as any provider's program.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from functools import partial

from ..diagnostics import CompilationStageError
from .execution import indexed_key, indexed_target, torch_storage
from .provider import EnvironmentCheck, LocalExecution, Provider
from .specification import require_matching_target

INSTALLATION = {
    "modules": ("torch",),
    "requirements": (),
    "toolchain": "ROCm 7 hipcc for gfx950; PyTorch-ROCm; libintent_hip.so built in-tree",
}

SUPPORTED_ARCHITECTURES = ("gfx950",)
EXECUTION_MODEL = "hip-direct"


# backend_options={"workspace": ...}: where the device memory a kernel needs beyond its operands
# comes from.
#   "prepare" (default)  allocated once per prepared call: the SpMV plan and the split
#                        partial sums of small attention-backward grids; a view whose layout
#                        the kernel does not take is staged through a contiguous copy.
#   "static"             the provider allocates nothing at prepare: SpMV runs on the library's
#                        static per-GPU scratch (intent_hip_csr_spmv_f32_static, problems up to
#                        INTENT_HIP_STATIC_SCRATCH_BYTES of plan), the attention backward runs its
#                        unsplit kernels, and a view that would need staging is rejected
#                        (ValueError). Out buffers the caller does not pass are still allocated.
#                        Calls on one GPU that overlap share the SpMV scratch and race.
WORKSPACE_POLICIES = ("prepare", "static")


@dataclass(frozen=True, slots=True)
class HipCompilationTarget:
    """Compiler facts of a hip program; constructing one queries no device."""

    provider: str
    architecture: str
    wavefront_size: int
    lds_per_workgroup: int

    def __post_init__(self) -> None:
        from .provider import provider

        if provider(self.provider).execution_model != EXECUTION_MODEL:
            raise ValueError(f"{self.provider!r} is not a {EXECUTION_MODEL} provider")
        if self.architecture not in SUPPORTED_ARCHITECTURES:
            raise ValueError(f"the hip provider is built for {', '.join(SUPPORTED_ARCHITECTURES)}, "
                             f"not {self.architecture!r}")
        for name in ("wavefront_size", "lds_per_workgroup"):
            value = getattr(self, name)
            if type(value) is not int or value <= 0:
                raise ValueError(f"{name} must be a positive integer, got {value!r}")

    def resolve(self) -> "HipCompilationTarget":
        return self

    def facts(self) -> dict:
        return {"architecture": self.architecture, "wavefront_size": self.wavefront_size,
                "lds_per_workgroup": self.lds_per_workgroup}

    def metadata(self) -> dict:
        """The `target` object of a saved program (`family` names the execution model)."""
        return {"family": EXECUTION_MODEL, **self.facts()}

    @property
    def compiler_options(self) -> tuple[str, ...]:
        return (f"--target={self.provider}", f"--target-options={json.dumps(self.facts(), sort_keys=True)}")

    @property
    def compiler_role(self) -> str:
        return f"Intent {self.provider} provider (hand-written {self.architecture} kernels, no compiler stage)"


def read_hip_target(provider_name: str, values: dict) -> HipCompilationTarget:
    """Saved target facts -> HipCompilationTarget; exactly the three facts, nothing defaulted."""
    expected = {"architecture", "wavefront_size", "lds_per_workgroup"}
    if set(values) != expected:
        raise ValueError(f"a hip target has exactly the fields {', '.join(sorted(expected))}; "
                         f"got {', '.join(sorted(values)) or 'none'}")
    return HipCompilationTarget(provider_name, values["architecture"], values["wavefront_size"],
                                values["lds_per_workgroup"])


@dataclass(frozen=True, slots=True)
class ResolvedHipTarget:
    device: int
    architecture: str
    compute_units: int
    wavefront_size: int
    lds_per_workgroup: int
    global_memory_bytes: int
    facts: dict = field(default_factory=dict, compare=False)
    workspace: str = "prepare"

    @property
    def provider(self) -> str:
        return "hip"

    @property
    def compilation(self) -> HipCompilationTarget:
        return HipCompilationTarget(self.provider, self.architecture, self.wavefront_size, self.lds_per_workgroup)

    def materialize(self, program):
        """Bind a generated or loaded program to this device, without regenerating it (the
        program's saved target must equal this device's compiler facts)."""
        require_matching_target(program.target, self.compilation)
        return _bind(program, self)


@dataclass(frozen=True, slots=True)
class HipTarget:
    device: int = 0
    workspace: str = "prepare"

    def __post_init__(self) -> None:
        if isinstance(self.device, bool) or not isinstance(self.device, int) or self.device < 0:
            raise ValueError(f"HipTarget device must be a non-negative integer, got {self.device!r}")
        if self.workspace not in WORKSPACE_POLICIES:
            raise ValueError(f"workspace must be one of {WORKSPACE_POLICIES}, got {self.workspace!r}")

    @property
    def provider(self) -> str:
        return "hip"

    def resolve(self) -> ResolvedHipTarget:
        from ..runtime.hip.library import library

        info = library().device_info(self.device)
        arch = info["arch"].split(":")[0]
        if arch not in SUPPORTED_ARCHITECTURES:
            raise CompilationStageError(
                "target_resolution", f"device {self.device} is {arch}; the hip provider is built for "
                f"{', '.join(SUPPORTED_ARCHITECTURES)} only")
        return ResolvedHipTarget(self.device, arch, info["compute_units"], info["wavefront_size"],
                                 info["lds_per_workgroup"], info["global_memory_bytes"], info, self.workspace)


def _read_facts(source, metadata, abi):
    """Provider facts of a saved program (`metadata["hip"]`), read without a device."""
    from ..compiler.artifact import read_hip_facts

    return read_hip_facts(metadata)


def _bind(program, target):
    from ..compiler.artifact import bind_program

    return bind_program(program, target)


def _generate(definition, *, target, compiler=None, constexprs=None, tuning_config=None, options=None):
    from ..compiler.artifact import generate

    return generate(definition, target=target, compiler=compiler, constexprs=constexprs,
                    tuning_config=tuning_config, options=options)


def _environment_checks(target):
    def native():
        from ..runtime.hip.library import library

        lib = library()
        return {"path": str(lib.path), "abi": lib.abi_version}

    return (EnvironmentCheck("hip native library", "provider_toolchain", native),)


PROVIDER = Provider(
    "gpu", HipTarget, _read_facts, _bind, _environment_checks,
    LocalExecution("cuda", True, frozenset({"workspace"}), partial(indexed_target, HipTarget), indexed_key,
                   torch_storage),
    EXECUTION_MODEL, read_hip_target, generate=_generate)
