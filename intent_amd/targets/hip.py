"""The `hip` provider: hand-written gfx950 kernels behind the `intent.jit` surface.

Registered in `components.json` as `"hip"`. Device kind is "cuda" because
PyTorch-ROCm exposes HIP devices as `torch.device("cuda", i)`, so
`select_device` and `register_operator`'s {"cpu","cuda"} check apply unchanged
(reference contract: `python/intent/targets/provider.py:26-48`, example provider
`python/intent/targets/triton.py:10-51`)."""
from __future__ import annotations

from dataclasses import dataclass, field
from functools import partial

from ..diagnostics import CompilationStageError
from .execution import indexed_key, indexed_target, torch_storage
from .provider import EnvironmentCheck, LocalExecution, Provider

INSTALLATION = {
    "modules": ("torch",),
    "requirements": (),
    "toolchain": "ROCm 7 hipcc for gfx950; PyTorch-ROCm; libintent_hip.so built in-tree",
}

SUPPORTED_ARCHITECTURES = ("gfx950",)


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


@dataclass(frozen=True, slots=True)
class HipTarget:
    device: int = 0
    workspace: str = "prepare"

    def __post_init__(self) -> None:
        if self.workspace not in WORKSPACE_POLICIES:
            raise ValueError(f"workspace must be one of {WORKSPACE_POLICIES}, got {self.workspace!r}")

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


def _materialize(target, definition, *, constexprs=None, tuning_config=None, options=None):
    from ..runtime.hip.program import materialize_hip_artifact

    return materialize_hip_artifact(target, definition, constexprs=constexprs or {},
                                    tuning_config=tuning_config, options=options)


def _environment_checks(target):
    def native():
        from ..runtime.hip.library import library

        lib = library()
        return {"path": str(lib.path), "abi": lib.abi_version}

    return (EnvironmentCheck("hip native library", "provider_toolchain", native),)


PROVIDER = Provider(
    "gpu", HipTarget, None, None, _environment_checks,
    LocalExecution("cuda", True, frozenset({"workspace"}), partial(indexed_target, HipTarget), indexed_key,
                   torch_storage),
    "hip-direct", None, materialize=_materialize)
