"""The hip runtime object behind `CompiledArtifact.runtime`.

Implements the runtime contract the reference's `CompiledArtifact` expects
(`python/intent/runtime/artifact.py:16-58`, `integrations/torch.py:11-14`):
`prepare_call`, `run`, `launch`, `interface`, `infer_outputs`, `observation`,
`close`. Its prepared call follows `python/intent/runtime/block/program.py:33-82`:
binding happens once, `launch()` replays the bound native call on the caller's
current stream, asynchronously; `result()` does not synchronize.
"""
from __future__ import annotations

import threading

from ...diagnostics import CompilationStageError
from ..artifact import CompiledArtifact
from ..diagnostics import ConfigurationAssessment, NativeObservation, NativeResource
from ..interface import PublicInterface, ViewParameter
from ..invocation import bind_arguments
from ..torch_views import allocate_output, observe_view
from .library import library
from .operators import OperatorSpec, numerics_policy, tuning_policy, workspace_policy
from .tuning import FAMILY_OF, SPLIT, TuningConfiguration


def _symbols(definition, constexprs) -> dict[str, int]:
    """Symbol name -> dimension identity, numbered as `PublicInterface.from_definition` does."""
    symbols: dict[str, int] = {}
    for parameter in definition.signature.parameters.values():
        annotation = parameter.annotation
        if all(hasattr(annotation, f) for f in ("kind", "dtype", "shape", "constraints")):
            for extent in annotation.shape:
                if isinstance(extent, str) and extent not in constexprs:
                    symbols.setdefault(extent, len(symbols) + 1)
    return symbols


def _constexpr_parameters(definition) -> tuple[tuple[str, object], ...]:
    out = []
    for name, parameter in definition.signature.parameters.items():
        annotation = parameter.annotation
        if hasattr(annotation, "value_type") and not hasattr(annotation, "kind"):
            out.append((name, parameter.default))
    return tuple(out)


def _raw_stream_getter():
    """Fast accessor of the current HIP stream handle of a device (an int)."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw
    return lambda index: torch.cuda.current_stream(index).cuda_stream


class HipPreparedCall:
    """Bound arguments, allocated outputs/workspace and the native call that uses them."""

    def __init__(self, program: "HipProgram", bound, launch):
        import torch

        self._program, self._bound, self._launch = program, bound, launch
        self._index = program.device.index
        self._run = launch.run
        self._before, self._after = launch.before, launch.after
        self._current_device = torch.cuda.current_device
        self._stream = _raw_stream_getter()
        self._launched = False

    def compile(self) -> None:
        """Kernels are compiled ahead of time into libintent_hip.so; nothing to do."""

    def launch(self) -> None:
        index = self._index
        previous = self._current_device()
        if previous != index:
            import torch

            torch.cuda.set_device(index)
        try:
            for step in self._before:
                step()
            status = self._run(self._stream(index))
            if status != 0:
                raise CompilationStageError("provider_invocation",
                                            f"{self._launch.entry}: {self._program.library.error(status)}")
            for step in self._after:
                step()
        finally:
            if previous != index:
                import torch

                torch.cuda.set_device(previous)
        self._launched = True
        self._program._last_launch = self._launch

    def result(self):
        return self._bound.result()

    @property
    def observation(self):
        """Facts of the kernel this call launched (read on demand; None before the first launch)."""
        return self._program.observe(self._launch) if self._launched else None

    def inspect_configurations(self) -> tuple:
        """Every row of the definition's tuning family (the chosen one first) with its eligibility
        and the reasons of an ineligible one; one fixed configuration otherwise."""
        candidates = self._launch.candidates
        if not candidates:
            return (ConfigurationAssessment(self._launch.configuration, True, ()),)
        chosen = dict(self._launch.configuration).get("split")
        ordered = sorted(candidates, key=lambda c: (c[0][0] != chosen or not c[1]))
        return tuple(ConfigurationAssessment(self._launch.configuration if row[0] == chosen else (("split", row[0]),),
                                             eligible, reasons)
                     for row, eligible, reasons in ordered)


class HipProgram:
    def __init__(self, spec: OperatorSpec, interface: PublicInterface, symbols: dict, constexprs: dict, target,
                 *, numerics: str = "source", tuning: dict | None = None):
        import torch

        from .tuning import DEFAULT_FAMILIES

        self.spec, self.interface, self.constexprs, self.target = spec, interface, dict(constexprs), target
        self.numerics = numerics
        self.tuning_family = FAMILY_OF.get(spec.name)
        table = DEFAULT_FAMILIES if tuning is None else tuning
        self.tuning_rows = table.get(self.tuning_family) if self.tuning_family else None
        self.workspace = getattr(target, "workspace", "prepare")
        self.device = torch.device("cuda", target.device)
        self.library = library()
        self._derived = {symbols[name]: (symbols[source], offset) for name, source, offset in spec.derived
                         if name in symbols and source in symbols}
        self._last_launch = None
        self._lock = threading.Lock()
        self._closed = False

    @property
    def derivable_dimensions(self) -> frozenset:
        """Dimension identities whose extents follow from other dimensions (csr_spmv's R = R1 - 1)."""
        return frozenset(self._derived)

    # -- binding ------------------------------------------------------------------------------
    def _bind(self, arguments, outputs, *, abstract=False):
        device = self.device
        return bind_arguments(
            self.interface, tuple(arguments), outputs,
            observe_view=lambda p, v: observe_view(p, v, device=device, abstract=abstract),
            allocate_output=lambda p, shape: allocate_output(p, shape, device=device, abstract=abstract),
            abstract=abstract, derived=self._derived)

    def _check_writable_overlap(self, bound) -> None:
        """Writable views may not overlap another view, except an exact in-place alias that the
        kernel supports (same address and strides; each element is read before it is written)."""
        views = [(p, f) for p, f in zip(self.interface.parameters, bound.views) if isinstance(p, ViewParameter)]
        for i, (left, lf) in enumerate(views):
            for right, rf in views[i + 1:]:
                if not (left.writable or right.writable):
                    continue
                if not (lf.begin < lf.end and rf.begin < rf.end and lf.begin < rf.end and rf.begin < lf.end):
                    continue
                exact = (lf.pointer == rf.pointer and lf.shape == rf.shape and lf.strides == rf.strides)
                if exact and self.spec.inplace_safe and not (left.writable and right.writable):
                    continue
                raise ValueError(f"{left.name} and {right.name} overlap; the hip kernel for "
                                 f"{self.spec.name} requires writable views that do not alias other views")

    def prepare_call(self, arguments: tuple, *, outputs: tuple | None = None) -> HipPreparedCall:
        if self._closed:
            raise RuntimeError("hip program is closed")
        if outputs is not None and not isinstance(outputs, tuple):
            raise TypeError("outputs must be a tuple in declared Out order")
        bound = self._bind(arguments, outputs)
        self._check_writable_overlap(bound)
        with workspace_policy(self.workspace), numerics_policy(self.numerics), tuning_policy(self.tuning_rows):
            launch = self.spec.plan(self.library, bound, self.constexprs, self.device)
        return HipPreparedCall(self, bound, launch)

    def run(self, *arguments):
        call = self.prepare_call(arguments)
        call.launch()
        return call.result()

    def launch(self, *arguments) -> None:
        inputs, outputs = self.interface.split_arguments(tuple(arguments))
        self.prepare_call(inputs, outputs=outputs).launch()

    def tuning_configurations(self, *arguments) -> tuple:
        """The eligible rows of this definition's tuning family for `arguments` (every runtime
        argument, explicit Out buffers included), in table order; () for a definition the hip
        kernels run in one fixed configuration. Binding may allocate, nothing is launched."""
        if self.tuning_family is None:
            return ()
        inputs, outputs = self.interface.split_arguments(tuple(arguments))
        call = self.prepare_call(inputs, outputs=outputs)
        return tuple(TuningConfiguration((SPLIT,), row) for row, eligible, _ in call._launch.candidates if eligible)

    def infer_outputs(self, arguments: tuple):
        """Out buffers for `arguments` without touching device pointers (fake/meta tensors)."""
        import torch

        device = arguments[0].device if arguments and hasattr(arguments[0], "device") else self.device
        bound = bind_arguments(
            self.interface, tuple(arguments), None,
            observe_view=lambda p, v: observe_view(p, v, device=device, abstract=True),
            allocate_output=lambda p, shape: allocate_output(p, shape, device=device, abstract=True),
            abstract=True, derived=self._derived)
        del torch
        return bound.result()

    # -- observation ----------------------------------------------------------------------------
    def observe(self, launch) -> NativeObservation:
        facts = launch.resources() or {}
        resources = tuple(NativeResource(name, facts.get(name), unit, "hipFuncGetAttributes", "launch",
                                         None if name in facts else "not reported")
                          for name, unit in (("vgprs", "registers"), ("lds_bytes", "bytes"),
                                             ("scratch_bytes", "bytes"), ("block_threads", "threads")))
        return NativeObservation("hip", launch.entry, facts.get("kernel", ""), launch.configuration, resources)

    @property
    def observation(self):
        """Facts of the most recent launch of this program, or None before one."""
        return None if self._last_launch is None else self.observe(self._last_launch)

    def close(self) -> None:
        self._closed = True
