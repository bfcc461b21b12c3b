"""Generated programs of the hip provider: generate, save, load and bind.

The reference keeps a generated program as three files (`python/intent/compiler/artifact.py:105-157`):
`kernel.source`, `kernel.mlir` and `artifact.json`, and reads `artifact.json` through its program
contract (`python/intent/runtime/contract.py:98-121`). That reader requires:

  provider          the registered provider name ("hip");
  entry_name        the diagnostic name;
  target            compiler facts whose `family` is the provider's execution model, read by the
                    provider's `read_target` (`python/intent/targets/specification.py:70-79`);
  compile_options   exactly numerics, optimizations and optimization_remarks
                    (`python/intent/compiler/options.py:51-58`);
  interface         the public parameter list (`python/intent/runtime/interface.py:110-150`);
  native            for a non-block execution model, the native slots, workspaces and entry
                    requirements (`python/intent/runtime/native.py:77-130`,
                    `python/intent/runtime/native_requirements.py:29-65`);

and hands the whole object to the provider's `read_facts`. A hip program writes all of these, so
the reference's own `GeneratedProgram.load(...)` accepts it, plus a `hip` object with the
provider's facts: the definition it maps to, its runtime signature, constexpr values, dimension
symbols, the C-ABI entry point, the library ABI version and the effective tuning table (the
provider's configuration rows, tuning_config families in place of their defaults).

The `native` section describes the C-ABI binding of every public parameter: a pointer, then an
i64 extent and an i64 stride per view axis, and each scalar by value. Views are "strided" (a
kernel reads unit-inner-stride rows, and other layouts are staged by the provider) and aligned to
their element. Every pair of views with a writable member must not overlap, except the exact
in-place alias of an Out and an input that the softmax kernels support.

`kernel.source` names the definition, the C-ABI entry point and the ABI version; `kernel.mlir`
states that the hip path has no KIR stage and lists the public interface.
"""
from __future__ import annotations

import enum
import inspect
import json
import tempfile
from dataclasses import dataclass
from pathlib import Path

from ..diagnostics import CompilationStageError
from .options import CompileOptions, read_options

FORMAT = "intent_amd.hip-program/2"

_SCALAR_CARRIERS = {"bool": "bool", "i8": "i8", "i16": "i16", "i32": "i32", "i64": "i64", "index": "i64",
                    "f32": "f32", "f64": "f64"}


def _encode_constexpr(value):
    if isinstance(value, enum.Enum):
        return {"enum": type(value).__name__, "name": value.name, "value": value.value}
    if isinstance(value, (bool, int, float, str)) or value is None:
        return value
    raise CompilationStageError("generated_program_export", f"constexpr value {value!r} is not serializable")


def _decode_constexpr(value):
    if isinstance(value, dict) and "enum" in value:
        return value["value"]          # the plans read enum constexprs by value
    return value


# ------------------------------------------------------------------------------ the program contract
@dataclass(frozen=True)
class HipFacts:
    """The hip provider's facts of one program (`artifact.json["hip"]`)."""

    definition: str
    signature: tuple
    constexprs: dict
    symbols: dict
    entry_point: str
    abi_version: int
    tuning: dict


def read_hip_facts(metadata: dict) -> HipFacts:
    """Read and check `metadata["hip"]`; the definition must match a kernel of this provider."""
    from ..runtime.hip.operators import recognize_saved

    hip = metadata["hip"]
    if not isinstance(hip, dict) or hip.get("format") != FORMAT:
        raise ValueError(f"artifact.json holds no hip program facts of format {FORMAT}")
    for key in ("definition", "signature", "constexprs", "symbols", "entry_point", "abi_version"):
        if key not in hip:
            raise KeyError(key)
    if type(hip["abi_version"]) is not int or hip["abi_version"] <= 0:
        raise ValueError("the hip ABI version is a positive integer")
    if not isinstance(hip["constexprs"], dict) or not isinstance(hip["symbols"], dict):
        raise TypeError("hip constexprs and symbols are JSON objects")
    signature = tuple(tuple(entry) for entry in hip["signature"])
    recognize_saved(hip["definition"], signature, tuple(hip["constexprs"]))
    from ..runtime.hip.tuning import table_from_metadata

    return HipFacts(hip["definition"], signature, dict(hip["constexprs"]), dict(hip["symbols"]),
                    hip["entry_point"], hip["abi_version"], table_from_metadata(hip.get("tuning")))


def _native_section(interface, inplace_safe: bool) -> dict:
    from ..runtime.interface import ViewParameter

    slots, views, disjoint = [], [], []
    for p in interface.parameters:
        if isinstance(p, ViewParameter):
            slots.append({"parameter": p.position, "role": "pointer", "carrier": "ptr", "element": p.dtype.name})
            for axis in range(len(p.shape)):
                slots.append({"parameter": p.position, "role": "extent", "carrier": "i64", "axis": axis})
                slots.append({"parameter": p.position, "role": "stride", "carrier": "i64", "axis": axis})
            views.append({"parameter": p.position, "layout": "strided", "alignment": p.dtype.itemsize})
        else:
            carrier = _SCALAR_CARRIERS.get(p.dtype.name)
            if carrier is None:
                raise CompilationStageError("provider_recognition",
                                            f"scalar {p.name} of dtype {p.dtype.name} has no native carrier")
            slots.append({"parameter": p.position, "role": "scalar", "carrier": carrier})
    view_params = [p for p in interface.parameters if isinstance(p, ViewParameter)]
    for i, left in enumerate(view_params):
        for right in view_params[i + 1:]:
            if not (left.writable or right.writable):
                continue
            if inplace_safe and left.writable != right.writable:
                continue                      # the exact in-place alias is allowed; other overlaps are refused
            disjoint.append({"left": left.position, "right": right.position})
    return {"slots": slots, "workspaces": [], "requirements": {"views": views, "disjoint": disjoint}}


def _check_native(native, interface) -> None:
    """The completeness rules of the reference's native ABI reader: every public parameter bound,
    every view axis with its extent and stride, a requirement per view, workspaces after the
    public arguments."""
    from ..runtime.interface import ViewParameter

    if not isinstance(native, dict):
        raise TypeError("native ABI metadata must be an object")
    count = len(interface.parameters)
    for offset, entry in enumerate(native["workspaces"]):
        if entry.get("position") != count + offset:
            raise ValueError("native workspaces must follow the public arguments in declaration order")
    seen = set()
    for entry in native["slots"]:
        position, role = entry["parameter"], entry["role"]
        if type(position) is not int or not 0 <= position < count + len(native["workspaces"]):
            raise ValueError("a native slot references an unknown parameter")
        identity = (position, role, entry.get("axis"))
        if identity in seen:
            raise ValueError("the native ABI binds a parameter slot twice")
        seen.add(identity)
    for p in interface.parameters:
        if isinstance(p, ViewParameter):
            if (p.position, "pointer", None) not in seen or any(
                    (p.position, role, axis) not in seen for axis in range(len(p.shape)) for role in ("extent", "stride")):
                raise ValueError(f"the native ABI does not bind every slot of view {p.name}")
        elif (p.position, "scalar", None) not in seen:
            raise ValueError(f"the native ABI does not bind scalar {p.name}")
    requirements = native["requirements"]
    declared = {entry["parameter"] for entry in requirements["views"]}
    for entry in requirements["views"]:
        if entry["layout"] not in ("strided", "contiguous") or type(entry["alignment"]) is not int \
                or entry["alignment"] <= 0:
            raise ValueError("a native view requirement has an unknown layout or a bad alignment")
    if declared != {p.position for p in interface.parameters if isinstance(p, ViewParameter)}:
        raise ValueError("the native entry must declare requirements for every public view")
    for entry in requirements["disjoint"]:
        left, right = entry["left"], entry["right"]
        if not (type(left) is int and type(right) is int and 0 <= left < right < count):
            raise ValueError("a native disjointness requirement names two ordered public views")


@dataclass(frozen=True)
class ProgramContract:
    """One parsed reading of a program's `artifact.json` (reference `runtime/contract.py:66-121`)."""

    provider: str
    target: object
    options: CompileOptions
    interface: object
    facts: object
    metadata: dict

    @classmethod
    def read(cls, source: str, metadata) -> "ProgramContract":
        from ..runtime.interface import PublicInterface
        from ..targets.provider import provider as get_provider
        from ..targets.specification import read_compilation_target

        if not isinstance(source, str) or not source.strip():
            raise ValueError("generated program source must be nonempty text")
        if not isinstance(metadata, dict):
            raise TypeError("generated program metadata must be an object")
        data = json.loads(json.dumps(metadata))
        try:
            name = data["provider"]
            if not isinstance(name, str) or not name:
                raise ValueError("provider must be a nonempty name")
            if not isinstance(data["entry_name"], str) or not data["entry_name"]:
                raise ValueError("generated entry name must be a nonempty name")
            target = read_compilation_target(name, data["target"])
            options = CompileOptions.read(data["compile_options"])
            interface = PublicInterface.read(data["interface"])
            adapter = get_provider(name)
            _check_native(data["native"], interface)
            if adapter.read_facts is None:
                raise NotImplementedError(f"provider {name!r} cannot read saved program facts")
            facts = adapter.read_facts(source, data, None)
        except KeyError as error:
            raise ValueError(f"generated program lacks required field {error}; regenerate it from its definition") \
                from error
        return cls(name, target, options, interface, facts, data)


# ------------------------------------------------------------------------------ GeneratedProgram
class GeneratedProgram:
    """Provider source, IR and metadata, with an optional process-local binding.

    load() restores the contract only; materialize() binds a runtime (reference
    `python/intent/compiler/artifact.py:39-185`)."""

    __slots__ = ("source", "ir", "cache_directory", "entry_name", "_binding", "_contract")

    def __init__(self, source: str, ir: str, metadata: dict, cache_directory, entry_name: str, _binding=None):
        contract = ProgramContract.read(source, metadata)
        if not isinstance(ir, str) or not ir.strip():
            raise ValueError("generated program IR must be nonempty text")
        if not isinstance(entry_name, str) or not entry_name.strip():
            raise ValueError("generated program requires a nonempty diagnostic name")
        self.source, self.ir, self.entry_name = source, ir, entry_name
        self.cache_directory = None if cache_directory is None else Path(cache_directory)
        self._binding, self._contract = _binding, contract

    def __repr__(self):
        return f"GeneratedProgram({self.entry_name!r}, provider={self._contract.provider!r})"

    @property
    def metadata(self) -> dict:
        """An inspection copy of the saved metadata; editing it changes nothing bound."""
        return json.loads(json.dumps(self._contract.metadata))

    @property
    def compile_options(self) -> CompileOptions:
        return self._contract.options

    @property
    def target(self):
        """The compiler facts this program was generated for."""
        return self._contract.target

    @property
    def interface(self):
        return self._contract.interface

    def save(self, directory) -> Path:
        """Write kernel.source, kernel.mlir and artifact.json into a new directory."""
        path = Path(directory).expanduser().absolute()
        try:
            if path.exists():
                raise FileExistsError(f"generated program destination already exists: {path}")
            path.parent.mkdir(parents=True, exist_ok=True)
            with tempfile.TemporaryDirectory(prefix=f".{path.name}-", dir=path.parent) as temporary:
                staging = Path(temporary) / "program"
                staging.mkdir()
                (staging / "kernel.source").write_text(self.source, encoding="utf-8")
                (staging / "kernel.mlir").write_text(self.ir, encoding="utf-8")
                (staging / "artifact.json").write_text(
                    json.dumps(self._contract.metadata, ensure_ascii=False, indent=2) + "\n", encoding="utf-8")
                staging.rename(path)
        except (OSError, UnicodeError, TypeError, ValueError) as error:
            raise CompilationStageError("generated_program_export", str(error)) from error
        return path

    @classmethod
    def load(cls, directory, *, name: str | None = None) -> "GeneratedProgram":
        """Load a saved program without loading native code; materialize() then needs a target."""
        path = Path(directory).expanduser().absolute()
        try:
            source = (path / "kernel.source").read_text(encoding="utf-8")
            ir = (path / "kernel.mlir").read_text(encoding="utf-8")
            metadata = json.loads((path / "artifact.json").read_text(encoding="utf-8"))
            if not source.strip() or not ir.strip() or not isinstance(metadata, dict):
                raise ValueError("generated program requires nonempty source, IR and object metadata")
            diagnostic = metadata["entry_name"] if name is None else name
            return cls(source, ir, metadata, path, diagnostic)
        except CompilationStageError as error:
            raise CompilationStageError("generated_program_loading", str(error)) from error
        except (OSError, UnicodeError, ValueError, KeyError, TypeError, NotImplementedError) as error:
            raise CompilationStageError("generated_program_loading", str(error)) from error

    def materialize(self, *, target=None):
        """Bind this program to a runtime target without regenerating it. A program generated
        for a local target reuses that binding; a loaded one needs `target` (a HipTarget, or an
        already resolved target)."""
        from ..targets.base import ResolvedTarget

        try:
            binding = target.resolve() if target is not None and not isinstance(target, ResolvedTarget) \
                else (target if target is not None else self._binding)
            if binding is None:
                raise ValueError("materialize requires an explicit runtime target for this generated program")
            if not isinstance(binding, ResolvedTarget):
                raise NotImplementedError("the selected target supplies compiler facts only; pass a runtime target")
            artifact = binding.materialize(self)
        except CompilationStageError:
            raise
        except Exception as error:
            raise CompilationStageError("generated_source_materialization", str(error)) from error
        artifact.cache_directory = self.cache_directory
        return artifact


# ------------------------------------------------------------------------------ binding
def bind_program(program, target):
    """The hip provider's `bind`: a CompiledArtifact of `program` on the resolved `target`.

    Reads only the program's public attributes and its metadata, so a program object of the
    reference's own package binds the same way as this package's."""
    from ..runtime.artifact import CompiledArtifact
    from ..runtime.hip.library import library
    from ..runtime.hip.operators import recognize_saved
    from ..runtime.hip.program import HipProgram
    from ..runtime.interface import PublicInterface

    metadata = program.metadata
    facts = read_hip_facts(metadata)
    options = CompileOptions.read(metadata["compile_options"])
    if library().abi_version < facts.abi_version:
        raise CompilationStageError("native_loading",
                                    f"libintent_hip.so has ABI {library().abi_version}, the program needs "
                                    f"{facts.abi_version}")
    spec = recognize_saved(facts.definition, facts.signature, tuple(facts.constexprs))
    constexprs = {name: _decode_constexpr(value) for name, value in facts.constexprs.items()}
    interface = PublicInterface.read(metadata["interface"])
    runtime = HipProgram(spec, interface, dict(facts.symbols), constexprs, target, numerics=options.numerics,
                         tuning=facts.tuning)
    return CompiledArtifact(program.source, program.ir, target.device, runtime, None, device_type="cuda",
                            cache_directory=program.cache_directory)


# ------------------------------------------------------------------------------ generation
def _resolve(target):
    """(compiler facts, runtime binding or None) of `target` (reference `compiler/pipeline.py:126-135`)."""
    from ..targets.base import ResolvedTarget
    from ..targets.specification import CompilationTarget

    try:
        resolved = target if isinstance(target, ResolvedTarget) else target.resolve()
        if isinstance(resolved, ResolvedTarget):
            return resolved.compilation, resolved
        if isinstance(resolved, CompilationTarget):
            return resolved, None
        raise TypeError("target resolution must provide compiler facts or a runtime binding")
    except CompilationStageError:
        raise
    except Exception as error:
        raise CompilationStageError("target_resolution", str(error)) from error


def constexpr_values(definition, constexprs: dict) -> dict:
    """Every constexpr parameter's value: the caller's, else the declared default."""
    from ..runtime.hip.program import _constexpr_parameters

    declared = _constexpr_parameters(definition)
    names = tuple(name for name, _ in declared)
    unknown = set(constexprs) - set(names)
    if unknown:
        raise CompilationStageError("frontend", f"unknown constexpr argument {sorted(unknown)[0]!r}")
    values = {}
    for name, default in declared:
        if name in constexprs:
            values[name] = constexprs[name]
        elif default is not inspect.Parameter.empty:
            values[name] = default
        else:
            raise CompilationStageError("frontend", f"constexpr parameter {name!r} requires a value")
    return values


def generate(definition, *, target, compiler=None, constexprs: dict | None = None, tuning_config=None,
             options=None) -> GeneratedProgram:
    """Map `definition` to its hip kernel and return the program without launching anything
    (reference signature: `python/intent/compiler/pipeline.py:37-49`).

    `target` is a HipTarget, a resolved hip target (kept as the program's process-local binding)
    or a HipCompilationTarget (compiler facts only: the program can be saved, and materialized
    later with a runtime target)."""
    from ..runtime.hip.library import ABI_VERSION
    from ..runtime.hip.operators import recognize, signature_of
    from ..runtime.hip.program import _symbols
    from ..runtime.interface import PublicInterface

    if compiler is not None:
        raise CompilationStageError("provider_configuration",
                                    "the hip provider has no compiler stage; compiler must be None")
    from ..runtime.hip.tuning import DEFAULT_FAMILIES, read_tuning_config, table_metadata

    table = dict(DEFAULT_FAMILIES) if tuning_config is None else read_tuning_config(tuning_config)
    try:
        policy = read_options(options)
    except (TypeError, ValueError) as error:
        raise CompilationStageError("provider_configuration", str(error)) from error
    compilation, binding = _resolve(target)
    values = constexpr_values(definition, dict(constexprs or {}))
    interface = PublicInterface.from_definition(definition, values)
    spec = recognize(definition, interface, tuple(values))
    entry = spec.entry_point
    source = (f"// hip provider program: {spec.name}\n"
              f"// definition {spec.name} runs a hand-written {compilation.architecture} kernel of "
              f"libintent_hip.so through {entry} (C ABI version {ABI_VERSION}, include/intent_hip.h).\n")
    parameters = "\n".join(f"//   {p.name}: {p}" for p in interface.parameters)
    ir = (f"// The hip path has no KIR stage: the definition is recognised by name and signature.\n"
          f"// Public interface of {spec.name}:\n{parameters}\n")
    metadata = {
        "provider": compilation.provider,
        "entry_name": spec.name,
        "target": compilation.metadata(),
        "compile_options": policy.metadata(),
        "interface": interface.to_json(),
        "native": _native_section(interface, spec.inplace_safe),
        "hip": {"format": FORMAT, "definition": spec.name,
                "signature": [list(item) for item in signature_of(interface)],
                "constexprs": {name: _encode_constexpr(value) for name, value in values.items()},
                "symbols": _symbols(definition, values), "entry_point": entry, "abi_version": ABI_VERSION,
                "tuning": table_metadata(table)},
    }
    try:
        return GeneratedProgram(source, ir, metadata, None, spec.name, _binding=binding)
    except (ValueError, KeyError, TypeError, NotImplementedError) as error:
        raise CompilationStageError("provider_generation", str(error)) from error
