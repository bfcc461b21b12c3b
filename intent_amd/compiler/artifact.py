"""Saved programs of the hip provider.

The reference saves a generated program as a directory with three files (reference
`python/intent/compiler/artifact.py:105-157`): `kernel.source` (provider source), `kernel.mlir`
(final IR) and `artifact.json` (compiler metadata), and restores it without loading native code;
`materialize(target=...)` binds it to a runtime (`:159-...`). On the hip path a program is the
binding of a recognised definition to a hand-written kernel of libintent_hip.so, so:

  kernel.source  names the definition, the C-ABI entry point and the library ABI version;
  kernel.mlir    states that the hip path has no KIR stage, and lists the public interface;
  artifact.json  holds everything materialize() needs without the definition object: entry name,
                 definition name and signature, constexpr values, dimension symbols, the public
                 interface (the reference compiler's JSON form), target facts, ABI version and
                 compile options.
"""
from __future__ import annotations

import enum
import json
import tempfile
from pathlib import Path

from ..diagnostics import CompilationStageError

FORMAT = "intent_amd.hip-program/1"


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


class GeneratedProgram:
    """Provider source, IR and metadata, with an optional process-local target binding."""

    __slots__ = ("source", "ir", "cache_directory", "entry_name", "_metadata", "_binding")

    def __init__(self, source: str, ir: str, metadata: dict, cache_directory: Path | None, entry_name: str,
                 _binding=None):
        if not isinstance(source, str) or not source.strip() or not isinstance(ir, str) or not ir.strip():
            raise ValueError("generated program requires nonempty source and IR text")
        if not isinstance(metadata, dict) or metadata.get("format") != FORMAT:
            raise ValueError(f"artifact.json is not a hip program ({FORMAT})")
        for key in ("definition", "signature", "constexprs", "symbols", "interface", "abi_version"):
            if key not in metadata:
                raise KeyError(f"artifact.json lacks {key!r}")
        if not isinstance(entry_name, str) or not entry_name.strip():
            raise ValueError("generated program requires a nonempty diagnostic name")
        self.source, self.ir, self.entry_name = source, ir, entry_name
        self.cache_directory = None if cache_directory is None else Path(cache_directory)
        self._metadata = json.loads(json.dumps(metadata))
        self._binding = _binding

    def __repr__(self):
        return f"GeneratedProgram({self.entry_name!r}, definition={self._metadata['definition']!r})"

    @property
    def metadata(self) -> dict:
        """An inspection copy of the saved metadata."""
        return json.loads(json.dumps(self._metadata))

    @property
    def compile_options(self) -> dict:
        return dict(self._metadata.get("options", {"numerics": "source"}))

    @property
    def target(self) -> dict:
        return dict(self._metadata.get("target", {}))

    @property
    def interface(self):
        from ..runtime.interface import PublicInterface

        return PublicInterface.read(self._metadata["interface"])

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
                (staging / "artifact.json").write_text(json.dumps(self._metadata, ensure_ascii=False, indent=2) + "\n",
                                                       encoding="utf-8")
                staging.rename(path)
        except (OSError, UnicodeError, TypeError, ValueError) as error:
            raise CompilationStageError("generated_program_export", str(error)) from error
        return path

    @classmethod
    def load(cls, directory, *, name: str | None = None) -> "GeneratedProgram":
        """Load a saved program without loading native code; materialize() needs a target."""
        path = Path(directory).expanduser().absolute()
        try:
            source = (path / "kernel.source").read_text(encoding="utf-8")
            ir = (path / "kernel.mlir").read_text(encoding="utf-8")
            metadata = json.loads((path / "artifact.json").read_text(encoding="utf-8"))
            if not isinstance(metadata, dict):
                raise ValueError("artifact.json must hold an object")
            return cls(source, ir, metadata, path, metadata.get("entry_name") if name is None else name)
        except (OSError, UnicodeError, ValueError, KeyError, TypeError) as error:
            raise CompilationStageError("generated_program_loading", str(error)) from error

    def materialize(self, *, target=None):
        """Bind this program to a hip target (a resolved target, or a HipTarget to resolve)."""
        from ..runtime.artifact import CompiledArtifact
        from ..runtime.hip.library import library
        from ..runtime.hip.operators import recognize_saved
        from ..runtime.hip.program import HipProgram

        if target is None:
            target = self._binding
        if target is None:
            raise CompilationStageError("generated_program_materialization",
                                        "a loaded program has no runtime device; pass target=")
        if hasattr(target, "resolve") and not hasattr(target, "architecture"):
            target = target.resolve()
        architecture = getattr(target, "architecture", None)
        saved = self._metadata.get("target", {}).get("architecture")
        if saved and architecture and saved != architecture:
            raise CompilationStageError("target_resolution",
                                        f"program was generated for {saved}, target is {architecture}")
        if library().abi_version < int(self._metadata["abi_version"]):
            raise CompilationStageError("native_loading", "libintent_hip.so is older than this program's ABI")
        meta = self._metadata
        constexprs = {name: _decode_constexpr(value) for name, value in meta["constexprs"].items()}
        spec = recognize_saved(meta["definition"], tuple(tuple(entry) for entry in meta["signature"]),
                               tuple(meta["constexprs"]))
        program = HipProgram(spec, self.interface, dict(meta["symbols"]), constexprs, target)
        return CompiledArtifact(self.source, self.ir, target.device, program, None, device_type="cuda",
                                cache_directory=self.cache_directory)


def generate(definition, *, target, compiler=None, constexprs: dict | None = None, tuning_config=None,
             options=None) -> GeneratedProgram:
    """Map `definition` to its hip kernel and return the program without launching anything
    (reference signature: `python/intent/compiler/pipeline.py:37-49`). `target` is a HipTarget or a
    resolved hip target; it is kept as the program's process-local binding."""
    import inspect

    from ..runtime.hip.library import ABI_VERSION
    from ..runtime.hip.operators import recognize, signature_of
    from ..runtime.hip.program import _constexpr_parameters, _symbols
    from ..runtime.interface import PublicInterface

    if tuning_config is not None:
        raise CompilationStageError("provider_configuration",
                                    "the hip provider has fixed kernel configurations; tuning_config is not accepted")
    numerics = getattr(options, "numerics", "source") if options is not None else "source"
    if numerics != "source":
        raise CompilationStageError("provider_configuration", "the hip provider supports numerics='source' only")
    constexprs = dict(constexprs or {})
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
    interface = PublicInterface.from_definition(definition, values)
    spec = recognize(definition, interface, names)
    resolved = target.resolve() if hasattr(target, "resolve") and not hasattr(target, "architecture") else target
    entry = getattr(spec.plan, "__name__", spec.name)
    source = (f"// hip provider program: {spec.name}\n"
              f"// definition {spec.name} runs a hand-written gfx950 kernel of libintent_hip.so "
              f"(C ABI version {ABI_VERSION}, include/intent_hip.h); launch plan {entry}.\n")
    parameters = "\n".join(f"//   {p.name}: {p}" for p in interface.parameters)
    ir = (f"// The hip path has no KIR stage: the definition is recognised by name and signature.\n"
          f"// Public interface of {spec.name}:\n{parameters}\n")
    metadata = {
        "format": FORMAT,
        "entry_name": spec.name,
        "definition": spec.name,
        "signature": [list(entry) for entry in signature_of(interface)],
        "constexprs": {name: _encode_constexpr(value) for name, value in values.items()},
        "symbols": _symbols(definition, values),
        "interface": interface.to_json(),
        "target": {"provider": "hip", "architecture": getattr(resolved, "architecture", None)},
        "abi_version": ABI_VERSION,
        "options": {"numerics": numerics},
    }
    return GeneratedProgram(source, ir, metadata, None, spec.name, _binding=resolved)
