"""The hip provider against the reference's target and program contracts, without a GPU.

The protocols below are restated from the reference, member for member:
  ResolvedTarget     python/intent/targets/base.py:12-19 (compilation, materialize);
  CompilationTarget  python/intent/targets/specification.py:56-67 (provider, compiler_options,
                     compiler_role).
The reference's JIT refuses a backend whose resolved local target is not a ResolvedTarget
(jit/kernel.py:55-57), and GeneratedProgram.materialize requires one (compiler/artifact.py:169-177).
A saved program is read by the reference's ProgramContract.read (runtime/contract.py:98-121): the
fields checked below are the ones that reader takes, with the shapes its readers require.
"""
from __future__ import annotations

import json
from types import SimpleNamespace
from typing import Protocol, runtime_checkable

import pytest

import intent_amd as intent
from intent_amd.examples.kernels.contraction.gemm import Activation, gemm
from intent_amd.examples.kernels.normalization.softmax import stable_softmax_f16
from intent_amd.examples.kernels.sparse.csr_spmv import csr_spmv
from intent_amd.examples.kernels.streaming.attention import flash_attention_fwd
from intent_amd.runtime.interface import PublicInterface
from intent_amd.targets.hip import PROVIDER, HipCompilationTarget, HipTarget, ResolvedHipTarget


@runtime_checkable
class ReferenceResolvedTarget(Protocol):
    @property
    def compilation(self): ...

    def materialize(self, program): ...


@runtime_checkable
class ReferenceCompilationTarget(Protocol):
    @property
    def provider(self) -> str: ...

    @property
    def compiler_options(self) -> tuple[str, ...]: ...

    @property
    def compiler_role(self) -> str: ...


def resolved(**changes):
    """A resolved gfx950 device as HipTarget.resolve() returns it, built without a GPU."""
    fields = dict(device=0, architecture="gfx950", compute_units=256, wavefront_size=64,
                  lds_per_workgroup=163840, global_memory_bytes=288 << 30)
    fields.update(changes)
    return ResolvedHipTarget(**fields)


def test_resolved_target_satisfies_the_reference_protocols():
    target = resolved()
    assert isinstance(target, ReferenceResolvedTarget)
    facts = target.compilation
    assert isinstance(facts, ReferenceCompilationTarget) and not isinstance(facts, ReferenceResolvedTarget)
    assert facts == HipCompilationTarget("hip", "gfx950", 64, 163840)
    assert facts.resolve() is facts
    assert facts.compiler_options[0] == "--target=hip"
    assert json.loads(facts.compiler_options[1].split("=", 1)[1]) == {
        "architecture": "gfx950", "lds_per_workgroup": 163840, "wavefront_size": 64}
    # the compute units and memory size are runtime facts, not compiler facts
    assert resolved(compute_units=32, global_memory_bytes=1).compilation == facts
    assert resolved(wavefront_size=32).compilation != facts
    with pytest.raises(ValueError):
        HipCompilationTarget("hip", "gfx942", 64, 163840)


def test_provider_exports_every_contract_callable():
    """targets/provider.py:40-49: read_facts, bind and read_target are callables the reference
    calls when it loads and binds a saved program."""
    assert PROVIDER.execution_model == "hip-direct"
    assert callable(PROVIDER.read_facts) and callable(PROVIDER.bind) and callable(PROVIDER.read_target)
    target = PROVIDER.read_target("hip", {"architecture": "gfx950", "wavefront_size": 64, "lds_per_workgroup": 163840})
    assert target == resolved().compilation
    for bad in ({"architecture": "gfx950", "wavefront_size": 64},
                {"architecture": "gfx950", "wavefront_size": 64, "lds_per_workgroup": 163840, "extra": 1}):
        with pytest.raises(ValueError):
            PROVIDER.read_target("hip", bad)
    assert PROVIDER.local.device_kind == "cuda" and PROVIDER.local.indexed
    with pytest.raises(ValueError):
        HipTarget(-1)


def test_jit_refuses_a_local_target_that_is_not_resolved(monkeypatch):
    """jit/kernel.py:55-57: NotImplementedError('<backend> has no local executable target')."""
    import importlib

    jit_module = importlib.import_module("intent_amd.jit.kernel")

    monkeypatch.setattr(jit_module, "resolve_local", lambda *a, **k: SimpleNamespace(device=0))
    kernel = intent.jit(stable_softmax_f16, backend="hip", device="cuda:0")
    with pytest.raises(NotImplementedError, match="hip has no local executable target"):
        kernel.prepare(SimpleNamespace(shape=(2, 2), device="cuda:0"))     # a stand-in tensor placed on cuda:0


def test_saved_program_carries_the_reference_contract(tmp_path):
    program = intent.generate(gemm, target=resolved().compilation, constexprs={"ACTIVATION": Activation.RELU})
    path = program.save(tmp_path / "gemm_relu")
    assert sorted(p.name for p in path.iterdir()) == ["artifact.json", "kernel.mlir", "kernel.source"]
    metadata = json.loads((path / "artifact.json").read_text())
    assert {"provider", "entry_name", "target", "compile_options", "interface", "native"} <= set(metadata)
    assert metadata["provider"] == "hip" and metadata["entry_name"] == "gemm"
    assert metadata["target"] == {"family": "hip-direct", "architecture": "gfx950", "wavefront_size": 64,
                                  "lds_per_workgroup": 163840}
    assert metadata["compile_options"] == {"numerics": "source", "optimizations": {}, "optimization_remarks": False}
    assert metadata["hip"]["entry_point"] == "intent_hip_gemm"
    assert metadata["hip"]["constexprs"]["ACTIVATION"] == {"enum": "Activation", "name": "RELU", "value": 1}
    native = metadata["native"]
    # three rank-2 views: a pointer, then an extent and a stride per axis
    assert len(native["slots"]) == 3 * 5 and native["workspaces"] == []
    assert [s["role"] for s in native["slots"][:5]] == ["pointer", "extent", "stride", "extent", "stride"]
    assert native["slots"][0] == {"parameter": 0, "role": "pointer", "carrier": "ptr", "element": "f16"}
    assert native["requirements"]["views"] == [{"parameter": i, "layout": "strided", "alignment": 2} for i in range(3)]
    assert native["requirements"]["disjoint"] == [{"left": 0, "right": 2}, {"left": 1, "right": 2}]
    loaded = intent.GeneratedProgram.load(path)
    assert loaded.metadata == program.metadata and loaded.target == program.target
    assert loaded.compile_options == intent.CompileOptions()
    assert loaded.interface.to_json() == PublicInterface.from_definition(
        gemm, {"ACTIVATION": Activation.RELU}).to_json()
    with pytest.raises(intent.CompilationStageError):
        program.save(path)                                     # never overwrites


@pytest.mark.parametrize("definition,constexprs,slots,disjoint", [
    (stable_softmax_f16, {}, 2 * 5, []),                       # Out may be exactly the input
    (csr_spmv, {}, 5 * 3, [{"left": i, "right": 4} for i in range(4)]),
    (flash_attention_fwd, {"CAUSAL": True}, 4 * 9 + 1, [{"left": i, "right": 3} for i in range(3)]),
])
def test_native_section_binds_every_parameter(definition, constexprs, slots, disjoint):
    metadata = intent.generate(definition, target=resolved(), constexprs=constexprs).metadata
    assert len(metadata["native"]["slots"]) == slots
    assert metadata["native"]["requirements"]["disjoint"] == disjoint
    if definition is flash_attention_fwd:
        assert metadata["native"]["slots"][-1] == {"parameter": 4, "role": "scalar", "carrier": "f32"}


def test_materialize_binds_through_the_resolved_target(tmp_path):
    path = intent.generate(gemm, target=HipCompilationTarget("hip", "gfx950", 64, 163840),
                           constexprs={"ACTIVATION": Activation.RELU}).save(tmp_path / "p")
    loaded = intent.GeneratedProgram.load(path)
    with pytest.raises(intent.CompilationStageError) as error:
        loaded.materialize()                                   # a loaded program has no device
    assert error.value.stage == "generated_source_materialization"
    with pytest.raises(intent.CompilationStageError):
        loaded.materialize(target=HipCompilationTarget("hip", "gfx950", 64, 163840))   # facts only
    artifact = loaded.materialize(target=resolved())
    assert artifact.cache_directory == path
    assert artifact.interface.to_json() == loaded.interface.to_json()
    assert artifact.runtime.constexprs == {"ACTIVATION": 1} and artifact.runtime.numerics == "source"
    with pytest.raises(intent.CompilationStageError):
        loaded.materialize(target=resolved(wavefront_size=32))   # other compiler facts
    # the reference's GeneratedProgram binds through the same bind with only its public attributes
    foreign = SimpleNamespace(source=loaded.source, ir=loaded.ir, metadata=loaded.metadata, target=loaded.target,
                              cache_directory=path, entry_name=loaded.entry_name)
    assert resolved().materialize(foreign).runtime.spec.name == "gemm"
    relaxed = intent.generate(gemm, target=resolved(), constexprs={"ACTIVATION": Activation.NONE},
                              options=intent.CompileOptions(numerics="relaxed_normalization")).materialize()
    assert relaxed.runtime.numerics == "relaxed_normalization"


@pytest.mark.parametrize("field,edit", [
    ("compile_options", lambda m: m["compile_options"].pop("optimizations")),
    ("target", lambda m: m["target"].update(family="block")),
    ("target", lambda m: m["target"].pop("lds_per_workgroup")),
    ("native", lambda m: m["native"]["slots"].pop()),
    ("native", lambda m: m["native"]["requirements"]["views"].pop()),
    ("hip", lambda m: m["hip"]["signature"][0].__setitem__(2, "bf16")),
    ("provider", lambda m: m.pop("provider")),
])
def test_load_rejects_a_broken_contract(tmp_path, field, edit):
    path = intent.generate(gemm, target=resolved(), constexprs={"ACTIVATION": Activation.RELU}).save(tmp_path / "p")
    metadata = json.loads((path / "artifact.json").read_text())
    edit(metadata)
    (path / "artifact.json").write_text(json.dumps(metadata))
    with pytest.raises(intent.CompilationStageError) as error:
        intent.GeneratedProgram.load(path)
    assert error.value.stage == "generated_program_loading"


def test_generate_refuses_what_the_hip_path_cannot_honour():
    with pytest.raises(intent.CompilationStageError):
        intent.generate(gemm, target=resolved(), compiler="/usr/bin/intent-compile")
    with pytest.raises(intent.CompilationStageError) as error:
        intent.generate(gemm, target=SimpleNamespace(device=0))
    assert error.value.stage == "target_resolution"


def test_tuning_config_rows_are_read_and_saved(tmp_path):
    """jit/generate(tuning_config=path): the reference's table form ({"columns", "families"}); a
    supplied family replaces its default rows, others keep theirs; rows outside what the kernels
    implement, unknown families and malformed files are CompilationStageError at generation; a
    saved program keeps its rows."""
    from intent_amd.examples.kernels.backward.attention import attention_backward_dq
    from intent_amd.runtime.hip.tuning import DEFAULT_FAMILIES

    config = tmp_path / "tuning.json"
    config.write_text(json.dumps({"columns": ["split"], "families": {"hip.attention_backward": [[0]]}}))
    program = intent.generate(attention_backward_dq, target=resolved(), tuning_config=config,
                              constexprs={"HEAD_GROUP": 1, "CAUSAL": True})
    tuning = program.metadata["hip"]["tuning"]
    assert tuning["families"]["hip.attention_backward"] == [[0]]
    assert tuning["families"]["hip.latent_prefill"] == [list(r) for r in DEFAULT_FAMILIES["hip.latent_prefill"]]
    loaded = intent.GeneratedProgram.load(program.save(tmp_path / "p"))
    artifact = loaded.materialize(target=resolved())
    assert artifact.runtime.tuning_family == "hip.attention_backward" and artifact.runtime.tuning_rows == ((0,),)
    default = intent.generate(attention_backward_dq, target=resolved(), constexprs={"HEAD_GROUP": 1, "CAUSAL": True})
    assert default.materialize().runtime.tuning_rows == ((1,), (0,))
    assert intent.generate(gemm, target=resolved(), tuning_config=config,
                           constexprs={"ACTIVATION": Activation.NONE}).materialize().runtime.tuning_family is None
    from intent_amd.examples.kernels.streaming.attention import (flash_attention_bf16_fwd, flash_attention_fwd,
                                                                  flash_gqa_attention_fwd)
    for defn, constexprs in ((flash_attention_fwd, {"CAUSAL": True}),
                             (flash_gqa_attention_fwd, {"HEAD_GROUP": 2, "CAUSAL": True}),
                             (flash_attention_bf16_fwd, {"HEAD_GROUP": 2, "CAUSAL": False})):
        runtime = intent.generate(defn, target=resolved(), constexprs=constexprs).materialize().runtime
        assert runtime.tuning_family == "hip.attention_forward" and runtime.tuning_rows == ((1,), (0,))
    for bad in ({"columns": ["split"], "families": {"hip.attention_backward": [[2]]}},
                {"columns": ["split"], "families": {"hip.nonexistent": [[0]]}},
                {"columns": ["tile"], "families": {}},
                {"columns": ["split"], "families": {"hip.latent_prefill": []}},
                {"families": {}}):
        config.write_text(json.dumps(bad))
        with pytest.raises(intent.CompilationStageError) as error:
            intent.generate(attention_backward_dq, target=resolved(), tuning_config=config,
                            constexprs={"HEAD_GROUP": 1, "CAUSAL": True})
        assert error.value.stage == "provider_configuration"
    with pytest.raises(intent.CompilationStageError):
        intent.generate(gemm, target=resolved(), tuning_config=tmp_path / "missing.json",
                        constexprs={"ACTIVATION": Activation.NONE})
