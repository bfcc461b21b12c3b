"""CPU tests of the host surface: annotations, definitions, device selection, the JIT call split,
tensor observation, PyTorch operator registration and the attention-backward program.

Error classes follow the reference's surface (python/intent/language/annotations.py,
api/definitions.py, targets/local.py:33-68, jit/kernel.py:14-133, runtime/torch_views.py:23-88,
integrations/torch.py:27-93)."""
from types import SimpleNamespace

import pytest
import torch

import intent_amd as intent
import intent_amd.language as I
from intent_amd.integrations.torch import operator_schema, register_operator, torch_dtype
from intent_amd.jit.kernel import _CallRoles
from intent_amd.runtime.interface import PublicInterface
from intent_amd.runtime.torch_views import allocate_output, byte_span, observe_view
from intent_amd.targets.local import LocalDevice, resolve_local, select_device


# ------------------------------------------------------------------------------ annotations
@pytest.mark.parametrize("make, error", [
    (lambda: I.In[I.f32, ("M", -1)], ValueError),
    (lambda: I.In[I.f32, ("not a name",)], ValueError),
    (lambda: I.In[I.f32, (True,)], TypeError),
    (lambda: I.In[I.f32, (1.5,)], TypeError),
    (lambda: I.In[I.f32, "M"], TypeError),
    (lambda: I.In[I.f32], TypeError),
    (lambda: I.In[I.f32, ("M",), I.constraints(), 1], TypeError),
    (lambda: I.In[I.f32, ("M",), {"noalias": True}], TypeError),
    (lambda: I.In["f32", ("M",)], TypeError),
    (lambda: I.In[I.f32, ("M", "N"), I.constraints(strides=(1,))], ValueError),
    (lambda: I.constraints(strides=(True,)), TypeError),
    (lambda: I.constraints(strides=("1x",)), TypeError),
    (lambda: I.constraints(alias=""), ValueError),
    (lambda: I.constraints(alias="g", noalias=True), ValueError),
    (lambda: I.Constexpr[None], TypeError),
])
def test_annotation_errors(make, error):
    with pytest.raises(error):
        make()


def test_annotation_specs():
    view = I.Out[I.bf16, ["M", 8], I.constraints(strides=("S", None), alias="g")]
    assert (view.kind, view.dtype, view.shape) == (I.ViewKind.OUT, I.bf16, ("M", 8))
    assert view.constraints.strides == ("S", None) and view.constraints.alias == "g"
    assert I.InOut[I.f16, ()].kind == I.ViewKind.INOUT and I.In[I.i32, (0,)].shape == (0,)
    assert I.Constexpr[int].value_type is int
    assert I.ViewKind.IN == 0 and I.ViewKind.OUT == 1 and I.ViewKind.INOUT == 2


# ------------------------------------------------------------------------------ definitions
def test_definitions():
    def body(x: I.In[I.f32, ("N",)], y: I.Out[I.f32, ("N",)], SCALE: I.Constexpr[float] = 2.0):
        """doc"""

    kernel = intent.kernel(body)
    assert isinstance(kernel, intent.KernelDefinition) and kernel.kind is intent.DefinitionKind.KERNEL
    assert kernel.__name__ == "body" and kernel.__doc__ == "doc" and kernel.python_function is body
    assert list(kernel.signature.parameters) == ["x", "y", "SCALE"]
    assert kernel.source.first_line == body.__code__.co_firstlineno and "def body" in kernel.source_text()
    assert repr(kernel).startswith("<intent kernel ")
    assert isinstance(intent.kernel()(body), intent.KernelDefinition)
    helper = intent.fn(lambda a: a)
    assert helper.kind is intent.DefinitionKind.HELPER and isinstance(intent.fn()(body), intent.HelperDefinition)
    with pytest.raises(intent.LanguageUseError):
        kernel(torch.zeros(1), torch.zeros(1))
    with pytest.raises(intent.LanguageUseError):
        helper(1)
    with pytest.raises(intent.DefinitionError):
        intent.kernel(print)
    with pytest.raises(intent.DefinitionError):
        intent.fn(SimpleNamespace())


# ------------------------------------------------------------------------------ device selection
def _tensor(device):
    return SimpleNamespace(shape=(1,), device=device)


@pytest.mark.parametrize("tensors, explicit, want", [
    (("cuda:0",), None, LocalDevice("cuda", 0)),
    (("cuda:1", "cuda:1"), None, LocalDevice("cuda", 1)),
    (("cuda:1",), "cuda", LocalDevice("cuda", 1)),
    (("cuda:2",), "cuda:2", LocalDevice("cuda", 2)),
    (("cuda:2",), 2, LocalDevice("cuda", 2)),
    ((), "cuda:3", LocalDevice("cuda", 3)),
    ((), 0, LocalDevice("cuda", 0)),
])
def test_select_device(tensors, explicit, want):
    arguments = tuple(_tensor(d) for d in tensors) + (1.0, "not a tensor")
    assert select_device("hip", arguments, explicit) == want
    assert str(want) == f"cuda:{want.index}"


@pytest.mark.parametrize("tensors, explicit", [
    (("cuda:0", "cuda:1"), None),          # tensors on several devices
    (("cpu",), None),                      # another device kind
    ((), None),                            # nothing names a device
    ((), "cuda"),                          # no ordinal
    (("cuda:0",), "cuda:1"),               # explicit and tensors disagree
    (("cuda:0",), "cpu"),
    (("cuda:0",), "cuda:0:1"),
    (("cuda:0",), "cuda:"),
    (("cuda:0",), "cuda:x"),
    (("cuda:0",), -1),
])
def test_select_device_errors(tensors, explicit):
    with pytest.raises(ValueError):
        select_device("hip", tuple(_tensor(d) for d in tensors), explicit)


def test_resolve_local_rejects_before_touching_a_device():
    with pytest.raises(ValueError):
        resolve_local("hip", LocalDevice("cpu"))
    with pytest.raises(ValueError):
        resolve_local("hip", LocalDevice("cuda", 0), backend_options={"no_such_option": 1})
    with pytest.raises(ValueError):
        select_device("no_such_backend", ())


# ------------------------------------------------------------------------------ jit
def test_call_roles_split_outputs_in_declaration_order():
    @intent.kernel
    def mixed(a: I.In[I.f32, ("N",)], out1: I.Out[I.f32, ("N",)], s: I.f32, b: I.InOut[I.f32, ("N",)],
              out2: I.Out[I.f32, ("N",)], FLAG: I.Constexpr[bool]):
        pass

    roles = _CallRoles(mixed)
    assert roles.count == 5 and roles.out_positions == (1, 4)
    assert roles.split(("a", "o1", 2.0, "b", "o2")) == (("a", 2.0, "b"), ("o1", "o2"))
    with pytest.raises(TypeError):
        roles.split(("a", "o1"))


def test_jit_rejects_and_closes():
    from intent_amd.examples.kernels.normalization.softmax import stable_softmax

    with pytest.raises(TypeError):
        intent.jit(stable_softmax.python_function, backend="hip")
    with intent.jit(stable_softmax, backend="hip", constexprs={}, backend_options={}) as kernel:
        assert kernel.artifacts == () and kernel.__name__ == "stable_softmax"
    with pytest.raises(RuntimeError):
        kernel.prepare(_tensor("cuda:0"))


# ------------------------------------------------------------------------------ tensor observation
def test_byte_span():
    assert byte_span(1000, (3, 4), (4, 1), 4) == (1000, 1048)
    assert byte_span(1000, (3, 4), (8, 1), 2) == (1000, 1000 + 2 * (2 * 8 + 3 + 1))
    assert byte_span(1000, (3, 0), (4, 1), 4) == (1000, 1000)
    assert byte_span(1000, (3,), (-2,), 4) == (1000 - 16, 1004)
    assert byte_span(1000, (5,), (0,), 8) == (1000, 1008)


def test_observe_and_allocate():
    from intent_amd.examples.kernels.normalization.softmax import stable_softmax

    x_param, y_param = PublicInterface.from_definition(stable_softmax).parameters
    cpu = torch.device("cpu")
    base = torch.zeros(6, 10)
    view = base[1:4, 2:7]
    facts = observe_view(x_param, view, device=cpu)
    assert facts.shape == (3, 5) and facts.strides == (10, 1) and facts.pointer == view.data_ptr()
    assert facts.allocation == base.data_ptr() and facts.allocation_end == base.data_ptr() + 240
    assert (facts.begin, facts.end) == (view.data_ptr(), view.data_ptr() + 4 * (2 * 10 + 4 + 1))
    assert facts.offset == 12 and facts.allocation_identity == (cpu, base.data_ptr())
    assert observe_view(x_param, view, device=cpu, abstract=True).pointer is None
    empties = [torch.zeros(0, 3), torch.zeros(0, 3)]
    empty = [observe_view(x_param, e, device=cpu) for e in empties]
    assert empty[0].allocation_identity != empty[1].allocation_identity      # distinct storages
    assert observe_view(x_param, empties[0][:, 1:], device=cpu).allocation_identity == empty[0].allocation_identity
    out, out_facts = allocate_output(y_param, (2, 3), device=cpu)
    assert out.shape == (2, 3) and out.dtype == torch.float32 and out_facts.strides == (3, 1)
    with pytest.raises(TypeError):
        observe_view(x_param, [1.0], device=cpu)
    with pytest.raises(TypeError):
        observe_view(x_param, torch.zeros(2, 2, dtype=torch.float64), device=cpu)
    with pytest.raises(ValueError):
        observe_view(x_param, torch.zeros(2), device=cpu)
    with pytest.raises(ValueError):
        observe_view(x_param, torch.zeros(2, 2, device="meta"), device=cpu)


def test_torch_dtype_covers_every_intent_dtype():
    want = {"bool": torch.bool, "index": torch.int64, "i8": torch.int8, "i16": torch.int16, "i32": torch.int32,
            "i64": torch.int64, "u8": torch.uint8, "f16": torch.float16, "bf16": torch.bfloat16,
            "f32": torch.float32, "f64": torch.float64, "f8e4m3fn": torch.float8_e4m3fn,
            "f8e5m2": torch.float8_e5m2}
    for name, dtype in want.items():
        assert torch_dtype(I.dtype(name)) is dtype
    for name in ("u16", "u32", "u64"):
        assert torch_dtype(I.dtype(name)) is getattr(torch, "uint" + name[1:])


# ------------------------------------------------------------------------------ PyTorch operators
@intent.kernel
def scaled_update(x: I.In[I.f32, ("N",)], acc: I.InOut[I.f32, ("N",)], y: I.Out[I.f32, ("N",)], alpha: I.f32,
                  count: I.i32, flag: I.bool):
    pass


class _CpuRuntime:
    """Stands in for a device runtime: runs the maths on the CPU, infers outputs from inputs."""

    def infer_outputs(self, arguments):
        return torch.empty_like(arguments[0])


def _cpu_artifact(definition, run):
    return SimpleNamespace(interface=PublicInterface.from_definition(definition), device_type="cpu",
                           runtime=_CpuRuntime(), run=run)


def test_operator_schema():
    schema = operator_schema(PublicInterface.from_definition(scaled_update))
    assert schema.text == "(Tensor arg0, Tensor(a1!) arg1, float arg2, SymInt arg3, bool arg4) -> Tensor"
    assert schema.mutated == ("arg1",) and schema.exclusive == ((0, 1),)


def test_register_operator_runs_checks_aliasing_and_traces():
    def run(x, acc, alpha, count, flag):
        acc.add_(x)
        return x * alpha + count

    op = register_operator(_cpu_artifact(scaled_update, run), "intent_amd_host_test::scaled_update")
    x, acc = torch.arange(4.0), torch.zeros(4)
    assert torch.equal(op(x, acc, 2.0, 1, True), x * 2.0 + 1) and torch.equal(acc, x)
    with pytest.raises(NotImplementedError):
        op(acc, acc, 2.0, 1, True)                       # a mutated input shares storage with another input
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode() as mode:
        out = op(mode.from_tensor(x), mode.from_tensor(acc), 2.0, 1, True)
        assert out.shape == (4,)
    with pytest.raises(ValueError):
        register_operator(_cpu_artifact(scaled_update, run), "no_namespace")
    with pytest.raises(NotImplementedError):
        register_operator(SimpleNamespace(interface=None, device_type="meta", runtime=_CpuRuntime()), "a::b")

    @intent.kernel
    def no_tensor_input(s: I.f32, y: I.Out[I.f32, (4,)]):
        pass

    with pytest.raises(NotImplementedError):
        register_operator(_cpu_artifact(no_tensor_input, run), "intent_amd_host_test::no_tensor_input")


# ------------------------------------------------------------------------------ attention backward program
def test_attention_backward_program_order_and_outputs():
    from intent_amd.examples.programs.attention_backward import AttentionBackward

    log = []

    class Call:
        def __init__(self, name, result):
            self.name, self._result = name, result

        def launch(self):
            log.append(("launch", self.name))

        def result(self):
            return self._result

    class Kernel:
        def __init__(self, definition, constexprs=None):
            self.name, self.constexprs = definition.__name__, constexprs

        def prepare(self, *arguments, outputs=None):
            log.append(("prepare", self.name, len(arguments), outputs))
            results = {"attention_backward_delta": "delta", "attention_backward_dkdv": ("dk", "dv"),
                       "attention_backward_dq": "dq"}
            return Call(self.name, results[self.name] if outputs is None else
                        (outputs[0] if len(outputs) == 1 else outputs))

    program = AttentionBackward.from_jit(lambda d, **kw: Kernel(d, **kw), head_group=4, causal=True)
    assert program.dkdv.constexprs == program.dq.constexprs == {"HEAD_GROUP": 4, "CAUSAL": True}
    assert program.delta.constexprs is None
    assert program.run("q", "k", "v", "o", "do", "lse", 0.125) == ("dq", "dk", "dv")
    assert [entry[:3] for entry in log] == [
        ("prepare", "attention_backward_delta", 2), ("prepare", "attention_backward_dkdv", 7),
        ("prepare", "attention_backward_dq", 7), ("launch", "attention_backward_delta"),
        ("launch", "attention_backward_dkdv"), ("launch", "attention_backward_dq")]
    log.clear()
    result = program.prepare("q", "k", "v", "o", "do", "lse", 0.125, outputs=("gq", "gk", "gv"), workspace="ws")
    assert result.result() == ("gq", "gk", "gv")
    assert [entry[3] for entry in log] == [("ws",), ("gk", "gv"), ("gq",)]
    with pytest.raises(TypeError):
        program.prepare("q", "k", "v", "o", "do", "lse", 0.125, outputs=("gq",))


# ------------------------------------------------------------------------------ backend options
def test_workspace_option_values_and_staging_refusal():
    from intent_amd.runtime.hip import operators
    from intent_amd.targets.hip import HipTarget

    assert HipTarget(0).workspace == "prepare" and HipTarget(0, "static").workspace == "static"
    with pytest.raises(ValueError):
        HipTarget(0, "pinned")
    transposed = torch.zeros(4, 6).t()
    keep, before = [], []
    assert operators._readable(transposed, keep, before) is not transposed and len(before) == 1
    with operators.workspace_policy("static"):
        with pytest.raises(ValueError):
            operators._readable(transposed, [], [])
        with pytest.raises(ValueError):
            operators._writable(transposed, [], [])
        plain = torch.zeros(4, 6)
        assert operators._readable(plain, [], []) is plain
    assert not operators._static_workspace()
