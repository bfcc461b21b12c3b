"""PyTorch integration: element types and custom-operator registration of an artifact.

`register_operator(artifact, name)` is the reference's entry point
(`python/intent/integrations/torch.py:27`, reached through `CompiledArtifact.as_torch_op`) and
keeps its contract:

* the op takes the runtime inputs of the public interface in order, named `arg0, arg1, ...`, and
  returns the declared Out buffers (one Tensor, or a tuple). InOut inputs are declared mutated;
* scalars map to `bool`, `SymInt` (every integer kind) or `float` (every float kind);
* the fake (meta) implementation is the runtime's `infer_outputs`, which reads no device pointer;
* a call in which a mutated input shares storage with another tensor input is refused: torch may
  clone mutated arguments on their own when it functionalizes a graph, which would split what the
  caller meant as one buffer;
* failures raise NotImplementedError (no tensor runtime, no tensor input, Outs that cannot be
  allocated, an unmapped scalar, aliased mutable storage) or ValueError (a malformed name).

Out allocation may use the relations the runtime derives between dimensions (the hip runtime's
`derivable_dimensions`, e.g. csr_spmv's R = R1 - 1), so an op whose Out extents follow from such a
relation registers too.
"""
from __future__ import annotations

from dataclasses import dataclass
from inspect import Parameter, Signature
from typing import Protocol, runtime_checkable

from ..language.dtypes import DType, DTypeCategory
from ..runtime.interface import ScalarParameter, ViewParameter

_FLOAT8_NAMES = {"f8e4m3fn": "float8_e4m3fn", "f8e5m2": "float8_e5m2"}
_SCALAR_SCHEMA = {DTypeCategory.BOOL: "bool", DTypeCategory.SIGNED_INTEGER: "SymInt",
                  DTypeCategory.UNSIGNED_INTEGER: "SymInt", DTypeCategory.INDEX: "SymInt",
                  DTypeCategory.FLOAT: "float", DTypeCategory.BFLOAT: "float"}


@runtime_checkable
class TorchOutputInference(Protocol):
    """A runtime that can produce a call's Out buffers from the inputs alone (fake tensors)."""

    def infer_outputs(self, arguments: tuple) -> object: ...


def _torch_name(element: DType) -> str:
    category = element.category
    if category is DTypeCategory.BOOL:
        return "bool"
    if category is DTypeCategory.INDEX:
        return "int64"
    if category is DTypeCategory.BFLOAT:
        return "bfloat16"
    if category is DTypeCategory.SIGNED_INTEGER:
        return f"int{element.bits}"
    if category is DTypeCategory.UNSIGNED_INTEGER:
        return f"uint{element.bits}"
    return _FLOAT8_NAMES.get(element.name, f"float{element.bits}")


def torch_dtype(element: DType):
    """The torch dtype of an Intent element type (I.f32 -> torch.float32, I.index -> torch.int64)."""
    import torch

    result = getattr(torch, _torch_name(element), None)
    if not isinstance(result, torch.dtype):
        raise TypeError(f"{element!r} has no torch element type")
    return result


@dataclass(frozen=True)
class OperatorSchema:
    """The torch schema of an interface, and the input pairs that must not share storage."""

    text: str
    mutated: tuple[str, ...]
    exclusive: tuple[tuple[int, int], ...]
    names: tuple[str, ...]


def operator_schema(interface) -> OperatorSchema:
    inputs = interface.inputs
    names = tuple(f"arg{i}" for i in range(len(inputs)))
    fields = []
    for parameter, name in zip(inputs, names):
        if isinstance(parameter, ViewParameter):
            fields.append(f"Tensor(a{parameter.position}!) {name}" if parameter.writable else f"Tensor {name}")
            continue
        kind = _SCALAR_SCHEMA.get(parameter.dtype.category) if isinstance(parameter, ScalarParameter) else None
        if kind is None:
            raise NotImplementedError(f"{parameter.name}: no PyTorch schema type for {parameter.dtype!r}")
        fields.append(f"{kind} {name}")
    tensors = [i for i, p in enumerate(inputs) if isinstance(p, ViewParameter)]
    exclusive = tuple((i, j) for k, i in enumerate(tensors) for j in tensors[k + 1:]
                      if inputs[i].writable or inputs[j].writable)
    count = len(interface.outputs)
    returns = "Tensor" if count == 1 else f"({', '.join(['Tensor'] * count)})"
    mutated = tuple(names[i] for i in tensors if inputs[i].writable)
    return OperatorSchema(f"({', '.join(fields)}) -> {returns}", mutated, exclusive, names)


def _refuse_shared_storage(schema: OperatorSchema, inputs, body):
    """`body(*args)` after checking that no mutated input shares storage with another tensor input
    (storage identity works for real and fake tensors alike and reads no data)."""
    import torch

    signature = Signature([Parameter(name, Parameter.POSITIONAL_OR_KEYWORD) for name in schema.names])

    def checked(*args, **kwargs):
        args = signature.bind(*args, **kwargs).args
        for i, j in schema.exclusive:
            if torch._C._is_alias_of(args[i], args[j]):
                raise NotImplementedError(
                    f"{inputs[i].name} and {inputs[j].name} share storage and one of them is written; the "
                    "PyTorch operator needs separate buffers (call the artifact directly for in-place use)")
        return body(*args)

    return checked


def register_operator(artifact, name: str):
    """Register `artifact` as the PyTorch custom op `name` ("namespace::operator")."""
    import torch

    if artifact.device_type not in ("cpu", "cuda") or not isinstance(artifact.runtime, TorchOutputInference):
        raise NotImplementedError("a PyTorch operator needs a CPU or CUDA tensor runtime that can infer its outputs")
    interface = artifact.interface
    if not any(isinstance(p, ViewParameter) for p in interface.inputs):
        raise NotImplementedError("a PyTorch operator needs a tensor input to dispatch on")
    interface.require_output_allocation(frozenset(getattr(artifact.runtime, "derivable_dimensions", ())))
    namespace, _, operator = name.partition("::")
    if not (namespace.isidentifier() and operator.isidentifier()):
        raise ValueError(f"operator names read 'namespace::operator' with identifiers on both sides, got {name!r}")
    schema = operator_schema(interface)
    inputs = interface.inputs
    op = torch.library.custom_op(name, _refuse_shared_storage(schema, inputs, artifact.run),
                                 mutates_args=schema.mutated, device_types=artifact.device_type, schema=schema.text)
    op.register_fake(_refuse_shared_storage(schema, inputs, lambda *args: artifact.runtime.infer_outputs(args)))
    return op
