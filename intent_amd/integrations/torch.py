"""PyTorch integration: dtype mapping and custom-operator registration.

Behaviour of `register_operator` follows the reference's
`python/intent/integrations/torch.py:27-93`: the schema is derived from the public
interface (`Tensor` / `Tensor(aN!)` for InOut / `float` / `SymInt` / `bool`), the
return is one Tensor or a tuple of the declared Outs, mutable inputs may not share
storage with another input, and the fake implementation uses output inference
without touching device pointers."""
from __future__ import annotations

from inspect import Parameter, Signature
from typing import Protocol, runtime_checkable

from ..language.dtypes import DType, DTypeCategory
from ..runtime.interface import ScalarParameter, ViewParameter

_TORCH_NAMES = {"index": "int64", "bool": "bool", "i8": "int8", "i16": "int16", "i32": "int32",
                "i64": "int64", "u8": "uint8", "u16": "uint16", "u32": "uint32", "u64": "uint64",
                "f16": "float16", "bf16": "bfloat16", "f32": "float32", "f64": "float64",
                "f8e4m3fn": "float8_e4m3fn", "f8e5m2": "float8_e5m2"}


@runtime_checkable
class TorchOutputInference(Protocol):
    def infer_outputs(self, arguments: tuple) -> object: ...


def torch_dtype(element: DType):
    import torch

    return getattr(torch, _TORCH_NAMES[element.name])


def _scalar_schema(parameter: ScalarParameter) -> str:
    category = parameter.dtype.category
    if category is DTypeCategory.BOOL:
        return "bool"
    if category in (DTypeCategory.SIGNED_INTEGER, DTypeCategory.UNSIGNED_INTEGER, DTypeCategory.INDEX):
        return "SymInt"
    if category in (DTypeCategory.FLOAT, DTypeCategory.BFLOAT):
        return "float"
    raise NotImplementedError(f"PyTorch scalar schema for {parameter.dtype}")


def register_operator(artifact, name: str):
    import torch

    interface = artifact.interface
    if artifact.device_type not in {"cpu", "cuda"} or not isinstance(artifact.runtime, TorchOutputInference):
        raise NotImplementedError("PyTorch registration requires a CPU or CUDA tensor runtime with output inference")
    inputs = interface.inputs
    views = [(i, p) for i, p in enumerate(inputs) if isinstance(p, ViewParameter)]
    if not views:
        raise NotImplementedError("PyTorch registration requires an input tensor to determine device dispatch")
    interface.require_output_allocation()
    pieces = name.split("::")
    if len(pieces) != 2 or not all(piece.isidentifier() for piece in pieces):
        raise ValueError("operator name must be 'your_namespace::your_operator'")
    mutable = tuple(f"arg{i}" for i, p in views if p.writable)
    pairs = [(li, ri, lp.name, rp.name) for k, (li, lp) in enumerate(views)
             for ri, rp in views[k + 1:] if lp.writable or rp.writable]
    fields = []
    for i, p in enumerate(inputs):
        kind = (f"Tensor(a{i}!)" if p.writable else "Tensor") if isinstance(p, ViewParameter) else _scalar_schema(p)
        fields.append(f"{kind} arg{i}")
    count = len(interface.outputs)
    returns = "()" if count == 0 else ("Tensor" if count == 1 else "(" + ", ".join(["Tensor"] * count) + ")")
    schema = f"({', '.join(fields)}) -> {returns}"
    signature = Signature([Parameter(f"arg{i}", Parameter.POSITIONAL_OR_KEYWORD) for i in range(len(inputs))])

    def guarded(invoke):
        def operator(*args, **kwargs):
            args = signature.bind(*args, **kwargs).args
            for left, right, lname, rname in pairs:
                if torch._C._is_alias_of(args[left], args[right]):
                    raise NotImplementedError(
                        f"PyTorch mutable calls require independent input storage: {lname} and {rname} "
                        "share storage; use ordinary artifact calls for this binding")
            return invoke(*args)
        return operator

    op = torch.library.custom_op(name, guarded(artifact.run), mutates_args=mutable,
                                 device_types=artifact.device_type, schema=schema)
    op.register_fake(guarded(lambda *args: artifact.runtime.infer_outputs(args)))
    return op
