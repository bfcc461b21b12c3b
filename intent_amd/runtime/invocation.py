"""Binding of concrete arguments to a `PublicInterface`.

Enforces the reference's binding contract (`python/intent/runtime/invocation.py:56-159`,
`python/intent/runtime/interface.py:187-245`): argument count (TypeError), per-view
dtype/device/rank (`torch_views.observe_view`), shape relations through dimension
identities and static extents (ValueError), stride constraints including shared
stride symbols (ValueError), Out allocation from input extents (NotImplementedError
when impossible), and noalias / named-alias allocation relations (ValueError).
The reference generates a Python function per mode with `exec`; this binder walks
the same schema directly.
"""
from __future__ import annotations

from dataclasses import dataclass

from .interface import PublicInterface, StrideSymbol, ViewParameter


@dataclass(slots=True)
class ViewFacts:
    shape: tuple
    strides: tuple
    pointer: int | None
    allocation: int | None
    allocation_end: int | None
    offset: int | None
    dtype: object
    begin: int | None
    end: int | None
    allocation_identity: object


def invocation_result(outputs: tuple):
    """Return only declared Out buffers: None, one value, or an ordered tuple."""
    if not outputs:
        return None
    return outputs[0] if len(outputs) == 1 else outputs


@dataclass(slots=True)
class BoundPublicArguments:
    arguments: tuple          # every runtime argument, declaration order
    outputs: tuple            # declared Out buffers, declaration order
    views: tuple              # ViewFacts per parameter (None for scalars)
    extents: dict             # dimension identity -> bound extent

    def result(self):
        return invocation_result(self.outputs)


def _spans_overlap(a: tuple, b: tuple) -> bool:
    return a[0] < a[1] and b[0] < b[1] and a[0] < b[1] and b[0] < a[1]


def bind_arguments(interface: PublicInterface, arguments: tuple, outputs: tuple | None, *,
                   observe_view, allocate_output, abstract: bool = False,
                   derived: dict | None = None) -> BoundPublicArguments:
    """Bind `arguments` (inputs, declaration order) and optional explicit `outputs`.

    `observe_view(parameter, value) -> ViewFacts` and
    `allocate_output(parameter, shape) -> (value, ViewFacts)` are the device family's
    observers. Abstract binding checks shapes and strides only (no addresses).
    `derived` maps a dimension identity to (source identity, offset): when the source
    is bound and the identity is not, its extent is source + offset (for relations such
    as R1 = R + 1 that symbols alone cannot state).
    """
    derived = dict(derived or {})
    explicit = outputs is not None
    if explicit:
        supplied = interface.parameters
        values = interface.explicit_arguments(tuple(arguments), tuple(outputs))
    else:
        supplied = interface.inputs
        if len(arguments) != len(supplied):
            raise TypeError(f"expected {len(supplied)} runtime arguments, got {len(arguments)}")
        interface.require_output_allocation(frozenset(derived))
        values = None
    static: dict[int, int] = {}
    for view in interface.views:
        for extent, identity in zip(view.shape, view.dimensions):
            if extent >= 0 and identity > 0:
                static.setdefault(identity, extent)
    extents: dict[int, int] = dict(static)
    stride_symbols: dict[str, int] = {}
    facts: dict[int, ViewFacts] = {}
    bound: dict[int, object] = {}

    def check(view: ViewParameter, fact: ViewFacts, allocated: bool) -> None:
        for axis, (extent, identity) in enumerate(zip(view.shape, view.dimensions)):
            actual = fact.shape[axis]
            if extent >= 0 and actual != extent:
                raise ValueError(f"{view.name}.shape[{axis}] violates the declared interface relation")
            if identity > 0:
                known = extents.setdefault(identity, actual)
                if known != actual:
                    raise ValueError(f"{view.name}.shape[{axis}] violates the declared interface relation")
        for axis, constraint in enumerate(view.strides):
            if constraint is None:
                continue
            actual = fact.strides[axis]
            if isinstance(constraint, StrideSymbol):
                expected = stride_symbols.setdefault(constraint.name, actual)
            else:
                expected = constraint
            if actual != expected:
                message = f"{view.name}.strides[{axis}] violates the declared interface relation"
                if allocated:
                    message += "; provide explicit output buffers with the required layout"
                raise ValueError(message)

    ordered = values if explicit else tuple(arguments)
    for parameter, value in zip(supplied, ordered):
        bound[parameter.position] = value
        if isinstance(parameter, ViewParameter):
            fact = observe_view(parameter, value)
            check(parameter, fact, False)
            facts[parameter.position] = fact
    for identity, (source, offset) in derived.items():
        if identity not in extents and source in extents:
            extents[identity] = extents[source] + offset
            if extents[identity] < 0:
                raise ValueError("a derived extent is negative; check the input extents")
    if not explicit:
        for view in interface.outputs:
            shape = tuple(e if e >= 0 else extents[i] for e, i in zip(view.shape, view.dimensions))
            value, fact = allocate_output(view, shape)
            check(view, fact, True)
            bound[view.position] = value
            facts[view.position] = fact
    if not abstract:
        views = interface.views
        for index, left in enumerate(views):
            for right in views[index + 1:]:
                lf, rf = facts[left.position], facts[right.position]
                if (left.noalias or right.noalias) and _spans_overlap(
                        (lf.allocation, lf.allocation_end), (rf.allocation, rf.allocation_end)):
                    raise ValueError(f"{left.name} and {right.name} violate an author noalias allocation constraint")
                if left.alias and left.alias == right.alias and lf.allocation_identity != rf.allocation_identity:
                    raise ValueError(f"{left.name} and {right.name} violate an author named allocation-alias constraint")
    all_values = tuple(bound[p.position] for p in interface.parameters)
    outs = tuple(bound[v.position] for v in interface.outputs)
    view_facts = tuple(facts.get(p.position) for p in interface.parameters)
    return BoundPublicArguments(all_values, outs, view_facts, extents)
