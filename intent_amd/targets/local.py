"""The local device of a JIT call, and the provider target for it.

`select_device` reads two sources: where the call's tensors are (every argument with a `.shape`),
and an optional explicit device (an ordinal, or "kind" / "kind:ordinal"). A kind-only explicit
device takes its ordinal from the tensors. An indexed device kind, such as the hip provider's
"cuda", must end with a concrete ordinal. Tensors on several devices, a device of another kind, or
an explicit device that disagrees with the tensors raise ValueError. So does an indexed call that
names no ordinal at all. This is the behaviour of the reference's `select_device` and
`resolve_local` (`python/intent/targets/local.py:33-68`).
"""
from __future__ import annotations

from dataclasses import dataclass

from .provider import provider


@dataclass(frozen=True)
class LocalDevice:
    kind: str
    index: int | None = None

    def __str__(self):
        return self.kind if self.index is None else f"{self.kind}:{self.index}"


def _parse(value, execution) -> LocalDevice:
    """A LocalDevice of the execution's kind from an ordinal, a string or a torch.device."""
    if isinstance(value, int) and not isinstance(value, bool):
        device = LocalDevice(execution.device_kind, value)
    else:
        kind, colon, ordinal = str(value).partition(":")
        if not kind or ":" in ordinal or (colon and not ordinal):
            raise ValueError(f"{value!r} is not a device (expected 'kind' or 'kind:ordinal')")
        device = LocalDevice(kind, int(ordinal) if colon else None)
    if device.kind != execution.device_kind:
        raise ValueError(f"{device} is not a {execution.device_kind} device")
    if device.index is not None:
        if device.index < 0:
            raise ValueError(f"device ordinal {device.index} is negative")
        if not execution.indexed:
            raise ValueError(f"{device.kind} devices take no ordinal, got {device}")
    return device


def _merge(explicit: LocalDevice | None, placed: LocalDevice | None) -> LocalDevice | None:
    """The one device both sources describe; a kind-only explicit device defers to the tensors."""
    if explicit is None or (placed is not None and explicit.index is None):
        return placed if placed is not None else explicit
    if placed is not None and placed != explicit:
        raise ValueError(f"the explicit device {explicit} differs from the tensors' device {placed}")
    return explicit


def select_device(backend: str, arguments: tuple, explicit=None) -> LocalDevice:
    execution = provider(backend).local
    placed = {_parse(getattr(value, "device", "cpu"), execution) for value in arguments if hasattr(value, "shape")}
    if len(placed) > 1:
        raise ValueError(f"the tensor arguments are on several devices: {', '.join(sorted(map(str, placed)))}")
    chosen = _merge(None if explicit is None else _parse(explicit, execution), next(iter(placed), None))
    if chosen is None:
        if execution.indexed:
            raise ValueError(f"a {backend} call needs a tensor argument or an explicit device to run on")
        return LocalDevice(execution.device_kind)
    if execution.indexed and chosen.index is None:
        raise ValueError(f"{chosen} names no ordinal; pass '{chosen.kind}:<ordinal>' or a tensor on the device")
    return chosen


def resolve_local(backend: str, device: LocalDevice, *, workers=None, backend_options=None):
    """The provider's resolved target for `device`, with the backend's own options applied."""
    execution = provider(backend).local
    if device.kind != execution.device_kind:
        raise ValueError(f"the {backend} backend runs on {execution.device_kind} devices, not {device}")
    options = dict(backend_options or {})
    unknown = sorted(set(options).difference(execution.options))
    if unknown:
        accepted = ", ".join(sorted(execution.options)) or "none"
        raise ValueError(f"the {backend} backend does not take the options {unknown} (accepted: {accepted})")
    return execution.resolve(device, workers=workers, **options)
