"""What the binder learns from a torch tensor, and how Out buffers are allocated.

Checks and their error classes follow the reference's `python/intent/runtime/torch_views.py:23-88`.
Passing a non-tensor or a tensor of the wrong dtype raises TypeError. A tensor on another device,
or of another rank, raises ValueError. An Out buffer is a fresh contiguous `torch.empty` on the
call's device.

A tensor's facts are its shape and strides, plus its address range for alias checks. The range
runs from the first to one past the last byte that its elements reach. `byte_span` accepts
strides of either sign; torch strides are never negative, so for a tensor the range starts at
`data_ptr()`. An allocation is identified by its device and
base address. A storage of zero bytes holds nothing two views could disagree about, so every
empty storage counts as one allocation. Abstract binding (fake tensors, `torch.compile` tracing)
records shape, strides and dtype only.
"""
from __future__ import annotations

from ..integrations.torch import torch_dtype
from .interface import ViewParameter
from .invocation import ViewFacts

def byte_span(pointer: int, shape: tuple, strides: tuple, itemsize: int) -> tuple[int, int]:
    """[begin, end) of the bytes a strided view's elements occupy (empty views: an empty range)."""
    if 0 in shape:
        return pointer, pointer
    below = sum((extent - 1) * stride for extent, stride in zip(shape, strides) if stride < 0)
    above = sum((extent - 1) * stride for extent, stride in zip(shape, strides) if stride > 0)
    return pointer + below * itemsize, pointer + (above + 1) * itemsize


def _check(parameter: ViewParameter, value, device):
    import torch

    if not isinstance(value, torch.Tensor):
        raise TypeError(f"{parameter.name} takes a torch.Tensor, got {type(value).__name__}")
    wanted = torch_dtype(parameter.dtype)
    if value.dtype != wanted:
        raise TypeError(f"{parameter.name} takes {wanted} elements, got {value.dtype}")
    if value.device != device:
        raise ValueError(f"{parameter.name} is on {value.device}; this call runs on {device}")
    if value.dim() != parameter.rank:
        raise ValueError(f"{parameter.name} takes a rank-{parameter.rank} tensor, got rank {value.dim()}")


def observe_view(parameter: ViewParameter, value, *, device, abstract: bool = False) -> ViewFacts:
    _check(parameter, value, device)
    shape, strides = tuple(value.shape), tuple(value.stride())
    if abstract:
        return ViewFacts(shape, strides, None, None, None, None, value.dtype, None, None, None)
    storage = value.untyped_storage()
    base, size = storage.data_ptr(), storage.nbytes()
    # A zero-byte storage has no meaningful address (several may report the same or a null
    # pointer), so each is identified by its own storage object, never by the pointer: two
    # distinct empty buffers are two allocations (reference runtime/torch_views.py:53).
    identity = (value.device, base) if size else (value.device, "empty", storage._cdata)
    begin, end = byte_span(value.data_ptr(), shape, strides, value.element_size())
    return ViewFacts(shape, strides, value.data_ptr(), base, base + size, value.storage_offset(), value.dtype,
                     begin, end, identity)


def allocate_output(parameter: ViewParameter, shape: tuple, *, device, abstract: bool = False):
    """A fresh contiguous Out buffer and its facts."""
    import torch

    value = torch.empty(shape, dtype=torch_dtype(parameter.dtype), device=device)
    return value, observe_view(parameter, value, device=device, abstract=abstract)
