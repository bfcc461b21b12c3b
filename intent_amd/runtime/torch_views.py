"""Observation and allocation of torch tensors for binding.

Behaviour follows the reference's `python/intent/runtime/torch_views.py:23-88`:
dtype mismatch is a TypeError, device or rank mismatch a ValueError, outputs are
`torch.empty` on the call's device with contiguous strides."""
from __future__ import annotations

from ..integrations.torch import torch_dtype
from .interface import ViewParameter
from .invocation import ViewFacts


def byte_span(pointer: int, shape: tuple, strides: tuple, itemsize: int) -> tuple[int, int]:
    if any(e == 0 for e in shape):
        return pointer, pointer
    low = high = 0
    for extent, stride in zip(shape, strides):
        d = (extent - 1) * stride
        low += min(0, d)
        high += max(0, d)
    return pointer + low * itemsize, pointer + (high + 1) * itemsize


def observe_view(parameter: ViewParameter, value, *, device, abstract: bool = False) -> ViewFacts:
    import torch

    if not isinstance(value, torch.Tensor):
        raise TypeError(f"{parameter.name} must be a torch.Tensor")
    expected = torch_dtype(parameter.dtype)
    if value.dtype != expected:
        raise TypeError(f"{parameter.name} must have dtype {expected}, got {value.dtype}")
    if value.device != device:
        raise ValueError(f"{parameter.name} must be on {device}, got {value.device}")
    shape, strides = tuple(value.shape), tuple(value.stride())
    if len(shape) != parameter.rank:
        raise ValueError(f"{parameter.name} must have rank {parameter.rank}, got {len(shape)}")
    if abstract:
        return ViewFacts(shape, strides, None, None, None, None, value.dtype, None, None, None)
    storage = value.untyped_storage()
    allocation, nbytes = storage.data_ptr(), storage.nbytes()
    pointer = value.data_ptr()
    identity = (value.device, allocation) if nbytes else (value.device, "empty", storage._cdata)
    begin, end = byte_span(pointer, shape, strides, value.element_size())
    return ViewFacts(shape, strides, pointer, allocation, allocation + nbytes, value.storage_offset(),
                     value.dtype, begin, end, identity)


def allocate_output(parameter: ViewParameter, shape: tuple, *, device, abstract: bool = False):
    import torch

    value = torch.empty(shape, dtype=torch_dtype(parameter.dtype), device=device)
    return value, observe_view(parameter, value, device=device, abstract=abstract)
