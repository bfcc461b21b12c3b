"""Reusable execution constraints (reference: `python/intent/targets/execution.py:7-32`)."""
from __future__ import annotations


def indexed_key(device):
    return device


def torch_storage(device, options):
    from ..integrations.torch_staging import TorchStorage

    return TorchStorage(device)


def indexed_target(target, device, *, workers, **options):
    if workers is not None:
        raise ValueError("workers is a CPU execution budget")
    return target(device=device.index, **options).resolve()
