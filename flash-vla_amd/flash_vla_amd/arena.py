"""Scratch buffers that survive hipGraph capture.

The interface (`get(role, shape, dtype, device)`, `freeze()`) is the one the
reference's wrappers route scratch through (`src/flash_vla/runtime/cuda/arena.py:19-42`):
a call site names a role and the shape it needs and gets the same device tensor
back on every call. Buffers are created only while the pool is open (the warmup
passes); `freeze()` closes it before capture, after which a request for a slot
the warmup never created is a programming error -- it would put an allocation
inside the graph -- and raises `LookupError`.
"""
from __future__ import annotations

from typing import NamedTuple

import torch


class _Slot(NamedTuple):
    role: str
    shape: tuple
    dtype: torch.dtype
    device: str


class ScratchPool:
    """Role-keyed, zero-initialised device scratch, open until `freeze()`."""

    def __init__(self) -> None:
        self._slots: dict[_Slot, torch.Tensor] = {}
        self._open = True

    def get(self, role: str, shape, dtype, device) -> torch.Tensor:
        slot = _Slot(role, tuple(int(d) for d in shape), dtype, str(device))
        try:
            return self._slots[slot]
        except KeyError:
            pass
        if not self._open:
            raise LookupError(
                f"scratch slot {slot.role!r} {slot.shape} {slot.dtype} on {slot.device} was not "
                "created during warmup; the pool is closed for graph capture")
        tensor = torch.zeros(slot.shape, dtype=dtype, device=device)
        self._slots[slot] = tensor
        return tensor

    def freeze(self) -> None:
        self._open = False

    @property
    def frozen(self) -> bool:
        return not self._open

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self._slots.values())

    def __len__(self) -> int:
        return len(self._slots)
