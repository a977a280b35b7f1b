"""Graph-safe scratch memory (mirrors `src/flash_vla/runtime/cuda/arena.py:19-42`).

Each (role, shape, dtype, device) buffer is allocated once, zeroed, and reused.
After warmup the pool is frozen: a request that warmup did not cover raises
instead of allocating inside a hipGraph capture.
"""
from __future__ import annotations

import torch


class ScratchPool:
    def __init__(self) -> None:
        self._buffers: dict = {}
        self._frozen = False

    def get(self, role: str, shape, dtype, device) -> torch.Tensor:
        key = (role, tuple(shape), dtype, str(device))
        buffer = self._buffers.get(key)
        if buffer is None:
            if self._frozen:
                raise RuntimeError(
                    f"ScratchPool is frozen but {key} was requested: warmup did not cover this "
                    "shape, so it would allocate mid-capture.")
            buffer = torch.zeros(shape, dtype=dtype, device=device)
            self._buffers[key] = buffer
        return buffer

    def freeze(self) -> None:
        self._frozen = True

    @property
    def frozen(self) -> bool:
        return self._frozen

    def __len__(self) -> int:
        return len(self._buffers)
