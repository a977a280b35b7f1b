"""HIP (gfx950) backend for the Pi0 decoder call sites.

Backend contract (`backends/__init__.py:10-14` of the reference):
    ALL_WRAPPERS   dict[str, Callable]   every decoder call site
    FUSED_WRAPPERS dict[str, Callable]   fused overlays
"""
from __future__ import annotations

from . import fused_wrappers, wrappers
from .wrappers import prepare_weights, use_pool

ALL_WRAPPERS = dict(wrappers.ALL_WRAPPERS)
FUSED_WRAPPERS = dict(fused_wrappers.FUSED_WRAPPERS)

__all__ = ["ALL_WRAPPERS", "FUSED_WRAPPERS", "prepare_weights", "use_pool", "wrappers",
           "fused_wrappers"]
