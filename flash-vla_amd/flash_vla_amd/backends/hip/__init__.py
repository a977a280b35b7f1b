"""HIP (gfx950) backend for the Pi0 decoder and prefix-encoder call sites.

Backend contract (`backends/__init__.py:10-14` of the reference):
    ALL_WRAPPERS   dict[str, Callable]   every decoder and encoder call site
    FUSED_WRAPPERS dict[str, Callable]   fused overlays
"""
from __future__ import annotations

from . import encoder_wrappers, fused_wrappers, wrappers
from .wrappers import prepare_weights, use_pool

# decoder + encoder call sites (wrappers.py:393-403 of the reference), plus
# `encoder_attention`, the function the reference pipeline calls directly
ALL_WRAPPERS = {**wrappers.ALL_WRAPPERS, **encoder_wrappers.ENCODER_WRAPPERS,
                "encoder_attention": encoder_wrappers.encoder_attention}
FUSED_WRAPPERS = dict(fused_wrappers.FUSED_WRAPPERS)

__all__ = ["ALL_WRAPPERS", "FUSED_WRAPPERS", "prepare_weights", "use_pool", "wrappers",
           "fused_wrappers", "encoder_wrappers"]
