"""HIP (gfx950) backend for the Pi0 vision, prefix-encoder and decoder call sites.

Backend contract (`backends/__init__.py:10-14` of the reference):
    ALL_WRAPPERS   dict[str, Callable]   every vision, encoder and decoder call site
    FUSED_WRAPPERS dict[str, Callable]   fused overlays
"""
from __future__ import annotations

from . import encoder_wrappers, vision_wrappers, wrappers
from .wrappers import (attention_prefetch_for, check_pinned, pin_packed_weights, prepare_weights,
                       repack_stale, use_pool)

# vision + encoder + decoder call sites (wrappers.py:393-403 of the reference), plus
# `vision_attention` / `encoder_attention`, the functions the reference pipeline
# calls directly (kernels/attention.py:20-34)
ALL_WRAPPERS = {**vision_wrappers.VISION_WRAPPERS, **encoder_wrappers.ENCODER_WRAPPERS,
                **wrappers.ALL_WRAPPERS,
                "vision_attention": vision_wrappers.vision_attention,
                "encoder_attention": encoder_wrappers.encoder_attention,
                "embed_prompt": encoder_wrappers.embed_prompt}
FUSED_WRAPPERS = dict(wrappers.FUSED_WRAPPERS)
# Engine-level option outside the op table: `attention_prefetch_for(op)` returns the form
# of this backend's decoder_attention that also prefetches the layer's FFN weights.

__all__ = ["ALL_WRAPPERS", "FUSED_WRAPPERS", "attention_prefetch_for", "check_pinned",
           "pin_packed_weights", "prepare_weights", "repack_stale", "use_pool",
           "wrappers",
           "encoder_wrappers", "vision_wrappers"]
