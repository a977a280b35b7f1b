"""Fused call sites of the HIP backend (the overlay `op_table(fused=True)` selects).

The names, signatures and semantics are those of the reference's fused overlay
(`backends/tilelang/fused_wrappers.py:45-122`):
  decoder_norm_gated_ffn   RMS factor computed inside the dual GEMM from its own A
                           fragments and applied to the fp32 accumulators (fused_norm.py:26-78)
  decoder_action_out_proj  the same for the Euler out-projection (fused_norm.py:81-125)
  decoder_attention        FlashDecoding split + combine, the score matrix never leaves
                           the kernel and `scores` is ignored (base.py:801-923)
The unfused forms in `ALL_WRAPPERS` round x * f (and the scores) to bf16 instead.
"""
from __future__ import annotations

from . import wrappers

FUSED_WRAPPERS = {
    "decoder_norm_gated_ffn": wrappers.decoder_norm_gated_ffn,
    "decoder_action_out_proj": wrappers.decoder_action_out_proj,
    "decoder_attention": wrappers.decoder_attention,
}
