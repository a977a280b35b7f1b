"""Fused call sites of the HIP backend (the overlay `op_table(fused=True)` selects).

The names and signatures are those of the reference's fused overlay
(`backends/tilelang/fused_wrappers.py:118-122`). In this backend the plain
wrappers already are the fused kernels (the RMS factor is computed inside the
consuming GEMM and attention is split + combine), so the overlay maps to them.
"""
from __future__ import annotations

from . import wrappers

FUSED_WRAPPERS = {
    "decoder_norm_gated_ffn": wrappers.decoder_norm_gated_ffn,
    "decoder_action_out_proj": wrappers.decoder_action_out_proj,
    "decoder_attention": wrappers.decoder_attention,
}
