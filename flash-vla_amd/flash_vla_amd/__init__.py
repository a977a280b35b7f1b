"""MI355X-native (gfx950) HIP implementation of the Pi0 action-expert denoising loop.

    from flash_vla_amd import Pi0DecoderEngine, decoder_checkpoint, op_table

The public names follow the reference package facade (`src/flash_vla/__init__.py:19-34`):
`random_checkpoint` and `op_table`; the decoder loop engine is `Pi0DecoderEngine`.
"""
from __future__ import annotations

__all__ = ["Pi0Inference", "Pi0DecoderEngine", "Pi0EncoderEngine", "random_checkpoint", "decoder_checkpoint", "decoder_inputs",
           "op_table"]


def __getattr__(name: str):
    if name in ("random_checkpoint", "decoder_checkpoint", "decoder_inputs"):
        from . import weights

        value = getattr(weights, name)
    elif name == "op_table":
        from .ops import op_table as value
    elif name == "Pi0DecoderEngine":
        from .engine import Pi0DecoderEngine as value
    elif name == "Pi0EncoderEngine":
        from .engine import Pi0EncoderEngine as value
    elif name == "Pi0Inference":
        from .engine import Pi0Inference as value
    else:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    globals()[name] = value
    return value
