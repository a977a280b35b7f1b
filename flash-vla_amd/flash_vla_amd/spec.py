"""Pi0 constants and the packed checkpoint schema.

The schema is an interface shared with the reference, so names and shapes are
identical to `src/flash_vla/models/pi0/spec.py:10-47`: weights are stored
`[in, out]` (K x N) row-major bf16, per-layer tensors stacked on a leading
layer axis, Q/K columns in adjacent-pair (interleaved) RoPE order.
"""
from __future__ import annotations

VISION_LAYERS = 27
ENCODER_LAYERS = 18
DECODER_LAYERS = 18
HEAD_DIM = 256
DECODER_HEADS = 8
ROPE_THETA = 10000
DECODER_WIDTH = 1024
ENCODER_WIDTH = 2048
ENCODER_FFN = 16384
VISION_WIDTH = 1152
VISION_TOKENS = 256
DECODER_FFN = 4096
ACTION_DIM = 32
NUM_STEPS = 10
RMS_EPS = 1e-6

# Decoder tensors, in the order the seeded generator draws them.
DECODER_WEIGHT_NAMES = (
    "decoder_state_in_proj_w", "decoder_state_in_proj_b",
    "decoder_action_fused_in_proj_w", "decoder_action_fused_time_biases",
    "decoder_action_mlp_w", "decoder_action_mlp_b",
    "decoder_attn_qkv_w", "decoder_attn_o_w",
    "decoder_ffn_gate_w", "decoder_ffn_up_w", "decoder_ffn_down_w",
    "decoder_action_fused_out_proj_w", "decoder_action_fused_out_proj_b",
)


def weight_shapes(prompt_len: int) -> dict[str, tuple[int, ...]]:
    """Every checkpoint tensor of a Pi0 model with this prompt length."""
    L, V = ENCODER_LAYERS, VISION_LAYERS
    return {
        "vision_patch_embedding_w": (14, 14, 3, 1152), "vision_patch_embedding_b": (1152,),
        "vision_position_embedding": (256, 1152),
        "vision_attn_qkv_w": (V, 1152, 3 * 1152), "vision_attn_qkv_b": (V, 3 * 1152),
        "vision_attn_o_w": (V, 1152, 1152), "vision_attn_o_b": (V, 1152),
        "vision_ffn_up_w": (V, 1152, 4304), "vision_ffn_up_b": (V, 4304),
        "vision_ffn_down_w": (V, 4304, 1152), "vision_ffn_down_b": (V, 1152),
        "vision_pre_attn_norm_w": (V, 1152), "vision_pre_attn_norm_b": (V, 1152),
        "vision_pre_ffn_norm_w": (V, 1152), "vision_pre_ffn_norm_b": (V, 1152),
        "vision_final_norm_w": (1152,), "vision_final_norm_b": (1152,),
        "encoder_multi_modal_projector_w": (1152, 2048),
        "encoder_multi_modal_projector_b": (2048,),
        "encoder_attn_qkv_w": (L, 2048, 2560),
        "encoder_attn_o_w": (L, 2048, 2048),
        "encoder_ffn_gate_w": (L, 2048, 16384),
        "encoder_ffn_up_w": (L, 2048, 16384),
        "encoder_ffn_down_w": (L, 16384, 2048),
        **decoder_weight_shapes(DECODER_LAYERS),
        "language_embeds": (prompt_len, 2048),
    }


def decoder_weight_shapes(layers: int = DECODER_LAYERS, width: int = DECODER_WIDTH,
                          ffn: int = DECODER_FFN, heads: int = DECODER_HEADS,
                          head_dim: int = HEAD_DIM, action_dim: int = ACTION_DIM,
                          steps: int = NUM_STEPS) -> dict[str, tuple[int, ...]]:
    """The 13 decoder tensors (`spec.py:35-45` of the reference), optionally at reduced size."""
    qkv = (heads + 2) * head_dim
    return {
        "decoder_state_in_proj_w": (action_dim, width), "decoder_state_in_proj_b": (width,),
        "decoder_action_fused_in_proj_w": (action_dim, width),
        "decoder_action_fused_time_biases": (steps, width),
        "decoder_action_mlp_w": (width, width), "decoder_action_mlp_b": (width,),
        "decoder_attn_qkv_w": (layers, width, qkv),
        "decoder_attn_o_w": (layers, heads * head_dim, width),
        "decoder_ffn_gate_w": (layers, width, ffn), "decoder_ffn_up_w": (layers, width, ffn),
        "decoder_ffn_down_w": (layers, ffn, width),
        "decoder_action_fused_out_proj_w": (width, action_dim),
        "decoder_action_fused_out_proj_b": (action_dim,),
    }
