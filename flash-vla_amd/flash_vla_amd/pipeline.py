"""The encoder and decoder execution plans (mirror `hardware/nvidia/h100/pi0/pipeline.py:57-135`).

These functions allocate nothing and branch on nothing but shapes: each one
issues a fixed sequence of op-table calls against buffers that already exist,
which is what lets the engines record a whole forward as a single hipGraph.
The decoder's token rows are the state token followed by the action chunk.
Per Euler step the noise is projected back into the residual stream, the
layers attend over the prefix K/V cache plus their own rows, and the
out-projection adds the step's velocity into `diffusion_noise` in place.

When the buffers also hold `diffusion_noise_f32`, that fp32 tensor is the Euler
accumulator (read by the in-projection, updated by the out-projection) and is
rounded into the bf16 `diffusion_noise` once, after the last step; otherwise
the bf16 buffer itself is updated every step, as in the reference.
"""
from __future__ import annotations

from .spec import HEAD_DIM


def _batch(buffers) -> int:
    """Requests in flight: the per-request caches are [B, layers, rows, head_dim] when B > 1."""
    k = buffers["encoder_K"]
    return k.shape[0] if k.dim() == 4 else 1


def _layer_cache(buffers, name, i, rows=None):
    """Layer i's K or V cache rows (`rows` a slice) for one request ([rows, hd]) or a batch
    ([B, rows, hd])."""
    c = buffers[name]
    if c.dim() == 4:
        return c[:, i] if rows is None else c[:, i, rows]
    return c[i] if rows is None else c[i][rows]


def vision_encoder(ops, weights, buffers, num_views, layers=None):
    """Patch-embed the images and run the SigLIP layers, in place on `vision_x`
    (pipeline.py:21-54). `ops.vision_attention` is the op-table form of the
    function the reference pipeline calls directly (`kernels/attention.py:20-26`)."""
    if num_views == 2:
        raise ValueError("the num_views == 2 two-part vision branch is not implemented "
                         "(as in the reference, pipeline.py:23)")
    ops.vision_patch_embed(
        buffers["observation_images_normalized"], weights["vision_patch_embedding_w"],
        weights["vision_patch_embedding_b"], weights["vision_position_embedding"],
        buffers["vision_x"])
    n = weights["vision_attn_qkv_w"].shape[0] if layers is None else layers
    for i in range(n):
        ops.vision_norm_qkv(
            buffers["vision_x"],
            weights["vision_pre_attn_norm_w"][i], weights["vision_pre_attn_norm_b"][i],
            weights["vision_attn_qkv_w"][i], weights["vision_attn_qkv_b"][i],
            buffers["vision_QKV"], buffers["vision_x_norm"])
        attn = ops.vision_attention(buffers["vision_QKV"])
        ops.vision_out_proj_residual(
            attn, weights["vision_attn_o_w"][i], weights["vision_attn_o_b"][i],
            buffers["vision_x"], buffers["vision_x"])
        ops.vision_norm_ffn_up(
            buffers["vision_x"],
            weights["vision_pre_ffn_norm_w"][i], weights["vision_pre_ffn_norm_b"][i],
            weights["vision_ffn_up_w"][i], weights["vision_ffn_up_b"][i],
            buffers["vision_hidden"], buffers["vision_x_norm"])
        ops.vision_ffn_down_residual(
            buffers["vision_hidden"],
            weights["vision_ffn_down_w"][i], weights["vision_ffn_down_b"][i],
            buffers["vision_x"], buffers["vision_x"])


def transformer_encoder(ops, weights, buffers, encoder_seq_len, layers=None, project=True):
    """Prefix encoder (pipeline.py:57-89): optional vision projector, then the Gemma layers.

    The last layer runs only its norm + QKV + RoPE: only its K and V are read
    (by the decoder). `project=False` starts from an `encoder_x` already in
    place (the config-3 workload, whose input is the [M, 2048] activation).
    `ops.encoder_attention` is the op-table form of the function the
    reference pipeline calls directly (`kernels/attention.py:29-34`).
    """
    B = _batch(buffers)
    if project:
        views = buffers["vision_x"].shape[0] // B
        for b in range(B):                 # request b's vision rows open its prefix
            ops.encoder_projector(
                buffers["vision_x"][b * views:(b + 1) * views],
                weights["vision_final_norm_w"], weights["vision_final_norm_b"],
                weights["encoder_multi_modal_projector_w"],
                weights["encoder_multi_modal_projector_b"],
                buffers["encoder_x"][b * encoder_seq_len:(b + 1) * encoder_seq_len],
                buffers["vision_x_norm"][b * views:(b + 1) * views])

    scale = HEAD_DIM ** -0.5
    if layers is None:
        layers = weights["encoder_attn_qkv_w"].shape[0]
    prefix = slice(0, encoder_seq_len)
    for i in range(layers):
        k_i = _layer_cache(buffers, "encoder_K", i, prefix)
        v_i = _layer_cache(buffers, "encoder_V", i, prefix)
        ops.encoder_norm_qkv_rope(
            buffers["encoder_x"], weights["encoder_attn_qkv_w"][i],
            buffers["encoder_rope_weights"], buffers["encoder_Q"], k_i, v_i,
            buffers["encoder_x_norm"])
        if i == layers - 1:
            break
        attn = ops.encoder_attention(buffers["encoder_Q"], k_i, v_i, scale)
        ops.encoder_out_proj_residual(attn, weights["encoder_attn_o_w"][i], buffers["encoder_x"])
        ops.encoder_norm_gated_ffn(
            buffers["encoder_x"], weights["encoder_ffn_gate_w"][i], weights["encoder_ffn_up_w"][i],
            buffers["encoder_hidden"], buffers["encoder_x_norm"])
        ops.encoder_ffn_down_residual(
            buffers["encoder_hidden"], weights["encoder_ffn_down_w"][i], buffers["encoder_x"])


def transformer_decoder(ops, weights, buffers, encoder_seq_len, steps=10, layers=18,
                        attention_prefetch=None):
    B = _batch(buffers)
    ops.decoder_state_proj(
        buffers["observation_state_normalized"], weights["decoder_state_in_proj_w"],
        weights["decoder_state_in_proj_b"], buffers["decoder_state_buf"])

    noise = buffers.get("diffusion_noise_f32", buffers["diffusion_noise"])
    dec_rows = slice(encoder_seq_len, None)
    for step in range(steps):
        buffers["decoder_x"][:B].copy_(buffers["decoder_state_buf"])
        ops.decoder_action_in_proj(
            noise, weights["decoder_action_fused_in_proj_w"],
            weights["decoder_action_fused_time_biases"][step % 10], buffers["decoder_x_buf"])
        ops.decoder_action_mlp(
            buffers["decoder_x_buf"], weights["decoder_action_mlp_w"],
            weights["decoder_action_mlp_b"], buffers["decoder_x"][B:])

        for i in range(layers):
            ops.decoder_norm_qkv_rope(
                buffers["decoder_x"], weights["decoder_attn_qkv_w"][i],
                buffers["decoder_rope_weights"], buffers["decoder_q_buf"],
                _layer_cache(buffers, "encoder_K", i, dec_rows),
                _layer_cache(buffers, "encoder_V", i, dec_rows),
                buffers["decoder_norm_factor_buf"])
            attn_args = (buffers["decoder_q_buf"], _layer_cache(buffers, "encoder_K", i),
                         _layer_cache(buffers, "encoder_V", i),
                         buffers["decoder_attn_buf"], buffers["decoder_q_buf"], encoder_seq_len)
            if attention_prefetch is None:
                ops.decoder_attention(*attn_args)
            else:   # same result; also pulls this layer's FFN weights into L2
                attention_prefetch(*attn_args, weights["decoder_ffn_gate_w"][i],
                                   weights["decoder_ffn_up_w"][i], weights["decoder_ffn_down_w"][i],
                                   down_x=buffers["decoder_hidden"])
            ops.decoder_out_proj_residual(
                buffers["decoder_q_buf"].view(buffers["decoder_x"].shape[0], -1), weights["decoder_attn_o_w"][i],
                buffers["decoder_x"])
            ops.decoder_norm_gated_ffn(
                buffers["decoder_x"], weights["decoder_ffn_gate_w"][i],
                weights["decoder_ffn_up_w"][i], buffers["decoder_hidden"],
                buffers["decoder_norm_factor_buf"])
            ops.decoder_ffn_down_residual(
                buffers["decoder_hidden"], weights["decoder_ffn_down_w"][i], buffers["decoder_x"])

        ops.decoder_action_out_proj(
            buffers["decoder_x"][B:], weights["decoder_action_fused_out_proj_w"],
            weights["decoder_action_fused_out_proj_b"], noise,
            buffers["decoder_norm_factor_buf"])

    if noise is not buffers["diffusion_noise"]:
        buffers["diffusion_noise"].copy_(noise)
