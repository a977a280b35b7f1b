"""The decoder execution plan (mirrors `hardware/nvidia/h100/pi0/pipeline.py:92-135`).

Pure orchestration: every line is an op-table call on static buffers, so the
loop captures into one hipGraph. Sequence = one state token + the action
chunk; each Euler step re-projects the noise, runs the layers against the
prefix KV cache and updates `diffusion_noise` in place.

When the buffers also hold `diffusion_noise_f32`, that fp32 tensor is the Euler
accumulator (read by the in-projection, updated by the out-projection) and is
rounded into the bf16 `diffusion_noise` once, after the last step; otherwise
the bf16 buffer itself is updated every step, as in the reference.
"""
from __future__ import annotations


def transformer_decoder(ops, weights, buffers, encoder_seq_len, steps=10, layers=18):
    ops.decoder_state_proj(
        buffers["observation_state_normalized"], weights["decoder_state_in_proj_w"],
        weights["decoder_state_in_proj_b"], buffers["decoder_state_buf"])

    noise = buffers.get("diffusion_noise_f32", buffers["diffusion_noise"])
    for step in range(steps):
        buffers["decoder_x"][:1].copy_(buffers["decoder_state_buf"])
        ops.decoder_action_in_proj(
            noise, weights["decoder_action_fused_in_proj_w"],
            weights["decoder_action_fused_time_biases"][step % 10], buffers["decoder_x_buf"])
        ops.decoder_action_mlp(
            buffers["decoder_x_buf"], weights["decoder_action_mlp_w"],
            weights["decoder_action_mlp_b"], buffers["decoder_x"][1:])

        for i in range(layers):
            ops.decoder_norm_qkv_rope(
                buffers["decoder_x"], weights["decoder_attn_qkv_w"][i],
                buffers["decoder_rope_weights"], buffers["decoder_q_buf"],
                buffers["encoder_K"][i][encoder_seq_len:],
                buffers["encoder_V"][i][encoder_seq_len:],
                buffers["decoder_norm_factor_buf"])
            ops.decoder_attention(
                buffers["decoder_q_buf"], buffers["encoder_K"][i], buffers["encoder_V"][i],
                buffers["decoder_attn_buf"], buffers["decoder_q_buf"], encoder_seq_len)
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
            buffers["decoder_x"][1:], weights["decoder_action_fused_out_proj_w"],
            weights["decoder_action_fused_out_proj_b"], noise,
            buffers["decoder_norm_factor_buf"])

    if noise is not buffers["diffusion_noise"]:
        buffers["diffusion_noise"].copy_(noise)
