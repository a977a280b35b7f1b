"""Seeded Pi0 checkpoints and decoder inputs.

Everything is drawn from one CPU `torch.Generator`, so the same seed gives the
same bits on any machine (the CUDA/ROCm Philox streams differ between vendors),
then moved to the requested device.

Two generators:

* `random_checkpoint` keeps the reference's public helper
  (`src/flash_vla/models/pi0/weights.py:10-24`): every packed tensor is
  N(0, 1) * wscale in fp32, cast to bf16, drawn in schema order.
* `decoder_checkpoint` builds the decoder tensors the way a real checkpoint is
  produced: it draws the *unfolded* action-expert parameters (OpenPI layout,
  RMSNorm weights 0 so that 1 + w = 1) and folds them into the packed schema
  with `fold_decoder`, the algebra of `eval/baselines/openpi.py:86-125,270-302`.
"""
from __future__ import annotations

import math

import torch

from .spec import (ACTION_DIM, DECODER_FFN, DECODER_HEADS, DECODER_LAYERS, DECODER_WIDTH,
                   ENCODER_FFN, ENCODER_LAYERS, ENCODER_WIDTH, HEAD_DIM, NUM_STEPS, weight_shapes)

EULER_DT = -0.1
TIME_MIN_PERIOD = 4e-3
TIME_MAX_PERIOD = 4.0


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)


def random_checkpoint(num_views: int = 3, chunk_size: int = 50, prompt_len: int = 256,
                      wscale: float = 0.05, seed: int = 0, device: str = "cuda",
                      draw_on_device: bool = False) -> dict:
    """Synthetic packed checkpoint, N(0,1)*wscale per tensor in schema order.

    `draw_on_device=True` draws on `device`'s own seeded generator (fast for the
    2.7 B-parameter model; the values then differ from the CPU draw)."""
    del num_views, chunk_size
    gen = (torch.Generator(device=device).manual_seed(seed) if draw_on_device else _gen(seed))
    out = {}
    for name, shape in weight_shapes(prompt_len).items():
        t = torch.randn(shape, dtype=torch.float32, generator=gen, device=gen.device) * wscale
        out[name] = t.to(torch.bfloat16).to(device)
    return out


def openpi_decoder_params(seed: int = 0, std: float = 0.02, layers: int = DECODER_LAYERS,
                          width: int = DECODER_WIDTH, ffn: int = DECODER_FFN,
                          heads: int = DECODER_HEADS, head_dim: int = HEAD_DIM,
                          action_dim: int = ACTION_DIM, dtype=torch.float32) -> dict:
    """Unfolded action-expert parameters, `[in, out]` matrices, N(0, std) each.

    Q/K projections are in OpenPI's half-split RoPE column order. Norm weights
    are zero (Gemma's RMSNorm multiplies by 1 + w).
    """
    gen = _gen(seed)

    def draw(*shape):
        return (torch.randn(shape, dtype=torch.float32, generator=gen) * std).to(dtype)

    p = {
        "state_proj_w": draw(action_dim, width), "state_proj_b": draw(width),
        "action_in_w": draw(action_dim, width), "action_in_b": draw(width),
        "time_mlp_in_w": draw(2 * width, width), "time_mlp_in_b": draw(width),
        "time_mlp_out_w": draw(width, width), "time_mlp_out_b": draw(width),
    }
    per_layer = {k: [] for k in ("q_w", "k_w", "v_w", "o_w", "gate_w", "up_w", "down_w")}
    for _ in range(layers):
        per_layer["q_w"].append(draw(width, heads * head_dim))
        per_layer["k_w"].append(draw(width, head_dim))
        per_layer["v_w"].append(draw(width, head_dim))
        per_layer["o_w"].append(draw(heads * head_dim, width))
        per_layer["gate_w"].append(draw(width, ffn))
        per_layer["up_w"].append(draw(width, ffn))
        per_layer["down_w"].append(draw(ffn, width))
    for k, v in per_layer.items():
        p[k] = torch.stack(v)
    p["action_out_w"] = draw(width, action_dim)
    p["action_out_b"] = draw(action_dim)
    p["input_norm_w"] = torch.zeros(layers, width, dtype=dtype)
    p["post_attn_norm_w"] = torch.zeros(layers, width, dtype=dtype)
    p["final_norm_w"] = torch.zeros(width, dtype=dtype)
    return p


def euler_times(steps: int = NUM_STEPS, dt: float = EULER_DT) -> torch.Tensor:
    """t = 1, 1+dt, ... accumulated in fp32 (`openpi.py:282-287`)."""
    t = torch.tensor(1.0, dtype=torch.float32)
    step = torch.tensor(dt, dtype=torch.float32)
    out = []
    for _ in range(steps):
        out.append(t.clone())
        t = t + step
    return torch.stack(out)


def sinusoidal_time_embedding(times: torch.Tensor, width: int,
                              min_period: float = TIME_MIN_PERIOD,
                              max_period: float = TIME_MAX_PERIOD) -> torch.Tensor:
    """Pi0's sine-cosine time embedding, [sin | cos] halves, computed in fp64.

    period_i = min_period * (max_period / min_period) ** (i / (width/2 - 1)),
    emb = [sin(2*pi*t/period), cos(2*pi*t/period)].
    """
    half = width // 2
    frac = torch.linspace(0.0, 1.0, half, dtype=torch.float64)
    period = min_period * (max_period / min_period) ** frac
    phase = times.to(torch.float64)[:, None] * (2.0 * math.pi / period)[None, :]
    return torch.cat([torch.sin(phase), torch.cos(phase)], dim=1)


def interleave_rope_columns(weight: torch.Tensor, heads: int) -> torch.Tensor:
    """Half-split RoPE column order -> adjacent-pair order (`openpi.py:101-109`)."""
    inputs, outputs = weight.shape[-2:]
    hd = outputs // heads
    lead = weight.shape[:-2]
    return (weight.reshape(*lead, inputs, heads, 2, hd // 2)
            .transpose(-1, -2).reshape(*lead, inputs, outputs))


def fold_gemma_layers(p: dict) -> tuple:
    """Fold the stacked Gemma layers of `p` into (qkv, o, gate, up, down), `[in, out]`.

    Input-norm (1 + w) scales the rows of Q, K and V; the post-attention norm
    scales the rows of gate and up (`openpi.py:86-90`); Q and K columns move
    from half-split to adjacent-pair RoPE order (`openpi.py:101-125`).
    """
    heads = p["q_w"].shape[-1] // p["k_w"].shape[-1]
    in_scale = (1.0 + p["input_norm_w"])[:, :, None]
    post_scale = (1.0 + p["post_attn_norm_w"])[:, :, None]
    qkv = torch.cat([
        interleave_rope_columns(p["q_w"] * in_scale, heads),
        interleave_rope_columns(p["k_w"] * in_scale, 1),
        p["v_w"] * in_scale,
    ], dim=-1)
    return qkv, p["o_w"], p["gate_w"] * post_scale, p["up_w"] * post_scale, p["down_w"]


def fold_decoder(p: dict, steps: int = NUM_STEPS, dt: float = EULER_DT,
                 out_dtype=torch.bfloat16) -> dict:
    """Fold unfolded parameters into the packed decoder schema.

    * RMSNorm (1 + w) scales fold into the rows of the consuming projection.
    * action_in_proj and the time half of action_time_mlp_in fold into one
      32 -> width projection plus one bias per Euler step.
    * final norm (1 + w) and the Euler dt fold into the output projection, so
      the step becomes `noise += b' + rms(x) @ W'`.
    """
    width = p["time_mlp_out_w"].shape[0]
    qkv, o_w, gate, up, down = fold_gemma_layers(p)
    mix_a = p["time_mlp_in_w"][:width]
    mix_t = p["time_mlp_in_w"][width:]
    temb = sinusoidal_time_embedding(euler_times(steps, dt), width).to(p["action_in_w"].dtype)
    time_biases = p["action_in_b"] @ mix_a + temb @ mix_t + p["time_mlp_in_b"]
    final = (1.0 + p["final_norm_w"])[:, None]
    out = {
        "decoder_state_in_proj_w": p["state_proj_w"], "decoder_state_in_proj_b": p["state_proj_b"],
        "decoder_action_fused_in_proj_w": p["action_in_w"] @ mix_a,
        "decoder_action_fused_time_biases": time_biases,
        "decoder_action_mlp_w": p["time_mlp_out_w"], "decoder_action_mlp_b": p["time_mlp_out_b"],
        "decoder_attn_qkv_w": qkv,
        "decoder_attn_o_w": o_w,
        "decoder_ffn_gate_w": gate,
        "decoder_ffn_up_w": up,
        "decoder_ffn_down_w": down,
        "decoder_action_fused_out_proj_w": dt * final * p["action_out_w"],
        "decoder_action_fused_out_proj_b": dt * p["action_out_b"],
    }
    return {k: v.to(out_dtype).contiguous() for k, v in out.items()}


def decoder_checkpoint(seed: int = 0, std: float = 0.02, layers: int = DECODER_LAYERS,
                       device: str = "cpu", **dims) -> dict:
    """Packed decoder tensors folded from seeded unfolded parameters (BASELINE config 1/2)."""
    packed = fold_decoder(openpi_decoder_params(seed, std, layers, **dims))
    return {k: v.to(device) for k, v in packed.items()}


def decoder_inputs(seed: int = 1, encoder_seq_len: int = 768, chunk_size: int = 50,
                   layers: int = DECODER_LAYERS, head_dim: int = HEAD_DIM,
                   action_dim: int = ACTION_DIM, kv_std: float = 1.0,
                   device: str = "cpu") -> dict:
    """State [32], noise [chunk, 32] and the prefix K/V cache, all N(0,1) (K/V N(0, kv_std)).

    The K/V caches are allocated at their full `[layers, enc + chunk + 1, head_dim]`
    size with the decoder rows zeroed; the decoder writes those rows itself.
    """
    gen = _gen(seed)
    bf16 = torch.bfloat16
    state = torch.randn(action_dim, generator=gen).to(bf16)
    noise = torch.randn(chunk_size, action_dim, generator=gen).to(bf16)
    total = encoder_seq_len + chunk_size + 1
    k = torch.zeros(layers, total, head_dim, dtype=bf16)
    v = torch.zeros(layers, total, head_dim, dtype=bf16)
    k[:, :encoder_seq_len] = (torch.randn(layers, encoder_seq_len, head_dim, generator=gen)
                              * kv_std).to(bf16)
    v[:, :encoder_seq_len] = (torch.randn(layers, encoder_seq_len, head_dim, generator=gen)
                              * kv_std).to(bf16)
    return {"observation_state_normalized": state.to(device),
            "diffusion_noise": noise.to(device),
            "encoder_K": k.to(device), "encoder_V": v.to(device)}


ENCODER_WEIGHT_NAMES = ("encoder_attn_qkv_w", "encoder_attn_o_w", "encoder_ffn_gate_w",
                        "encoder_ffn_up_w", "encoder_ffn_down_w")


def encoder_checkpoint(seed: int = 2, std: float = 0.02, layers: int = ENCODER_LAYERS,
                       width: int = ENCODER_WIDTH, ffn: int = ENCODER_FFN,
                       heads: int = DECODER_HEADS, head_dim: int = HEAD_DIM,
                       device: str = "cpu", draw_on_device: bool = False) -> dict:
    """Packed prefix-encoder tensors, N(0, std) per element.

    With Gemma RMSNorm weights 0 the fold of `fold_decoder` multiplies the
    projections by 1 and only permutes Q/K columns, which leaves i.i.d. normal
    entries i.i.d. normal: drawing the packed tensors directly gives the same
    distribution (the fold algebra itself is pinned against the unfolded layer
    at small size by the oracle tests). Drawn layer by layer on the CPU
    generator, rounded to bf16 at once, so the 18-layer set (~4 GB) never exists
    in fp32. `draw_on_device=True` draws on `device`'s own seeded generator
    instead (fast; the values then differ from the CPU draw).
    """
    gen = (torch.Generator(device=device).manual_seed(seed) if draw_on_device else _gen(seed))
    shapes = {
        "encoder_attn_qkv_w": (width, (heads + 2) * head_dim),
        "encoder_attn_o_w": (heads * head_dim, width),
        "encoder_ffn_gate_w": (width, ffn),
        "encoder_ffn_up_w": (width, ffn),
        "encoder_ffn_down_w": (ffn, width),
    }
    out = {n: torch.empty((layers, *sh), dtype=torch.bfloat16, device=device)
           for n, sh in shapes.items()}
    for i in range(layers):
        for n, sh in shapes.items():
            draw = torch.randn(sh, generator=gen, device=gen.device)
            out[n][i].copy_((draw * std).to(torch.bfloat16))
    return out


def encoder_inputs(seed: int = 3, encoder_seq_len: int = 768, width: int = ENCODER_WIDTH,
                   device: str = "cpu") -> torch.Tensor:
    """The config-3 encoder input: a seeded N(0, 1) bf16 [encoder_seq_len, width] activation."""
    gen = _gen(seed)
    return torch.randn(encoder_seq_len, width, generator=gen).to(torch.bfloat16).to(device)
