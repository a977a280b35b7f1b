"""Static decoder buffers and the RoPE table (mirrors `hardware/nvidia/h100/pi0/buffers.py`).

Layout in HBM (all bf16, row-major, allocated once; the hot loop only writes
in place):
  encoder_K / encoder_V  [18, enc_len + chunk + 1, 256]  prefix rows then decoder rows
  decoder_x              [chunk + 1, 1024]               residual stream (row 0 = state)
  decoder_q_buf          [(chunk + 1) * 8, 256]          flat (token * 8 + head) queries,
                                                         reused as the attention output
  decoder_hidden         [chunk + 1, 4096]               GeGLU activations
Encoder (prefix) buffers, M = encoder_seq_len token rows:
  encoder_x / encoder_x_norm  [M, 2048]      residual stream / its RMS-normalised copy
  encoder_Q                   [M * 8, 256]   flat queries (token * 8 + head)
  encoder_hidden              [M, 16384]     GeGLU activations
  encoder_rope_weights        [M, 256]       positions 0 .. M - 1
"""
from __future__ import annotations

import torch

from .spec import (DECODER_FFN, DECODER_HEADS, DECODER_LAYERS, DECODER_WIDTH, ENCODER_FFN,
                   ENCODER_LAYERS, ENCODER_WIDTH, HEAD_DIM, ROPE_THETA, VISION_WIDTH)


def rope_table(seq_len: int, offset: int, head_dim: int, device) -> torch.Tensor:
    """RoPE operand of the QKV kernels: bf16 [seq_len, head_dim] (reference `buffers.py:15-23`).

    Row r is position p = offset + r. Column pair (2j, 2j + 1) holds
    (cos(p * w_j), sin(p * w_j)) with w_j = 1 / theta^(2j / head_dim), the
    adjacent-pair rotation the packed Q/K columns use. Angles and their
    cosines / sines are evaluated on the host in fp32 and rounded to bf16
    once, so the table is the same bits whatever device it is copied to.
    """
    half = head_dim // 2
    exponents = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    w = torch.pow(ROPE_THETA, exponents).reciprocal()
    p = torch.arange(offset, offset + seq_len, dtype=torch.float32)
    angles = torch.outer(p, w)                                    # [seq_len, half]
    table = torch.empty(seq_len, half, 2, dtype=torch.bfloat16)
    table[..., 0] = angles.cos()
    table[..., 1] = angles.sin()
    return table.reshape(seq_len, head_dim).to(device)


def allocate_decoder_buffers(encoder_seq_len: int, chunk_size: int, device,
                             layers: int = DECODER_LAYERS, width: int = DECODER_WIDTH,
                             ffn: int = DECODER_FFN, heads: int = DECODER_HEADS,
                             head_dim: int = HEAD_DIM, action_dim: int = 32,
                             batch: int = 1) -> dict:
    """Every persistent buffer the decoder loop touches (buffers.py:37-64, decoder part).

    batch > 1 (the reference is batch-1 only): B requests share
    every GEMM; their rows are stacked "states first" (the B state tokens, then the
    B x chunk action tokens), each request has its own K/V cache
    (`encoder_K/V` [B, layers, cache_len, head_dim]), state is [B, 32] and the noise
    [B * chunk, 32]."""
    bf16 = torch.bfloat16
    dec_len = chunk_size + 1
    cache_len = encoder_seq_len + dec_len
    B = batch

    def buf(*shape, dtype=bf16):
        return torch.zeros(shape, dtype=dtype, device=device)

    cache = (layers, cache_len, head_dim) if B == 1 else (B, layers, cache_len, head_dim)
    buffers = {
        "observation_state_normalized": buf(action_dim) if B == 1 else buf(B, action_dim),
        "diffusion_noise": buf(B * chunk_size, action_dim),
        "encoder_K": buf(*cache),
        "encoder_V": buf(*cache),
        "decoder_rope_weights": buf(dec_len, head_dim),
        "decoder_x": buf(B * dec_len, width),
        "decoder_x_buf": buf(B * chunk_size, width),
        "decoder_state_buf": buf(B, width),
        "decoder_norm_factor_buf": buf(B * dec_len),
        "decoder_q_buf": buf(B * dec_len * heads, head_dim),
        # probabilities of the unfused attention (op_table(fused=False), one request);
        # the fused attention ignores it
        "decoder_attn_buf": buf(dec_len * heads, cache_len) if B == 1 else buf(1, 1),
        "decoder_hidden": buf(B * dec_len, ffn),
    }
    buffers["decoder_rope_weights"].copy_(rope_table(dec_len, encoder_seq_len, head_dim, device))
    return buffers


def allocate_encoder_buffers(encoder_seq_len: int, device, buffers: dict | None = None,
                             layers: int = ENCODER_LAYERS, width: int = ENCODER_WIDTH,
                             ffn: int = ENCODER_FFN, heads: int = DECODER_HEADS,
                             head_dim: int = HEAD_DIM, cache_len: int | None = None,
                             num_views: int = 3, batch: int = 1) -> dict:
    """The encoder part of `buffers.py:37-64`; adds to `buffers` (sharing its K/V cache).
    With batch B the B prefixes are stacked: encoder_x [B * encoder_seq_len, width]."""
    bf16 = torch.bfloat16
    buffers = {} if buffers is None else buffers
    if cache_len is None:
        cache_len = encoder_seq_len

    def buf(*shape):
        return torch.zeros(shape, dtype=bf16, device=device)

    B = batch
    buffers.update({
        "encoder_rope_weights": buf(encoder_seq_len, head_dim),
        "encoder_x": buf(B * encoder_seq_len, width),
        "encoder_x_norm": buf(B * encoder_seq_len, width),
        "encoder_Q": buf(B * encoder_seq_len * heads, head_dim),
        "encoder_hidden": buf(B * encoder_seq_len, ffn),
        "vision_x_norm": buf(B * num_views, 256, VISION_WIDTH),
    })
    if "encoder_K" not in buffers:
        cache = (layers, cache_len, head_dim) if B == 1 else (B, layers, cache_len, head_dim)
        buffers["encoder_K"] = buf(*cache)
        buffers["encoder_V"] = buf(*cache)
    buffers["encoder_rope_weights"].copy_(rope_table(encoder_seq_len, 0, head_dim, device))
    return buffers


def allocate_static_buffers(num_views: int, chunk_size: int, prompt_len: int, device,
                            batch: int = 1) -> tuple[dict, int]:
    """Every persistent buffer of the full forward (buffers.py:25-64 of the reference):
    images, state, noise, vision, encoder and decoder buffers, the K/V cache sized for
    prefix + decoder rows, and both RoPE tables. Returns (buffers, encoder_seq_len).
    batch > 1 stacks B requests (images [B * views, 224, 224, 3])."""
    bf16 = torch.bfloat16
    B = batch
    encoder_seq_len = num_views * 256 + prompt_len
    buffers = allocate_decoder_buffers(encoder_seq_len, chunk_size, device, batch=B)
    cache_len = encoder_seq_len + chunk_size + 1
    allocate_encoder_buffers(encoder_seq_len, device, buffers=buffers, cache_len=cache_len,
                             num_views=num_views, batch=B)

    def buf(*shape):
        return torch.zeros(shape, dtype=bf16, device=device)

    buffers.update({
        "observation_images_normalized": buf(B * num_views, 224, 224, 3),
        "vision_x": buf(B * num_views, 256, VISION_WIDTH),
        "vision_x_norm": buf(B * num_views, 256, VISION_WIDTH),
        "vision_QKV": buf(B * num_views, 256, 3 * VISION_WIDTH),
        "vision_hidden": buf(B * num_views, 256, 4304),
    })
    return buffers, encoder_seq_len
