"""CPU oracle for the Pi0 SigLIP vision tower (TEST INFRASTRUCTURE ONLY).

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg may
import this module, and only as the checker; the HIP product path never calls it.

Restates `vision_encoder` (`hardware/nvidia/h100/pi0/pipeline.py:21-54`) and its
wrappers (`backends/tilelang/wrappers.py:232-315`): 14 x 14 patch embedding as a
GEMM over (iy, ix, c)-ordered patches plus bias plus the 256-row position
embedding, then 27 pre-LN layers at width 1152 (LayerNorm eps 1e-5 with
E[x^2] - mean^2 statistics, packed QKV + bias, 16-head attention per view,
o-proj + bias + residual, LayerNorm, up + bias + tanh-GELU 1152 -> 4304,
down + bias + residual). With `bf16=True` every stored tensor is rounded as the
reference stores it; attention (torch SDPA in the reference,
`kernels/attention.py:20-26`) is exact softmax in fp32 with a bf16 output.
"""
from __future__ import annotations

import math

import torch

from .pi0_decoder import _bf, gelu_tanh
from .pi0_encoder import enc_layer_norm

TOKENS, DIM, HEADS, HEAD_DIM, FFN = 256, 1152, 16, 72, 4304


def patchify(images):
    """[views, 224, 224, 3] -> [views * 256, 588], features in (iy, ix, c) order."""
    v = images.shape[0]
    return (images.reshape(v, 16, 14, 16, 14, 3).permute(0, 1, 3, 2, 4, 5)
            .reshape(v * TOKENS, 14 * 14 * 3))


def patch_embed(images, w, b, pos, bf16=True):
    """patches @ w.reshape(588, 1152) + b + pos[row % 256] (wrappers.py:257-269)."""
    p = patchify(images.to(w.dtype))
    out = p @ w.reshape(-1, DIM) + b
    out = out.reshape(-1, TOKENS, DIM) + pos
    return _bf(out.reshape(-1, DIM), bf16)


def vision_attention(qkv, views, bf16=True):
    """Per view and head softmax(q k^T / sqrt(72)) v over the 256 tokens (attention.py:20-26)."""
    x = qkv.reshape(views, TOKENS, 3, HEADS, HEAD_DIM).permute(0, 2, 3, 1, 4)
    q, k, v = x[:, 0], x[:, 1], x[:, 2]                  # [views, heads, tokens, 72]
    s = (q @ k.transpose(-1, -2)) / math.sqrt(HEAD_DIM)
    o = torch.softmax(s, dim=-1) @ v
    return _bf(o.transpose(1, 2).reshape(views * TOKENS, DIM), bf16)


def vision_layer(x, w: dict, i: int, views: int, bf16=True):
    """One pre-LN SigLIP layer on [views * 256, 1152] (pipeline.py:33-54)."""
    xn = enc_layer_norm(x, w["vision_pre_attn_norm_w"][i], w["vision_pre_attn_norm_b"][i], 1e-5, bf16)
    qkv = _bf(xn @ w["vision_attn_qkv_w"][i] + w["vision_attn_qkv_b"][i], bf16)
    o = vision_attention(qkv, views, bf16)
    x = _bf(o @ w["vision_attn_o_w"][i] + w["vision_attn_o_b"][i] + x, bf16)
    xn = enc_layer_norm(x, w["vision_pre_ffn_norm_w"][i], w["vision_pre_ffn_norm_b"][i], 1e-5, bf16)
    h = _bf(gelu_tanh(xn @ w["vision_ffn_up_w"][i] + w["vision_ffn_up_b"][i]), bf16)
    return _bf(h @ w["vision_ffn_down_w"][i] + w["vision_ffn_down_b"][i] + x, bf16)


def vision_tower(weights: dict, images, layers: int | None = None, bf16=True,
                 dtype=torch.float32):
    """Patch embedding + layers; returns vision_x [views * 256, 1152]."""
    w = {k: v.to(dtype) for k, v in weights.items() if k.startswith("vision_")}
    n = w["vision_attn_qkv_w"].shape[0] if layers is None else layers
    views = images.shape[0]
    x = patch_embed(images.to(dtype), w["vision_patch_embedding_w"], w["vision_patch_embedding_b"],
                    w["vision_position_embedding"], bf16)
    for i in range(n):
        x = vision_layer(x, w, i, views, bf16)
    return x


def full_forward(weights: dict, images, state, noise, num_views: int = 3, steps: int = 10,
                 bf16=True, dtype=torch.float32, fp32_noise=True):
    """Pi0Inference._run (engine.py:58-65): vision tower, projector, prefix encoder over
    [vision tokens | language_embeds], then the decoder loop against the resulting K/V.
    Layer counts follow the stacks in `weights`. Returns (noise, K, V)."""
    from . import pi0_decoder as O
    from . import pi0_encoder as E
    w = {k: v.to(dtype) for k, v in weights.items()}
    vx = vision_tower(w, images.to(dtype), bf16=bf16, dtype=dtype)
    enc_in = E.enc_projector(vx, w["vision_final_norm_w"], w["vision_final_norm_b"],
                             w["encoder_multi_modal_projector_w"],
                             w["encoder_multi_modal_projector_b"], bf16)
    lang = w["language_embeds"]
    x = torch.cat([enc_in, lang], 0) if lang.shape[0] else enc_in
    K, V, _ = E.encoder_packed(w, x, bf16=bf16, dtype=dtype)
    enc_len = x.shape[0]
    layers = w["decoder_attn_qkv_w"].shape[0]
    total = enc_len + noise.shape[0] + 1
    Kc = torch.zeros(layers, total, K.shape[-1], dtype=dtype)
    Vc = torch.zeros_like(Kc)
    n = min(layers, K.shape[0])
    Kc[:n, :enc_len], Vc[:n, :enc_len] = K[:n], V[:n]
    out = O.decoder_packed(w, state, noise, Kc, Vc, enc_len, steps=steps, layers=layers,
                           bf16=bf16, dtype=dtype, fp32_noise=fp32_noise)
    return out[0], K, V
