"""OpenPI-form Pi0 reference written directly on a raw OpenPI state dict (test helper).

Shared by the CPU conversion tests and the GPU test that runs converted weights
through the HIP engine. It uses `nn.Linear`-layout `[out, in]` weights through
`F.linear`, Gemma RMSNorm with `1 + w`, rotate-half RoPE at absolute positions
and `F.scaled_dot_product_attention`, and shares no code with the converter
or the packed oracle. It follows the sampling loop the reference's OpenPI
baseline drives (`eval/baselines/openpi.py:270-302`): Euler from t = 1 with
dt = -0.1, the sinusoidal time embedding with periods geometric from 4e-3 to 4.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from flash_vla_amd import convert as C

DT = -0.1          # the converter folds dt as this double into the output projection


@dataclass(frozen=True)
class Dims:
    """Widths of a (possibly reduced) Pi0: Gemma prefix encoder, action expert, SigLIP."""
    enc_width: int = 48
    enc_ffn: int = 80
    enc_layers: int = 2
    dec_width: int = 64
    dec_ffn: int = 96
    dec_layers: int = 2
    heads: int = 2
    head_dim: int = 16
    action: int = 8
    vis_width: int = 24
    vis_ffn: int = 40
    vis_layers: int = 2
    vis_tokens: int = 256


SMALL = Dims()
# the action expert at its real size (2 layers); encoder and vision stay reduced
FULL_DECODER = Dims(enc_width=48, enc_ffn=64, enc_layers=1, dec_width=1024, dec_ffn=4096,
                    dec_layers=2, heads=8, head_dim=256, action=32, vis_width=16,
                    vis_ffn=16, vis_layers=1)


def openpi_state(d: Dims = SMALL, seed: int = 0, std: float = 0.15, norm_std: float = 0.3,
                 dtype=torch.float64) -> dict:
    """A seeded OpenPI Pi0 state dict with the checkpoint's own tensor names.

    Norm weights and biases are drawn non-zero so that every fold is exercised.
    """
    g = torch.Generator().manual_seed(seed)
    sd = {}

    def put(name, *shape, scale=std):
        sd[name] = (torch.randn(shape, generator=g, dtype=torch.float64) * scale).to(dtype)

    vw, vf = d.vis_width, d.vis_ffn
    v = C.VISION
    put(f"{v}.embeddings.patch_embedding.weight", vw, 3, 14, 14, scale=0.05)
    put(f"{v}.embeddings.patch_embedding.bias", vw)
    put(f"{v}.embeddings.position_embedding.weight", d.vis_tokens, vw)
    for i in range(d.vis_layers):
        lay = f"{v}.encoder.layers.{i}"
        for p in ("q", "k", "v"):
            put(f"{lay}.self_attn.{p}_proj.weight", vw, vw, scale=std / 2)
            put(f"{lay}.self_attn.{p}_proj.bias", vw)
        put(f"{lay}.self_attn.out_proj.weight", vw, vw, scale=std / 2)
        put(f"{lay}.self_attn.out_proj.bias", vw)
        put(f"{lay}.mlp.fc1.weight", vf, vw, scale=std / 2)
        put(f"{lay}.mlp.fc1.bias", vf)
        put(f"{lay}.mlp.fc2.weight", vw, vf, scale=std / 2)
        put(f"{lay}.mlp.fc2.bias", vw)
        for n in ("layer_norm1", "layer_norm2"):
            put(f"{lay}.{n}.weight", vw)
            sd[f"{lay}.{n}.weight"] += 1.0
            put(f"{lay}.{n}.bias", vw)
    put(f"{v}.post_layernorm.weight", vw)
    put(f"{v}.post_layernorm.bias", vw)
    put(f"{C.PROJECTOR}.weight", d.enc_width, vw)
    put(f"{C.PROJECTOR}.bias", d.enc_width)

    def gemma(root, width, ffn, layers):
        hq = d.heads * d.head_dim
        for i in range(layers):
            lay = f"{root}.layers.{i}"
            put(f"{lay}.self_attn.q_proj.weight", hq, width)
            put(f"{lay}.self_attn.k_proj.weight", d.head_dim, width)
            put(f"{lay}.self_attn.v_proj.weight", d.head_dim, width)
            put(f"{lay}.self_attn.o_proj.weight", width, hq)
            put(f"{lay}.mlp.gate_proj.weight", ffn, width)
            put(f"{lay}.mlp.up_proj.weight", ffn, width)
            put(f"{lay}.mlp.down_proj.weight", width, ffn)
            put(f"{lay}.input_layernorm.weight", width, scale=norm_std)
            put(f"{lay}.post_attention_layernorm.weight", width, scale=norm_std)
        put(f"{root}.norm.weight", width, scale=norm_std)

    gemma(C.ENCODER, d.enc_width, d.enc_ffn, d.enc_layers)
    gemma(C.DECODER, d.dec_width, d.dec_ffn, d.dec_layers)
    dw, a = d.dec_width, d.action
    put("state_proj.weight", dw, a)
    put("state_proj.bias", dw)
    put("action_in_proj.weight", dw, a)
    put("action_in_proj.bias", dw)
    put("action_time_mlp_in.weight", dw, 2 * dw)
    put("action_time_mlp_in.bias", dw)
    put("action_time_mlp_out.weight", dw, dw)
    put("action_time_mlp_out.bias", dw)
    put("action_out_proj.weight", a, dw)
    put("action_out_proj.bias", a)
    return sd


def rms(x, w):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + w)


def rotate_half_rope(x, pos, head_dim):
    """HF Gemma RoPE: x * cos + rotate_half(x) * sin, frequencies duplicated over halves."""
    n = x.shape[-1] // head_dim
    inv = 1.0 / (10000.0 ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    ang = pos.to(torch.float64)[:, None] * inv[None]
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos()[:, None].to(x.dtype), emb.sin()[:, None].to(x.dtype)
    xh = x.reshape(x.shape[0], n, head_dim)
    rot = torch.cat([-xh[..., head_dim // 2:], xh[..., :head_dim // 2]], -1)
    return (xh * cos + rot * sin).reshape(x.shape)


def gemma_qkv(sd, root, i, x, pos, d: Dims):
    lay = f"{root}.layers.{i}"
    h = rms(x, sd[f"{lay}.input_layernorm.weight"])
    q = rotate_half_rope(F.linear(h, sd[f"{lay}.self_attn.q_proj.weight"]), pos, d.head_dim)
    k = rotate_half_rope(F.linear(h, sd[f"{lay}.self_attn.k_proj.weight"]), pos, d.head_dim)
    v = F.linear(h, sd[f"{lay}.self_attn.v_proj.weight"])
    return q, k, v


def gemma_rest(sd, root, i, x, q, K, V, mask, d: Dims):
    lay = f"{root}.layers.{i}"
    T = x.shape[0]
    qh = q.reshape(T, d.heads, d.head_dim).transpose(0, 1)
    o = F.scaled_dot_product_attention(qh, K[None].expand(d.heads, -1, -1),
                                       V[None].expand(d.heads, -1, -1), attn_mask=mask)
    x = x + F.linear(o.transpose(0, 1).reshape(T, d.heads * d.head_dim),
                     sd[f"{lay}.self_attn.o_proj.weight"])
    h = rms(x, sd[f"{lay}.post_attention_layernorm.weight"])
    g = F.gelu(F.linear(h, sd[f"{lay}.mlp.gate_proj.weight"]), approximate="tanh")
    u = F.linear(h, sd[f"{lay}.mlp.up_proj.weight"])
    return x + F.linear(g * u, sd[f"{lay}.mlp.down_proj.weight"])


def openpi_prefix(sd, x, d: Dims = SMALL):
    """Gemma prefix encoder: bidirectional; returns per-layer rotated K and V."""
    pos = torch.arange(x.shape[0])
    Ks, Vs = [], []
    for i in range(d.enc_layers):
        q, k, v = gemma_qkv(sd, C.ENCODER, i, x, pos, d)
        Ks.append(k), Vs.append(v)
        x = gemma_rest(sd, C.ENCODER, i, x, q, k, v, None, d)
    return Ks, Vs


def time_embedding(t: float, width: int, dtype=torch.float64) -> torch.Tensor:
    """[sin | cos] of 2*pi*t / period, periods geometric from 4e-3 to 4 over width/2 entries."""
    frac = torch.linspace(0, 1, width // 2, dtype=torch.float64)
    period = 4e-3 * (4.0 / 4e-3) ** frac
    ph = float(t) * 2 * math.pi / period
    return torch.cat([ph.sin(), ph.cos()]).to(dtype)


def openpi_decode(sd, Ks, Vs, state, noise, d: Dims = SMALL, steps: int = 10):
    """Pi0 flow-matching sampling over the action expert against prefix K/V per layer
    (OpenPI's rotate-half column order)."""
    M, T = Ks[0].shape[0], noise.shape[0] + 1
    pos = torch.arange(M, M + T)
    mask = torch.ones(T, M + T, dtype=torch.bool)
    mask[0, M + 1:] = False                        # the state token sees prefix + itself
    x_t = noise.clone()
    t = torch.tensor(1.0, dtype=torch.float32)
    dt = torch.tensor(-0.1, dtype=torch.float32)
    for _ in range(steps):
        s = F.linear(state[None], sd["state_proj.weight"], sd["state_proj.bias"])
        a = F.linear(x_t, sd["action_in_proj.weight"], sd["action_in_proj.bias"])
        temb = time_embedding(float(t), d.dec_width, a.dtype)[None].expand(a.shape[0], -1)
        h = F.linear(torch.cat([a, temb], 1), sd["action_time_mlp_in.weight"],
                     sd["action_time_mlp_in.bias"])
        h = F.linear(F.silu(h), sd["action_time_mlp_out.weight"], sd["action_time_mlp_out.bias"])
        x = torch.cat([s, h], 0)
        for i in range(d.dec_layers):
            q, k, v = gemma_qkv(sd, C.DECODER, i, x, pos, d)
            K = torch.cat([Ks[i], k])
            V = torch.cat([Vs[i], v])
            x = gemma_rest(sd, C.DECODER, i, x, q, K, V, mask, d)
        vel = F.linear(rms(x[1:], sd[f"{C.DECODER}.norm.weight"]), sd["action_out_proj.weight"],
                       sd["action_out_proj.bias"])
        x_t = x_t + DT * vel
        t = t + dt
    return x_t


def openpi_sample(sd, prefix_x, state, noise, d: Dims = SMALL, steps: int = 10):
    """Prefix encoder, then the decoder loop; returns (actions, Ks, Vs)."""
    Ks, Vs = openpi_prefix(sd, prefix_x, d)
    return openpi_decode(sd, Ks, Vs, state, noise, d, steps), Ks, Vs


def half_split_order(k: torch.Tensor, head_dim: int) -> torch.Tensor:
    """Adjacent-pair RoPE column order (the packed cache) -> rotate-half order (OpenPI)."""
    return k.reshape(*k.shape[:-1], head_dim // 2, 2).transpose(-1, -2).reshape(k.shape)
