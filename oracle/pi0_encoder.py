"""CPU oracle for the Pi0 prefix encoder (TEST INFRASTRUCTURE ONLY).

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg may
import this module, and only as the checker; the HIP product path never calls it.

Restates `transformer_encoder` (`hardware/nvidia/h100/pi0/pipeline.py:57-89`)
without the vision projector (BASELINE config 3 starts from the [M, 2048]
encoder input): 18 Gemma layers at width 2048, 8 query heads + 1 KV head of
256, bidirectional attention, GeGLU 2048 -> 2 x 16384. The last layer runs
only its norm + QKV + RoPE (only its K/V are consumed). Rounding points with
`bf16=True` follow the reference's encoder kernels:
  * RMSNorm emits the normalised tensor in bf16, factor unrounded (base.py:373-403);
  * the QKV GEMM output is bf16 and RoPE rotates the bf16 values (base.py:672-726);
  * attention: bf16 logits, fused fp32 scale + softmax, bf16 P, bf16 P @ V
    (attention.py:29-34, compiled);
  * residual GEMMs round once (base.py:115-154); GeGLU on fp32 accumulators
    (base.py:508-549).
`encoder_unfolded` is an independent fp32/fp64 restatement in the OpenPI form
(half-split RoPE, RMSNorm with 1 + w) used to pin the packed plan.
"""
from __future__ import annotations

import math

import torch

from .pi0_decoder import RMS_EPS, _bf, _rms_norm, _rope_half_split, gelu_tanh, rope_interleaved


def enc_rms_norm(x, bf16=True):
    """x * rsqrt(mean(x^2) + 1e-6), rounded per element (base.py:373-403)."""
    f = torch.rsqrt((x * x).mean(-1, keepdim=True) + RMS_EPS)
    return _bf(x * f, bf16)


def enc_layer_norm(x, w, b, eps=1e-5, bf16=True):
    """(x - mean) * rsqrt(E[x^2] - mean^2 + eps) * w + b, statistics in fp32 (base.py:405-447)."""
    mean = x.mean(-1, keepdim=True)
    inv = torch.rsqrt((x * x).mean(-1, keepdim=True) - mean * mean + eps)
    return _bf((x - mean) * inv * w + b, bf16)


def enc_projector(x, norm_w, norm_b, proj_w, proj_b, bf16=True):
    """Vision final LayerNorm then the projection to encoder width (wrappers.py:336-344)."""
    xn = enc_layer_norm(x, norm_w, norm_b, 1e-5, bf16)
    return _bf(xn @ proj_w.to(x.dtype) + proj_b, bf16)


def enc_norm_qkv_rope(x, w, rope, heads, bf16=True):
    """RMSNorm, bf16 projection, RoPE on the rounded values, scatter (wrappers.py:335-355)."""
    hd = rope.shape[-1]
    xn = enc_rms_norm(x, bf16)
    proj = _bf(xn @ w.to(x.dtype), bf16)
    qk = _bf(rope_interleaved(proj[:, :(heads + 1) * hd], rope), bf16)
    q = qk[:, :heads * hd].reshape(-1, hd)
    k = qk[:, heads * hd:]
    v = proj[:, (heads + 1) * hd:]
    return q, k, v


def enc_attention(q, k, v, bf16=True):
    """softmax(q k^T * hd^-0.5) v for every flat row, no mask (attention.py:29-34).

    The reference function is `torch.compile`d: the bf16 logits of the first
    matmul are scaled and soft-maxed in one fused fp32 kernel, so the logits
    are rounded once and the probabilities once."""
    hd = q.shape[-1]
    s = _bf(q @ k.t(), bf16) * (hd ** -0.5)
    p = _bf(torch.softmax(s, dim=-1), bf16)
    return _bf(p @ v, bf16)


def enc_residual(x, w, r, bf16=True):
    return _bf(r + x @ w.to(r.dtype), bf16)


def enc_norm_gated_ffn(x, wg, wu, bf16=True):
    xn = enc_rms_norm(x, bf16)
    return _bf(gelu_tanh(xn @ wg.to(x.dtype)) * (xn @ wu.to(x.dtype)), bf16)


def encoder_packed(weights: dict, x, layers: int | None = None, heads: int = 8, bf16=True,
                   dtype=torch.float32, rope=None):
    """The encoder plan on packed weights. Returns (K, V, x): K/V [layers, M, hd]."""
    w = {k: v.to(dtype) for k, v in weights.items()}
    n = w["encoder_attn_qkv_w"].shape[0] if layers is None else layers
    x = x.to(dtype).clone()
    M = x.shape[0]
    hd = (w["encoder_attn_qkv_w"].shape[-1] - w["encoder_attn_o_w"].shape[1]) // 2
    if rope is None:
        from .pi0_decoder import rope_table
        rope = rope_table(M, 0, hd)
    rope = rope.to(dtype)
    K = torch.zeros(n, M, hd, dtype=dtype)
    V = torch.zeros(n, M, hd, dtype=dtype)
    for i in range(n):
        q, k, v = enc_norm_qkv_rope(x, w["encoder_attn_qkv_w"][i], rope, heads, bf16)
        K[i], V[i] = k, v
        if i == n - 1:
            break
        o = enc_attention(q, k, v, bf16).reshape(M, -1)
        x = enc_residual(o, w["encoder_attn_o_w"][i], x, bf16)
        h = enc_norm_gated_ffn(x, w["encoder_ffn_gate_w"][i], w["encoder_ffn_up_w"][i], bf16)
        x = enc_residual(h, w["encoder_ffn_down_w"][i], x, bf16)
    return K, V, x


def encoder_unfolded(p: dict, x, layers: int | None = None, dtype=torch.float64):
    """OpenPI-form prefix encoder: Gemma layers with RMSNorm(1 + w), half-split RoPE at
    positions 0..M-1, full bidirectional MQA. `p` uses the keys of
    `flash_vla_amd.weights.openpi_decoder_params` (the layers have the same form)."""
    P = {k: v.to(dtype) for k, v in p.items()}
    n = P["q_w"].shape[0] if layers is None else layers
    hd = P["k_w"].shape[-1]
    heads = P["q_w"].shape[-1] // hd
    x = x.to(dtype).clone()
    M = x.shape[0]
    pos = torch.arange(M)
    K = torch.zeros(n, M, hd, dtype=dtype)
    V = torch.zeros(n, M, hd, dtype=dtype)
    for i in range(n):
        r = _rms_norm(x, P["input_norm_w"][i])
        q = _rope_half_split(r @ P["q_w"][i], pos, hd)
        k = _rope_half_split(r @ P["k_w"][i], pos, hd)
        v = r @ P["v_w"][i]
        K[i], V[i] = k, v
        if i == n - 1:
            break
        qh = q.reshape(M, heads, hd).transpose(0, 1)
        o = torch.softmax((qh @ k.t()) / math.sqrt(hd), dim=-1) @ v
        x = x + o.transpose(0, 1).reshape(M, heads * hd) @ P["o_w"][i]
        r = _rms_norm(x, P["post_attn_norm_w"][i])
        x = x + (torch.nn.functional.gelu(r @ P["gate_w"][i], approximate="tanh")
                 * (r @ P["up_w"][i])) @ P["down_w"][i]
    return K, V, x
