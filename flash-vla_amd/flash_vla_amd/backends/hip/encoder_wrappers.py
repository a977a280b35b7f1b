"""HIP backend call sites for the Pi0 prefix encoder (M = 768..816 token rows).

Names and signatures are the reference's `ENCODER_WRAPPERS`
(`backends/tilelang/wrappers.py:336-401`) plus `encoder_attention`
(`kernels/attention.py:29-34`, which the reference pipeline calls directly).
The GEMMs run on the LDS-tiled MFMA kernels of `csrc/pi0_encoder.hip`; the
weights are read in the 32x32x16 B-fragment order (packed once, layout 32 of the
shared packed-weight cache).
"""
from __future__ import annotations

import torch

from . import _abi
from .wrappers import _check, _ptr, _stream, packed_weight_ptr, scratch

VISION_DIM = 1152
VISION_TOKENS = 256
LN_EPS = 1e-5
# ffn-down (K = 16384): split K so that the 96 output tiles of 128 x 128 become 384
# workgroups (1.5 per CU), partials summed in split order by a second launch
_DOWN_SPLITK = 4


def encoder_projector(x, norm_w, norm_b, proj_w, proj_b, out, x_norm):
    """Vision final LayerNorm (eps 1e-5), then out[:M] = x_norm @ proj_w + proj_b (wrappers.py:336-344)."""
    M = x.shape[0] * VISION_TOKENS
    x2, xn2 = x.reshape(M, VISION_DIM), x_norm.view(M, VISION_DIM)
    _check(x2, "x", 2); _check(xn2, "x_norm", 2); _check(out, "out", 2)
    _check(norm_w, "norm_w", 1); _check(norm_b, "norm_b", 1); _check(proj_b, "proj_b", 1)
    N = proj_w.shape[1]
    if proj_w.shape[0] != VISION_DIM or out.shape[0] < M or out.shape[1] != N:
        raise ValueError("encoder_projector: shape mismatch")
    _abi.call("pi0hip_layer_norm", _ptr(x2), x2.stride(0), _ptr(norm_w), _ptr(norm_b), _ptr(xn2),
              xn2.stride(0), M, VISION_DIM, LN_EPS, _stream())
    _abi.call("pi0hip_tile_linear", _ptr(xn2), xn2.stride(0), packed_weight_ptr(proj_w, 32),
              _ptr(proj_b), _ptr(out), out.stride(0), M, N, VISION_DIM, _stream())
    return out


def encoder_norm_qkv_rope(x, weight_qkv, rope, Q, K, V, x_norm):
    """RMSNorm into x_norm, QKV projection, RoPE on the rounded values, scatter (wrappers.py:347-363).

    Batched form (config 5): K / V are [requests, L, head_dim] views of the per-request
    caches and x holds the requests' L prefix rows one request after another."""
    _check(x, "x", 2); _check(x_norm, "x_norm", 2); _check(rope, "rope", 2); _check(Q, "Q", 2)
    batch = K.shape[0] if K.dim() == 3 else 1
    K2, V2 = (K[0], V[0]) if K.dim() == 3 else (K, V)
    _check(K2, "K", 2); _check(V2, "V", 2)
    M, Kdim = x.shape
    head_dim = V2.shape[1]
    heads = Q.shape[0] // M
    L = K2.shape[0]
    if (Q.shape != (M * heads, head_dim) or not Q.is_contiguous() or M != batch * L
            or V.shape != K.shape or K2.stride(0) != V2.stride(0) or K.stride() != V.stride()
            or weight_qkv.shape != (Kdim, (heads + 2) * head_dim)
            or rope.shape[0] < L or rope.shape[1] != head_dim or not rope.is_contiguous()
            or x_norm.shape[0] < M or x_norm.shape[1] != Kdim):
        raise ValueError("encoder_norm_qkv_rope: shape mismatch")
    _abi.call("pi0hip_rms_norm", _ptr(x), x.stride(0), _ptr(x_norm), x_norm.stride(0), M, Kdim,
              _stream())
    _abi.call("pi0hip_tile_qkv_rope_batched", _ptr(x_norm), x_norm.stride(0),
              packed_weight_ptr(weight_qkv, 32), _ptr(rope), _ptr(Q), _ptr(K2), _ptr(V2),
              K2.stride(0), K.stride(0) if batch > 1 else 0, L, M, Kdim, heads, head_dim,
              _stream())


def _tile_residual(x, weight, out, splitk, role):
    _check(x, "x", 2); _check(out, "out", 2)
    M, K = x.shape
    N = weight.shape[1]
    if weight.shape[0] != K or out.shape != (M, N):
        raise ValueError(f"{role}: shape mismatch")
    lib = _abi.lib()
    nbytes = lib.pi0hip_tile_workspace_bytes(M, N, splitk)
    ws = scratch(f"tile_ws_{role}", (nbytes,), torch.uint8, x.device).data_ptr() if nbytes else None
    _abi.call("pi0hip_tile_linear_residual", _ptr(x), x.stride(0), packed_weight_ptr(weight, 32),
              _ptr(out), out.stride(0), M, N, K, splitk, ws, nbytes, _stream())
    return out


def encoder_out_proj_residual(x, weight, out):
    """out += attn @ weight in place (wrappers.py:366-371)."""
    return _tile_residual(x, weight, out, 1, "enc_o_proj")


def encoder_norm_gated_ffn(x, gate_w, up_w, out, x_norm):
    """RMSNorm into x_norm, then out = gelu_tanh(x_norm @ Wg) * (x_norm @ Wu) (wrappers.py:374-380)."""
    _check(x, "x", 2); _check(x_norm, "x_norm", 2); _check(out, "out", 2)
    M, K = x.shape
    N = gate_w.shape[1]
    if (gate_w.shape != (K, N) or up_w.shape != (K, N) or out.shape[0] < M or out.shape[1] != N
            or x_norm.shape[0] < M or x_norm.shape[1] != K):
        raise ValueError("encoder_norm_gated_ffn: shape mismatch")
    _abi.call("pi0hip_rms_norm", _ptr(x), x.stride(0), _ptr(x_norm), x_norm.stride(0), M, K,
              _stream())
    _abi.call("pi0hip_tile_gated_ffn", _ptr(x_norm), x_norm.stride(0), packed_weight_ptr(gate_w, 32),
              packed_weight_ptr(up_w, 32), _ptr(out), out.stride(0), M, N, K, _stream())
    return out


def encoder_ffn_down_residual(x, weight, out):
    """out += hidden @ weight in place (wrappers.py:383-392). K = 16384 is split four ways at
    the single-request size; from 2048 rows up the row tiles alone fill the chip."""
    M, K = x.shape
    s = _DOWN_SPLITK if (K // 64) % _DOWN_SPLITK == 0 and M < 2048 else 1
    return _tile_residual(x, weight, out, s, "enc_ffn_down")


def encoder_attention(Q, K, V, scale):
    """softmax(scale * Q K^T) V over all keys, one shared KV head; returns [M, heads * head_dim]
    (kernels/attention.py:29-34). Batched form: K / V [requests, L, head_dim], Q the
    requests' rows one after another. The result lives in a pool buffer reused by the
    next call."""
    _check(Q, "Q", 2)
    batch = K.shape[0] if K.dim() == 3 else 1
    K2, V2 = (K[0], V[0]) if K.dim() == 3 else (K, V)
    _check(K2, "K", 2); _check(V2, "V", 2)
    rows, head_dim = Q.shape
    keys = K2.shape[0]
    if (V.shape != K.shape or K2.shape[1] != head_dim or K2.stride(0) != V2.stride(0)
            or K.stride() != V.stride() or rows % batch):
        raise ValueError("encoder_attention: shape mismatch")
    out = scratch("encoder_attn_out", (rows, head_dim), Q.dtype, Q.device)
    nbytes = _abi.lib().pi0hip_encoder_attention_batched_workspace_bytes(keys, batch)
    ws = scratch("encoder_attn_ws", (nbytes,), torch.uint8, Q.device)
    _abi.call("pi0hip_encoder_attention_batched", _ptr(Q), Q.stride(0), _ptr(K2), _ptr(V2),
              K2.stride(0), K.stride(0) if batch > 1 else 0, _ptr(out), out.stride(0),
              rows // batch, keys, head_dim, float(scale), batch, ws.data_ptr(), nbytes,
              _stream())
    width = 2048 if (rows * head_dim) % 2048 == 0 else head_dim
    return out.view(-1, width)


def embed_prompt(token_ids, table, out, row0, rows_per_request, scale):
    """Prompt token embedding, scaled (the reference takes precomputed
    `language_embeds`, spec.py:46): out[b * rows_per_request + row0 + j] =
    bf16(table[token_ids[b, j]] * scale)."""
    if token_ids.dtype != torch.int32 or not token_ids.is_cuda or not token_ids.is_contiguous():
        raise TypeError("token_ids must be a contiguous int32 GPU tensor")
    _check(table, "table", 2); _check(out, "out", 2)
    batch, n_tok = token_ids.shape if token_ids.dim() == 2 else (1, token_ids.shape[0])
    vocab, dim = table.shape
    if out.shape[1] != dim or out.shape[0] < batch * rows_per_request:
        raise ValueError("embed_prompt: shape mismatch")
    _abi.call("pi0hip_embed_tokens", _ptr(token_ids), n_tok, batch, _ptr(table), vocab, dim,
              float(scale), _ptr(out), out.stride(0), row0, rows_per_request, _stream())
    return out


ENCODER_WRAPPERS = {
    "encoder_projector": encoder_projector,
    "encoder_norm_qkv_rope": encoder_norm_qkv_rope,
    "encoder_out_proj_residual": encoder_out_proj_residual,
    "encoder_norm_gated_ffn": encoder_norm_gated_ffn,
    "encoder_ffn_down_residual": encoder_ffn_down_residual,
}
