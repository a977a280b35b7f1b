"""HIP backend call sites for the Pi0 SigLIP vision tower (M = views x 256 rows, width 1152).

Names and signatures are the reference's `VISION_WRAPPERS`
(`backends/tilelang/wrappers.py:252-315`) plus `vision_attention`
(`kernels/attention.py:20-26`, which the reference pipeline calls directly).
The two ragged axes (the 588-wide patches and the 4304-wide FFN) run on whole
tiles: their weights are packed zero-padded (588 -> 640, 4304 -> 4352) and only
the valid output columns are stored.
"""
from __future__ import annotations

import torch

from . import _abi
from .wrappers import _check, _ptr, _stream, packed_weight_ptr, scratch

TOKENS = 256
DIM = 1152
FFN = 4304
FFN_PAD = 4352          # 34 x 128
PATCH = 588             # 14 x 14 x 3
PATCH_PAD = 640         # 5 x 128
HEADS, HEAD_DIM = 16, 72
LN_EPS = 1e-5


def _rows(t, width):
    """[views, 256, width] (or [M, width]) -> a row-major [M, width] view."""
    v = t.reshape(-1, width)
    if v.stride(-1) != 1 or v.stride(0) != width:
        raise ValueError("expected a contiguous row-major tensor")
    return v


def _layer_norm(x2, w, b, out2):
    _abi.call("pi0hip_layer_norm", _ptr(x2), x2.stride(0), _ptr(w), _ptr(b), _ptr(out2),
              out2.stride(0), x2.shape[0], x2.shape[1], LN_EPS, _stream())


def _bias_res(x2, weight, bias, res2, out2, res_mod=0, pad=None):
    K, N = weight.shape
    kp, np_ = pad if pad is not None else (K, N)
    _abi.call("pi0hip_tile_linear_bias_res", _ptr(x2), x2.stride(0),
              packed_weight_ptr(weight, 32, (kp, np_)), _ptr(bias), _ptr(res2), res2.stride(0),
              res_mod, _ptr(out2), out2.stride(0), out2.shape[0], N, K, np_, kp, _stream())


def vision_patch_embed(images, patch_w, patch_b, pos_emb, out):
    """Patchify, project, add bias and the per-position embedding (wrappers.py:257-269)."""
    _check(images, "images", 4); _check(patch_b, "patch_b", 1); _check(pos_emb, "pos_emb", 2)
    views = images.shape[0]
    if tuple(images.shape[1:]) != (224, 224, 3) or not images.is_contiguous():
        raise ValueError("vision_patch_embed: images must be contiguous [views, 224, 224, 3]")
    M = views * TOKENS
    out2 = _rows(out, DIM)
    if out2.shape[0] != M or tuple(pos_emb.shape) != (TOKENS, DIM):
        raise ValueError("vision_patch_embed: shape mismatch")
    patches = scratch("vision_patches", (M, PATCH_PAD), images.dtype, images.device)
    _abi.call("pi0hip_im2col_patches", _ptr(images), views, _ptr(patches), PATCH_PAD, _stream())
    w2 = patch_w.reshape(PATCH, DIM)
    _bias_res(patches, w2, patch_b, pos_emb, out2, res_mod=TOKENS, pad=(PATCH_PAD, DIM))
    return out


def vision_norm_qkv(x, norm_w, norm_b, qkv_w, qkv_b, out, x_norm):
    """LayerNorm into x_norm, then out = x_norm @ qkv_w + qkv_b (wrappers.py:272-280)."""
    x2, xn2, out2 = _rows(x, DIM), _rows(x_norm, DIM), _rows(out, qkv_w.shape[1])
    _check(qkv_b, "qkv_b", 1)
    M = x2.shape[0]
    _layer_norm(x2, norm_w, norm_b, xn2[:M])
    _abi.call("pi0hip_tile_linear", _ptr(xn2), xn2.stride(0), packed_weight_ptr(qkv_w, 32),
              _ptr(qkv_b), _ptr(out2), out2.stride(0), M, qkv_w.shape[1], DIM, _stream())
    return out


def vision_out_proj_residual(x, weight, bias, res, out):
    """out = attn @ weight + bias + res; `res` and `out` may alias (wrappers.py:283-291)."""
    _bias_res(_rows(x, DIM), weight, bias, _rows(res, DIM), _rows(out, DIM))
    return out


def vision_norm_ffn_up(x, norm_w, norm_b, weight, bias, out, x_norm):
    """LayerNorm into x_norm, then out = gelu_tanh(x_norm @ weight + bias) (wrappers.py:292-299)."""
    x2, xn2, out2 = _rows(x, DIM), _rows(x_norm, DIM), _rows(out, FFN)
    M = x2.shape[0]
    _layer_norm(x2, norm_w, norm_b, xn2[:M])
    _abi.call("pi0hip_tile_linear_bias_gelu", _ptr(xn2), xn2.stride(0),
              packed_weight_ptr(weight, 32, (DIM, FFN_PAD)), _ptr(bias), _ptr(out2),
              out2.stride(0), M, FFN, DIM, FFN_PAD, DIM, _stream())
    return out


def vision_ffn_down_residual(x, weight, bias, res, out):
    """out = hidden @ weight + bias + res (wrappers.py:302-306). The packed weight's zero rows
    4304..4351 meet the next row's (finite) hidden values, contributing exactly 0."""
    _bias_res(_rows(x, FFN), weight, bias, _rows(res, DIM), _rows(out, DIM), pad=(FFN_PAD, DIM))
    return out


def vision_attention(QKV):
    """Per-view multi-head attention over a packed QKV buffer, (views, 256, 3*1152) ->
    (views, 256, 1152) (kernels/attention.py:20-26). The result lives in a pool buffer."""
    _check(QKV, "QKV")
    views = QKV.shape[0] if QKV.dim() == 3 else QKV.shape[0] // TOKENS
    q2 = _rows(QKV, 3 * DIM)
    out = scratch("vision_attn_out", (views, TOKENS, DIM), QKV.dtype, QKV.device)
    nbytes = _abi.lib().pi0hip_vision_attention_workspace_bytes(views, HEADS)
    ws = scratch("vision_attn_ws", (nbytes,), torch.uint8, QKV.device)
    _abi.call("pi0hip_vision_attention", _ptr(q2), q2.stride(0), _ptr(out), DIM, views, TOKENS,
              HEADS, HEAD_DIM, HEAD_DIM ** -0.5, ws.data_ptr(), nbytes, _stream())
    return out


VISION_WRAPPERS = {
    "vision_patch_embed": vision_patch_embed,
    "vision_norm_qkv": vision_norm_qkv,
    "vision_out_proj_residual": vision_out_proj_residual,
    "vision_norm_ffn_up": vision_norm_ffn_up,
    "vision_ffn_down_residual": vision_ffn_down_residual,
}
