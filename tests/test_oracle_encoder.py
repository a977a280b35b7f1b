"""Pins the prefix-encoder oracle (oracle/pi0_encoder.py) without retyping it."""
import math

import torch

from oracle import pi0_decoder as O
from oracle import pi0_encoder as E
from flash_vla_amd import weights as W

DIMS = dict(width=64, ffn=96, heads=2, head_dim=16, action_dim=8)


def _packed_encoder(p):
    """Fold unfolded Gemma-layer params into the encoder's packed tensor names."""
    f = W.fold_decoder(p, out_dtype=torch.float64)
    return {"encoder_attn_qkv_w": f["decoder_attn_qkv_w"], "encoder_attn_o_w": f["decoder_attn_o_w"],
            "encoder_ffn_gate_w": f["decoder_ffn_gate_w"], "encoder_ffn_up_w": f["decoder_ffn_up_w"],
            "encoder_ffn_down_w": f["decoder_ffn_down_w"]}


def _deinterleave(k):
    hd = k.shape[-1]
    return k.reshape(*k.shape[:-1], hd // 2, 2).transpose(-1, -2).reshape(k.shape)


def test_encoder_fold_identity_fp64():
    """Packed plan (interleaved RoPE, exact table) == OpenPI-form Gemma encoder, fp64."""
    layers, M = 3, 12
    p = W.openpi_decoder_params(seed=5, std=0.1, layers=layers, dtype=torch.float64, **DIMS)
    x = torch.randn(M, DIMS["width"], generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    Ku, Vu, xu = E.encoder_unfolded(p, x)
    rope = O.rope_table(M, 0, DIMS["head_dim"], exact=True)
    Kp, Vp, xp = E.encoder_packed(_packed_encoder(p), x, heads=DIMS["heads"], bf16=False,
                                  dtype=torch.float64, rope=rope)
    assert torch.allclose(_deinterleave(Kp), Ku, atol=1e-10)   # keys carry the interleave permutation
    assert torch.allclose(Vp, Vu, atol=1e-10)
    assert torch.allclose(xp, xu, atol=1e-10)                   # residual after layers 0..L-2
    # and the packed K is exactly the permuted unfolded K (not merely close): dot products agree
    assert not torch.allclose(Kp, Ku, atol=1e-3)


def test_rms_norm_closed_form():
    x = torch.tensor([[3.0, 4.0], [0.0, 0.0]], dtype=torch.float64)
    y = E.enc_rms_norm(x, bf16=False)
    assert torch.allclose(y[0], torch.tensor([3.0, 4.0], dtype=torch.float64) / math.sqrt(12.5 + 1e-6))
    assert torch.equal(y[1], torch.zeros(2, dtype=torch.float64))
    assert E.enc_rms_norm(x.float(), bf16=True).dtype == torch.float32


def test_encoder_attention_is_unmasked_softmax():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(6, 8, generator=g, dtype=torch.float64)
    k = torch.randn(5, 8, generator=g, dtype=torch.float64)
    v = torch.randn(5, 8, generator=g, dtype=torch.float64)
    got = E.enc_attention(q, k, v, bf16=False)
    for r in range(6):
        s = torch.tensor([float(q[r] @ k[j]) / math.sqrt(8) for j in range(5)], dtype=torch.float64)
        pr = torch.exp(s - s.max()); pr = pr / pr.sum()
        assert torch.allclose(got[r], (pr[:, None] * v).sum(0))
    # the decoder attention with no state rows and every key visible is the same function
    assert torch.allclose(O.op_attention(q, k, v, enc_len=5, heads=0, bf16=False), got)


def test_rope_after_rounding_differs_from_rope_before():
    """The encoder rotates rounded values (base.py:672-726), the decoder the fp32 accumulator."""
    g = torch.Generator().manual_seed(8)
    x = torch.randn(4, 32, generator=g)
    w = torch.randn(32, 4 * 16, generator=g)
    rope = O.rope_table(4, 100, 16)
    q_enc, k_enc, v_enc = E.enc_norm_qkv_rope(x, w, rope, heads=2)
    q_dec, k_dec, v_dec, _ = O.op_norm_qkv_rope(x, w, rope, heads=2)
    # same up to bf16 rounding, but not identical in general
    assert torch.allclose(q_enc, q_dec, atol=0.1, rtol=0.05)
    assert torch.equal(v_enc, _bf16(v_enc))


def _bf16(t):
    return t.bfloat16().float()


def test_layer_norm_matches_torch():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(5, 48, generator=g, dtype=torch.float64) * 3 + 1
    w = torch.randn(48, generator=g, dtype=torch.float64)
    b = torch.randn(48, generator=g, dtype=torch.float64)
    ref = torch.nn.functional.layer_norm(x, (48,), w, b, eps=1e-5)
    assert torch.allclose(E.enc_layer_norm(x, w, b, bf16=False), ref, atol=1e-10)


# ---- vision tower pins ---------------------------------------------------------------
from oracle import pi0_vision as Vn


def test_patch_embed_is_a_14x14_stride_14_convolution():
    """The GEMM over (iy, ix, c) patches == conv2d with the [14, 14, 3, D] kernel."""
    g = torch.Generator().manual_seed(11)
    img = torch.randn(2, 224, 224, 3, generator=g, dtype=torch.float64)
    w = torch.randn(14, 14, 3, 1152, generator=g, dtype=torch.float64) * 0.05
    b = torch.randn(1152, generator=g, dtype=torch.float64)
    pos = torch.randn(256, 1152, generator=g, dtype=torch.float64)
    got = Vn.patch_embed(img, w, b, pos, bf16=False).reshape(2, 16, 16, 1152)
    conv = torch.nn.functional.conv2d(img.permute(0, 3, 1, 2), w.permute(3, 2, 0, 1), b, stride=14)
    ref = conv.permute(0, 2, 3, 1) + pos.reshape(16, 16, 1152)
    assert torch.allclose(got, ref, atol=1e-9)


def test_vision_attention_brute_force():
    g = torch.Generator().manual_seed(12)
    qkv = torch.randn(2 * 256, 3 * 1152, generator=g, dtype=torch.float64)
    got = Vn.vision_attention(qkv, 2, bf16=False)
    for view, head, t in ((0, 0, 0), (1, 15, 255), (1, 7, 100)):
        rows = qkv[view * 256:(view + 1) * 256]
        q = rows[t, head * 72:(head + 1) * 72]
        k = rows[:, 1152 + head * 72:1152 + (head + 1) * 72]
        v = rows[:, 2304 + head * 72:2304 + (head + 1) * 72]
        s = k @ q / math.sqrt(72)
        p = torch.exp(s - s.max()); p = p / p.sum()
        assert torch.allclose(got[view * 256 + t, head * 72:(head + 1) * 72], p @ v)
