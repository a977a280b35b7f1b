"""OpenPI checkpoint conversion (flash_vla_amd/convert.py), pinned end to end.

The pin is an OpenPI-form forward written directly on the raw state dict
(`tests/openpi_form.py`: `nn.Linear` `[out, in]` weights through `F.linear`,
Gemma RMSNorm with `1 + w`, rotate-half RoPE at absolute positions,
`F.scaled_dot_product_attention`; here also the patch embedding as `F.conv2d`
and `F.layer_norm`). It shares no code with the converter or the packed oracle, so a transposed weight, a norm
folded into the wrong side, a wrong RoPE column permutation, a wrong time
bias or a wrong dt fold makes the fp64 comparison fail. Norm weights and
biases are drawn non-zero so every fold is exercised.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from flash_vla_amd import convert as C
from flash_vla_amd import spec
from oracle import pi0_decoder as O
from oracle import pi0_encoder as E
from oracle import pi0_vision as Vn

from openpi_form import SMALL, Dims, half_split_order, openpi_sample, openpi_state, time_embedding

D = SMALL
ENC = dict(width=D.enc_width, ffn=D.enc_ffn, layers=D.enc_layers)
DEC = dict(width=D.dec_width, ffn=D.dec_ffn, layers=D.dec_layers)
HEADS, HD, ACT = D.heads, D.head_dim, D.action


def _openpi_state(seed=0, std=0.15, vision=None):
    if vision is not None:
        d = Dims(vis_width=vision["width"], vis_ffn=vision["ffn"], vis_layers=vision["layers"],
                 vis_tokens=vision["tokens"])
    else:
        d = D
    return openpi_state(d, seed=seed, std=std)


def _deinterleave(k):
    return half_split_order(k, HD)


# ---- tests ----------------------------------------------------------------------------------

def test_converted_checkpoint_reproduces_openpi_sampling_fp64():
    sd = _openpi_state()
    packed = C.convert_state_dict(sd, strict=False, compute_dtype=torch.float64,
                                  out_dtype=torch.float64)
    g = torch.Generator().manual_seed(1)
    M, chunk = 12, 5
    prefix_x = torch.randn(M, ENC["width"], generator=g, dtype=torch.float64)
    state = torch.randn(ACT, generator=g, dtype=torch.float64)
    noise = torch.randn(chunk, ACT, generator=g, dtype=torch.float64)
    ref, Ks, Vs = openpi_sample(sd, prefix_x, state, noise, D)

    Kp, Vp, _ = E.encoder_packed(packed, prefix_x, heads=HEADS, bf16=False, dtype=torch.float64,
                                 rope=O.rope_table(M, 0, HD, exact=True))
    for i in range(ENC["layers"]):
        assert torch.allclose(_deinterleave(Kp[i]), Ks[i], atol=1e-10)
        assert torch.allclose(Vp[i], Vs[i], atol=1e-10)
    T = chunk + 1
    Kc = torch.cat([Kp, torch.zeros(DEC["layers"], T, HD, dtype=torch.float64)], 1)
    Vc = torch.cat([Vp, torch.zeros(DEC["layers"], T, HD, dtype=torch.float64)], 1)
    got, _, _, _ = O.decoder_packed(packed, state, noise, Kc, Vc, M, steps=10, bf16=False,
                                    dtype=torch.float64, heads=HEADS,
                                    rope=O.rope_table(T, M, HD, exact=True))
    assert torch.allclose(got, ref, atol=1e-9, rtol=1e-9)
    assert (got - noise).abs().max() > 1e-2          # the loop moved the actions


def test_converted_vision_reproduces_siglip_fp64():
    """Full SigLIP dims, one layer, one view: conv2d patch embedding + pre-LN layer."""
    full = dict(width=Vn.DIM, ffn=Vn.FFN, layers=1, tokens=Vn.TOKENS)
    sd = _openpi_state(seed=4, std=0.04, vision=full)
    packed = C.convert_state_dict(sd, strict=False, compute_dtype=torch.float64,
                                  out_dtype=torch.float64)
    img = torch.rand(1, 224, 224, 3, generator=torch.Generator().manual_seed(2),
                     dtype=torch.float64) * 2 - 1
    got = Vn.vision_tower(packed, img, bf16=False, dtype=torch.float64)

    v = C.VISION
    x = F.conv2d(img.permute(0, 3, 1, 2), sd[f"{v}.embeddings.patch_embedding.weight"],
                 sd[f"{v}.embeddings.patch_embedding.bias"], stride=14)
    x = x.flatten(2).transpose(1, 2)[0] + sd[f"{v}.embeddings.position_embedding.weight"]
    lay = f"{v}.encoder.layers.0"
    D, H = Vn.DIM, Vn.HEADS

    def lin(h, name):
        return F.linear(h, sd[f"{lay}.{name}.weight"], sd[f"{lay}.{name}.bias"])

    h = F.layer_norm(x, (D,), sd[f"{lay}.layer_norm1.weight"], sd[f"{lay}.layer_norm1.bias"], 1e-5)
    q, k, vv = (lin(h, f"self_attn.{p}_proj").reshape(-1, H, D // H).transpose(0, 1) for p in "qkv")
    o = F.scaled_dot_product_attention(q, k, vv).transpose(0, 1).reshape(-1, D)
    x = x + lin(o, "self_attn.out_proj")
    h = F.layer_norm(x, (D,), sd[f"{lay}.layer_norm2.weight"], sd[f"{lay}.layer_norm2.bias"], 1e-5)
    ref = x + lin(F.gelu(lin(h, "mlp.fc1"), approximate="tanh"), "mlp.fc2")
    assert torch.allclose(got, ref, atol=1e-9)
    # the projector input: post_layernorm then the projector linear
    enc_in = E.enc_projector(got, packed["vision_final_norm_w"], packed["vision_final_norm_b"],
                             packed["encoder_multi_modal_projector_w"],
                             packed["encoder_multi_modal_projector_b"], bf16=False)
    ref_in = F.linear(F.layer_norm(ref, (D,), sd[f"{v}.post_layernorm.weight"],
                                   sd[f"{v}.post_layernorm.bias"], 1e-5),
                      sd[f"{C.PROJECTOR}.weight"], sd[f"{C.PROJECTOR}.bias"])
    assert torch.allclose(enc_in, ref_in, atol=1e-9)


def test_safetensors_file_round_trip(tmp_path):
    from safetensors.torch import save_file
    sd = {k: v.float() for k, v in _openpi_state(seed=7).items()}
    save_file(sd, str(tmp_path / "model.safetensors"))
    from_file = C.convert_checkpoint(tmp_path, strict=False)       # directory form
    direct = C.convert_state_dict(sd, strict=False)
    assert set(from_file) == set(direct)
    for k in direct:
        assert from_file[k].dtype == torch.bfloat16
        assert torch.equal(from_file[k], direct[k]), k
    assert from_file["language_embeds"].shape == (0, ENC["width"])
    assert from_file["decoder_action_fused_time_biases"].shape == (10, DEC["width"])


def test_cli_writes_packed_file(tmp_path):
    from safetensors.torch import load_file, save_file
    sd = {k: v.float() for k, v in _openpi_state(seed=8).items()}
    save_file(sd, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="expected"):       # strict schema check on a reduced model
        C.main(["--checkpoint", str(tmp_path), "--out", str(tmp_path / "packed.safetensors")])


def test_strict_schema_and_missing_names():
    sd = _openpi_state(seed=9)
    with pytest.raises(ValueError, match="has shape"):
        C.convert_state_dict(sd)
    del sd["action_out_proj.bias"]
    with pytest.raises(KeyError, match="action_out_proj.bias"):
        C.convert_state_dict(sd, strict=False)
    with pytest.raises(FileNotFoundError):
        C.load_openpi_state("/nonexistent/dir")


def test_packed_names_are_the_schema():
    """Every name the converter emits is a schema name, and it emits all of them."""
    packed = C.convert_state_dict(_openpi_state(seed=10), strict=False)
    assert set(packed) == set(spec.weight_shapes(prompt_len=0))


def test_error_metrics_closed_form():
    ref = torch.tensor([1.0, 0.0, 0.0, 0.0])
    out = torch.tensor([1.0, 0.0, 0.0, 1.0])
    m = C.error_metrics(ref, out)
    assert m["max_abs"] == 1.0 and m["mean_abs"] == 0.25
    assert math.isclose(m["rms_error"], 0.5)
    assert math.isclose(m["cosine_similarity"], 1 / math.sqrt(2), rel_tol=1e-6)
    assert math.isclose(m["p99_abs"], 0.97, rel_tol=1e-6)   # linear interpolation at 0.99 * 3
    with pytest.raises(ValueError):
        C.error_metrics(ref, out[:3])
