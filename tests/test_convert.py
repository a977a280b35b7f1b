"""OpenPI checkpoint conversion (flash_vla_amd/convert.py), pinned end to end.

The pin is an OpenPI-form forward written directly on the raw state dict
(`nn.Linear` `[out, in]` weights through `F.linear`, Gemma RMSNorm with
`1 + w`, rotate-half RoPE at absolute positions, the patch embedding as
`F.conv2d`, `F.layer_norm` and `F.scaled_dot_product_attention`). It shares no
code with the converter or the packed oracle, so a transposed weight, a norm
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

ENC = dict(width=48, ffn=80, layers=2)
DEC = dict(width=64, ffn=96, layers=2)
HEADS, HD, ACT = 2, 16, 8
VIS = dict(width=24, ffn=40, layers=2, tokens=256)
DT = -0.1          # the converter folds dt as this double into the output projection


def _openpi_state(seed=0, std=0.15, vision=VIS, dtype=torch.float64) -> dict:
    """A reduced OpenPI Pi0 state dict with the checkpoint's own tensor names."""
    g = torch.Generator().manual_seed(seed)
    sd = {}

    def put(name, *shape, scale=std):
        sd[name] = (torch.randn(shape, generator=g, dtype=torch.float64) * scale).to(dtype)

    vw, vf = vision["width"], vision["ffn"]
    v = C.VISION
    put(f"{v}.embeddings.patch_embedding.weight", vw, 3, 14, 14, scale=0.05)
    put(f"{v}.embeddings.patch_embedding.bias", vw)
    put(f"{v}.embeddings.position_embedding.weight", vision["tokens"], vw)
    for i in range(vision["layers"]):
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
    put(f"{C.PROJECTOR}.weight", ENC["width"], vw)
    put(f"{C.PROJECTOR}.bias", ENC["width"])

    def gemma(root, width, ffn, layers):
        for i in range(layers):
            lay = f"{root}.layers.{i}"
            put(f"{lay}.self_attn.q_proj.weight", HEADS * HD, width)
            put(f"{lay}.self_attn.k_proj.weight", HD, width)
            put(f"{lay}.self_attn.v_proj.weight", HD, width)
            put(f"{lay}.self_attn.o_proj.weight", width, HEADS * HD)
            put(f"{lay}.mlp.gate_proj.weight", ffn, width)
            put(f"{lay}.mlp.up_proj.weight", ffn, width)
            put(f"{lay}.mlp.down_proj.weight", width, ffn)
            put(f"{lay}.input_layernorm.weight", width, scale=0.3)
            put(f"{lay}.post_attention_layernorm.weight", width, scale=0.3)
        put(f"{root}.norm.weight", width, scale=0.3)

    gemma(C.ENCODER, ENC["width"], ENC["ffn"], ENC["layers"])
    gemma(C.DECODER, DEC["width"], DEC["ffn"], DEC["layers"])
    dw = DEC["width"]
    put("state_proj.weight", dw, ACT)
    put("state_proj.bias", dw)
    put("action_in_proj.weight", dw, ACT)
    put("action_in_proj.bias", dw)
    put("action_time_mlp_in.weight", dw, 2 * dw)
    put("action_time_mlp_in.bias", dw)
    put("action_time_mlp_out.weight", dw, dw)
    put("action_time_mlp_out.bias", dw)
    put("action_out_proj.weight", ACT, dw)
    put("action_out_proj.bias", ACT)
    return sd


# ---- the OpenPI-form forward on the raw state dict ----------------------------------------

def _rms(x, w):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + w)


def _rotate_half_rope(x, pos):
    """HF Gemma RoPE: x * cos + rotate_half(x) * sin, frequencies duplicated over halves."""
    n = x.shape[-1] // HD
    inv = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, dtype=torch.float64) / HD))
    ang = pos.to(torch.float64)[:, None] * inv[None]
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos()[:, None], emb.sin()[:, None]
    xh = x.reshape(x.shape[0], n, HD)
    rot = torch.cat([-xh[..., HD // 2:], xh[..., :HD // 2]], -1)
    return (xh * cos + rot * sin).reshape(x.shape)


def _gemma_qkv(sd, root, i, x, pos):
    lay = f"{root}.layers.{i}"
    h = _rms(x, sd[f"{lay}.input_layernorm.weight"])
    q = _rotate_half_rope(F.linear(h, sd[f"{lay}.self_attn.q_proj.weight"]), pos)
    k = _rotate_half_rope(F.linear(h, sd[f"{lay}.self_attn.k_proj.weight"]), pos)
    v = F.linear(h, sd[f"{lay}.self_attn.v_proj.weight"])
    return q, k, v


def _gemma_rest(sd, root, i, x, q, K, V, mask):
    lay = f"{root}.layers.{i}"
    T = x.shape[0]
    qh = q.reshape(T, HEADS, HD).transpose(0, 1)
    o = F.scaled_dot_product_attention(qh, K[None].expand(HEADS, -1, -1),
                                       V[None].expand(HEADS, -1, -1), attn_mask=mask)
    x = x + F.linear(o.transpose(0, 1).reshape(T, HEADS * HD), sd[f"{lay}.self_attn.o_proj.weight"])
    h = _rms(x, sd[f"{lay}.post_attention_layernorm.weight"])
    g = F.gelu(F.linear(h, sd[f"{lay}.mlp.gate_proj.weight"]), approximate="tanh")
    u = F.linear(h, sd[f"{lay}.mlp.up_proj.weight"])
    return x + F.linear(g * u, sd[f"{lay}.mlp.down_proj.weight"])


def _openpi_prefix(sd, x):
    """Gemma prefix encoder: bidirectional; returns per-layer rotated K and V."""
    M = x.shape[0]
    pos = torch.arange(M)
    Ks, Vs = [], []
    for i in range(ENC["layers"]):
        q, k, v = _gemma_qkv(sd, C.ENCODER, i, x, pos)
        Ks.append(k), Vs.append(v)
        x = _gemma_rest(sd, C.ENCODER, i, x, q, k, v, None)
    return Ks, Vs


def _openpi_sample(sd, prefix_x, state, noise, steps=10):
    """Pi0 flow-matching sampling: Euler from t=1 with dt=-0.1 over the action expert."""
    Ks, Vs = _openpi_prefix(sd, prefix_x)
    M, T = prefix_x.shape[0], noise.shape[0] + 1
    pos = torch.arange(M, M + T)
    mask = torch.ones(T, M + T, dtype=torch.bool)
    mask[0, M + 1:] = False                        # the state token sees prefix + itself
    x_t = noise.clone()
    t = torch.tensor(1.0, dtype=torch.float32)
    dt = torch.tensor(-0.1, dtype=torch.float32)
    dw = DEC["width"]
    for _ in range(steps):
        s = F.linear(state[None], sd["state_proj.weight"], sd["state_proj.bias"])
        a = F.linear(x_t, sd["action_in_proj.weight"], sd["action_in_proj.bias"])
        # sinusoidal embedding: periods geometric from 4e-3 to 4, [sin | cos]
        frac = torch.linspace(0, 1, dw // 2, dtype=torch.float64)
        period = 4e-3 * (4.0 / 4e-3) ** frac
        ph = float(t) * 2 * math.pi / period
        temb = torch.cat([ph.sin(), ph.cos()])[None].expand(a.shape[0], -1)
        h = F.linear(torch.cat([a, temb], 1), sd["action_time_mlp_in.weight"],
                     sd["action_time_mlp_in.bias"])
        h = F.linear(F.silu(h), sd["action_time_mlp_out.weight"], sd["action_time_mlp_out.bias"])
        x = torch.cat([s, h], 0)
        for i in range(DEC["layers"]):
            q, k, v = _gemma_qkv(sd, C.DECODER, i, x, pos)
            K = torch.cat([Ks[i], k]); V = torch.cat([Vs[i], v])
            x = _gemma_rest(sd, C.DECODER, i, x, q, K, V, mask)
        vel = F.linear(_rms(x[1:], sd[f"{C.DECODER}.norm.weight"]), sd["action_out_proj.weight"],
                       sd["action_out_proj.bias"])
        x_t = x_t + DT * vel
        t = t + dt
    return x_t, Ks, Vs


def _deinterleave(k):
    return k.reshape(*k.shape[:-1], HD // 2, 2).transpose(-1, -2).reshape(k.shape)


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
    ref, Ks, Vs = _openpi_sample(sd, prefix_x, state, noise)

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
