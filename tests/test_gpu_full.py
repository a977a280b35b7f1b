"""Parity of the SigLIP vision kernels and of the one-graph full forward
with the CPU oracle (oracle/pi0_vision.py, pi0_encoder.py, pi0_decoder.py).

Per-op tolerance as for the encoder ops: max|got - ref| <= 2**-6 * max|ref|,
cosine >= 0.99999 (attention 2**-5: P is rounded before normalisation). The
whole forward runs at reduced depth (2 vision, 2 encoder, 2 decoder layers,
2 Euler steps) on full-width random_checkpoint() tensors and uniform[-1, 1]
images; its criterion is relative to exact bf16 emulation (x1.5 of the bf16
oracle's distance from fp32, cosine >= 0.999).
"""
import pytest
import torch

from oracle import pi0_vision as Vn
from oracle import pi0_encoder as E
from flash_vla_amd.arena import ScratchPool
from flash_vla_amd.backends.hip import vision_wrappers as VW
from flash_vla_amd.backends.hip import wrappers as W

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2.0 ** -6


@pytest.fixture(autouse=True)
def _pool():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.set_num_threads(min(16, torch.get_num_threads()))
    with W.use_pool(ScratchPool()):
        yield


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def metrics(got, ref):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    err = (got - ref).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten().double(), ref.flatten().double(),
                                                dim=0).item()
    return err, cos


def close(got, ref, tol=TOL, what=""):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert torch.isfinite(got).all(), what
    err, cos = metrics(got, ref)
    scale = ref.abs().max().item()
    print(f"{what}: max err {err:.3e} (scale {scale:.3e}) cos {cos:.8f}", flush=True)
    assert err <= tol * scale + 1e-6, f"{what}: max err {err} vs scale {scale}"
    assert cos >= 0.99999, f"{what}: cosine {cos}"


def test_patch_embed():
    img = (torch.rand(3, 224, 224, 3, generator=torch.Generator().manual_seed(60)) * 2 - 1
           ).to(torch.bfloat16)
    w, b, pos = rnd((14, 14, 3, 1152), 61, 0.05), rnd(1152, 62, 0.5), rnd((256, 1152), 63, 0.5)
    out = torch.zeros(3, 256, 1152, dtype=torch.bfloat16, device=DEV)
    VW.vision_patch_embed(img.to(DEV), w.to(DEV), b.to(DEV), pos.to(DEV), out)
    ref = Vn.patch_embed(img.float(), w.float(), b.float(), pos.float())
    close(out.reshape(768, 1152), ref, what="patch_embed")


def test_norm_qkv():
    x = rnd((3, 256, 1152), 64)
    nw, nb = rnd(1152, 65, 0.5), rnd(1152, 66, 0.5)
    w, b = rnd((1152, 3456), 67, 0.03), rnd(3456, 68, 0.5)
    out = torch.zeros(3, 256, 3456, dtype=torch.bfloat16, device=DEV)
    xn = torch.zeros(3, 256, 1152, dtype=torch.bfloat16, device=DEV)
    VW.vision_norm_qkv(x.to(DEV), nw.to(DEV), nb.to(DEV), w.to(DEV), b.to(DEV), out, xn)
    ref_n = E.enc_layer_norm(x.float().reshape(768, 1152), nw.float(), nb.float())
    close(xn.reshape(768, 1152), ref_n, what="vision layer_norm")
    close(out.reshape(768, 3456), (ref_n @ w.float() + b.float()).bfloat16().float(),
          what="vision qkv")


@pytest.mark.parametrize("views", [3, 1])
def test_vision_attention(views):
    qkv = rnd((views, 256, 3456), 69)
    out = VW.vision_attention(qkv.to(DEV))
    ref = Vn.vision_attention(qkv.float().reshape(views * 256, 3456), views)
    close(out.reshape(views * 256, 1152), ref, tol=2.0 ** -5, what=f"vision attention {views}")


def test_out_proj_residual_in_place():
    x, w, b, r = rnd((3, 256, 1152), 70), rnd((1152, 1152), 71, 0.03), rnd(1152, 72), rnd((3, 256, 1152), 73)
    out = r.to(DEV).clone()
    VW.vision_out_proj_residual(x.to(DEV), w.to(DEV), b.to(DEV), out, out)
    ref = x.float().reshape(768, 1152) @ w.float() + b.float() + r.float().reshape(768, 1152)
    close(out.reshape(768, 1152), ref.bfloat16().float(), what="vision o_proj")


def test_ffn_up_gelu_ragged_n():
    """N = 4304 (16 x 269): padded to 4352 in the packed weight, only 4304 columns stored."""
    x = rnd((3, 256, 1152), 74)
    nw, nb = rnd(1152, 75, 0.5), rnd(1152, 76, 0.5)
    w, b = rnd((1152, 4304), 77, 0.03), rnd(4304, 78, 0.5)
    store = torch.full((768 * 4304 + 64,), 7.0, dtype=torch.bfloat16, device=DEV)
    out = store[:768 * 4304].view(3, 256, 4304)         # a sentinel right after the last row
    xn = torch.zeros(3, 256, 1152, dtype=torch.bfloat16, device=DEV)
    VW.vision_norm_ffn_up(x.to(DEV), nw.to(DEV), nb.to(DEV), w.to(DEV), b.to(DEV), out, xn)
    ref_n = E.enc_layer_norm(x.float().reshape(768, 1152), nw.float(), nb.float())
    from oracle.pi0_decoder import gelu_tanh
    ref = gelu_tanh(ref_n @ w.float() + b.float())
    close(out.reshape(768, 4304), ref.bfloat16().float(), what="vision ffn_up")
    assert torch.all(store[768 * 4304:] == 7.0), "stored past the 4304 valid columns"


@pytest.mark.parametrize("views", [12])
def test_large_m_vision_gemms(views):
    """Batched profile (4 requests x 3 views = 3072 rows): QKV, o-proj and FFN-down run on the
    taller large-M tiles; references in fp32 on the device."""
    M = views * 256
    x = rnd((views, 256, 1152), 83)
    nw, nb = rnd(1152, 84, 0.5), rnd(1152, 85, 0.5)
    wq, bq = rnd((1152, 3456), 86, 0.03), rnd(3456, 87, 0.5)
    qkv = torch.zeros(views, 256, 3456, dtype=torch.bfloat16, device=DEV)
    xn = torch.zeros(views, 256, 1152, dtype=torch.bfloat16, device=DEV)
    VW.vision_norm_qkv(x.to(DEV), nw.to(DEV), nb.to(DEV), wq.to(DEV), bq.to(DEV), qkv, xn)
    ref_n = E.enc_layer_norm(x.to(DEV).float().reshape(M, 1152), nw.to(DEV).float(), nb.to(DEV).float())
    close(qkv.reshape(M, 3456), (ref_n @ wq.to(DEV).float() + bq.to(DEV).float()).bfloat16().float(),
          what=f"vision qkv M={M}")
    a, wo, bo, r = rnd((views, 256, 1152), 88), rnd((1152, 1152), 89, 0.03), rnd(1152, 90), rnd((views, 256, 1152), 91)
    out = r.to(DEV).clone()
    VW.vision_out_proj_residual(a.to(DEV), wo.to(DEV), bo.to(DEV), out, out)
    ref = a.to(DEV).float().reshape(M, 1152) @ wo.to(DEV).float() + bo.to(DEV).float() + r.to(DEV).float().reshape(M, 1152)
    close(out.reshape(M, 1152), ref.bfloat16().float(), what=f"vision o_proj M={M}")
    h, wd, bd = rnd((views, 256, 4304), 92, 0.5), rnd((4304, 1152), 93, 0.02), rnd(1152, 94)
    out = r.to(DEV).clone()
    VW.vision_ffn_down_residual(h.to(DEV), wd.to(DEV), bd.to(DEV), out, out)
    ref = h.to(DEV).float().reshape(M, 4304) @ wd.to(DEV).float() + bd.to(DEV).float() + r.to(DEV).float().reshape(M, 1152)
    close(out.reshape(M, 1152), ref.bfloat16().float(), what=f"vision ffn_down M={M}")


def test_padded_layer_views_resolve_exactly():
    """Layer views of a zero-padded packed stack land exactly on layer boundaries of the
    packed copy (a float ratio of padded / unpadded sizes put layers 3, 6, 11-13 and 21-26
    of the 27-layer vision FFN one byte off: misaligned bf16, NaN outputs)."""
    stack = rnd((27, 1152, 4304), 84, 0.02).to(DEV)
    base = W.packed_weight_ptr(stack[0], 32, (1152, 4352))
    for i in (1, 3, 6, 13, 26):
        assert W.packed_weight_ptr(stack[i], 32, (1152, 4352)) == base + i * 1152 * 4352 * 2


def test_ffn_down_ragged_k():
    """K = 4304: the packed weight's zero rows 4304..4351 meet the next row's values."""
    h, w, b, r = rnd((3, 256, 4304), 79, 0.5), rnd((4304, 1152), 80, 0.02), rnd(1152, 81), rnd((3, 256, 1152), 82)
    out = r.to(DEV).clone()
    VW.vision_ffn_down_residual(h.to(DEV), w.to(DEV), b.to(DEV), out, out)
    ref = h.float().reshape(768, 4304) @ w.float() + b.float() + r.float().reshape(768, 1152)
    close(out.reshape(768, 1152), ref.bfloat16().float(), what="vision ffn_down")


def _shallow_checkpoint(seed=90, vis=2, enc=2, dec=2, prompt_len=0):
    """random_checkpoint()'s tensors (N(0,1) x 0.05, schema order) with short layer stacks."""
    from flash_vla_amd.spec import weight_shapes
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in weight_shapes(prompt_len).items():
        if name.startswith(("vision_attn", "vision_ffn", "vision_pre")):
            shape = (vis,) + tuple(shape[1:])
        elif name.startswith(("encoder_attn", "encoder_ffn")):
            shape = (enc,) + tuple(shape[1:])
        elif name.startswith(("decoder_attn", "decoder_ffn")):
            shape = (dec,) + tuple(shape[1:])
        out[name] = (torch.randn(shape, generator=g) * 0.05).to(torch.bfloat16)
    return out


@pytest.fixture(scope="module")
def full_case():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    ck = _shallow_checkpoint()
    g = torch.Generator().manual_seed(91)
    images = (torch.rand(3, 224, 224, 3, generator=g) * 2 - 1).to(torch.bfloat16)
    state = torch.randn(32, generator=g).to(torch.bfloat16)
    noise = torch.randn(50, 32, generator=g).to(torch.bfloat16)
    return ck, images, state, noise


def test_full_forward_shallow(full_case):
    from flash_vla_amd import Pi0Inference
    ck, images, state, noise = full_case
    eng = Pi0Inference({k: v.to(DEV) for k, v in ck.items()}, num_views=3, chunk_size=50,
                       steps=2, capture=False)
    out = eng.forward(images.to(DEV), state.to(DEV), noise.to(DEV)).clone()
    bn, bK, bV = Vn.full_forward(ck, images, state, noise, steps=2, bf16=True)
    fn, fK, fV = Vn.full_forward(ck, images, state, noise, steps=2, bf16=False)
    for name, got, b, f in (("K", eng.buffers["encoder_K"][:2, :768], bK, fK),
                            ("V", eng.buffers["encoder_V"][:2, :768], bV, fV),
                            ("noise", out, bn, fn)):
        g_err, g_cos = metrics(got, f)
        e_err, e_cos = metrics(b, f)
        print(f"full forward {name}: gpu vs fp32 err {g_err:.3e} 1-cos {1 - g_cos:.2e}; "
              f"bf16 oracle err {e_err:.3e} 1-cos {1 - e_cos:.2e}", flush=True)
        assert g_cos >= 0.999
        assert (1 - g_cos) <= 1.5 * (1 - e_cos) + 1e-6 and g_err <= 1.5 * e_err + 2e-3


def test_full_forward_default_prompt_256():
    """random_checkpoint()'s default prompt_len=256 (weights.py:10 of the reference): prefix
    1024 tokens, decoder keys 1075 (9 key chunks), 1 layer each, 1 Euler step."""
    from flash_vla_amd import Pi0Inference
    ck = _shallow_checkpoint(seed=95, vis=1, enc=1, dec=1, prompt_len=256)
    g = torch.Generator().manual_seed(96)
    images = (torch.rand(3, 224, 224, 3, generator=g) * 2 - 1).to(torch.bfloat16)
    state = torch.randn(32, generator=g).to(torch.bfloat16)
    noise = torch.randn(50, 32, generator=g).to(torch.bfloat16)
    eng = Pi0Inference({k: v.to(DEV) for k, v in ck.items()}, num_views=3, chunk_size=50,
                       steps=1)
    assert eng.encoder_seq_len == 1024 and eng.buffers["encoder_K"].shape[1] == 1075
    out = eng.forward(images.to(DEV), state.to(DEV), noise.to(DEV)).clone()
    bn, _, _ = Vn.full_forward(ck, images, state, noise, steps=1, bf16=True)
    fn, _, _ = Vn.full_forward(ck, images, state, noise, steps=1, bf16=False)
    g_err, g_cos = metrics(out, fn)
    e_err, e_cos = metrics(bn, fn)
    print(f"prompt 256 forward: gpu vs fp32 err {g_err:.3e} 1-cos {1 - g_cos:.2e}; "
          f"bf16 oracle err {e_err:.3e} 1-cos {1 - e_cos:.2e}", flush=True)
    assert g_cos >= 0.999
    assert (1 - g_cos) <= 1.5 * (1 - e_cos) + 1e-6 and g_err <= 1.5 * e_err + 2e-3


@pytest.mark.parametrize("views", [1, 4])
def test_full_forward_other_view_counts(views):
    """num_views other than 3 (the reference rejects only 2, pipeline.py:22): one view puts
    256 rows through the vision and encoder GEMMs and 307 keys before the decoder rows;
    four views 1024 rows and 1075 keys. 1 layer each, 1 Euler step, graph captured."""
    from flash_vla_amd import Pi0Inference
    ck = _shallow_checkpoint(seed=97 + views, vis=1, enc=1, dec=1)
    g = torch.Generator().manual_seed(98 + views)
    images = (torch.rand(views, 224, 224, 3, generator=g) * 2 - 1).to(torch.bfloat16)
    state = torch.randn(32, generator=g).to(torch.bfloat16)
    noise = torch.randn(50, 32, generator=g).to(torch.bfloat16)
    print(f"full forward with {views} view(s)", flush=True)
    eng = Pi0Inference({k: v.to(DEV) for k, v in ck.items()}, num_views=views, chunk_size=50,
                       steps=1)
    assert eng.encoder_seq_len == 256 * views
    assert eng.buffers["encoder_K"].shape[1] == 256 * views + 51
    out = eng.forward(images.to(DEV), state.to(DEV), noise.to(DEV)).clone()
    bn, _, _ = Vn.full_forward(ck, images, state, noise, num_views=views, steps=1, bf16=True)
    fn, _, _ = Vn.full_forward(ck, images, state, noise, num_views=views, steps=1, bf16=False)
    g_err, g_cos = metrics(out, fn)
    e_err, e_cos = metrics(bn, fn)
    print(f"{views} view(s): gpu vs fp32 err {g_err:.3e} 1-cos {1 - g_cos:.2e}; "
          f"bf16 oracle err {e_err:.3e} 1-cos {1 - e_cos:.2e}", flush=True)
    assert g_cos >= 0.999
    assert (1 - g_cos) <= 1.5 * (1 - e_cos) + 1e-6 and g_err <= 1.5 * e_err + 2e-3


def test_full_forward_graph_equals_eager(full_case):
    from flash_vla_amd import Pi0Inference
    ck, images, state, noise = full_case
    w = {k: v.to(DEV) for k, v in ck.items()}
    eager = Pi0Inference(w, steps=2, capture=False)
    a = eager.forward(images.to(DEV), state.to(DEV), noise.to(DEV)).clone()
    graph = Pi0Inference(w, steps=2, capture=True)
    b1 = graph.forward(images.to(DEV), state.to(DEV), noise.to(DEV)).clone()
    b2 = graph.forward(images.to(DEV), state.to(DEV), noise.to(DEV)).clone()
    assert torch.equal(a, b1) and torch.equal(b1, b2)
