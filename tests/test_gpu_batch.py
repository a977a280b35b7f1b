"""Batch-4 / prompt-token profile (not in the reference, which is
batch-1 with precomputed language embeddings).

The batched kernels must give every request exactly what a batch-1 run of that request
gives: each row's arithmetic does not depend on how rows are grouped into blocks, so the
checks are bitwise (Q / K / V scatter, RoPE positions, per-request caches, the attention's
state-row mask and its "states first" output order). The batched forward is also checked
against the CPU oracle run request by request (relative criterion as for the full forward).
"""
import pytest
import torch

from oracle import pi0_vision as Vn
from flash_vla_amd.arena import ScratchPool
from flash_vla_amd.backends.hip import encoder_wrappers as EW
from flash_vla_amd.backends.hip import wrappers as W
from flash_vla_amd.buffers import rope_table

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _pool():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.set_num_threads(min(16, torch.get_num_threads()))
    with W.use_pool(ScratchPool()):
        yield


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def states_first(rows_per_request, B):
    """Row of token t of request b in the "states first" order (B states, then actions)."""
    T = rows_per_request - 1
    return lambda b, t: b if t == 0 else B + b * T + (t - 1)


@pytest.mark.parametrize("B", [4, 2])
def test_decoder_qkv_and_attention_batched_equal_per_request(B):
    enc, T1, L = 816, 51, 18
    x = rnd((B * T1, 1024), 100)
    w = rnd((1024, 2560), 101, 0.02)
    rope = rope_table(T1, enc, 256, DEV)
    cache_k = rnd((B, L, enc + T1, 256), 102)
    cache_v = rnd((B, L, enc + T1, 256), 103)
    kb, vb = cache_k.clone(), cache_v.clone()
    q = torch.zeros(B * T1 * 8, 256, dtype=torch.bfloat16, device=DEV)
    nf = torch.zeros(B * T1, dtype=torch.bfloat16, device=DEV)
    W.decoder_norm_qkv_rope(x, w, rope, q, kb[:, 3, enc:], vb[:, 3, enc:], nf)
    pos = states_first(T1, B)
    for b in range(B):
        xb = torch.stack([x[pos(b, t)] for t in range(T1)])          # request b, token order
        qb = torch.zeros(T1 * 8, 256, dtype=torch.bfloat16, device=DEV)
        k1, v1 = cache_k[b, 3].clone(), cache_v[b, 3].clone()
        W.decoder_norm_qkv_rope(xb, w, rope, qb, k1[enc:], v1[enc:], None)
        assert torch.equal(qb, q[b * T1 * 8:(b + 1) * T1 * 8]), f"Q of request {b}"
        assert torch.equal(k1, kb[b, 3]) and torch.equal(v1, vb[b, 3]), f"K/V of request {b}"
    out = torch.zeros_like(q)
    W.decoder_attention(q, kb[:, 3], vb[:, 3], None, out, enc)
    for b in range(B):
        qb = q[b * T1 * 8:(b + 1) * T1 * 8].clone()
        ob = torch.zeros_like(qb)
        W.decoder_attention(qb, kb[b, 3], vb[b, 3], None, ob, enc)
        for t in range(T1):
            r = pos(b, t)
            assert torch.equal(out[r * 8:(r + 1) * 8], ob[t * 8:(t + 1) * 8]), f"request {b} token {t}"
    # in place (out is Q), as the pipeline calls it
    W.decoder_attention(q, kb[:, 3], vb[:, 3], None, q, enc)
    assert torch.equal(q, out)


def test_encoder_qkv_and_attention_batched_equal_per_request():
    B, Lp = 2, 816
    x = rnd((B * Lp, 2048), 110)
    w = rnd((2048, 2560), 111, 0.02)
    rope = rope_table(Lp, 0, 256, DEV)
    ck = torch.zeros(B, 3, Lp + 51, 256, dtype=torch.bfloat16, device=DEV)
    cv = torch.zeros_like(ck)
    q = torch.zeros(B * Lp * 8, 256, dtype=torch.bfloat16, device=DEV)
    xn = torch.zeros(B * Lp, 2048, dtype=torch.bfloat16, device=DEV)
    EW.encoder_norm_qkv_rope(x, w, rope, q, ck[:, 1, :Lp], cv[:, 1, :Lp], xn)
    att = EW.encoder_attention(q, ck[:, 1, :Lp], cv[:, 1, :Lp], 256 ** -0.5).clone()
    for b in range(B):
        qb = torch.zeros(Lp * 8, 256, dtype=torch.bfloat16, device=DEV)
        k1 = torch.zeros(Lp, 256, dtype=torch.bfloat16, device=DEV)
        v1 = torch.zeros_like(k1)
        xn1 = torch.zeros(Lp, 2048, dtype=torch.bfloat16, device=DEV)
        EW.encoder_norm_qkv_rope(x[b * Lp:(b + 1) * Lp], w, rope, qb, k1, v1, xn1)
        assert torch.equal(qb, q[b * Lp * 8:(b + 1) * Lp * 8])
        assert torch.equal(k1, ck[b, 1, :Lp]) and torch.equal(v1, cv[b, 1, :Lp])
        a1 = EW.encoder_attention(qb, k1, v1, 256 ** -0.5)
        assert torch.equal(a1, att[b * Lp:(b + 1) * Lp])
    assert not ck[:, 1, Lp:].any(), "wrote decoder rows"


def test_embed_prompt():
    vocab, B, n = 1000, 3, 48
    table = rnd((vocab, 2048), 120)
    ids = torch.randint(0, vocab, (B, n), generator=torch.Generator().manual_seed(121),
                        dtype=torch.int32).to(DEV)
    L = 816
    out = torch.zeros(B * L, 2048, dtype=torch.bfloat16, device=DEV)
    EW.embed_prompt(ids, table, out, 768, L, 2048 ** 0.5)
    for b in range(B):
        ref = (table[ids[b].long()].float() * 2048 ** 0.5).bfloat16()
        assert torch.equal(out[b * L + 768:(b + 1) * L], ref)
        assert not out[b * L:b * L + 768].any()


def _shallow_checkpoint(seed=130, vocab=1000):
    from flash_vla_amd.spec import weight_shapes
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in weight_shapes(0).items():
        if name.startswith(("vision_attn", "vision_ffn", "vision_pre", "encoder_attn",
                            "encoder_ffn", "decoder_attn", "decoder_ffn")):
            shape = (2,) + tuple(shape[1:])
        out[name] = (torch.randn(shape, generator=g) * 0.05).to(torch.bfloat16)
    out["embed_tokens"] = (torch.randn(vocab, 2048, generator=g) * 0.05).to(torch.bfloat16)
    return out


def test_batched_forward_with_prompt_tokens():
    from flash_vla_amd import Pi0Inference
    B, P, vocab = 2, 48, 1000
    ck = _shallow_checkpoint(vocab=vocab)
    g = torch.Generator().manual_seed(131)
    images = (torch.rand(B, 3, 224, 224, 3, generator=g) * 2 - 1).to(torch.bfloat16)
    state = torch.randn(B, 32, generator=g).to(torch.bfloat16)
    noise = torch.randn(B, 50, 32, generator=g).to(torch.bfloat16)
    ids = torch.randint(0, vocab, (B, P), generator=g, dtype=torch.int32)
    eng = Pi0Inference({k: v.to(DEV) for k, v in ck.items()}, steps=2, batch=B,
                       prompt_tokens=P, capture=True)
    out = eng.forward(images.to(DEV), state.to(DEV), noise.to(DEV), ids.to(DEV)).clone()
    assert out.shape == (B * 50, 32)
    for b in range(B):
        w1 = dict(ck)
        w1.pop("embed_tokens")
        w1["language_embeds"] = (ck["embed_tokens"][ids[b].long()].float() * 2048 ** 0.5).bfloat16()
        # the batched request b ~ a batch-1 engine fed the same request (not bitwise: at
        # M = 102 rows the decoder's split-K GEMMs split K 2 ways instead of 4, so fp32
        # partial sums are added in another order)
        one = Pi0Inference({k: v.to(DEV) for k, v in w1.items()}, steps=2, capture=False)
        o1 = one.forward(images[b].to(DEV), state[b].to(DEV), noise[b].to(DEV)).float().cpu()
        ob = out[b * 50:(b + 1) * 50].float().cpu()
        d_err = (o1 - ob).abs().max().item()
        d_cos = torch.nn.functional.cosine_similarity(o1.flatten().double(), ob.flatten().double(),
                                                      dim=0).item()
        scale = o1.abs().max().item()
        print(f"request {b}: batched vs batch-1 max abs {d_err:.3e} (scale {scale:.2f}) "
              f"cos {d_cos:.7f}", flush=True)
        # about two bf16 ulps at the largest magnitude
        assert d_err <= 2.0 ** -6 * scale and d_cos >= 0.9999, f"request {b} differs from batch-1"
        bn, bK, bV = Vn.full_forward(w1, images[b], state[b], noise[b], steps=2, bf16=True)
        fn, fK, fV = Vn.full_forward(w1, images[b], state[b], noise[b], steps=2, bf16=False)
        got = out[b * 50:(b + 1) * 50].float().cpu()

        def cos(x, y):
            return torch.nn.functional.cosine_similarity(x.flatten().double(), y.flatten().double(),
                                                         dim=0).item()
        g_err, e_err = (got - fn).abs().max().item(), (bn.float() - fn).abs().max().item()
        g_cos, e_cos = cos(got, fn), cos(bn.float(), fn)
        kb_ = eng.buffers["encoder_K"][b, :2, :816].float().cpu()
        print(f"request {b}: gpu vs fp32 err {g_err:.3e} 1-cos {1 - g_cos:.2e}; bf16 oracle err "
              f"{e_err:.3e} 1-cos {1 - e_cos:.2e}; gpu vs bf16 oracle 1-cos {1 - cos(got, bn.float()):.2e}; "
              f"prefix K 1-cos gpu {1 - cos(kb_, fK):.2e} bf16 {1 - cos(bK.float(), fK):.2e}", flush=True)
        assert g_cos >= 0.999
        assert (1 - g_cos) <= 1.5 * (1 - e_cos) + 1e-6 and g_err <= 2.0 * e_err + 2e-3
