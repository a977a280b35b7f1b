"""The unfused decoder call sites (op_table(fused=False)) against the oracle's unfused
ops, and the fused-vs-unfused gate of the reference
(eval/correctness/pi0/fused_vs_unfused.py:34-82).

Per-op tolerance as for the fused ops (tests/test_gpu_ops.py): the kernels and the
oracle round at the same points and differ only in fp32 summation order, so
max|got - ref| <= 2**-6 * max|ref| and cosine >= 0.99999 (2**-5 for the attention
output, whose bf16 probabilities can land one ulp apart).
"""
import pytest
import torch

from oracle import pi0_decoder as O
from flash_vla_amd import Pi0DecoderEngine
from flash_vla_amd.arena import ScratchPool
from flash_vla_amd.backends.hip import wrappers as W
from flash_vla_amd.ops import op_table
from flash_vla_amd.weights import decoder_checkpoint, decoder_inputs

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


def close(got, ref, tol=TOL, what=""):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert torch.isfinite(got).all(), what
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten().double(), ref.flatten().double(),
                                                dim=0).item()
    print(f"{what}: max err {err:.3e} (scale {scale:.3e}) cos {cos:.8f}", flush=True)
    assert err <= tol * scale + 1e-6, f"{what}: max err {err} vs scale {scale}"
    assert cos >= 0.99999, f"{what}: cosine {cos}"


def test_tables_differ_exactly_at_the_fused_call_sites():
    fused, unfused = op_table(True), op_table(False)
    differ = {n for n in vars(fused) if getattr(fused, n) is not getattr(unfused, n)}
    assert differ == {"decoder_norm_gated_ffn", "decoder_action_out_proj", "decoder_attention"}


@pytest.mark.parametrize("M", [51, 7])
def test_unfused_gate(M):
    x = rnd((M, 1024), 40)
    wg, wu = rnd((1024, 4096), 41, 0.02), rnd((1024, 4096), 42, 0.02)
    out = torch.zeros(M, 4096, dtype=torch.bfloat16, device=DEV)
    nf = torch.zeros(M, dtype=torch.bfloat16, device=DEV)
    W.decoder_norm_gated_ffn_unfused(x.to(DEV), wg.to(DEV), wu.to(DEV), out, nf)
    ref, f = O.op_norm_gated_ffn_unfused(x.float(), wg.float(), wu.float())
    assert torch.equal(nf.cpu().float(), f), "rms factor"
    close(out, ref, what=f"unfused gate M={M}")
    fused = O.op_norm_gated_ffn(x.float(), wg.float(), wu.float())
    assert not torch.equal(ref, fused)       # the rounding point is really different


@pytest.mark.parametrize("fp32_out", [False, True])
def test_unfused_action_out_proj(fp32_out):
    x, w, b = rnd((50, 1024), 43), rnd((1024, 32), 44, 0.02), rnd(32, 45, 0.1)
    r = rnd((50, 32), 46)
    dt = torch.float32 if fp32_out else torch.bfloat16
    out = r.to(DEV).to(dt)
    nf = torch.zeros(51, dtype=torch.bfloat16, device=DEV)
    W.decoder_action_out_proj_unfused(x.to(DEV), w.to(DEV), b.to(DEV), out, nf)
    ref = O.op_action_out_proj_unfused(x.float(), w.float(), b.float(), r.float(), bf16=True,
                                       round_out=not fp32_out)
    close(out, ref, what=f"unfused out-proj fp32={fp32_out}")


@pytest.mark.parametrize("rows,keys,enc", [(408, 819, 768), (408, 1075, 1024), (16, 64, 40)])
def test_unfused_attention(rows, keys, enc):
    q, k, v = rnd((rows, 256), 47), rnd((keys, 256), 48), rnd((keys, 256), 49)
    Q = q.to(DEV)
    probs = torch.zeros(rows, keys, dtype=torch.bfloat16, device=DEV)
    W.decoder_attention_unfused(Q, k.to(DEV), v.to(DEV), probs, Q, enc)     # out aliases Q
    ref, p = O.op_attention_unfused(q.float(), k.float(), v.float(), enc, 8)
    close(probs, p, tol=2.0 ** -5, what="unfused probabilities")
    assert torch.all(probs[:8, enc + 1:] == 0)
    close(Q, ref, tol=2.0 ** -5, what=f"unfused attention keys={keys}")


def test_fused_vs_unfused_one_step():
    """The reference's regression gate at --steps 1 (18 layers): the two tables on identical
    buffers agree within allclose(0.5) (its TOLERANCE), and each agrees tightly with the
    oracle of its own rounding points."""
    ck = decoder_checkpoint(seed=0)
    inp = decoder_inputs(seed=1)
    outs = {}
    for fused in (True, False):
        eng = Pi0DecoderEngine({k: v.to(DEV) for k, v in ck.items()}, steps=1, fused=fused,
                               fp32_euler=False)
        eng.load_prefix(inp["encoder_K"].to(DEV), inp["encoder_V"].to(DEV))
        outs[fused] = eng.forward(inp["observation_state_normalized"].to(DEV),
                                  inp["diffusion_noise"].to(DEV)).float().cpu()
    diff = (outs[True] - outs[False]).abs().max().item()
    print(f"\nfused vs unfused (1 step x 18 layers): max abs {diff:.3e}")
    assert torch.allclose(outs[True], outs[False], atol=5e-1, rtol=5e-1)
    assert not torch.equal(outs[True], outs[False])
    args = (ck, inp["observation_state_normalized"], inp["diffusion_noise"], inp["encoder_K"],
            inp["encoder_V"], 768)
    for fused in (True, False):
        ref = O.decoder_packed(*args, steps=1, bf16=True, unfused=not fused)[0]
        err = (outs[fused] - ref).abs().max().item()
        cos = torch.nn.functional.cosine_similarity(outs[fused].flatten().double(),
                                                    ref.flatten().double(), dim=0).item()
        print(f"{'fused' if fused else 'unfused'} vs its oracle: max abs {err:.3e} cos {cos:.7f}")
        assert err <= 2e-2 and cos >= 0.99999
