"""Parity of the prefix-encoder HIP kernels with the CPU oracle.

Per-op tests call the backend wrappers (ctypes -> libpi0hip.so) at the
encoder's real shapes (M = 768, ragged 816 and small M) on seeded bf16 inputs,
against oracle/pi0_encoder.py in fp32 with the reference's rounding points.
Per-op tolerance: outputs differ only by fp32 summation order, so
max|got - ref| <= 2**-6 * max|ref| and cosine >= 0.99999 (attention:
2**-5, since the kernel rounds unnormalised probabilities to bf16 where the
reference rounds normalised ones).

Layer-stack tests compare against the fp32 oracle with a relative criterion,
as bf16 rounding noise grows through the residual stream: the GPU must be no
farther from fp32 than exact bf16 emulation, within a factor 1.5.
"""
import pytest
import torch

from oracle import pi0_encoder as E
from oracle import pi0_decoder as O
from flash_vla_amd.arena import ScratchPool
from flash_vla_amd.backends.hip import encoder_wrappers as EW
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


def test_pack_weight32_layout():
    """16 k x 32 n fragments: [b][nt][kt][lane][j] = W[b][16 kt + 8 (lane // 32) + j][32 nt + lane % 32]."""
    w = rnd((2, 64, 64), 10)
    wd = w.to(DEV)
    p = torch.empty_like(wd)
    W._abi.call("pi0hip_pack_weight32", wd.data_ptr(), p.data_ptr(), 64, 64, 2, W._stream())
    torch.cuda.synchronize()
    exp = w.reshape(2, 4, 2, 8, 2, 32).permute(0, 4, 1, 2, 5, 3).reshape(-1)
    assert torch.equal(p.cpu().reshape(-1), exp)


@pytest.mark.parametrize("M", [768, 816, 5])
def test_rms_norm(M):
    x = rnd((M, 2048), 11, 2.0)
    out = torch.zeros(M, 2048, dtype=torch.bfloat16, device=DEV)
    W._abi.call("pi0hip_rms_norm", x.to(DEV).data_ptr(), 2048, out.data_ptr(), 2048, M, 2048,
                W._stream())
    close(out, E.enc_rms_norm(x.float()), what=f"rms_norm M={M}")


def test_projector():
    """LayerNorm(eps 1e-5) over 1152 + bias GEMM 1152 -> 2048 on 3 views x 256 tokens."""
    x = rnd((3, 256, 1152), 12, 1.5)
    nw, nb = rnd(1152, 13, 0.5), rnd(1152, 14, 0.5)
    pw, pb = rnd((1152, 2048), 15, 0.03), rnd(2048, 16, 0.5)
    out = torch.zeros(768, 2048, dtype=torch.bfloat16, device=DEV)
    xn = torch.zeros(3, 256, 1152, dtype=torch.bfloat16, device=DEV)
    EW.encoder_projector(x.to(DEV), nw.to(DEV), nb.to(DEV), pw.to(DEV), pb.to(DEV), out, xn)
    ref_n = E.enc_layer_norm(x.float().reshape(768, 1152), nw.float(), nb.float())
    close(xn.reshape(768, 1152), ref_n, what="projector layer_norm")
    close(out, E.enc_projector(x.float().reshape(768, 1152), nw.float(), nb.float(), pw.float(),
                               pb.float()), what="projector")


@pytest.mark.parametrize("M", [768, 816, 40, 3264])
def test_norm_qkv_rope(M):
    x = rnd((M, 2048), 17, 1.0)
    w = rnd((2048, 2560), 18, 0.02)
    rope = O.rope_table(M, 0, 256).to(torch.bfloat16)
    Q = torch.zeros(M * 8, 256, dtype=torch.bfloat16, device=DEV)
    K = torch.zeros(M + 51, 256, dtype=torch.bfloat16, device=DEV)   # cache with decoder rows
    V = torch.zeros_like(K)
    xn = torch.zeros(M, 2048, dtype=torch.bfloat16, device=DEV)
    EW.encoder_norm_qkv_rope(x.to(DEV), w.to(DEV), rope.to(DEV), Q, K[:M], V[:M], xn)
    q, k, v = E.enc_norm_qkv_rope(x.float(), w.float(), rope.float(), heads=8)
    close(Q, q, what=f"Q M={M}")
    close(K[:M], k, what=f"K M={M}")
    close(V[:M], v, what=f"V M={M}")
    assert not K[M:].any() and not V[M:].any(), "wrote past the prefix rows"


@pytest.mark.parametrize("rows,keys", [(6144, 768), (6528, 816), (64, 40), (24, 7)])
def test_encoder_attention(rows, keys):
    q, k, v = rnd((rows, 256), 19), rnd((keys, 256), 20), rnd((keys, 256), 21)
    out = EW.encoder_attention(q.to(DEV), k.to(DEV), v.to(DEV), 256 ** -0.5)
    ref = E.enc_attention(q.float(), k.float(), v.float())
    close(out.reshape(rows, 256), ref, tol=2.0 ** -5, what=f"attention {rows}x{keys}")


@pytest.mark.parametrize("M", [768, 100, 3264])
def test_out_proj_residual(M):
    x, w, r = rnd((M, 2048), 22), rnd((2048, 2048), 23, 0.02), rnd((M, 2048), 24)
    out = r.to(DEV).clone()
    EW.encoder_out_proj_residual(x.to(DEV), w.to(DEV), out)
    close(out, E.enc_residual(x.float(), w.float(), r.float()), what=f"o_proj M={M}")


def test_ffn_down_splitk_deterministic():
    """K = 16384 split four ways; partials summed in split order: bitwise repeatable."""
    M = 768
    x, w, r = rnd((M, 16384), 25, 0.5), rnd((16384, 2048), 26, 0.02), rnd((M, 2048), 27)
    xd, wd = x.to(DEV), w.to(DEV)
    out1 = r.to(DEV).clone()
    EW.encoder_ffn_down_residual(xd, wd, out1)
    out2 = r.to(DEV).clone()
    EW.encoder_ffn_down_residual(xd, wd, out2)
    assert torch.equal(out1, out2)
    close(out1, E.enc_residual(x.float(), w.float(), r.float()), what="ffn_down")


def test_ffn_down_large_m():
    """Batched prefix (4 x 816 rows): the row tiles fill the chip, K is not split; the fp32
    oracle arithmetic runs on the device to keep the 219-GFLOP reference fast."""
    M = 3264
    x, w, r = rnd((M, 16384), 31, 0.5), rnd((16384, 2048), 32, 0.02), rnd((M, 2048), 33)
    out = r.to(DEV).clone()
    EW.encoder_ffn_down_residual(x.to(DEV), w.to(DEV), out)
    ref = E.enc_residual(x.to(DEV).float(), w.to(DEV).float(), r.to(DEV).float())
    close(out, ref, what="ffn_down M=3264")


@pytest.mark.parametrize("M", [768, 816])
def test_norm_gated_ffn(M):
    x = rnd((M, 2048), 28, 1.0)
    wg, wu = rnd((2048, 16384), 29, 0.02), rnd((2048, 16384), 30, 0.02)
    out = torch.zeros(M, 16384, dtype=torch.bfloat16, device=DEV)
    xn = torch.zeros(M, 2048, dtype=torch.bfloat16, device=DEV)
    EW.encoder_norm_gated_ffn(x.to(DEV), wg.to(DEV), wu.to(DEV), out, xn)
    close(out, E.enc_norm_gated_ffn(x.float(), wg.float(), wu.float()), what=f"gated_ffn M={M}")


def test_gated_ffn_row_blocks_bitwise():
    """From 512 rows the gated FFN runs on 384-row 8-wave blocks with both operands in LDS,
    below on the 128-row strip kernel; both accumulate every output in the same k order, so
    the first 200 rows of an M = 768 (and of a ragged M = 600) product equal an M = 200
    product bit for bit."""
    x = rnd((768, 2048), 31, 1.0).to(DEV)
    wg, wu = rnd((2048, 16384), 32, 0.02).to(DEV), rnd((2048, 16384), 33, 0.02).to(DEV)
    outs = {}
    for M in (768, 600, 200):
        out = torch.zeros(M, 16384, dtype=torch.bfloat16, device=DEV)
        xn = torch.zeros(M, 2048, dtype=torch.bfloat16, device=DEV)
        EW.encoder_norm_gated_ffn(x[:M].contiguous(), wg, wu, out, xn)
        outs[M] = out.cpu()
    assert torch.equal(outs[768][:200], outs[200])
    assert torch.equal(outs[600][:200], outs[200])
    assert torch.equal(outs[768][:600], outs[600])


def _encoder_case(layers, M, seed=40):
    from flash_vla_amd.weights import encoder_checkpoint, encoder_inputs
    ck = encoder_checkpoint(seed=seed, layers=layers)
    x = encoder_inputs(seed=seed + 1, encoder_seq_len=M)
    return ck, x


def _run_engine(ck, x, capture):
    from flash_vla_amd import Pi0EncoderEngine
    eng = Pi0EncoderEngine(ck, encoder_seq_len=x.shape[0], capture=capture)
    K, V = eng.forward(x.to(DEV))
    return eng, K, V


@pytest.mark.parametrize("layers,M", [(2, 768), (18, 64)])
def test_encoder_stack(layers, M):
    """Whole encoder stacks (last layer QKV only) against the oracle; the 18-layer stack
    runs at M = 64 so the CPU oracle stays within seconds."""
    ck, x = _encoder_case(layers, M)
    eng, K, V = _run_engine(ck, x, capture=False)
    bK, bV, bx = E.encoder_packed(ck, x, bf16=True)
    fK, fV, fx = E.encoder_packed(ck, x, bf16=False)
    for name, got, b, f in (("K", K[:, :M], bK, fK), ("V", V[:, :M], bV, fV)):
        g_err, g_cos = metrics(got, f)
        e_err, e_cos = metrics(b, f)
        print(f"{layers} layers M={M} {name}: gpu vs fp32 err {g_err:.3e} 1-cos {1 - g_cos:.2e}; "
              f"bf16 oracle err {e_err:.3e} 1-cos {1 - e_cos:.2e}", flush=True)
        assert g_cos >= 0.999
        assert (1 - g_cos) <= 1.5 * (1 - e_cos) + 1e-7 and g_err <= 1.5 * e_err + 1e-3


def test_encoder_graph_equals_eager():
    ck, x = _encoder_case(3, 768, seed=50)
    _, K1, V1 = _run_engine(ck, x, capture=False)
    K1, V1 = K1.clone(), V1.clone()
    eng, K2, V2 = _run_engine(ck, x, capture=True)
    assert torch.equal(K1, K2) and torch.equal(V1, V2)
    # replay again on the same input: the graph re-reads encoder_x after forward re-copies it
    K3, V3 = eng.forward(x.to(DEV))
    assert torch.equal(K1, K3) and torch.equal(V1, V3)
