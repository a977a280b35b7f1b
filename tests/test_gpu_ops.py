"""Per-op parity of the HIP kernels against the CPU oracle, at the decoder's real shapes.

Every op is called through the backend wrappers (ctypes -> libpi0hip.so) on
seeded bf16 inputs and compared with oracle/pi0_decoder.py evaluated in fp32
on the same bf16 values, with the oracle rounding where the kernels store bf16.
Tolerance (stated per test): the kernels and the oracle differ only in fp32
summation order, so outputs agree to a couple of bf16 ulps:
max|got - ref| <= 2**-6 * max|ref| (about two ulps at the largest magnitude)
and cosine >= 0.99999.
"""
import math

import pytest
import torch

from oracle import pi0_decoder as O
from flash_vla_amd.backends.hip import wrappers as W
from flash_vla_amd.arena import ScratchPool

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2.0 ** -6


@pytest.fixture(autouse=True)
def _pool():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    with W.use_pool(ScratchPool()):
        yield


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def close(got, ref, tol=TOL, what=""):
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert torch.isfinite(got).all(), what
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten().double(), ref.flatten().double(),
                                                dim=0).item()
    assert err <= tol * scale + 1e-6, f"{what}: max err {err} vs scale {scale}"
    assert cos >= 0.99999, f"{what}: cosine {cos}"


def test_pack_weight_layout():
    from flash_vla_amd.backends.hip import _abi
    w = rnd((2, 64, 48), 1)
    wd = w.to(DEV)
    p = torch.empty_like(wd)
    _abi.call("pi0hip_pack_weight", wd.data_ptr(), p.data_ptr(), 64, 48, 2,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    # expected: [b][nt][kt][lane][j] = W[b][kt*32 + (lane//16)*8 + j][nt*16 + lane%16]
    exp = w.reshape(2, 2, 4, 8, 3, 16).permute(0, 4, 1, 2, 5, 3).reshape(-1)
    assert torch.equal(p.cpu().reshape(-1), exp)


def test_state_proj():
    x, w, b = rnd(32, 2), rnd((32, 1024), 3, 0.02), rnd(1024, 4, 0.02)
    out = torch.zeros(1, 1024, dtype=torch.bfloat16, device=DEV)
    W.decoder_state_proj(x.to(DEV), w.to(DEV), b.to(DEV), out)
    close(out, O.op_state_proj(x.float(), w.float(), b.float()), what="state_proj")


def test_action_in_proj():
    x, w, b = rnd((50, 32), 5), rnd((32, 1024), 6, 0.02), rnd(1024, 7, 0.5)
    out = torch.zeros(50, 1024, dtype=torch.bfloat16, device=DEV)
    W.decoder_action_in_proj(x.to(DEV), w.to(DEV), b.to(DEV), out)
    close(out, O.op_action_in_proj(x.float(), w.float(), b.float()), what="action_in")


def test_action_in_proj_fp32_input():
    x = torch.randn(50, 32, generator=torch.Generator().manual_seed(36))
    w, b = rnd((32, 1024), 37, 0.02), rnd(1024, 38, 0.5)
    out = torch.zeros(50, 1024, dtype=torch.bfloat16, device=DEV)
    W.decoder_action_in_proj(x.to(DEV), w.to(DEV), b.to(DEV), out)
    close(out, O.op_action_in_proj(x, w.float(), b.float()), what="action_in fp32 x")


def test_action_mlp_into_row_view():
    x, w, b = rnd((50, 1024), 8), rnd((1024, 1024), 9, 0.02), rnd(1024, 10, 0.02)
    xbuf = torch.full((51, 1024), 7.0, dtype=torch.bfloat16, device=DEV)
    W.decoder_action_mlp(x.to(DEV), w.to(DEV), b.to(DEV), xbuf[1:])
    close(xbuf[1:], O.op_action_mlp(x.float(), w.float(), b.float()), what="action_mlp")
    assert torch.all(xbuf[0] == 7.0)      # row 0 (state) untouched


@pytest.mark.parametrize("M", [51, 1, 56, 57, 64, 100])
def test_norm_qkv_rope(M):
    x = rnd((M, 1024), 11)
    w = rnd((1024, 2560), 12, 0.02)
    enc = 768
    rope = O.rope_table(M, enc, 256)
    Kc = torch.zeros(enc + M, 256, dtype=torch.bfloat16, device=DEV)
    Vc = torch.zeros_like(Kc)
    Q = torch.zeros(M * 8, 256, dtype=torch.bfloat16, device=DEV)
    nf = torch.zeros(M + 3, dtype=torch.bfloat16, device=DEV)
    W.decoder_norm_qkv_rope(x.to(DEV), w.to(DEV), rope.to(DEV), Q, Kc[enc:], Vc[enc:], nf)
    q, k, v, f = O.op_norm_qkv_rope(x.float(), w.float(), rope, 8)
    close(Q, q, what="Q")
    close(Kc[enc:], k, what="K")
    close(Vc[enc:], v, what="V")
    assert torch.equal(nf[:M].cpu().float(), f)
    assert torch.all(Kc[:enc] == 0) and torch.all(Vc[:enc] == 0)


@pytest.mark.parametrize("rows,keys,enc", [(408, 819, 768), (408, 867, 816), (16, 64, 40),
                                           (24, 100, 60), (8, 769, 768), (1632, 819, 768),
                                           (408, 1024, 973), (408, 1075, 1024), (408, 2048, 1997)])
def test_attention_matches_masked_softmax(rows, keys, enc):
    q = rnd((rows, 256), 13)
    k = rnd((keys, 256), 14)
    v = rnd((keys, 256), 15)
    Q = q.to(DEV)
    scores = torch.zeros(1, dtype=torch.bfloat16, device=DEV)
    W.decoder_attention(Q, k.to(DEV), v.to(DEV), scores, Q, enc)   # out aliases Q
    ref = O.op_attention(q.float(), k.float(), v.float(), enc, 8)
    close(Q, ref, tol=2.0 ** -5, what="attention")


def test_attention_rejects_more_than_2048_keys():
    q, k = rnd((16, 256), 13).to(DEV), rnd((2049, 256), 14).to(DEV)
    with pytest.raises(RuntimeError):
        W.decoder_attention(q, k, k, None, q, 1998)


def test_attention_state_rows_ignore_action_keys():
    q, k, v = rnd((408, 256), 16), rnd((819, 256), 17), rnd((819, 256), 18)
    k2, v2 = k.clone(), v.clone()
    k2[769:] = rnd((50, 256), 19) * 4
    v2[769:] = rnd((50, 256), 20) * 4
    outs = []
    for kk, vv in ((k, v), (k2, v2)):
        Q = q.to(DEV)
        W.decoder_attention(Q, kk.to(DEV), vv.to(DEV), None, Q, 768)
        outs.append(Q.cpu())
    assert torch.equal(outs[0][:8], outs[1][:8])
    assert not torch.equal(outs[0][8:], outs[1][8:])


@pytest.mark.parametrize("M,K,N", [(1, 512, 1024), (16, 1024, 1024), (17, 2048, 32),
                                   (51, 4096, 1024), (64, 4096, 48), (50, 2048, 1024)])
def test_residual_rows_kernel_shapes(M, K, N):
    """The row-split residual GEMM (one launch, 16-row workgroups over the whole K) at its
    edges: a single row, exact and ragged 16-row blocks, column counts that are and are not
    a multiple of 8 tiles (the XCD placement applies only to the former)."""
    from flash_vla_amd.backends.hip import _abi
    x, w, r = rnd((M, K), 121), rnd((K, N), 122, 0.02), rnd((M, N), 123)
    out = r.to(DEV).clone()
    xd, wd = x.to(DEV), w.to(DEV)          # the packed copy lives as long as wd
    _abi.call("pi0hip_linear_residual_rows", xd.data_ptr(), K, W.packed_weight_ptr(wd),
              out.data_ptr(), N, M, N, K, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    close(out, O.op_matmul_residual(x.float(), w.float(), r.float()), what=f"rows M={M} K={K}")


@pytest.mark.parametrize("M,K", [(51, 2048), (51, 4096), (204, 2048), (204, 4096), (100, 4096)])
def test_residual_gemm(M, K):
    """M > 64 (the batched decoder) runs on the tile kernel's split-K path."""
    x = rnd((M, K), 21)
    w = rnd((K, 1024), 22, 0.02)
    r = rnd((M, 1024), 23)
    out = r.to(DEV)
    W.decoder_out_proj_residual(x.to(DEV), w.to(DEV), out)
    close(out, O.op_matmul_residual(x.float(), w.float(), r.float()), what=f"res M={M} K={K}")


@pytest.mark.parametrize("M", [51, 204])
def test_residual_splitk_is_deterministic_and_reentrant(M):
    x, w, r = rnd((M, 4096), 24).to(DEV), rnd((4096, 1024), 25, 0.02).to(DEV), rnd((M, 1024), 26)
    outs = []
    for _ in range(3):
        out = r.to(DEV)
        W.decoder_ffn_down_residual(x, w, out)
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


@pytest.mark.parametrize("M", [51, 7, 56, 57, 64, 204, 100])
def test_norm_gated_ffn(M):
    """M > 64 runs on the tile kernel with the RMS factor fused (f rounded to bf16); up to
    56 rows the skinny kernel stages only rows 0-55 of its 64-row block."""
    x = rnd((M, 1024), 27)
    wg, wu = rnd((1024, 4096), 28, 0.02), rnd((1024, 4096), 29, 0.02)
    out = torch.zeros(M, 4096, dtype=torch.bfloat16, device=DEV)
    W.decoder_norm_gated_ffn(x.to(DEV), wg.to(DEV), wu.to(DEV), out, None)
    close(out, O.op_norm_gated_ffn(x.float(), wg.float(), wu.float()), what=f"gated_ffn M={M}")


def test_unstaged_rows_do_not_leak():
    """At M <= 56 the skinny GEMMs leave LDS rows 56-63 unloaded: NaNs staged there by a
    preceding 64-row launch (same kernels, same LDS) must not reach the 51 output rows."""
    wg, wu = rnd((1024, 4096), 28, 0.02).to(DEV), rnd((1024, 4096), 29, 0.02).to(DEV)
    xn = rnd((64, 1024), 30).to(DEV)
    xn[51:] = float("nan")
    W.decoder_norm_gated_ffn(xn, wg, wu, torch.empty(64, 4096, dtype=torch.bfloat16, device=DEV), None)
    x = rnd((51, 1024), 27)
    out = torch.zeros(51, 4096, dtype=torch.bfloat16, device=DEV)
    W.decoder_norm_gated_ffn(x.to(DEV), wg, wu, out, None)
    assert torch.isfinite(out.float()).all()
    close(out, O.op_norm_gated_ffn(x.float(), wg.cpu().float(), wu.cpu().float()), what="gated_ffn after NaN rows")


def test_action_out_proj_euler_update():
    xfull = rnd((51, 1024), 30)
    w, b = rnd((1024, 32), 31, 0.002), rnd(32, 32, 0.002)
    noise = rnd((50, 32), 33)
    out = noise.to(DEV)
    xd = xfull.to(DEV)
    W.decoder_action_out_proj(xd[1:], w.to(DEV), b.to(DEV), out, None)
    close(out, O.op_action_out_proj(xfull[1:].float(), w.float(), b.float(), noise.float()),
          what="out_proj")


def test_action_out_proj_fp32_accumulator():
    xfull = rnd((51, 1024), 46)
    w, b = rnd((1024, 32), 47, 0.002), rnd(32, 48, 0.002)
    noise = torch.randn(50, 32, generator=torch.Generator().manual_seed(49))
    out = noise.to(DEV)
    W.decoder_action_out_proj(xfull.to(DEV)[1:], w.to(DEV), b.to(DEV), out, None)
    x = xfull[1:].float()
    f = O.rms_factor(x, bf16=True)[:, None]          # the factor is rounded to bf16, as in the reference
    ref = noise + b.float() + (x @ w.float()) * f    # everything else stays fp32
    assert out.dtype == torch.float32
    err = (out.cpu() - ref).abs().max().item()
    assert err <= 1e-5, err          # only fp32 summation order differs


def test_layer_views_of_a_stacked_weight():
    """Per-layer views of one [L, K, N] stack resolve to the right packed layer."""
    ws = rnd((3, 2048, 1024), 34, 0.02).to(DEV)
    x = rnd((51, 2048), 35)
    for i in (2, 0, 1):
        out = torch.zeros(51, 1024, dtype=torch.bfloat16, device=DEV)
        W.decoder_out_proj_residual(x.to(DEV), ws[i], out)
        close(out, O.op_matmul_residual(x.float(), ws[i].cpu().float(), torch.zeros(51, 1024)),
              what=f"layer {i}")



def test_skinny_gemm_rejects_misaligned_operands():
    """The skinny GEMMs read x rows 16 bytes at a time (straight into LDS) and store four
    outputs at a time: a row pitch that is not a multiple of 8 elements, a pitch below K,
    or an x pointer off a 16-byte boundary is a shape error, raised before any launch."""
    from flash_vla_amd.backends.hip import _abi
    lib = _abi.lib()
    M, K, N = 51, 1024, 1024
    x = torch.zeros((M, K + 8), dtype=torch.bfloat16, device=DEV)
    wp = torch.zeros((K, N), dtype=torch.bfloat16, device=DEV)
    out = torch.zeros((M, N), dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.current_stream().cuda_stream

    def run(xptr, ldx):
        return lib.pi0hip_linear_residual(xptr, ldx, wp.data_ptr(), out.data_ptr(), N, M, N, K,
                                          1, None, 0, s)

    assert run(x.data_ptr(), K + 8) == 0
    torch.cuda.synchronize()
    assert run(x.data_ptr(), K + 4) == -2            # pitch not a multiple of 8
    assert run(x.data_ptr(), K - 8) == -2            # pitch below K
    assert run(x.data_ptr() + 8, K + 8) == -2        # x not 16-byte aligned


def test_attention_prefetch_is_bitwise_attention():
    """The prefetching attention (spare workgroups pull the layer's gate / up / down
    weights into L2) returns exactly what decoder_attention returns."""
    rows, keys, enc = 408, 819, 768
    q = rnd((rows, 256), 31).to(DEV)
    k = rnd((keys, 256), 32).to(DEV)
    v = rnd((keys, 256), 33).to(DEV)
    gate = rnd((1024, 4096), 34, 0.02).to(DEV)
    up = rnd((1024, 4096), 35, 0.02).to(DEV)
    down = rnd((4096, 1024), 36, 0.02).to(DEV)
    ref = W.decoder_attention(q.clone(), k, v, None, q.clone(), enc)
    out = torch.empty_like(q)
    got = W.decoder_attention_prefetch(q.clone(), k, v, None, out, enc, gate, up, down)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert W.attention_prefetch_for(W.decoder_attention) is W.decoder_attention_prefetch
    assert W.attention_prefetch_for(W.decoder_norm_gated_ffn) is None
