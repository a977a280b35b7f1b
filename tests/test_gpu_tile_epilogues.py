"""Tile GEMM epilogues at ragged row counts, through the C ABI.

The bias and residual pieces of `tile_gemm_kernel`'s epilogue are read while the k loop
runs, through buffer resources bounded to the valid rows and columns; these cases put the
last row block partly past M, use the position-table residual (`res_mod`) and padded
weight columns, and check that nothing is written past row M or column N. References are
fp32 products on the device, rounded once to bf16."""
import pytest
import torch

from flash_vla_amd.arena import ScratchPool
from flash_vla_amd.backends.hip import _abi
from flash_vla_amd.backends.hip import wrappers as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _pool():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    with W.use_pool(ScratchPool()):
        yield


def rnd(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def _gelu_tanh(v):
    return 0.5 * v * (1.0 + torch.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))


def _check(got, ref, what):
    got, ref = got.float(), ref.float()
    assert torch.isfinite(got).all(), what
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    assert err <= 2.0 ** -6 * scale + 1e-6, f"{what}: max err {err} vs scale {scale}"


def _out_with_sentinel(M, N, ld):
    """[M, N] rows of pitch ld with 7.0 in the padding columns and in 3 rows after M."""
    store = torch.full(((M + 3) * ld,), 7.0, dtype=torch.bfloat16, device=DEV)
    return store, store.view(M + 3, ld)


@pytest.mark.parametrize("M", [100, 300, 2100])      # 2100: the 128-row tiles used from 2048 rows
@pytest.mark.parametrize("res_mod", [0, 256])
def test_bias_residual_ragged(M, res_mod):
    K, N, N_pad, K_pad = 1152, 1144, 1152, 1152      # N = 1144: the last 8 packed columns padded
    x, w, b = rnd((M, K), 1), rnd((K, N), 2, 0.03), rnd(N, 3, 0.5)
    rrows = res_mod or M
    res = rnd((rrows, N_pad), 4)
    store, out = _out_with_sentinel(M, N, N_pad)
    _abi.call("pi0hip_tile_linear_bias_res", x.data_ptr(), K, W.packed_weight_ptr(w, 32, (K_pad, N_pad)),
              b.data_ptr(), res.data_ptr(), N_pad, res_mod, out.data_ptr(), N_pad, M, N, K, N_pad,
              K_pad, W._stream())
    torch.cuda.synchronize()
    ridx = torch.arange(M, device=DEV) % res_mod if res_mod else torch.arange(M, device=DEV)
    ref = (x.float() @ w.float() + b.float() + res[ridx, :N].float()).bfloat16()
    _check(out[:M, :N], ref, f"bias + residual M={M} res_mod={res_mod}")
    assert torch.all(out[:M, N:] == 7.0), "stored into the padded columns"
    assert torch.all(out[M:] == 7.0), "stored past row M"


@pytest.mark.parametrize("M", [100, 300])
def test_residual_in_place_ragged(M):
    K, N = 2048, 2048
    x, w, r = rnd((M, K), 5), rnd((K, N), 6, 0.02), rnd((M, N), 7)
    store, out = _out_with_sentinel(M, N, N)
    out[:M].copy_(r)
    _abi.call("pi0hip_tile_linear_residual", x.data_ptr(), K, W.packed_weight_ptr(w, 32),
              out.data_ptr(), N, M, N, K, 1, None, 0, W._stream())
    torch.cuda.synchronize()
    _check(out[:M], (x.float() @ w.float() + r.float()).bfloat16(), f"residual M={M}")
    assert torch.all(out[M:] == 7.0), "stored past row M"


@pytest.mark.parametrize("M", [100, 300])
def test_bias_gelu_and_bias_ragged(M):
    K, N, N_pad = 1152, 4304, 4352
    x, w, b = rnd((M, K), 8), rnd((K, N), 9, 0.03), rnd(N, 10, 0.5)
    store, out = _out_with_sentinel(M, N, N)
    _abi.call("pi0hip_tile_linear_bias_gelu", x.data_ptr(), K, W.packed_weight_ptr(w, 32, (K, N_pad)),
              b.data_ptr(), out.data_ptr(), N, M, N, K, N_pad, K, W._stream())
    torch.cuda.synchronize()
    _check(out[:M], _gelu_tanh(x.float() @ w.float() + b.float()).bfloat16(), f"bias + gelu M={M}")
    assert torch.all(out[M:] == 7.0), "stored past row M"

    N2 = 2048
    w2, b2 = rnd((K, N2), 11, 0.03), rnd(N2, 12, 0.5)
    store2, out2 = _out_with_sentinel(M, N2, N2)
    _abi.call("pi0hip_tile_linear", x.data_ptr(), K, W.packed_weight_ptr(w2, 32), b2.data_ptr(),
              out2.data_ptr(), N2, M, N2, K, W._stream())
    torch.cuda.synchronize()
    _check(out2[:M], (x.float() @ w2.float() + b2.float()).bfloat16(), f"bias M={M}")
    assert torch.all(out2[M:] == 7.0), "stored past row M"
