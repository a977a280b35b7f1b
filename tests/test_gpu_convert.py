"""Converted OpenPI weights through the HIP decoder engine on the GPU.

A seeded OpenPI-form state dict at the action expert's real size (width 1024,
8 query heads and 1 KV head of dim 256, FFN 4096, action dim 32; 2 layers;
non-zero Gemma norm weights and biases so every fold is exercised) goes
through `convert.convert_state_dict` -- the path the reference takes from an
OpenPI checkpoint to its engine (`eval/baselines/openpi.py:128-313` ->
`engine.py:35-56`) -- and then through `Pi0DecoderEngine` on the MI355X.
The comparator is the independent OpenPI-form fp64 forward on the raw state
dict (`tests/openpi_form.py`, rotate-half RoPE on the un-permuted weights),
fed the same prefix K/V in its own column order.

Tolerance: BASELINE's bf16 bound, max abs <= 2e-2 and cosine >= 0.999 on the
[50, 32] chunk (`eval/correctness/pi0/openpi_parity.py:14-28` metrics), at 1
and at 10 Euler steps (engine default: fp32 Euler accumulator). On the CPU the
fp32 packed oracle on the same bf16 weights is 4.9e-3 from this comparator
after 10 steps, so the bound leaves the kernels the same room as
`test_gpu_loop.py`.
"""
import pytest
import torch

from flash_vla_amd import Pi0DecoderEngine
from flash_vla_amd import convert as C
from openpi_form import FULL_DECODER as D
from openpi_form import half_split_order, openpi_decode, openpi_state

pytestmark = pytest.mark.gpu
ENC_LEN = 768


@pytest.fixture(scope="module")
def converted():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.set_num_threads(min(16, torch.get_num_threads()))
    sd = openpi_state(D, seed=11, std=0.02, norm_std=0.3)
    packed = C.convert_state_dict(sd, strict=False)
    g = torch.Generator().manual_seed(12)
    K = torch.randn(D.dec_layers, ENC_LEN, D.head_dim, generator=g).bfloat16()
    V = torch.randn(D.dec_layers, ENC_LEN, D.head_dim, generator=g).bfloat16()
    state = torch.randn(D.action, generator=g).bfloat16()
    noise = torch.randn(50, D.action, generator=g).bfloat16()
    return sd, packed, K, V, state, noise


@pytest.mark.parametrize("steps", [1, 10])
def test_converted_checkpoint_on_hip_engine(converted, steps):
    sd, packed, K, V, state, noise = converted
    print(f"[convert-gpu] steps={steps} layers={D.dec_layers}", flush=True)
    eng = Pi0DecoderEngine({k: v.cuda() for k, v in packed.items()}, encoder_seq_len=ENC_LEN,
                           steps=steps, layers=D.dec_layers)
    eng.load_prefix(K.cuda(), V.cuda())
    got = eng.forward(state.cuda(), noise.cuda()).double().cpu()
    Ks = [half_split_order(K[i].double(), D.head_dim) for i in range(D.dec_layers)]
    Vs = [V[i].double() for i in range(D.dec_layers)]
    ref = openpi_decode(sd, Ks, Vs, state.double(), noise.double(), D, steps)
    m = C.error_metrics(ref, got)
    print(f"[convert-gpu] steps={steps}: {m}", flush=True)
    assert (ref - noise.double()).abs().max() > 0.05          # the loop moved the actions
    assert m["max_abs"] <= 2e-2 and m["cosine_similarity"] >= 0.999, m
