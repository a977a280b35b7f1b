"""Host-side logic and the C ABI surface (no GPU needed)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from flash_vla_amd import op_table
from flash_vla_amd.arena import ScratchPool
from flash_vla_amd.backends import BACKENDS, register_backend
from flash_vla_amd.backends.hip import _abi, wrappers
from flash_vla_amd.spec import decoder_weight_shapes, weight_shapes

ROOT = Path(__file__).resolve().parents[1]
DECODER_OPS = {"decoder_state_proj", "decoder_action_in_proj", "decoder_action_mlp",
               "decoder_norm_qkv_rope", "decoder_attention", "decoder_out_proj_residual",
               "decoder_ffn_down_residual", "decoder_norm_gated_ffn", "decoder_action_out_proj"}


def _header_functions():
    text = (ROOT / "include" / "pi0_hip.h").read_text()
    return set(re.findall(r"^\s*(?:int|size_t)\s+(pi0hip_\w+)\s*\(", text, re.M))


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(_abi.library_path())
    names = _header_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    # the Python binding declares exactly the header's functions
    assert set(_abi.PROTOTYPES) == names


def test_workspace_sizes_are_host_computable():
    lib = _abi.lib()
    assert lib.pi0hip_version() >= 1
    assert lib.pi0hip_gemm_workspace_bytes(51, 1024, 1, 0) == 0
    ws = lib.pi0hip_gemm_workspace_bytes(51, 1024, 4, 0)
    # 64 tiles x 4 splits x (64x16 partials + 64 sums) floats
    assert ws == 64 * 4 * (64 * 16 + 64) * 4
    att = lib.pi0hip_attention_workspace_bytes(408, 819)
    # 26 tiles of 16 rows (416 padded), 7 chunks of 128 keys: lse, fp32 partials
    r256 = lambda v: (v + 255) // 256 * 256
    assert att == r256(7 * 416 * 4) + 7 * 416 * 256 * 4


def test_rejected_arguments_do_not_launch():
    lib = _abi.lib()
    # null pointers / bad shapes are rejected before any HIP call
    assert lib.pi0hip_linear_residual(None, 0, None, None, 0, 51, 1024, 2048, 4, None, 0,
                                      None) == -1
    assert lib.pi0hip_pack_weight(None, None, 33, 16, 1, None) == -1
    assert lib.pi0hip_attention(1, 256, 1, 1, 256, 1, 256, 408, 819, 768, 8, 128, 1, 1 << 30,
                                None) == -2
    assert lib.pi0hip_attention(1, 256, 1, 1, 256, 1, 256, 408, 819, 768, 8, 256, 1, 16,
                                None) == -3
    assert lib.pi0hip_linear_residual(1, 2048, 1, 1, 1024, 51, 1024, 2048, 4, None, 0,
                                      None) == -3
    assert lib.pi0hip_norm_gated_ffn(1, 1024, 1, 1, 1, 4096, 51, 4096, 1000, None) == -2
    with pytest.raises(_abi.HipLibraryError):
        _abi.check(-2, "x")


ENCODER_OPS = {"encoder_projector", "encoder_norm_qkv_rope", "encoder_out_proj_residual",
               "encoder_norm_gated_ffn", "encoder_ffn_down_residual", "encoder_attention",
               "vision_patch_embed", "vision_norm_qkv", "vision_out_proj_residual",
               "vision_norm_ffn_up", "vision_ffn_down_residual", "vision_attention",
               "embed_prompt"}


def test_op_table_contract():
    t = op_table(fused=True)
    assert set(vars(t)) == DECODER_OPS | ENCODER_OPS
    hip = BACKENDS["hip"]
    assert t.decoder_attention is hip.FUSED_WRAPPERS["decoder_attention"]
    t2 = op_table(fused=False, plan={"decoder_attention": "hip"})
    assert set(vars(t2)) == DECODER_OPS | ENCODER_OPS
    with pytest.raises(KeyError):
        op_table(plan={"not_an_op": "hip"})
    with pytest.raises(KeyError):
        op_table(plan={"decoder_attention": "tilelang"})


def test_register_backend_mixes_per_call_site():
    class Fake:
        ALL_WRAPPERS = {"decoder_attention": lambda *a: "fake"}
        FUSED_WRAPPERS = {}
    register_backend("fake", Fake)
    try:
        t = op_table(fused=True, plan={"decoder_attention": "fake"})
        assert t.decoder_attention() == "fake"
        assert t.decoder_norm_gated_ffn is BACKENDS["hip"].FUSED_WRAPPERS["decoder_norm_gated_ffn"]
        with pytest.raises(KeyError):
            op_table(plan={"decoder_state_proj": "fake"})
    finally:
        BACKENDS.pop("fake")
    with pytest.raises(TypeError):
        register_backend("bad", object())


def test_scratch_pool_freeze():
    pool = ScratchPool()
    a = pool.get("r", (4,), torch.float32, "cpu")
    assert torch.equal(a, torch.zeros(4))
    assert pool.get("r", (4,), torch.float32, "cpu") is a
    pool.freeze()
    assert pool.get("r", (4,), torch.float32, "cpu") is a
    with pytest.raises(LookupError):
        pool.get("r", (5,), torch.float32, "cpu")
    assert len(pool) == 1 and pool.nbytes() == 16 and pool.frozen


def test_splitk_choice_fills_the_chip():
    assert wrappers._splitk(51, 1024, 2048) == 4          # o-proj: 64 tiles x 4
    assert wrappers._splitk(51, 1024, 4096) == 4          # down
    assert wrappers._splitk(50, 1024, 1024) == 4          # action mlp
    assert wrappers._splitk(50, 32, 1024) == 8            # out-proj, capped by K
    assert wrappers._splitk(51, 4096, 1024) == 1
    for M, N, K in [(51, 1024, 2048), (50, 32, 1024), (51, 2560, 1024), (204, 1024, 4096)]:
        s = wrappers._splitk(M, N, K)
        assert (K // 32) % (4 * s) == 0


def test_schema_shapes():
    full = weight_shapes(0)
    dec = decoder_weight_shapes()
    for k, v in dec.items():
        assert full[k] == v
    assert dec["decoder_attn_qkv_w"] == (18, 1024, 2560)
    layer_bytes = 2 * sum(int(torch.tensor(dec[k][1:]).prod()) for k in (
        "decoder_attn_qkv_w", "decoder_attn_o_w", "decoder_ffn_gate_w", "decoder_ffn_up_w",
        "decoder_ffn_down_w"))
    assert layer_bytes == 34_603_008


def test_wrappers_reject_bad_inputs_on_cpu():
    x = torch.zeros(51, 1024, dtype=torch.bfloat16)
    with pytest.raises((ValueError, TypeError)):
        wrappers.decoder_out_proj_residual(x, torch.zeros(2048, 1024, dtype=torch.bfloat16), x)
    with pytest.raises(TypeError):
        wrappers.decoder_out_proj_residual(x.float(), x, x)
