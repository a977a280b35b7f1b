"""Offline conversion of a local OpenPI Pi0 checkpoint into the packed schema.

Follows `eval/baselines/openpi.py:75-313` of the reference, minus its model
import: the reference instantiates OpenPI's `PI0Pytorch` and reads
`model.state_dict()`. This module reads the same state dict straight from the
`model.safetensors` file with `safetensors.safe_open` (it executes nothing
from the file), so OpenPI itself is not needed. The algebra:

* `nn.Linear` weights are `[out, in]`; the packed schema is `[in, out]`.
* Gemma RMSNorm `(1 + w)` folds into the rows of the next projection
  (input norm into Q/K/V, post-attention norm into gate/up); Q and K columns
  move from half-split to adjacent-pair RoPE order (`openpi.py:86-125`).
* The SigLIP patch convolution `[out, in, kh, kw]` becomes the
  `[kh, kw, in, out]` GEMM operand (`openpi.py:161-163`).
* action_in_proj and the time half of action_time_mlp_in fold into one
  projection plus one bias per Euler step; the final norm and dt = -0.1 fold
  into action_out_proj (`openpi.py:270-302`).

All folding runs in fp32 and each packed tensor is rounded to bf16 once, in
the reference's order of operations. `error_metrics` is the reference's
parity report (`eval/correctness/pi0/openpi_parity.py:14-28`).

Command line::

    python -m flash_vla_amd.convert --checkpoint /path/model.safetensors --out packed.safetensors
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path

import torch
import torch.nn.functional as F

from . import spec
from .weights import EULER_DT, fold_decoder, fold_gemma_layers

# OpenPI module prefixes (`openpi.py:17-20`): these are the checkpoint's own names.
VISION = "paligemma_with_expert.paligemma.model.vision_tower.vision_model"
PROJECTOR = "paligemma_with_expert.paligemma.model.multi_modal_projector.linear"
ENCODER = "paligemma_with_expert.paligemma.model.language_model"
DECODER = "paligemma_with_expert.gemma_expert.model"


class _State:
    """Read-only view of a state dict that reports missing names clearly."""

    def __init__(self, tensors, dtype=torch.float32):
        self._t = tensors
        self._dtype = dtype

    def value(self, name: str) -> torch.Tensor:
        try:
            t = self._t[name]
        except KeyError as error:
            raise KeyError(f"OpenPI checkpoint is missing {name!r}") from error
        return t.detach().to(self._dtype)

    def linear(self, name: str) -> torch.Tensor:
        """`nn.Linear` weight as `[in, out]`."""
        return self.value(f"{name}.weight").t()

    def count_layers(self, root: str) -> int:
        n = 0
        while f"{root}.layers.{n}.self_attn.q_proj.weight" in self._t:
            n += 1
        return n


def _stack(count: int, make) -> torch.Tensor:
    return torch.stack([make(i) for i in range(count)])


def _gemma_params(st: _State, root: str, layers: int) -> dict:
    """Unfolded Gemma layers in `[in, out]` form, half-split RoPE columns."""
    def lin(i, name):
        return st.linear(f"{root}.layers.{i}.{name}")

    def norm(i, name):
        return st.value(f"{root}.layers.{i}.{name}.weight")

    return {
        "q_w": _stack(layers, lambda i: lin(i, "self_attn.q_proj")),
        "k_w": _stack(layers, lambda i: lin(i, "self_attn.k_proj")),
        "v_w": _stack(layers, lambda i: lin(i, "self_attn.v_proj")),
        "o_w": _stack(layers, lambda i: lin(i, "self_attn.o_proj")),
        "gate_w": _stack(layers, lambda i: lin(i, "mlp.gate_proj")),
        "up_w": _stack(layers, lambda i: lin(i, "mlp.up_proj")),
        "down_w": _stack(layers, lambda i: lin(i, "mlp.down_proj")),
        "input_norm_w": _stack(layers, lambda i: norm(i, "input_layernorm")),
        "post_attn_norm_w": _stack(layers, lambda i: norm(i, "post_attention_layernorm")),
    }


def _vision(st: _State, layers: int) -> dict:
    """SigLIP tower: layout changes only (`openpi.py:142-203`)."""
    def lay(i):
        return f"{VISION}.encoder.layers.{i}"

    def qkv_w(i):
        return torch.cat([st.linear(f"{lay(i)}.self_attn.{p}_proj") for p in "qkv"], dim=1)

    def qkv_b(i):
        return torch.cat([st.value(f"{lay(i)}.self_attn.{p}_proj.bias") for p in "qkv"])

    def per(name):
        return _stack(layers, lambda i: st.value(f"{lay(i)}.{name}"))

    return {
        "vision_patch_embedding_w":
            st.value(f"{VISION}.embeddings.patch_embedding.weight").permute(2, 3, 1, 0),
        "vision_patch_embedding_b": st.value(f"{VISION}.embeddings.patch_embedding.bias"),
        "vision_position_embedding": st.value(f"{VISION}.embeddings.position_embedding.weight"),
        "vision_attn_qkv_w": _stack(layers, qkv_w),
        "vision_attn_qkv_b": _stack(layers, qkv_b),
        "vision_attn_o_w": _stack(layers, lambda i: st.linear(f"{lay(i)}.self_attn.out_proj")),
        "vision_attn_o_b": per("self_attn.out_proj.bias"),
        "vision_ffn_up_w": _stack(layers, lambda i: st.linear(f"{lay(i)}.mlp.fc1")),
        "vision_ffn_up_b": per("mlp.fc1.bias"),
        "vision_ffn_down_w": _stack(layers, lambda i: st.linear(f"{lay(i)}.mlp.fc2")),
        "vision_ffn_down_b": per("mlp.fc2.bias"),
        "vision_pre_attn_norm_w": per("layer_norm1.weight"),
        "vision_pre_attn_norm_b": per("layer_norm1.bias"),
        "vision_pre_ffn_norm_w": per("layer_norm2.weight"),
        "vision_pre_ffn_norm_b": per("layer_norm2.bias"),
        "vision_final_norm_w": st.value(f"{VISION}.post_layernorm.weight"),
        "vision_final_norm_b": st.value(f"{VISION}.post_layernorm.bias"),
    }


def _count_vision_layers(tensors) -> int:
    n = 0
    while f"{VISION}.encoder.layers.{n}.self_attn.q_proj.weight" in tensors:
        n += 1
    return n


def convert_state_dict(tensors, strict: bool = True, steps: int = spec.NUM_STEPS,
                       dt: float = EULER_DT, compute_dtype=torch.float32,
                       out_dtype=torch.bfloat16) -> dict[str, torch.Tensor]:
    """OpenPI Pi0 state dict (name -> tensor) -> packed bf16 checkpoint.

    Layer counts and widths are read from the tensors. `strict=True` checks
    the result against the Pi0 schema (`spec.weight_shapes(prompt_len=0)`),
    as the reference does (`openpi.py:303-311`); `strict=False` accepts
    reduced models (used by the tests). Folding runs in `compute_dtype` (fp32,
    as the reference) and every tensor is rounded once to `out_dtype`.
    """
    st = _State(tensors, compute_dtype)
    out = _vision(st, _count_vision_layers(tensors))
    out["encoder_multi_modal_projector_w"] = st.linear(PROJECTOR)
    out["encoder_multi_modal_projector_b"] = st.value(f"{PROJECTOR}.bias")

    enc = _gemma_params(st, ENCODER, st.count_layers(ENCODER))
    qkv, o_w, gate, up, down = fold_gemma_layers(enc)
    out.update({"encoder_attn_qkv_w": qkv, "encoder_attn_o_w": o_w, "encoder_ffn_gate_w": gate,
                "encoder_ffn_up_w": up, "encoder_ffn_down_w": down})

    dec = _gemma_params(st, DECODER, st.count_layers(DECODER))
    dec.update({
        "state_proj_w": st.linear("state_proj"), "state_proj_b": st.value("state_proj.bias"),
        "action_in_w": st.linear("action_in_proj"), "action_in_b": st.value("action_in_proj.bias"),
        "time_mlp_in_w": st.linear("action_time_mlp_in"),
        "time_mlp_in_b": st.value("action_time_mlp_in.bias"),
        "time_mlp_out_w": st.linear("action_time_mlp_out"),
        "time_mlp_out_b": st.value("action_time_mlp_out.bias"),
        "action_out_w": st.linear("action_out_proj"),
        "action_out_b": st.value("action_out_proj.bias"),
        "final_norm_w": st.value(f"{DECODER}.norm.weight"),
    })
    packed = {k: v.to(out_dtype).contiguous() for k, v in out.items()}
    packed.update(fold_decoder(dec, steps=steps, dt=dt, out_dtype=out_dtype))
    width = packed["encoder_multi_modal_projector_w"].shape[1]
    packed["language_embeds"] = torch.empty(0, width, dtype=out_dtype)

    if strict:
        expected = spec.weight_shapes(prompt_len=0)
        if set(packed) != set(expected):
            missing = sorted(set(expected) - set(packed))
            extra = sorted(set(packed) - set(expected))
            raise ValueError(f"packed checkpoint keys do not match: missing={missing}, extra={extra}")
        for name, shape in expected.items():
            if tuple(packed[name].shape) != shape:
                raise ValueError(f"{name} has shape {tuple(packed[name].shape)}, expected {shape}")
    return packed


def load_openpi_state(checkpoint: str | Path) -> dict[str, torch.Tensor]:
    """Tensors of a local OpenPI `model.safetensors` (a file or its directory)."""
    from safetensors import safe_open

    path = Path(checkpoint)
    if path.is_dir():
        path = path / "model.safetensors"
    if not path.is_file():
        raise FileNotFoundError(path)
    with safe_open(str(path), framework="pt", device="cpu") as f:
        return {name: f.get_tensor(name) for name in f.keys()}


def convert_checkpoint(checkpoint: str | Path, device: str = "cpu",
                       strict: bool = True) -> dict[str, torch.Tensor]:
    """Load a local OpenPI checkpoint and return the packed schema on `device`."""
    packed = convert_state_dict(load_openpi_state(checkpoint), strict=strict)
    return {k: v.to(device) for k, v in packed.items()}


def error_metrics(reference: torch.Tensor, output: torch.Tensor) -> dict[str, float]:
    """max_abs, mean_abs, rms_error, p99_abs and cosine_similarity of `output` against
    `reference` (`openpi_parity.py:14-28`)."""
    if reference.shape != output.shape:
        raise ValueError(f"shape mismatch: reference={reference.shape}, output={output.shape}")
    ref = reference.float().flatten()
    out = output.float().flatten()
    err = (out - ref).abs()
    return {
        "max_abs": err.max().item(),
        "mean_abs": err.mean().item(),
        "rms_error": torch.sqrt(torch.mean((out - ref) ** 2)).item(),
        "p99_abs": torch.quantile(err, 0.99).item(),
        "cosine_similarity": F.cosine_similarity(ref, out, dim=0).item(),
    }


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description="Convert a local OpenPI Pi0 checkpoint.")
    parser.add_argument("--checkpoint", required=True,
                        help="OpenPI model.safetensors or its directory")
    parser.add_argument("--out", required=True, help="packed safetensors file to write")
    args = parser.parse_args(argv)
    from safetensors.torch import save_file

    packed = convert_checkpoint(args.checkpoint)
    save_file(packed, args.out)
    print(json.dumps({"tensors": len(packed),
                      "bytes": sum(t.numel() * t.element_size() for t in packed.values())}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
