"""ctypes binding of libpi0hip.so (the C ABI declared in include/pi0_hip.h).

The library is loaded once, from this package's `lib/` directory. There is no
fallback: if the library is missing or fails to load, every hip op raises.
"""
from __future__ import annotations

import ctypes
import os

_LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(
    os.path.abspath(__file__)))), "lib", "libpi0hip.so")

c_int, c_size_t, c_void_p, c_float = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float
P = c_void_p

# name -> (restype, argtypes); must match include/pi0_hip.h exactly.
PROTOTYPES = {
    "pi0hip_version": (c_int, []),
    "pi0hip_pack_weight": (c_int, [P, P, c_int, c_int, c_int, P]),
    "pi0hip_gemm_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "pi0hip_small_linear": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "pi0hip_small_linear_f32x": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "pi0hip_rms_linear_bias_residual_f32": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int,
                                                    c_int, P, c_size_t, P]),
    "pi0hip_linear_bias": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, c_int,
                                   P, c_size_t, P]),
    "pi0hip_linear_residual": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int,
                                       P, c_size_t, P]),
    "pi0hip_linear_residual_rows": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, P]),
    "pi0hip_rms_linear_bias_residual": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int,
                                                c_int, P, c_size_t, P]),
    "pi0hip_norm_qkv_rope": (c_int, [P, c_int, P, P, P, P, P, c_int, P, c_int, c_int, c_int,
                                     c_int, P]),
    "pi0hip_norm_gated_ffn": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, P]),
    "pi0hip_attention_workspace_bytes": (c_size_t, [c_int, c_int]),
    "pi0hip_attention": (c_int, [P, c_int, P, P, c_int, P, c_int, c_int, c_int, c_int, c_int,
                                 c_int, P, c_size_t, P]),
    "pi0hip_attention_noalloc_max_bytes": (c_size_t, []),
    "pi0hip_attention_noalloc_streams": (c_int, []),
    "pi0hip_attention_noalloc": (c_int, [P, c_int, P, P, c_int, P, c_int, c_int, c_int, c_int,
                                         c_int, c_int, P]),
    # unfused decoder call sites
    "pi0hip_rms_factor": (c_int, [P, c_int, P, c_int, c_int, P]),
    "pi0hip_scaled_gated_ffn": (c_int, [P, c_int, P, P, P, P, c_int, c_int, c_int, c_int, P]),
    "pi0hip_scaled_linear_bias_residual": (c_int, [P, c_int, P, P, P, P, c_int, c_int, c_int,
                                                   c_int, c_int, P, c_size_t, P]),
    "pi0hip_scaled_linear_bias_residual_f32": (c_int, [P, c_int, P, P, P, P, c_int, c_int, c_int,
                                                       c_int, c_int, P, c_size_t, P]),
    "pi0hip_attention_unfused": (c_int, [P, c_int, P, P, c_int, P, c_int, P, c_int, P, c_int, c_int,
                                         c_int, c_int, c_int, c_int, P]),
    # batched (config 5)
    "pi0hip_norm_qkv_rope_batched": (c_int, [P, c_int, P, P, P, P, P, c_int, ctypes.c_longlong, P,
                                             c_int, c_int, c_int, c_int, c_int, P]),
    "pi0hip_attention_batched_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "pi0hip_attention_batched": (c_int, [P, c_int, P, P, c_int, ctypes.c_longlong, P, c_int, c_int,
                                         c_int, c_int, c_int, c_int, c_int, P, c_size_t, P]),
    "pi0hip_attention_prefetch": (c_int, [P, c_int, P, P, c_int, P, c_int, c_int, c_int, c_int,
                                          c_int, c_int, P, c_size_t, P, c_size_t, c_int, P,
                                          c_size_t, c_int, P, c_size_t, c_int, P, c_size_t, c_int,
                                          P]),
    "pi0hip_tile_qkv_rope_batched": (c_int, [P, c_int, P, P, P, P, P, c_int, ctypes.c_longlong,
                                             c_int, c_int, c_int, c_int, c_int, P]),
    "pi0hip_encoder_attention_batched_workspace_bytes": (c_size_t, [c_int, c_int]),
    "pi0hip_encoder_attention_batched": (c_int, [P, c_int, P, P, c_int, ctypes.c_longlong, P, c_int,
                                                 c_int, c_int, c_int, c_float, c_int, P, c_size_t,
                                                 P]),
    "pi0hip_embed_tokens": (c_int, [P, c_int, c_int, P, c_int, c_int, c_float, P, c_int, c_int,
                                    c_int, P]),
    # prefix encoder
    "pi0hip_pack_weight32": (c_int, [P, P, c_int, c_int, c_int, P]),
    "pi0hip_pack_weight32_padded": (c_int, [P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "pi0hip_rms_norm": (c_int, [P, c_int, P, c_int, c_int, c_int, P]),
    "pi0hip_layer_norm": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_float, P]),
    "pi0hip_tile_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "pi0hip_tile_linear": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, P]),
    "pi0hip_tile_linear_residual": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int,
                                            P, c_size_t, P]),
    "pi0hip_tile_gated_ffn": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, P]),
    "pi0hip_tile_norm_gated_ffn": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, P]),
    "pi0hip_tile_qkv_rope": (c_int, [P, c_int, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int,
                                     P]),
    "pi0hip_encoder_attention_workspace_bytes": (c_size_t, [c_int]),
    "pi0hip_encoder_attention": (c_int, [P, c_int, P, P, c_int, P, c_int, c_int, c_int, c_int,
                                         c_float, P, c_size_t, P]),
    # vision tower
    "pi0hip_tile_linear_bias_res": (c_int, [P, c_int, P, P, P, c_int, c_int, P, c_int, c_int,
                                            c_int, c_int, c_int, c_int, P]),
    "pi0hip_tile_linear_bias_gelu": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int,
                                             c_int, c_int, P]),
    "pi0hip_im2col_patches": (c_int, [P, c_int, P, c_int, P]),
    "pi0hip_vision_attention_workspace_bytes": (c_size_t, [c_int, c_int]),
    "pi0hip_vision_attention": (c_int, [P, c_int, P, c_int, c_int, c_int, c_int, c_int, c_float,
                                        P, c_size_t, P]),
}

ERRORS = {-1: "invalid argument", -2: "unsupported shape", -3: "workspace missing or too small"}

_lib = None


class HipLibraryError(RuntimeError):
    pass


def library_path() -> str:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """The loaded library with prototypes applied (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise HipLibraryError(
                f"{_LIB_PATH} is not built; run `python flash-vla_amd/build_lib.py`")
        handle = ctypes.CDLL(_LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int, name: str) -> None:
    if rc != 0:
        what = ERRORS.get(rc, f"hipError_t {rc}")
        raise HipLibraryError(f"{name} failed: {what}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
