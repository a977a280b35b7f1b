"""HIP backend call-site wrappers for the Pi0 decoder.

One function per op-table entry, with the reference's signatures
(`backends/tilelang/wrappers.py:108-221`, `fused_wrappers.py:45-122`): tensors
in, destinations written in place, return value = the destination. Each
wrapper checks dtype / layout / shape on the host, maps tensors to raw
pointers and calls one C-ABI entry point of libpi0hip.so on the current
stream. Nothing here allocates after warmup: workspaces come from the active
ScratchPool and packed weights from the packed-weight cache, both filled
during warmup and frozen before capture.
"""
from __future__ import annotations

import contextlib
import weakref

import torch

from ...arena import ScratchPool
from . import _abi

DECODER_HEADS = 8
# Above one 64-row block (the batched decoder, M = B x 51) the decoder's GEMMs run on the
# prefix encoder's tile kernel: the skinny kernel would stream the weights once per row block.
_TILE_M = 64
_POOL = ScratchPool()


def set_pool(pool: ScratchPool) -> None:
    global _POOL
    _POOL = pool


@contextlib.contextmanager
def use_pool(pool: ScratchPool):
    """Route scratch allocation through `pool` (as `wrappers.py:42-51` of the reference)."""
    global _POOL
    previous = _POOL
    _POOL = pool
    try:
        yield
    finally:
        _POOL = previous


def scratch(role: str, shape, dtype, device) -> torch.Tensor:
    return _POOL.get(role, shape, dtype, device)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _capturing() -> bool:
    return torch.cuda.is_current_stream_capturing()


def _check(t: torch.Tensor, name: str, ndim: int | None = None, allow_f32: bool = False) -> None:
    if t.dtype != torch.bfloat16 and not (allow_f32 and t.dtype == torch.float32):
        raise TypeError(f"{name}: expected bfloat16, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name}: expected a GPU tensor")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name}: expected {ndim} dims, got shape {tuple(t.shape)}")
    if t.dim() >= 1 and t.stride(-1) != 1:
        raise ValueError(f"{name}: last dimension must be contiguous")


def _ptr(t: torch.Tensor):
    return t.data_ptr()


# ---------------------------------------------------------------------------
# Packed weights: the kernels stream W[K, N] in MFMA B-fragment order. A weight
# is packed once (a whole [L, K, N] stack at a time when it is a layer view)
# and looked up by address on every later call.
# ---------------------------------------------------------------------------
class _PackedEntry:
    """Packed copy of one source weight. The tensor that owns the source's storage
    (typically an engine's [L, K, N] stack) is held by weak reference: when it is freed,
    the entry and its packed copy are dropped with it, so the cache never keeps a model
    alive. The source itself (possibly a view, e.g. a reshape) is re-derived from the
    owner when it is needed."""
    __slots__ = ("owner_ref", "view", "packed", "base", "nbytes", "K", "N", "version", "layout",
                 "pad", "__weakref__")

    def __init__(self, src, packed, K, N, layout, pad):
        self.packed, self.K, self.N, self.layout, self.pad = packed, K, N, layout, pad
        self.base = src.data_ptr()
        self.nbytes = src.numel() * src.element_size()
        self.version = src._version
        owner = src if src._base is None else src._base
        self.view = (tuple(src.shape), tuple(src.stride()), src.storage_offset())
        self.owner_ref = weakref.ref(owner, self._drop)

    @property
    def src(self):
        owner = self.owner_ref()
        if owner is None:
            return None
        shape, stride, offset = self.view
        return owner.as_strided(shape, stride, offset)

    def _drop(self, _ref) -> None:
        if _PACKED is None:           # interpreter shutdown: module globals already cleared
            return
        try:
            _PACKED.remove(self)
        except ValueError:
            pass


_PACKED: list[_PackedEntry] = []


_PACKERS = {16: "pi0hip_pack_weight", 32: "pi0hip_pack_weight32"}


def _pack_into(src: torch.Tensor, dst: torch.Tensor, K: int, N: int, layout: int, pad) -> None:
    batch = src.numel() // (K * N)
    if pad is not None:
        _abi.call("pi0hip_pack_weight32_padded", _ptr(src), _ptr(dst), K, N, pad[0], pad[1], batch,
                  _stream())
    else:
        _abi.call(_PACKERS[layout], _ptr(src), _ptr(dst), K, N, batch, _stream())


def packed_weight_ptr(w: torch.Tensor, layout: int = 16, pad: tuple | None = None) -> int:
    """Device address of the packed copy of `w` ([K, N] bf16, possibly a layer view).

    layout 16: the decoder kernels' 32 k x 16 n fragments (pi0hip_pack_weight);
    layout 32: the encoder kernels' 16 k x 32 n fragments (pi0hip_pack_weight32);
    pad = (K_pad, N_pad): layout 32 zero-padded to whole tiles (pi0hip_pack_weight32_padded)."""
    _check(w, "weight", 2)
    if not w.is_contiguous():
        raise ValueError("weight must be contiguous [K, N]")
    K, N = w.shape
    if pad is not None:
        pad = (int(pad[0]), int(pad[1]))
        if layout != 32 or pad == (K, N):
            pad = None if pad == (K, N) else pad
        if pad is not None and (pad[0] < K or pad[1] < N):
            raise ValueError("padding smaller than the weight")
    def packed_offset(byte_off: int) -> int:
        """Byte offset in the packed copy of the weight at `byte_off` in the source stack:
        the same for unpadded layouts; for padded ones layer i of [L, K, N] starts at
        i * K_pad * N_pad elements (integer arithmetic: a float ratio can land a byte off)."""
        if pad is None:
            return byte_off
        layer_bytes = K * N * w.element_size()
        if byte_off % layer_bytes:
            raise ValueError("a padded weight must be a whole layer of its stack")
        return byte_off // layer_bytes * pad[0] * pad[1] * w.element_size()
    ptr = w.data_ptr()
    for e in list(_PACKED):     # a copy: a weakref callback may remove entries meanwhile
        if (e.K == K and e.N == N and e.layout == layout and e.pad == pad
                and e.base <= ptr < e.base + e.nbytes):
            src = e.src
            if src is None:
                continue
            if not _capturing() and e.version != src._version:
                _pack_into(src, e.packed, K, N, layout, pad)
                e.version = src._version
            return e.packed.data_ptr() + packed_offset(ptr - e.base)
    if _capturing():
        raise RuntimeError("weight was not packed before graph capture; run a warmup pass first")
    base = w._base if w._base is not None else w
    src = base if (base.dim() >= 2 and base.is_contiguous() and tuple(base.shape[-2:]) == (K, N)
                   and base.dtype == w.dtype) else w
    if pad is None:
        packed = torch.empty_like(src)
    else:
        packed = torch.empty(src.numel() // (K * N) * pad[0] * pad[1], dtype=src.dtype,
                             device=src.device)
    _pack_into(src, packed, K, N, layout, pad)
    entry = _PackedEntry(src, packed, K, N, layout, pad)
    _PACKED.append(entry)
    return packed.data_ptr() + packed_offset(ptr - entry.base)


def prepare_weights(weights: dict) -> None:
    """Pack every GEMM weight stack of the model up front (outside any capture)."""
    plan = {name: (16, None) for name in (
        "decoder_action_mlp_w", "decoder_attn_qkv_w", "decoder_attn_o_w", "decoder_ffn_gate_w",
        "decoder_ffn_up_w", "decoder_ffn_down_w", "decoder_action_fused_out_proj_w")}
    plan.update({name: (32, None) for name in (
        "encoder_multi_modal_projector_w", "encoder_attn_qkv_w", "encoder_attn_o_w",
        "encoder_ffn_gate_w", "encoder_ffn_up_w", "encoder_ffn_down_w",
        "vision_attn_qkv_w", "vision_attn_o_w")})
    plan["vision_ffn_up_w"] = (32, (1152, 4352))
    plan["vision_ffn_down_w"] = (32, (4352, 1152))
    for name, (layout, pad) in plan.items():
        if name in weights:
            w = weights[name]
            packed_weight_ptr(w if w.dim() == 2 else w[0], layout, pad)
    if "vision_patch_embedding_w" in weights:
        packed_weight_ptr(weights["vision_patch_embedding_w"].reshape(588, 1152), 32, (640, 1152))


def clear_packed_cache() -> None:
    _PACKED.clear()


def packed_cache_bytes() -> int:
    """Device bytes held by live packed copies."""
    return sum(e.packed.numel() * e.packed.element_size() for e in list(_PACKED)
               if e.src is not None)


def pin_packed_weights(weights) -> list:
    """Strong references to the packed copies of `weights` (an engine's tensors).

    A captured graph reads packed copies at fixed addresses. The cache itself holds
    each source weakly and drops the copy with it, so an engine keeps the list this
    returns for as long as its graph lives: then a source that is replaced rather
    than updated in place leaves the graph reading stale but valid memory, and
    `check_pinned` reports it."""
    spans = [(t.data_ptr(), t.data_ptr() + t.numel() * t.element_size()) for t in weights]
    return [e for e in list(_PACKED)
            if any(lo <= e.base < hi for lo, hi in spans)]


def check_pinned(pinned: list, weights) -> None:
    """Raise if a pinned copy's source is no longer one of `weights`' storages (the
    engine's weight was replaced by another tensor instead of updated in place)."""
    live = {t.untyped_storage().data_ptr() for t in weights}
    for e in pinned:
        src = e.src
        if src is None or src.untyped_storage().data_ptr() not in live:
            raise RuntimeError(
                "an engine weight was replaced rather than updated in place; the captured "
                "graph still reads the old packed copy. Update weights in place "
                "(engine.weights[name].copy_(new)) or build a new engine")


def repack_stale() -> int:
    """Re-pack, in place, every packed copy whose source weight changed since it was packed
    (outside graph capture). A captured graph reads the packed copies at fixed addresses,
    so after updating an engine's weights in place this makes replays use the new values.
    Returns the number of copies refreshed."""
    if _capturing():
        raise RuntimeError("repack_stale() cannot run during graph capture")
    n = 0
    for e in list(_PACKED):
        src = e.src
        if src is not None and src._version != e.version:
            _pack_into(src, e.packed, e.K, e.N, e.layout, e.pad)
            e.version = src._version
            n += 1
    return n


def _splitk(M: int, N: int, K: int, target: int = 256) -> int:
    """Split K across workgroups until the grid covers the 256 CUs, and at least until each
    wave's K range fits the kernel's unrolled widths (1..8 fragments of 32)."""
    tiles = ((M + 63) // 64) * (N // 16)
    kt = K // 32
    s = 1
    while (tiles * s < target or kt // (4 * s) > 8) and kt % (4 * s * 2) == 0:
        s *= 2
    return s


def _gemm_ws(role: str, M: int, N: int, splitk: int, dual: int, device):
    nbytes = _abi.lib().pi0hip_gemm_workspace_bytes(M, N, splitk, dual)
    if nbytes == 0:
        return None, 0
    buf = scratch(role, (nbytes,), torch.uint8, device)
    return buf.data_ptr(), nbytes


# ---------------------------------------------------------------------------
# Decoder call sites (pipeline.py:92-135 calls these by name)
# ---------------------------------------------------------------------------
def decoder_state_proj(x, weight, bias, out):
    """out = x @ weight + bias for the state token(s) (wrappers.py:108-112); x [32] or [B, 32]."""
    _check(x, "x"); _check(weight, "weight", 2); _check(bias, "bias", 1); _check(out, "out", 2)
    K, N = weight.shape
    B = out.shape[0]
    if x.numel() != B * K or out.shape != (B, N) or bias.shape != (N,) or not x.is_contiguous():
        raise ValueError("decoder_state_proj: shape mismatch")
    _abi.call("pi0hip_small_linear", _ptr(x), K, _ptr(weight), _ptr(bias), _ptr(out),
              out.stride(0), B, N, K, 0, _stream())
    return out


def decoder_action_in_proj(x, weight, bias, out):
    """out = silu(x @ weight + bias) (wrappers.py:115-120); x may be the fp32 noise accumulator."""
    _check(x, "x", 2, allow_f32=True); _check(weight, "weight", 2); _check(bias, "bias", 1)
    _check(out, "out", 2)
    M, K = x.shape
    N = weight.shape[1]
    if weight.shape[0] != K or out.shape != (M, N) or bias.shape != (N,):
        raise ValueError("decoder_action_in_proj: shape mismatch")
    fn = "pi0hip_small_linear_f32x" if x.dtype == torch.float32 else "pi0hip_small_linear"
    _abi.call(fn, _ptr(x), x.stride(0), _ptr(weight), _ptr(bias), _ptr(out), out.stride(0),
              M, N, K, 1, _stream())
    return out


def decoder_action_mlp(x, weight, bias, out):
    """out = x @ weight + bias, out = decoder_x[1:] (wrappers.py:123-128)."""
    _check(x, "x", 2); _check(bias, "bias", 1); _check(out, "out", 2)
    M, K = x.shape
    N = weight.shape[1]
    if weight.shape[0] != K or out.shape != (M, N) or bias.shape != (N,):
        raise ValueError("decoder_action_mlp: shape mismatch")
    wp = packed_weight_ptr(weight)
    s = _splitk(M, N, K)
    ws, nbytes = _gemm_ws("gemm_ws_mlp", M, N, s, 0, x.device)
    _abi.call("pi0hip_linear_bias", _ptr(x), x.stride(0), wp, _ptr(bias), _ptr(out),
              out.stride(0), M, N, K, s, ws, nbytes, _stream())
    return out


def decoder_norm_qkv_rope(x, weight_qkv, rope, Q, K, V, norm_factor):
    """RMS factor, QKV projection, RoPE, scatter into Q and the K/V cache rows (wrappers.py:131-144).

    Batched form: K / V are [requests, T + 1, head_dim] views of the
    per-request caches and x holds the requests' rows "states first" (the requests'
    state tokens, then each request's actions)."""
    _check(x, "x", 2); _check(rope, "rope", 2); _check(Q, "Q", 2)
    batch = K.shape[0] if K.dim() == 3 else 1
    K2, V2 = (K[0], V[0]) if K.dim() == 3 else (K, V)
    _check(K2, "K", 2); _check(V2, "V", 2)
    M, Kdim = x.shape
    head_dim = V2.shape[1]
    heads = Q.shape[0] // M
    rows = K2.shape[0]
    if (Q.shape != (M * heads, head_dim) or not Q.is_contiguous() or M != batch * rows
            or V.shape != K.shape or K2.stride(0) != V2.stride(0) or K.stride() != V.stride()
            or weight_qkv.shape != (Kdim, (heads + 2) * head_dim)
            or rope.shape[0] < rows or rope.shape[1] != head_dim or not rope.is_contiguous()):
        raise ValueError("decoder_norm_qkv_rope: shape mismatch")
    nf = 0
    if norm_factor is not None:
        _check(norm_factor, "norm_factor", 1)
        if norm_factor.shape[0] < M:
            raise ValueError("norm_factor too short")
        nf = _ptr(norm_factor)
    wp = packed_weight_ptr(weight_qkv)
    if batch == 1:
        _abi.call("pi0hip_norm_qkv_rope", _ptr(x), x.stride(0), wp, _ptr(rope), _ptr(Q), _ptr(K2),
                  _ptr(V2), K2.stride(0), nf, M, Kdim, heads, head_dim, _stream())
    else:
        _abi.call("pi0hip_norm_qkv_rope_batched", _ptr(x), x.stride(0), wp, _ptr(rope), _ptr(Q),
                  _ptr(K2), _ptr(V2), K2.stride(0), K.stride(0), nf, M, Kdim, heads, head_dim,
                  batch, _stream())


def decoder_attention(Q, K, V, scores, out, encoder_seq_len):
    """Masked single-KV-head attention; `out` may be `Q`, `scores` is unused (fused_wrappers.py:88-115).

    Batched form: K / V are [requests, keys, head_dim]; Q holds each request's query rows
    request-major and `out` receives them in the "states first" token order."""
    _check(Q, "Q", 2); _check(out, "out", 2)
    batch = K.shape[0] if K.dim() == 3 else 1
    K2, V2 = (K[0], V[0]) if K.dim() == 3 else (K, V)
    _check(K2, "K", 2); _check(V2, "V", 2)
    rows, head_dim = Q.shape
    keys = K2.shape[0]
    if (V.shape != K.shape or K2.shape[1] != head_dim or out.shape != Q.shape
            or K2.stride(0) != V2.stride(0) or K.stride() != V.stride() or rows % batch):
        raise ValueError("decoder_attention: shape mismatch")
    lib = _abi.lib()
    per = rows // batch
    nbytes = lib.pi0hip_attention_batched_workspace_bytes(per, keys, batch)
    ws = scratch("attn_ws", (nbytes,), torch.uint8, Q.device)
    _abi.call("pi0hip_attention_batched", _ptr(Q), Q.stride(0), _ptr(K2), _ptr(V2), K2.stride(0),
              K.stride(0) if batch > 1 else 0, _ptr(out), out.stride(0), per, keys,
              int(encoder_seq_len), DECODER_HEADS, head_dim, batch, ws.data_ptr(), nbytes,
              _stream())
    return out


def _consumer_slices(M: int, ld: int, addr: int, w) -> int:
    """Slices of packed `w` such that slice s is what workgroup s of its residual GEMM
    reads (and so lands on XCD s % 8) when its input is [M, K] with row pitch `ld` at
    `addr`: row-split -> one column tile per slice (the tile's workgroups sit on XCD
    nt % 8); split-K -> the (N / 16) x splitk K-slices. The choice is `_residual`'s own
    predicate on the same operand."""
    Kw, Nw = w.shape
    return (Nw // 16) * (1 if _rows_ok_for(M, ld, addr, Kw, Nw) else _splitk(M, Nw, Kw))


def decoder_attention_prefetch(Q, K, V, scores, out, encoder_seq_len, gate_w, up_w, down_w,
                               down_x=None):
    """`decoder_attention` whose spare workgroups also pull this layer's gate / up and
    down weights into the L2 of the XCDs that will read them (pi0hip_attention_prefetch).
    (Prefetching the o-proj's weights here, or the down's from spare workgroups of the
    o-proj launch, measured slower: the o-proj is bound by its CUs' load path.)

    Engine-level option of this backend, not a reference call site: the reference's
    decoder_attention (fused_wrappers.py:88-115) prefetches nothing. The result is bitwise
    that of decoder_attention. Used for one request whose GEMMs take the skinny kernels,
    where workgroup s of the gate / up launch reads packed tile s and the residual GEMMs'
    workgroups read the slices `_consumer_slices` describes; otherwise it is plain
    decoder_attention. `down_x` is the down projection's input (the GeGLU activations);
    without it an [M, K] row-major operand at a 16-byte aligned address is assumed."""
    rows = Q.shape[0]
    M = rows // DECODER_HEADS
    if K.dim() == 3 or M > _TILE_M:
        return decoder_attention(Q, K, V, scores, out, encoder_seq_len)
    _check(Q, "Q", 2); _check(out, "out", 2); _check(K, "K", 2); _check(V, "V", 2)
    keys, head_dim = K.shape
    if (V.shape != K.shape or head_dim != Q.shape[1] or out.shape != Q.shape
            or K.stride(0) != V.stride(0)):
        raise ValueError("decoder_attention: shape mismatch")
    regions = []
    for w in (gate_w, up_w):
        regions += [packed_weight_ptr(w), w.numel() * 2, w.shape[1] // 16]
    ld, addr = (down_w.shape[0], 0) if down_x is None else (down_x.stride(0), down_x.data_ptr())
    regions += [packed_weight_ptr(down_w), down_w.numel() * 2,
                _consumer_slices(M, ld, addr, down_w)]
    regions += [None, 0, 0]
    lib = _abi.lib()
    nbytes = lib.pi0hip_attention_batched_workspace_bytes(rows, keys, 1)
    ws = scratch("attn_ws", (nbytes,), torch.uint8, Q.device)
    _abi.call("pi0hip_attention_prefetch", _ptr(Q), Q.stride(0), _ptr(K), _ptr(V), K.stride(0),
              _ptr(out), out.stride(0), rows, keys, int(encoder_seq_len), DECODER_HEADS, head_dim,
              ws.data_ptr(), nbytes, *regions, _stream())
    return out


def attention_prefetch_for(attention_op):
    """The prefetching form of `attention_op` if it is this backend's decoder_attention."""
    return decoder_attention_prefetch if attention_op is decoder_attention else None


def _rows_ok_for(M: int, ld: int, addr: int, K: int, N: int) -> bool:
    """The row-split kernel's shape rules (pi0hip_linear_residual_rows) for an [M, K]
    operand with row pitch `ld` elements at device address `addr`."""
    return (RESIDUAL_MODE == "rows" and M <= _TILE_M and K in (512, 1024, 2048, 4096)
            and N % 16 == 0 and ld % 8 == 0 and addr % 16 == 0)


def _rows_ok(x, K: int, N: int) -> bool:
    return _rows_ok_for(x.shape[0], x.stride(0), x.data_ptr(), K, N)


# Residual GEMMs at M <= 64: "rows" = one launch of 16-row workgroups over the whole K
# (pi0hip_linear_residual_rows); "splitk" = split-K partials + a reduce launch.
RESIDUAL_MODE = "rows"


def _residual(x, weight, out, role):
    _check(x, "x", 2); _check(out, "out", 2)
    M, K = x.shape
    N = weight.shape[1]
    if weight.shape[0] != K or out.shape != (M, N):
        raise ValueError(f"{role}: shape mismatch")
    if _rows_ok(x, K, N):
        _abi.call("pi0hip_linear_residual_rows", _ptr(x), x.stride(0), packed_weight_ptr(weight),
                  _ptr(out), out.stride(0), M, N, K, _stream())
        return out
    if M > _TILE_M and K % 256 == 0 and N % 128 == 0:
        s = 4
        nbytes = _abi.lib().pi0hip_tile_workspace_bytes(M, N, s)
        ws = scratch(f"tile_ws_{role}", (nbytes,), torch.uint8, x.device)
        _abi.call("pi0hip_tile_linear_residual", _ptr(x), x.stride(0), packed_weight_ptr(weight, 32),
                  _ptr(out), out.stride(0), M, N, K, s, ws.data_ptr(), nbytes, _stream())
        return out
    wp = packed_weight_ptr(weight)
    s = _splitk(M, N, K)
    ws, nbytes = _gemm_ws(f"gemm_ws_{role}", M, N, s, 0, x.device)
    _abi.call("pi0hip_linear_residual", _ptr(x), x.stride(0), wp, _ptr(out), out.stride(0),
              M, N, K, s, ws, nbytes, _stream())
    return out


def decoder_out_proj_residual(x, weight, out):
    """out += x @ weight (wrappers.py:176-181)."""
    return _residual(x, weight, out, "o_proj")


def decoder_ffn_down_residual(x, weight, out):
    """out += x @ weight (wrappers.py:184-189)."""
    return _residual(x, weight, out, "ffn_down")


def _gated_ffn(x, gate_w, up_w, out):
    _check(x, "x", 2); _check(out, "out", 2)
    M, K = x.shape
    N = gate_w.shape[1]
    if gate_w.shape != (K, N) or up_w.shape != (K, N) or out.shape != (M, N):
        raise ValueError("decoder_norm_gated_ffn: shape mismatch")
    if M > _TILE_M and K % 128 == 0 and N % 128 == 0:
        _abi.call("pi0hip_tile_norm_gated_ffn", _ptr(x), x.stride(0), packed_weight_ptr(gate_w, 32),
                  packed_weight_ptr(up_w, 32), _ptr(out), out.stride(0), M, N, K, _stream())
        return out
    gp = packed_weight_ptr(gate_w)
    up = packed_weight_ptr(up_w)
    _abi.call("pi0hip_norm_gated_ffn", _ptr(x), x.stride(0), gp, up, _ptr(out), out.stride(0),
              M, N, K, _stream())
    return out


def decoder_norm_gated_ffn(x, gate_w, up_w, out, norm_factor):
    """out = gelu(f * x@Wg) * (f * x@Wu), f computed in-kernel (fused_norm.py:26-78)."""
    return _gated_ffn(x, gate_w, up_w, out)


def _action_out(x, weight, bias, out):
    _check(x, "x", 2); _check(bias, "bias", 1); _check(out, "out", 2, allow_f32=True)
    M, K = x.shape
    N = weight.shape[1]
    if weight.shape[0] != K or out.shape != (M, N) or bias.shape != (N,):
        raise ValueError("decoder_action_out_proj: shape mismatch")
    wp = packed_weight_ptr(weight)
    s = _splitk(M, N, K)
    ws, nbytes = _gemm_ws("gemm_ws_out", M, N, s, 0, x.device)
    fn = ("pi0hip_rms_linear_bias_residual_f32" if out.dtype == torch.float32
          else "pi0hip_rms_linear_bias_residual")
    _abi.call(fn, _ptr(x), x.stride(0), wp, _ptr(bias), _ptr(out), out.stride(0), M, N, K, s, ws,
              nbytes, _stream())
    return out


def decoder_action_out_proj(x, weight, bias, out, norm_factor):
    """Euler update out += bias + f * x@W (fused_norm.py:81-125); `norm_factor` untouched."""
    return _action_out(x, weight, bias, out)


# ---------------------------------------------------------------------------
# Unfused call sites: op_table(fused=False) (the reference's wrappers.py:147-173, 192-208).
# Same signatures; the reference's two-kernel rounding points.
# ---------------------------------------------------------------------------
def _rms_factor(x, norm_factor):
    """norm_factor[:M] = bf16(rsqrt(mean(x^2) + 1e-6)) (wrappers.py:101-105)."""
    _check(norm_factor, "norm_factor", 1)
    M, K = x.shape
    if norm_factor.shape[0] < M:
        raise ValueError("norm_factor too short")
    _abi.call("pi0hip_rms_factor", _ptr(x), x.stride(0), _ptr(norm_factor), M, K, _stream())
    return norm_factor


def decoder_norm_gated_ffn_unfused(x, gate_w, up_w, out, norm_factor):
    """out = gelu(bf16(x*f) @ Wg) * (bf16(x*f) @ Wu), f written to norm_factor first
    (wrappers.py:192-198 -> tl_rms_factor + tl_scaled_gate, base.py:453-505)."""
    _check(x, "x", 2); _check(out, "out", 2)
    M, K = x.shape
    N = gate_w.shape[1]
    if gate_w.shape != (K, N) or up_w.shape != (K, N) or out.shape != (M, N):
        raise ValueError("decoder_norm_gated_ffn: shape mismatch")
    _rms_factor(x, norm_factor)
    _abi.call("pi0hip_scaled_gated_ffn", _ptr(x), x.stride(0), _ptr(norm_factor),
              packed_weight_ptr(gate_w), packed_weight_ptr(up_w), _ptr(out), out.stride(0),
              M, N, K, _stream())
    return out


def decoder_action_out_proj_unfused(x, weight, bias, out, norm_factor):
    """Euler update out += bias + bf16(x*f) @ W, f written to norm_factor first
    (wrappers.py:201-208 -> tl_rms_factor + tl_scaled_matmul_bias_res, base.py:552-596)."""
    _check(x, "x", 2); _check(bias, "bias", 1); _check(out, "out", 2, allow_f32=True)
    M, K = x.shape
    N = weight.shape[1]
    if weight.shape[0] != K or out.shape != (M, N) or bias.shape != (N,):
        raise ValueError("decoder_action_out_proj: shape mismatch")
    _rms_factor(x, norm_factor)
    wp = packed_weight_ptr(weight)
    s = _splitk(M, N, K)
    ws, nbytes = _gemm_ws("gemm_ws_out", M, N, s, 0, x.device)
    fn = ("pi0hip_scaled_linear_bias_residual_f32" if out.dtype == torch.float32
          else "pi0hip_scaled_linear_bias_residual")
    _abi.call(fn, _ptr(x), x.stride(0), _ptr(norm_factor), wp, _ptr(bias), _ptr(out),
              out.stride(0), M, N, K, s, ws, nbytes, _stream())
    return out


def decoder_attention_unfused(Q, K, V, scores, out, encoder_seq_len):
    """softmax_mask0(Q K^T * scale) @ V with the bf16 score matrix materialised in scratch
    and the bf16 probabilities in `scores` ([rows, keys]); `out` may be `Q`
    (wrappers.py:147-173). One request only, as in the reference."""
    _check(Q, "Q", 2); _check(out, "out", 2)
    if K.dim() != 2:
        raise ValueError("the unfused decoder attention takes one request (K [keys, head_dim])")
    _check(K, "K", 2); _check(V, "V", 2)
    if scores is None:
        raise ValueError("the unfused decoder attention needs the [rows, keys] scores buffer")
    _check(scores, "scores", 2)
    rows, head_dim = Q.shape
    keys = K.shape[0]
    if (V.shape != K.shape or K.shape[1] != head_dim or out.shape != Q.shape
            or K.stride(0) != V.stride(0) or scores.shape[0] < rows or scores.shape[1] < keys):
        raise ValueError("decoder_attention: shape mismatch")
    raw = scratch("attn_scores", (rows, keys), torch.bfloat16, Q.device)
    _abi.call("pi0hip_attention_unfused", _ptr(Q), Q.stride(0), _ptr(K), _ptr(V), K.stride(0),
              _ptr(raw), raw.stride(0), _ptr(scores), scores.stride(0), _ptr(out), out.stride(0),
              rows, keys, int(encoder_seq_len), DECODER_HEADS, head_dim, _stream())
    return out


DECODER_WRAPPERS = {
    "decoder_state_proj": decoder_state_proj,
    "decoder_action_in_proj": decoder_action_in_proj,
    "decoder_action_mlp": decoder_action_mlp,
    "decoder_norm_qkv_rope": decoder_norm_qkv_rope,
    "decoder_attention": decoder_attention,
    "decoder_out_proj_residual": decoder_out_proj_residual,
    "decoder_ffn_down_residual": decoder_ffn_down_residual,
    "decoder_norm_gated_ffn": decoder_norm_gated_ffn,
    "decoder_action_out_proj": decoder_action_out_proj,
}

# op_table(fused=False): the unfused forms at the three call sites the reference's fused
# overlay replaces (backends/tilelang/fused_wrappers.py:118-122)
ALL_WRAPPERS = dict(DECODER_WRAPPERS)
ALL_WRAPPERS.update({
    "decoder_norm_gated_ffn": decoder_norm_gated_ffn_unfused,
    "decoder_action_out_proj": decoder_action_out_proj_unfused,
    "decoder_attention": decoder_attention_unfused,
})

# op_table(fused=True) overlay, the names and semantics of the reference's fused overlay
# (backends/tilelang/fused_wrappers.py:45-122): the gated FFN and the Euler out-projection
# form their RMS factor inside the GEMM from its own A fragments and apply it to the fp32
# accumulators (fused_norm.py:26-125); the attention keeps its score matrix inside the
# kernel and ignores `scores` (base.py:801-923)
FUSED_WRAPPERS = {
    "decoder_norm_gated_ffn": decoder_norm_gated_ffn,
    "decoder_action_out_proj": decoder_action_out_proj,
    "decoder_attention": decoder_attention,
}
