"""CPU oracle for the Pi0 action-expert denoising loop (TEST INFRASTRUCTURE ONLY).

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg
may import this module, and only as the checker; the HIP product path never
calls it.

Two restatements of the same maths, both plain PyTorch on the CPU:

* `decoder_unfolded` -- BASELINE config 1 in its explicit OpenPI form:
  action_in_proj, sinusoidal time embedding, concat + MLP (swish), 18 Gemma
  layers with half-split RoPE, final RMSNorm, action_out_proj, x += dt * v.
* `decoder_packed` -- the reference's packed execution plan
  (`hardware/nvidia/h100/pi0/pipeline.py:92-135`) on folded weights, op by op,
  with an optional `bf16=True` mode that rounds exactly where the reference's
  fused kernels store bf16 (factor, Q/K/V, probabilities before P@V, every
  activation buffer).

Each per-op function cites the reference lines it follows. How each one is
pinned (closed forms, invariants, fp64 identities, brute force) is listed in
`tests/test_oracle.py`; the time embedding is "parity unpinned" against OpenPI
(its module is absent), see `sinusoidal_time_embedding` in the package.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

RMS_EPS = 1e-6
GELU_C0 = 1.5957691216057308   # 2*sqrt(2/pi), base.py:69
GELU_C1 = 0.044715             # base.py:70
ROPE_THETA = 10000.0


def _bf(x: torch.Tensor, on: bool) -> torch.Tensor:
    """Round to bf16 (and back to the working dtype) when `on`."""
    return x.to(torch.bfloat16).to(x.dtype) if on else x


# ---------------------------------------------------------------------------
# Elementary pieces
# ---------------------------------------------------------------------------
def rope_table(seq_len: int, offset: int, head_dim: int, exact: bool = False) -> torch.Tensor:
    """Interleaved bf16 (cos, sin) rows for positions offset.. (buffers.py:15-23).

    `exact=True` returns the same table in fp64 without rounding.
    """
    dt = torch.float64 if exact else torch.float32
    pos = torch.arange(seq_len, dtype=dt) + offset
    inv_freq = 1.0 / (ROPE_THETA ** (torch.arange(0, head_dim, 2, dtype=dt) / head_dim))
    phase = inv_freq[None, :] * pos[:, None]
    table = torch.stack([torch.cos(phase), torch.sin(phase)], dim=2).reshape(seq_len, head_dim)
    return table if exact else table.to(torch.bfloat16)


def rms_factor(x: torch.Tensor, bf16: bool = True) -> torch.Tensor:
    """f[m] = rsqrt(mean_k x^2 + 1e-6), rounded to bf16 (base.py:344-370, fused_norm.py:72)."""
    ss = (x * x).sum(dim=-1)
    return _bf(torch.rsqrt(ss / x.shape[-1] + RMS_EPS), bf16)


def gelu_tanh(v: torch.Tensor) -> torch.Tensor:
    """v * sigmoid(C0 * v * (1 + C1 v^2)) (base.py:77-78)."""
    return v * torch.sigmoid(GELU_C0 * v * (1.0 + GELU_C1 * v * v))


def silu(v: torch.Tensor) -> torch.Tensor:
    return v * torch.sigmoid(v)


def rope_interleaved(x: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """Rotate adjacent pairs (2p, 2p+1) of each head row (base.py:651-661).

    x [..., T, heads*hd] or [T, hd]; table [T, hd] interleaved (cos, sin).
    """
    T_, n = x.shape[-2], x.shape[-1]
    hd = table.shape[-1]
    t = table.to(x.dtype)
    cos = t[:, 0::2]
    sin = t[:, 1::2]
    xr = x.reshape(*x.shape[:-2], T_, n // hd, hd // 2, 2)
    x0, x1 = xr[..., 0], xr[..., 1]
    c = cos[:, None, :]
    s = sin[:, None, :]
    out = torch.stack([x0 * c - x1 * s, x1 * c + x0 * s], dim=-1)
    return out.reshape(x.shape)


def attention_mask(rows: int, keys: int, enc_len: int, heads: int) -> torch.Tensor:
    """Pi0 decoder mask on the flat (token*heads + head) query axis (base.py:858-862).

    The state token (flat rows < heads) keeps keys j <= enc_len (prefix plus
    itself); action tokens keep every key j < keys.
    """
    r = torch.arange(rows)[:, None]
    j = torch.arange(keys)[None, :]
    return (r >= heads) | (j <= enc_len)


def num_splits(keys: int, block_n: int, requested: int) -> tuple[int, int]:
    """Largest split count <= requested with no empty split (fused_wrappers.py:70-85)."""
    def chunk_blocks(n: int) -> int:
        return ((keys + n - 1) // n + block_n - 1) // block_n

    while requested > 1 and (requested - 1) * chunk_blocks(requested) * block_n >= keys:
        requested -= 1
    return requested, chunk_blocks(requested)


# ---------------------------------------------------------------------------
# Per-op restatements of the decoder wrappers (packed schema)
# ---------------------------------------------------------------------------
def op_state_proj(x, w, b, bf16=True):
    """out = x @ w + b (wrappers.py:108-112 -> base.py:158-192)."""
    wt = x.dtype
    return _bf(x.reshape(1, -1) @ w.to(wt) + b.to(wt), bf16)


def op_action_in_proj(x, w, b, bf16=True):
    """out = silu(x @ w + b) (wrappers.py:115-120 -> base.py:304-335)."""
    wt = x.dtype
    return _bf(silu(x @ w.to(wt) + b.to(wt)), bf16)


def op_action_mlp(x, w, b, bf16=True):
    """out = x @ w + b (wrappers.py:123-128)."""
    wt = x.dtype
    return _bf(x @ w.to(wt) + b.to(wt), bf16)


def op_norm_qkv_rope(x, w, rope, heads, bf16=True):
    """Q, K, V of one layer (wrappers.py:131-144 -> base.py:607-669).

    acc = (x @ W) * f in fp32 with f the bf16 rms factor; RoPE on the fp32
    accumulator for the first (heads+1)*hd columns; each output rounded once.
    Returns Q [T*heads, hd] (flat row = token*heads + head), K [T, hd], V [T, hd].
    """
    wt = x.dtype
    hd = rope.shape[-1]
    f = rms_factor(x, bf16)
    acc = (x @ w.to(wt)) * f[:, None]
    qk = rope_interleaved(acc[:, :(heads + 1) * hd], rope)
    q = _bf(qk[:, :heads * hd], bf16).reshape(-1, hd)
    k = _bf(qk[:, heads * hd:], bf16)
    v = _bf(acc[:, (heads + 1) * hd:], bf16)
    return q, k, v, f


def op_attention(q, k, v, enc_len, heads, bf16=True):
    """softmax(mask(q k^T / sqrt(hd))) v on the flat query axis (fused_wrappers.py:88-115).

    With bf16=True the probabilities are rounded to bf16 before P @ V and
    normalised afterwards, as the reference's split kernel does (base.py:879-880).
    """
    hd = q.shape[-1]
    s = (q @ k.t()) * (hd ** -0.5)
    mask = attention_mask(q.shape[0], k.shape[0], enc_len, heads)
    s = s.masked_fill(~mask, float("-inf"))
    m = s.max(dim=-1, keepdim=True).values
    p = torch.exp(s - m)
    denom = p.sum(dim=-1, keepdim=True)
    o = (_bf(p, bf16) @ v) / denom
    return _bf(o, bf16)


def op_matmul_residual(x, w, r, bf16=True):
    """out = r + x @ w in fp32, rounded once (wrappers.py:176-189 -> base.py:115-154)."""
    wt = r.dtype
    return _bf(r + x.to(wt) @ w.to(wt), bf16)


def op_norm_gated_ffn(x, wg, wu, bf16=True):
    """gelu(f*(x@Wg)) * (f*(x@Wu)) with the factor on the fp32 accumulators (fused_norm.py:26-78)."""
    wt = x.dtype
    f = rms_factor(x, bf16)[:, None]
    return _bf(gelu_tanh((x @ wg.to(wt)) * f) * ((x @ wu.to(wt)) * f), bf16)


def op_action_out_proj(x, w, b, r, bf16=True):
    """out = r + b + f * (x @ w) (fused_norm.py:81-125); x is decoder_x[1:]."""
    wt = r.dtype
    f = rms_factor(x, bf16)[:, None]
    return _bf(r + b.to(wt) + (x @ w.to(wt)) * f, bf16)


# ---------------------------------------------------------------------------
# Unfused call sites (op_table(fused=False)): the same maths with the reference's
# two-kernel rounding points
# ---------------------------------------------------------------------------
UNFUSED_MASK_NEG = -3.0e38     # tl_softmax_mask0's fill value (base.py:780)


def op_attention_unfused(q, k, v, enc_len, heads, bf16=True):
    """Unfused decoder attention (wrappers.py:147-173): S = bf16((q k^T) * hd^-0.5)
    (tl_matmul_abT_scale, base.py:737-762); row softmax of the masked S in fp32 with a
    finite fill, P = bf16(e / sum) (tl_softmax_mask0, base.py:765-798); out = bf16(P @ v)
    (tl_matmul, base.py:84-111). Returns (out, P)."""
    hd = q.shape[-1]
    s = _bf((q @ k.t()) * (hd ** -0.5), bf16)
    mask = attention_mask(q.shape[0], k.shape[0], enc_len, heads)
    s = s.masked_fill(~mask, UNFUSED_MASK_NEG)
    e = torch.exp(s - s.max(dim=-1, keepdim=True).values)
    p = _bf(e / e.sum(dim=-1, keepdim=True), bf16)
    return _bf(p @ v, bf16), p


def op_norm_gated_ffn_unfused(x, wg, wu, bf16=True):
    """Unfused gate (wrappers.py:192-198): f from tl_rms_factor (bf16), then
    a = bf16(x * f) per element before the dual GEMM (tl_scaled_gate, base.py:496-497),
    out = bf16(gelu(a @ Wg) * (a @ Wu)). Returns (out, f)."""
    wt = x.dtype
    f = rms_factor(x, bf16)
    a = _bf(x * f[:, None], bf16)
    return _bf(gelu_tanh(a @ wg.to(wt)) * (a @ wu.to(wt)), bf16), f


def op_action_out_proj_unfused(x, w, b, r, bf16=True, round_out=True):
    """Unfused Euler out-projection (wrappers.py:201-208): a = bf16(x * f) with the bf16
    factor, out = r + b + a @ W in fp32 (tl_scaled_matmul_bias_res, base.py:552-596),
    rounded when `round_out`."""
    wt = r.dtype
    f = rms_factor(x, bf16)[:, None]
    a = _bf(x * f, bf16)
    return _bf(r + b.to(wt) + a @ w.to(wt), round_out)


# ---------------------------------------------------------------------------
# Whole loops
# ---------------------------------------------------------------------------
def decoder_packed(weights: dict, state, noise, enc_k, enc_v, enc_len: int,
                   steps: int = 10, layers: int | None = None, bf16: bool = True,
                   dtype=torch.float32, heads: int = 8, trace: list | None = None,
                   rope: torch.Tensor | None = None, fp32_noise: bool = False,
                   unfused: bool = False):
    """The packed decoder loop (pipeline.py:92-135) on CPU.

    `enc_k`/`enc_v` are the [layers, enc_len + T, hd] caches whose first
    `enc_len` rows hold the prefix; the decoder rows are overwritten here (a
    copy is made, the inputs are not modified). Returns (noise, x, K, V).
    `fp32_noise=True` keeps the Euler accumulator unrounded between steps (the
    fused HIP loop does this and rounds the chunk to bf16 once at the end).
    `rope` overrides the bf16 table of `rope_table` (an exact table is used by
    the fp64 folding identity).
    If `trace` is a list, per-step (noise, x) pairs are appended.
    `unfused=True` runs the op_table(fused=False) call sites (the `*_unfused` ops).
    """
    w = {k: v.to(dtype) for k, v in weights.items()}
    n_layers = w["decoder_attn_qkv_w"].shape[0] if layers is None else layers
    K = enc_k.to(dtype).clone()
    V = enc_v.to(dtype).clone()
    noise = noise.to(dtype).clone()
    T_ = noise.shape[0] + 1
    hd = K.shape[-1]
    if rope is None:
        rope = rope_table(T_, enc_len, hd)
    rope = rope.to(dtype)
    s_buf = op_state_proj(state.to(dtype), w["decoder_state_in_proj_w"],
                          w["decoder_state_in_proj_b"], bf16)
    x = None
    for step in range(steps):
        h = op_action_in_proj(noise, w["decoder_action_fused_in_proj_w"],
                              w["decoder_action_fused_time_biases"][step % 10], bf16)
        a = op_action_mlp(h, w["decoder_action_mlp_w"], w["decoder_action_mlp_b"], bf16)
        x = torch.cat([s_buf, a], dim=0)
        for i in range(n_layers):
            q, k, v, _ = op_norm_qkv_rope(x, w["decoder_attn_qkv_w"][i], rope, heads, bf16)
            K[i, enc_len:enc_len + T_] = k
            V[i, enc_len:enc_len + T_] = v
            if unfused:
                o, _ = op_attention_unfused(q, K[i, :enc_len + T_], V[i, :enc_len + T_],
                                            enc_len, heads, bf16)
            else:
                o = op_attention(q, K[i, :enc_len + T_], V[i, :enc_len + T_], enc_len, heads,
                                 bf16)
            x = op_matmul_residual(o.reshape(T_, -1), w["decoder_attn_o_w"][i], x, bf16)
            if unfused:
                hdn, _ = op_norm_gated_ffn_unfused(x, w["decoder_ffn_gate_w"][i],
                                                   w["decoder_ffn_up_w"][i], bf16)
            else:
                hdn = op_norm_gated_ffn(x, w["decoder_ffn_gate_w"][i], w["decoder_ffn_up_w"][i],
                                        bf16)
            x = op_matmul_residual(hdn, w["decoder_ffn_down_w"][i], x, bf16)
        if unfused:
            noise = op_action_out_proj_unfused(x[1:], w["decoder_action_fused_out_proj_w"],
                                               w["decoder_action_fused_out_proj_b"], noise,
                                               bf16, bf16 and not fp32_noise)
        else:
            noise = op_action_out_proj(x[1:], w["decoder_action_fused_out_proj_w"],
                                       w["decoder_action_fused_out_proj_b"], noise,
                                       bf16 and not fp32_noise)
        if trace is not None:
            trace.append((noise.clone(), x.clone()))
    return noise, x, K, V


def _rms_norm(x, w):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + RMS_EPS) * (1.0 + w)


def _rope_half_split(x, pos, hd):
    """OpenPI rotate-half RoPE on [T, n*hd] with pair (i, i + hd/2)."""
    inv_freq = 1.0 / (ROPE_THETA ** (torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    phase = pos.to(torch.float64)[:, None] * inv_freq[None, :]
    cos = torch.cos(phase).to(x.dtype)
    sin = torch.sin(phase).to(x.dtype)
    T_, n = x.shape
    xr = x.reshape(T_, n // hd, 2, hd // 2)
    x1, x2 = xr[:, :, 0], xr[:, :, 1]
    c, s = cos[:, None], sin[:, None]
    return torch.stack([x1 * c - x2 * s, x2 * c + x1 * s], dim=2).reshape(T_, n)


def decoder_unfolded(p: dict, state, noise, prefix_k, prefix_v, time_embedding,
                     steps: int = 10, dt: float = -0.1, layers: int | None = None,
                     dtype=torch.float32):
    """the explicit OpenPI-form decoder loop, no folding, no rounding.

    `prefix_k/v` [layers, enc_len, hd] are the cached prefix keys/values (already
    rotated). `time_embedding(times, width)` supplies the sinusoidal embedding.
    RoPE here is the half-split form on unpermuted Q/K projections; attention
    positions of the decoder rows start at enc_len.
    """
    P = {k: v.to(dtype) for k, v in p.items()}
    n_layers = P["q_w"].shape[0] if layers is None else layers
    hd = prefix_k.shape[-1]
    heads = P["q_w"].shape[-1] // hd
    width = P["time_mlp_out_w"].shape[0]
    enc_len = prefix_k.shape[1]
    x_t = noise.to(dtype).clone()
    T_ = x_t.shape[0] + 1
    pos = torch.arange(T_) + enc_len
    t = torch.tensor(1.0, dtype=torch.float32)
    dt32 = torch.tensor(dt, dtype=torch.float32)
    keys = enc_len + T_
    mask = torch.ones(T_, keys, dtype=torch.bool)
    mask[0, enc_len + 1:] = False
    x = None
    for _ in range(steps):
        s_emb = state.to(dtype)[None] @ P["state_proj_w"] + P["state_proj_b"]
        a = x_t @ P["action_in_w"] + P["action_in_b"]
        temb = time_embedding(t[None], width).to(dtype).expand(a.shape[0], -1)
        h = torch.cat([a, temb], dim=1) @ P["time_mlp_in_w"] + P["time_mlp_in_b"]
        h = F.silu(h) @ P["time_mlp_out_w"] + P["time_mlp_out_b"]
        x = torch.cat([s_emb, h], dim=0)
        for i in range(n_layers):
            r = _rms_norm(x, P["input_norm_w"][i])
            q = _rope_half_split(r @ P["q_w"][i], pos, hd)
            k = _rope_half_split(r @ P["k_w"][i], pos, hd)
            v = r @ P["v_w"][i]
            K = torch.cat([prefix_k[i].to(dtype), k], dim=0)
            V = torch.cat([prefix_v[i].to(dtype), v], dim=0)
            qh = q.reshape(T_, heads, hd).transpose(0, 1)            # [H, T, hd]
            s = (qh @ K.t()) / math.sqrt(hd)
            s = s.masked_fill(~mask[None], float("-inf"))
            o = torch.softmax(s, dim=-1) @ V                        # [H, T, hd]
            x = x + o.transpose(0, 1).reshape(T_, heads * hd) @ P["o_w"][i]
            r = _rms_norm(x, P["post_attn_norm_w"][i])
            g = F.gelu(r @ P["gate_w"][i], approximate="tanh")
            x = x + (g * (r @ P["up_w"][i])) @ P["down_w"][i]
        v_t = _rms_norm(x[1:], P["final_norm_w"]) @ P["action_out_w"] + P["action_out_b"]
        x_t = x_t + dt * v_t
        t = t + dt32
    return x_t, x
