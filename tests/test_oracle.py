"""Pins the CPU oracle (oracle/pi0_decoder.py) with checks that do not retype it.

Each oracle function is tied to something independent:
  * fold + packed loop  == unfolded OpenPI-form loop, fp64 (algebraic identity);
  * RoPE                == half-split RoPE under the column permutation
                           (through the identity above) + rotation invariants;
  * attention + mask    == brute-force per-row loops in fp64, and FlashDecoding
                           split/merge gives the same result for any split count;
  * rms factor / gelu   == closed forms and special values;
  * num_splits          == the known answers stated by the reference;
  * GEMM-shaped ops     == explicit triple loops on tiny shapes;
  * Euler update        == special cases (zero weights, zero steps).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import pi0_decoder as O
from flash_vla_amd import weights as W

SMALL = dict(width=64, ffn=96, heads=2, head_dim=16, action_dim=8)


def _small_case(layers=2, enc_len=20, chunk=5, seed=3, std=0.1):
    p = W.openpi_decoder_params(seed=seed, std=std, layers=layers, dtype=torch.float64, **SMALL)
    gen = torch.Generator().manual_seed(seed + 100)
    hd = SMALL["head_dim"]
    state = torch.randn(SMALL["action_dim"], generator=gen, dtype=torch.float64)
    noise = torch.randn(chunk, SMALL["action_dim"], generator=gen, dtype=torch.float64)
    pk = torch.randn(layers, enc_len, hd, generator=gen, dtype=torch.float64)
    pv = torch.randn(layers, enc_len, hd, generator=gen, dtype=torch.float64)
    return p, state, noise, pk, pv


def _deinterleave(k):
    """Inverse of the adjacent-pair permutation on the last axis (one head)."""
    hd = k.shape[-1]
    return k.reshape(*k.shape[:-1], hd // 2, 2).transpose(-1, -2).reshape(k.shape)


@pytest.mark.parametrize("steps", [1, 3])
def test_fold_identity_fp64(steps):
    layers, enc_len, chunk = 2, 20, 5
    p, state, noise, pk, pv = _small_case(layers, enc_len, chunk)
    # unfolded explicit loop
    ref_noise, ref_x = O.decoder_unfolded(p, state, noise, _deinterleave(pk), pv,
                                          W.sinusoidal_time_embedding, steps=steps,
                                          dtype=torch.float64)
    packed = W.fold_decoder(p, out_dtype=torch.float64)
    T_ = chunk + 1
    K = torch.cat([pk, torch.zeros(layers, T_, pk.shape[-1], dtype=torch.float64)], 1)
    V = torch.cat([pv, torch.zeros(layers, T_, pv.shape[-1], dtype=torch.float64)], 1)
    rope = O.rope_table(T_, enc_len, SMALL["head_dim"], exact=True)
    got_noise, got_x, _, _ = O.decoder_packed(packed, state, noise, K, V, enc_len, steps=steps,
                                              bf16=False, dtype=torch.float64,
                                              heads=SMALL["heads"], rope=rope)
    assert torch.allclose(got_noise, ref_noise, atol=1e-10, rtol=1e-10)
    assert torch.allclose(got_x, ref_x, atol=1e-9, rtol=1e-9)


def test_fold_detects_wrong_rope_layout():
    """Without the de-interleave of the cached prefix keys the identity must fail."""
    layers, enc_len, chunk = 1, 12, 3
    p, state, noise, pk, pv = _small_case(layers, enc_len, chunk, std=0.3)
    ref_noise, _ = O.decoder_unfolded(p, state, noise, pk, pv, W.sinusoidal_time_embedding,
                                      steps=1, dtype=torch.float64)
    packed = W.fold_decoder(p, out_dtype=torch.float64)
    T_ = chunk + 1
    K = torch.cat([pk, torch.zeros(layers, T_, pk.shape[-1], dtype=torch.float64)], 1)
    V = torch.cat([pv, torch.zeros(layers, T_, pv.shape[-1], dtype=torch.float64)], 1)
    rope = O.rope_table(T_, enc_len, SMALL["head_dim"], exact=True)
    got, _, _, _ = O.decoder_packed(packed, state, noise, K, V, enc_len, steps=1, bf16=False,
                                    dtype=torch.float64, heads=SMALL["heads"], rope=rope)
    assert not torch.allclose(got, ref_noise, atol=1e-6)


def test_time_embedding_shape_and_endpoints():
    t = W.euler_times()
    assert torch.allclose(t, torch.tensor([1.0 - 0.1 * i for i in range(10)]), atol=1e-6)
    emb = W.sinusoidal_time_embedding(torch.tensor([0.0, 1.0]), 8)
    # t = 0 -> sin 0, cos 1
    assert torch.equal(emb[0], torch.tensor([0, 0, 0, 0, 1, 1, 1, 1], dtype=torch.float64))
    # first period is min_period: sin(2*pi*1/0.004) = sin(500*pi) = 0
    assert abs(emb[1, 0].item()) < 1e-9
    # last period is max_period = 4: sin(2*pi/4) = 1
    assert abs(emb[1, 3].item() - 1.0) < 1e-12


def test_time_embedding_interior_known_answers():
    """Hand-worked values at interior indices (Pi0: periods geometric from 4e-3 to 4).

    Width 8 -> 4 periods 4e-3 * 1000^(i/3) = 0.004, 0.04, 0.4, 4. At t = 0.3 the
    phases 2*pi*t/period are 150*pi, 15*pi, 1.5*pi and 0.15*pi, so
    emb = [0, 0, -1, sin(0.15 pi) | 1, -1, 0, cos(0.15 pi)]. A linear period
    spacing (0.004, 1.336, 2.668, 4) or swapped sin/cos halves fails at i = 1, 2.
    Width 14 -> periods 4e-3 * 1000^(i/6): i = 2 is 0.04, i = 3 is 4e-3 * sqrt(1000).
    """
    from openpi_form import time_embedding

    s15, c15 = math.sin(0.15 * math.pi), math.cos(0.15 * math.pi)
    want8 = torch.tensor([0.0, 0.0, -1.0, s15, 1.0, -1.0, 0.0, c15], dtype=torch.float64)
    got8 = W.sinusoidal_time_embedding(torch.tensor([0.3], dtype=torch.float64), 8)[0]
    assert torch.allclose(got8, want8, atol=1e-9), got8
    # t = 0.1: phases 50 pi, 5 pi, pi/2, 0.05 pi
    want8b = torch.tensor([0.0, 0.0, 1.0, math.sin(0.05 * math.pi),
                           1.0, -1.0, 0.0, math.cos(0.05 * math.pi)], dtype=torch.float64)
    got8b = W.sinusoidal_time_embedding(torch.tensor([0.1], dtype=torch.float64), 8)[0]
    assert torch.allclose(got8b, want8b, atol=1e-9), got8b
    got14 = W.sinusoidal_time_embedding(torch.tensor([0.3], dtype=torch.float64), 14)[0]
    assert abs(got14[2].item() - 0.0) < 1e-9 and abs(got14[7 + 2].item() + 1.0) < 1e-9
    ph3 = 2 * math.pi * 0.3 / (4e-3 * math.sqrt(1000.0))
    assert math.isclose(got14[3].item(), math.sin(ph3), abs_tol=1e-12)
    assert math.isclose(got14[7 + 3].item(), math.cos(ph3), abs_tol=1e-12)
    # the OpenPI-form test reference uses the same law
    assert torch.allclose(time_embedding(0.3, 8), want8, atol=1e-9)
    # and the packed schema's fp32 time grid reaches t = 0.3 at step 7 (fp32 accumulation)
    assert abs(W.euler_times()[7].item() - 0.3) < 1e-6


def test_rope_table_values():
    tab = O.rope_table(3, 768, 256, exact=True)
    # pair 0 has inv_freq 1: (cos 768, sin 768)
    assert math.isclose(tab[0, 0].item(), math.cos(768), abs_tol=1e-12)
    assert math.isclose(tab[0, 1].item(), math.sin(768), abs_tol=1e-12)
    # last pair: inv_freq = 10000^(-254/256)
    f = 10000 ** (-254 / 256)
    assert math.isclose(tab[2, 255].item(), math.sin(770 * f), abs_tol=1e-12)
    assert O.rope_table(3, 768, 256).dtype == torch.bfloat16


def test_rope_invariants():
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(4, 3 * 32, generator=gen, dtype=torch.float64)
    tab = O.rope_table(4, 0, 32, exact=True)
    y = O.rope_interleaved(x, tab)
    # position 0 is the identity
    assert torch.allclose(y[0], x[0])
    # pair norms are preserved
    n0 = x.reshape(4, -1, 2).norm(dim=-1)
    n1 = y.reshape(4, -1, 2).norm(dim=-1)
    assert torch.allclose(n0, n1)
    # relative-position property: <R_a q, R_b k> depends on b - a only
    q = torch.randn(1, 32, generator=gen, dtype=torch.float64)
    k = torch.randn(1, 32, generator=gen, dtype=torch.float64)
    t1 = O.rope_table(8, 0, 32, exact=True)
    t2 = O.rope_table(8, 100, 32, exact=True)
    d1 = (O.rope_interleaved(q, t1[2:3]) * O.rope_interleaved(k, t1[5:6])).sum()
    d2 = (O.rope_interleaved(q, t2[2:3]) * O.rope_interleaved(k, t2[5:6])).sum()
    assert torch.allclose(d1, d2)


def test_rms_factor_closed_forms():
    x = torch.zeros(2, 1024)
    x[1] = 3.0
    f = O.rms_factor(x)
    assert f.dtype == torch.float32
    assert f[0].item() == 1000.0                 # rsqrt(1e-6), exactly representable in bf16
    assert f[1].item() == torch.tensor(1 / math.sqrt(9 + 1e-6)).bfloat16().float().item()
    g = torch.randn(5, 64, dtype=torch.float64)
    exact = 1.0 / torch.sqrt((g ** 2).mean(-1) + 1e-6)
    assert torch.allclose(O.rms_factor(g, bf16=False), exact)


def test_gelu_matches_tanh_gelu():
    v = torch.linspace(-8, 8, 2001, dtype=torch.float64)
    assert torch.allclose(O.gelu_tanh(v), F.gelu(v, approximate="tanh"), atol=1e-12)
    assert torch.allclose(O.silu(v), F.silu(v))


def _attention_bruteforce(q, k, v, enc_len, heads):
    rows, hd = q.shape
    out = torch.zeros_like(q)
    for r in range(rows):
        keys = [j for j in range(k.shape[0]) if r >= heads or j <= enc_len]
        s = torch.tensor([float((q[r] * k[j]).sum()) / math.sqrt(hd) for j in keys],
                         dtype=torch.float64)
        p = torch.exp(s - s.max())
        p = p / p.sum()
        for pj, j in zip(p, keys):
            out[r] += pj * v[j]
    return out


def _attention_split(q, k, v, enc_len, heads, n_split):
    """FlashDecoding: per-chunk normalised partials merged by log-sum-exp."""
    hd = q.shape[1]
    keys = k.shape[0]
    chunk = -(-keys // n_split)
    mask = O.attention_mask(q.shape[0], keys, enc_len, heads)
    parts, lses = [], []
    for s0 in range(0, keys, chunk):
        sc = (q @ k[s0:s0 + chunk].t()) / math.sqrt(hd)
        sc = sc.masked_fill(~mask[:, s0:s0 + chunk], float("-inf"))
        m = sc.max(-1, keepdim=True).values.clamp_min(-1e300)
        p = torch.exp(sc - m)
        l = p.sum(-1, keepdim=True)
        parts.append((p @ v[s0:s0 + chunk]) / l.clamp_min(1e-300))
        lses.append(torch.where(l > 0, m + torch.log(l.clamp_min(1e-300)),
                                torch.full_like(l, -1e300)))
    lse = torch.cat(lses, 1)
    wts = torch.softmax(lse, dim=1)
    return sum(wts[:, i:i + 1] * parts[i] for i in range(len(parts)))


def test_attention_bruteforce_and_mask():
    gen = torch.Generator().manual_seed(1)
    heads, T_, enc_len, hd = 2, 4, 9, 8
    q = torch.randn(T_ * heads, hd, generator=gen, dtype=torch.float64)
    k = torch.randn(enc_len + T_, hd, generator=gen, dtype=torch.float64)
    v = torch.randn(enc_len + T_, hd, generator=gen, dtype=torch.float64)
    got = O.op_attention(q, k, v, enc_len, heads, bf16=False)
    assert torch.allclose(got, _attention_bruteforce(q, k, v, enc_len, heads))
    # state rows see exactly enc_len + 1 keys: equal to attention over the truncated cache
    trunc = O.op_attention(q[:heads], k[:enc_len + 1], v[:enc_len + 1], enc_len, heads,
                           bf16=False)
    assert torch.allclose(got[:heads], trunc)
    assert int(O.attention_mask(16, 819, 768, 8)[:8].sum(1).unique().item()) == 769
    assert int(O.attention_mask(16, 819, 768, 8)[8:].sum(1).unique().item()) == 819


@pytest.mark.parametrize("n_split", [1, 2, 3, 7, 13])
def test_attention_split_invariance(n_split):
    gen = torch.Generator().manual_seed(2)
    heads, T_, enc_len, hd = 8, 6, 40, 16
    q = torch.randn(T_ * heads, hd, generator=gen, dtype=torch.float64)
    k = torch.randn(enc_len + T_, hd, generator=gen, dtype=torch.float64)
    v = torch.randn(enc_len + T_, hd, generator=gen, dtype=torch.float64)
    ref = O.op_attention(q, k, v, enc_len, heads, bf16=False)
    assert torch.allclose(_attention_split(q, k, v, enc_len, heads, n_split), ref)


def test_num_splits_known_answers():
    # fused_wrappers.py:77-78: keys=819 keeps the tuned 7 splits, keys=1075 selects 6
    assert O.num_splits(819, 64, 7) == (7, 2)
    assert O.num_splits(1075, 64, 7)[0] == 6
    assert O.num_splits(867, 64, 7) == (7, 2)
    for keys in range(1, 2000, 37):
        n, cb = O.num_splits(keys, 64, 7)
        assert (n - 1) * cb * 64 < keys          # no empty split
        assert n * cb * 64 >= keys               # every key covered


def _loop_matmul(x, w):
    M, K = x.shape
    N = w.shape[1]
    out = torch.zeros(M, N, dtype=torch.float64)
    for m in range(M):
        for n in range(N):
            out[m, n] = sum(float(x[m, k]) * float(w[k, n]) for k in range(K))
    return out


def test_gemm_ops_bruteforce():
    gen = torch.Generator().manual_seed(4)
    d = torch.float64
    x = torch.randn(3, 8, generator=gen, dtype=d)
    w = torch.randn(8, 5, generator=gen, dtype=d)
    b = torch.randn(5, generator=gen, dtype=d)
    r = torch.randn(3, 5, generator=gen, dtype=d)
    mm = _loop_matmul(x, w)
    assert torch.allclose(O.op_action_mlp(x, w, b, bf16=False), mm + b)
    assert torch.allclose(O.op_action_in_proj(x, w, b, bf16=False),
                          (mm + b) / (1 + torch.exp(-(mm + b))))
    assert torch.allclose(O.op_state_proj(x[0], w, b, bf16=False), mm[:1] + b)
    assert torch.allclose(O.op_matmul_residual(x, w, r, bf16=False), mm + r)
    f = 1.0 / torch.sqrt((x * x).mean(1) + 1e-6)
    assert torch.allclose(O.op_action_out_proj(x, w, b, r, bf16=False), r + b + mm * f[:, None])
    wu = torch.randn(8, 5, generator=gen, dtype=d)
    mu = _loop_matmul(x, wu)
    g = mm * f[:, None]
    gl = 0.5 * g * (1 + torch.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))
    assert torch.allclose(O.op_norm_gated_ffn(x, w, wu, bf16=False), gl * (mu * f[:, None]))


def test_qkv_rope_columns():
    """Q/K get rotated, V does not; flat Q row = token*heads + head."""
    gen = torch.Generator().manual_seed(5)
    heads, hd, D, T_ = 2, 8, 16, 3
    x = torch.randn(T_, D, generator=gen, dtype=torch.float64)
    w = torch.randn(D, (heads + 2) * hd, generator=gen, dtype=torch.float64)
    tab = O.rope_table(T_, 0, hd, exact=True)
    q, k, v, f = O.op_norm_qkv_rope(x, w, tab, heads, bf16=False)
    acc = _loop_matmul(x, w) * f[:, None]
    assert torch.allclose(v, acc[:, (heads + 1) * hd:])
    assert torch.allclose(q.reshape(T_, heads, hd)[0], acc[0, :heads * hd].reshape(heads, hd))
    th = tab[1]
    c, s = float(th[2]), float(th[3])     # pair 1 at position 1
    a0, a1 = acc[1, heads * hd + 2], acc[1, heads * hd + 3]
    assert math.isclose(k[1, 2].item(), a0 * c - a1 * s, abs_tol=1e-12)
    assert math.isclose(k[1, 3].item(), a1 * c + a0 * s, abs_tol=1e-12)


def test_euler_special_cases():
    layers, enc_len, chunk = 1, 10, 4
    p, state, noise, pk, pv = _small_case(layers, enc_len, chunk)
    packed = W.fold_decoder(p, out_dtype=torch.float64)
    T_ = chunk + 1
    K = torch.cat([pk, torch.zeros(layers, T_, pk.shape[-1], dtype=torch.float64)], 1)
    V = torch.cat([pv, torch.zeros(layers, T_, pv.shape[-1], dtype=torch.float64)], 1)
    n0, _, _, _ = O.decoder_packed(packed, state, noise, K, V, enc_len, steps=0, bf16=False,
                                   dtype=torch.float64, heads=SMALL["heads"])
    assert torch.equal(n0, noise)
    z = dict(packed)
    z["decoder_action_fused_out_proj_w"] = torch.zeros_like(z["decoder_action_fused_out_proj_w"])
    z["decoder_action_fused_out_proj_b"] = torch.zeros_like(z["decoder_action_fused_out_proj_b"])
    n1, _, _, _ = O.decoder_packed(z, state, noise, K, V, enc_len, steps=3, bf16=False,
                                   dtype=torch.float64, heads=SMALL["heads"])
    assert torch.equal(n1, noise)


def test_bf16_mode_close_to_fp32_small():
    layers, enc_len, chunk = 2, 20, 5
    p, state, noise, pk, pv = _small_case(layers, enc_len, chunk, std=0.05)
    packed = W.fold_decoder(p)
    T_ = chunk + 1
    K = torch.cat([pk, torch.zeros(layers, T_, pk.shape[-1], dtype=torch.float64)], 1)
    V = torch.cat([pv, torch.zeros(layers, T_, pv.shape[-1], dtype=torch.float64)], 1)
    a, _, _, _ = O.decoder_packed(packed, state, noise, K, V, enc_len, steps=2, bf16=True,
                                  heads=SMALL["heads"])
    b, _, _, _ = O.decoder_packed(packed, state, noise, K, V, enc_len, steps=2, bf16=False,
                                  heads=SMALL["heads"])
    assert (a - b).abs().max() < 3e-2


# ---------------------------------------------------------------------------
# Unfused call sites (op_table(fused=False))
# ---------------------------------------------------------------------------
def test_unfused_loop_equals_fused_without_rounding_fp64():
    """Without bf16 rounding the unfused and fused plans are the same function: the whole
    unfolded-vs-packed identity above then pins the unfused ops too (a dropped factor, a
    wrong mask fill or a transposed operand breaks the equality)."""
    layers, enc_len, chunk = 2, 20, 5
    p, state, noise, pk, pv = _small_case(layers, enc_len, chunk)
    packed = W.fold_decoder(p, out_dtype=torch.float64)
    T_ = chunk + 1
    K = torch.cat([pk, torch.zeros(layers, T_, pk.shape[-1], dtype=torch.float64)], 1)
    V = torch.cat([pv, torch.zeros(layers, T_, pv.shape[-1], dtype=torch.float64)], 1)
    kw = dict(steps=3, bf16=False, dtype=torch.float64, heads=SMALL["heads"])
    a = O.decoder_packed(packed, state, noise, K, V, enc_len, unfused=False, **kw)[0]
    b = O.decoder_packed(packed, state, noise, K, V, enc_len, unfused=True, **kw)[0]
    assert torch.allclose(a, b, atol=1e-11, rtol=1e-11)


def test_unfused_attention_brute_force_fp64():
    """Unfused attention without rounding == per-row loops with explicit mask; with
    rounding, P rows sum to 1 within bf16 rounding and masked keys get exactly 0."""
    g = torch.Generator().manual_seed(71)
    heads, T_, enc, hd = 2, 3, 5, 8
    q = torch.randn(T_ * heads, hd, generator=g, dtype=torch.float64)
    k = torch.randn(enc + T_, hd, generator=g, dtype=torch.float64)
    v = torch.randn(enc + T_, hd, generator=g, dtype=torch.float64)
    out, _ = O.op_attention_unfused(q, k, v, enc, heads, bf16=False)
    for r in range(q.shape[0]):
        keys = [j for j in range(k.shape[0]) if r >= heads or j <= enc]
        s = [sum(q[r, d] * k[j, d] for d in range(hd)) / math.sqrt(hd) for j in keys]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        z = sum(e)
        ref = [sum(e[i] / z * v[j, d] for i, j in enumerate(keys)) for d in range(hd)]
        assert torch.allclose(out[r], torch.tensor(ref, dtype=torch.float64), atol=1e-12)
    _, p = O.op_attention_unfused(q.float(), k.float(), v.float(), enc, heads, bf16=True)
    assert torch.all(p[:heads, enc + 1:] == 0)
    assert torch.allclose(p.sum(-1), torch.ones(p.shape[0]), atol=2e-2)


def test_unfused_rounding_points_known_answers():
    """Hand-worked values of the unfused rounding points.

    Gate / out-proj: x = 1 + 2^-7 in every column of a 256-wide row gives
    f = bf16(1/sqrt(1.0156..+1e-6)) = 0.9921875 and x*f = 0.99993896484375, which bf16 rounds
    to 1.0. With W = e_0 the unfused gate is bf16(gelu(1) * 1); with W = all ones and an fp32
    destination the unfused out-projection is exactly 256 while the fused one (factor on the
    fp32 accumulator) is 0.9921875 * 258 = 255.984375.
    Scores: q.k = 1.00390625 (1 + 2^-8) with hd = 1 is not a bf16 value and rounds to 1.0 (ties
    to even) before the softmax."""
    K = 256
    x = torch.full((1, K), 1.0 + 2.0 ** -7)
    f = O.rms_factor(x, True)
    assert f.item() == 0.9921875
    wg = torch.zeros(K, 1)
    wg[0, 0] = 1.0
    wu = wg.clone()
    out, _ = O.op_norm_gated_ffn_unfused(x, wg, wu, bf16=True)
    assert out.item() == O._bf(O.gelu_tanh(torch.tensor(1.0)) * 1.0, True).item()
    r = torch.zeros(1, 1)
    b = torch.zeros(1)
    ones = torch.ones(K, 1)
    assert O.op_action_out_proj_unfused(x, ones, b, r, bf16=True, round_out=False).item() == 256.0
    fused_fp32 = (x @ ones) * f                       # the fused form's fp32 value
    assert fused_fp32.item() == 255.984375
    q = torch.tensor([[1.0]])
    kk = torch.tensor([[1.00390625], [0.0]])
    vv = torch.tensor([[2.0], [0.0]])
    o, p = O.op_attention_unfused(q, kk, vv, enc_len=1, heads=1, bf16=True)
    # S = [1.0, 0.0] after rounding: p = [e/(e+1), 1/(e+1)] rounded to bf16
    e = math.exp(1.0)
    assert p[0, 0].item() == O._bf(torch.tensor(e / (e + 1.0)), True).item()
    assert p[0, 1].item() == O._bf(torch.tensor(1.0 / (e + 1.0)), True).item()


@pytest.mark.parametrize("offset", [0, 768, 816, 1024])
def test_engine_rope_table_is_the_oracle_table_bitwise(offset):
    """The engine's RoPE operand (built on the host) is the oracle's bf16 table bit for bit."""
    from flash_vla_amd.buffers import rope_table
    for rows in (51, 204):
        assert torch.equal(rope_table(rows, offset, 256, "cpu"), O.rope_table(rows, offset, 256))
