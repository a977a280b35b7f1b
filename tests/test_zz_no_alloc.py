"""The allocation-free decoder attention entry point (pi0hip_attention_noalloc) against the
workspace-taking one (pi0hip_attention), through the C ABI: same kernels, so the outputs
must be bitwise equal. Two calls in a row, the second with a smaller shape, so the second
reads a static scratch array the first left full; and a shape beyond the array's size is
rejected without a launch. Each stream has its own scratch slot: two streams running at
once both match, and streams beyond the slots are rejected."""
import pytest
import torch

from flash_vla_amd.backends.hip import _abi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rnd(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16).to(DEV)


def _case(rows, keys, seed):
    q, k, v = _rnd((rows, 256), seed), _rnd((keys, 256), seed + 1), _rnd((keys, 256), seed + 2)
    return q, k, v, torch.full((rows, 256), 7.0, dtype=torch.bfloat16, device=DEV)


def _reference(q, k, v, rows, keys, enc):
    lib = _abi.lib()
    out_ref = torch.zeros(rows, 256, dtype=torch.bfloat16, device=DEV)
    nbytes = lib.pi0hip_attention_workspace_bytes(rows, keys)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    _abi.call("pi0hip_attention", q.data_ptr(), 256, k.data_ptr(), v.data_ptr(), 256,
              out_ref.data_ptr(), 256, rows, keys, enc, 8, 256, ws.data_ptr(), nbytes,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out_ref


def _noalloc(q, k, v, out, rows, keys, enc, stream):
    return _abi.lib().pi0hip_attention_noalloc(q.data_ptr(), 256, k.data_ptr(), v.data_ptr(),
                                               256, out.data_ptr(), 256, rows, keys, enc, 8,
                                               256, stream)


def _run_both(rows, keys, enc, seed):
    q, k, v, out_new = _case(rows, keys, seed)
    out_ref = _reference(q, k, v, rows, keys, enc)
    assert _noalloc(q, k, v, out_new, rows, keys, enc,
                    torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    return out_ref, out_new


def test_noalloc_attention_matches_the_workspace_entry_point():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    print("noalloc attention: rows 408 keys 1075, then rows 24 keys 100", flush=True)
    a_ref, a_new = _run_both(408, 1075, 1024, 11)     # 9 key chunks: fills most of the array
    assert torch.isfinite(a_ref.float()).all()
    assert torch.equal(a_ref, a_new)
    b_ref, b_new = _run_both(24, 100, 60, 21)        # smaller, over the previous contents
    assert torch.equal(b_ref, b_new)
    c_ref, c_new = _run_both(408, 819, 768, 31)      # the decoder's shape (7 chunks)
    assert torch.equal(c_ref, c_new)


def test_noalloc_attention_rejects_shapes_beyond_its_scratch():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    lib = _abi.lib()
    limit = lib.pi0hip_attention_noalloc_max_bytes()
    assert lib.pi0hip_attention_workspace_bytes(408, 2048) <= limit
    assert lib.pi0hip_attention_workspace_bytes(2048, 2048) > limit
    q = torch.zeros(2048, 256, dtype=torch.bfloat16, device=DEV)
    rc = lib.pi0hip_attention_noalloc(q.data_ptr(), 256, q.data_ptr(), q.data_ptr(), 256,
                                      q.data_ptr(), 256, 2048, 2048, 1997, 8, 256,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == -3      # PI0HIP_ERR_WORKSPACE, nothing launched


def test_noalloc_attention_streams_have_their_own_scratch():
    """Two streams at once on the decoder's shape, different inputs: each matches the
    workspace entry point (shared scratch would mix their partials). Then fresh streams
    until the slots run out: the next one is rejected, the accepted ones keep working."""
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    lib = _abi.lib()
    slots = lib.pi0hip_attention_noalloc_streams()
    assert slots >= 2
    print(f"noalloc attention: 2 concurrent streams, then up to {slots + 1} streams",
          flush=True)
    rows, keys, enc = 408, 819, 768
    cases = [_case(rows, keys, 41), _case(rows, keys, 51)]
    refs = [_reference(q, k, v, rows, keys, enc) for q, k, v, _ in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]   # default priority
    torch.cuda.synchronize()
    for rep in range(3):
        for (q, k, v, out), st in zip(cases, streams):
            out.fill_(7.0)
        torch.cuda.synchronize()
        for (q, k, v, out), st in zip(cases, streams):
            assert _noalloc(q, k, v, out, rows, keys, enc, st.cuda_stream) == 0
        torch.cuda.synchronize()
        for (_, _, _, out), ref in zip(cases, refs):
            assert torch.equal(out, ref), f"replay {rep}"

    # fresh streams until one is rejected; a rejected call launches nothing
    q, k, v, out = cases[0]
    extra, rejected = [], False
    for _ in range(slots + 1):
        st = torch.cuda.Stream()
        out.fill_(7.0)
        torch.cuda.synchronize()
        rc = _noalloc(q, k, v, out, rows, keys, enc, st.cuda_stream)
        torch.cuda.synchronize()
        if rc == -3:                                       # PI0HIP_ERR_WORKSPACE
            assert (out.float() == 7.0).all()
            rejected = True
            break
        assert rc == 0 and torch.equal(out, refs[0])
        extra.append(st)
    assert rejected and len(extra) <= slots - 2
    for st in streams + extra:                             # slots are kept
        out.fill_(7.0)
        torch.cuda.synchronize()
        assert _noalloc(q, k, v, out, rows, keys, enc, st.cuda_stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, refs[0])
