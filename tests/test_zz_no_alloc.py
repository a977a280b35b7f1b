"""The allocation-free decoder attention entry point (pi0hip_attention_noalloc) against the
workspace-taking one (pi0hip_attention), through the C ABI: same kernels, so the outputs
must be bitwise equal. Two calls in a row, the second with a smaller shape, so the second
reads a static scratch array the first left full; and a shape beyond the array's size is
rejected without a launch."""
import pytest
import torch

from flash_vla_amd.backends.hip import _abi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rnd(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16).to(DEV)


def _run_both(rows, keys, enc, seed):
    lib = _abi.lib()
    stream = torch.cuda.current_stream().cuda_stream
    q, k, v = _rnd((rows, 256), seed), _rnd((keys, 256), seed + 1), _rnd((keys, 256), seed + 2)
    out_ref = torch.zeros(rows, 256, dtype=torch.bfloat16, device=DEV)
    out_new = torch.full((rows, 256), 7.0, dtype=torch.bfloat16, device=DEV)
    nbytes = lib.pi0hip_attention_workspace_bytes(rows, keys)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    _abi.call("pi0hip_attention", q.data_ptr(), 256, k.data_ptr(), v.data_ptr(), 256,
              out_ref.data_ptr(), 256, rows, keys, enc, 8, 256, ws.data_ptr(), nbytes, stream)
    _abi.call("pi0hip_attention_noalloc", q.data_ptr(), 256, k.data_ptr(), v.data_ptr(), 256,
              out_new.data_ptr(), 256, rows, keys, enc, 8, 256, stream)
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
