"""The oracle against the committed fixtures of tests/golden/ (see make_golden.py)."""
import os

import numpy as np
import torch

from oracle import pi0_decoder as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_num_splits_fixture():
    kat = np.load(os.path.join(HERE, "num_splits_kat.npy"))
    for keys, block, req, n, cb in kat:
        assert O.num_splits(int(keys), int(block), int(req)) == (n, cb)
    # the values the reference states (fused_wrappers.py:77-78)
    assert tuple(kat[kat[:, 0] == 819][0, 3:]) == (7, 2)
    assert kat[kat[:, 0] == 1075][0, 3] == 6


def test_small_decoder_fixture():
    f = np.load(os.path.join(HERE, "decoder_small_fp64.npz"))
    w = {k[2:]: torch.from_numpy(f[k]) for k in f.files if k.startswith("w_")}
    enc_len = 20
    T_ = f["noise"].shape[0] + 1
    rope = O.rope_table(T_, enc_len, f["K"].shape[-1], exact=True)
    out, x, _, _ = O.decoder_packed(w, torch.from_numpy(f["state"]), torch.from_numpy(f["noise"]),
                                    torch.from_numpy(f["K"]), torch.from_numpy(f["V"]), enc_len,
                                    steps=2, bf16=False, dtype=torch.float64, heads=2, rope=rope)
    assert np.allclose(out.numpy(), f["out"], atol=1e-12, rtol=1e-12)
    assert np.allclose(x.numpy(), f["x"], atol=1e-12, rtol=1e-12)
