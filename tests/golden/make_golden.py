"""Writes the small committed fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors for the decoder path, so these are the
build's own: a reduced-width decoder (width 64, 2 heads x 16, FFN 96, 2 layers,
prefix 20 rows, chunk 5) evaluated two independent ways in fp64 (unfolded
OpenPI form and the folded packed plan), plus the split-count known answers the
reference states. tests/test_golden.py checks the oracle still reproduces them.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flash-vla_amd")]

from oracle import pi0_decoder as O  # noqa: E402
from flash_vla_amd import weights as W  # noqa: E402

DIMS = dict(width=64, ffn=96, heads=2, head_dim=16, action_dim=8)


def small_case(steps=2, layers=2, enc_len=20, chunk=5, seed=11):
    p = W.openpi_decoder_params(seed=seed, std=0.1, layers=layers, dtype=torch.float64, **DIMS)
    g = torch.Generator().manual_seed(seed + 1)
    hd = DIMS["head_dim"]
    state = torch.randn(DIMS["action_dim"], generator=g, dtype=torch.float64)
    noise = torch.randn(chunk, DIMS["action_dim"], generator=g, dtype=torch.float64)
    pk = torch.randn(layers, enc_len, hd, generator=g, dtype=torch.float64)
    pv = torch.randn(layers, enc_len, hd, generator=g, dtype=torch.float64)
    packed = W.fold_decoder(p, out_dtype=torch.float64)
    T_ = chunk + 1
    K = torch.cat([pk, torch.zeros(layers, T_, hd, dtype=torch.float64)], 1)
    V = torch.cat([pv, torch.zeros(layers, T_, hd, dtype=torch.float64)], 1)
    rope = O.rope_table(T_, enc_len, hd, exact=True)
    out, x, _, _ = O.decoder_packed(packed, state, noise, K, V, enc_len, steps=steps,
                                    bf16=False, dtype=torch.float64, heads=DIMS["heads"],
                                    rope=rope)
    return dict(state=state, noise=noise, K=K, V=V, out=out, x=x,
                **{f"w_{k}": v for k, v in packed.items()})


def main():
    case = small_case()
    np.savez_compressed(os.path.join(HERE, "decoder_small_fp64.npz"),
                        **{k: v.numpy() for k, v in case.items()})
    splits = np.array([[keys, 64, 7, *O.num_splits(keys, 64, 7)] for keys in
                       (64, 128, 819, 867, 1075, 1100, 2048)], dtype=np.int64)
    np.save(os.path.join(HERE, "num_splits_kat.npy"), splits)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
