"""Measurement probe (not part of the library): the same four decoder GEMM call sites as
`persistent_chain.hip` -- norm + QKV + RoPE, o-proj + residual, norm + gated FFN, ffn-down +
residual -- for 18 layers, through the hip backend, captured in one hipGraph (one kernel per
call site), at BASELINE config 2's M = 51. Prints the median time per layer of 30 replays.

    python3 flash-vla_amd/probes/graph_chain.py
"""
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(HERE)]

import torch  # noqa: E402

from flash_vla_amd import Pi0DecoderEngine  # noqa: E402
from flash_vla_amd.pipeline import _layer_cache  # noqa: E402
from flash_vla_amd.weights import decoder_checkpoint  # noqa: E402

LAYERS, ENC = 18, 768


def main() -> None:
    ck = {k: v.cuda() for k, v in decoder_checkpoint(seed=0).items()}
    eng = Pi0DecoderEngine(ck, encoder_seq_len=ENC, capture=False, prefetch=False)
    ops, w, b = eng.ops, eng.weights, eng.buffers
    rows = b["decoder_x"].shape[0]
    dec = slice(ENC, None)

    def chain():
        for i in range(LAYERS):
            ops.decoder_norm_qkv_rope(b["decoder_x"], w["decoder_attn_qkv_w"][i],
                                      b["decoder_rope_weights"], b["decoder_q_buf"],
                                      _layer_cache(b, "encoder_K", i, dec),
                                      _layer_cache(b, "encoder_V", i, dec),
                                      b["decoder_norm_factor_buf"])
            ops.decoder_out_proj_residual(b["decoder_q_buf"].view(rows, -1),
                                          w["decoder_attn_o_w"][i], b["decoder_x"])
            ops.decoder_norm_gated_ffn(b["decoder_x"], w["decoder_ffn_gate_w"][i],
                                       w["decoder_ffn_up_w"][i], b["decoder_hidden"],
                                       b["decoder_norm_factor_buf"])
            ops.decoder_ffn_down_residual(b["decoder_hidden"], w["decoder_ffn_down_w"][i],
                                          b["decoder_x"])

    with eng.backend.use_pool(eng.pool):
        for _ in range(3):
            chain()
        torch.cuda.synchronize()
        eng.pool.freeze()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        with torch.cuda.stream(side), torch.cuda.graph(graph, stream=side):
            chain()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    for _ in range(5):
        graph.replay()
    times = []
    for _ in range(30):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    print(f"graph of the 4 decoder GEMM call sites x {LAYERS} layers: "
          f"{statistics.median(times) * 1000 / LAYERS:.2f} us per layer (median of 30)")


if __name__ == "__main__":
    main()
