"""Measurement probe (not part of the library): this library's tile GEMMs against the vendor
GEMM that torch.mm / torch.addmm dispatch to on ROCm (hipBLASLt / rocBLAS), at the prefix
encoder's and the vision tower's shapes (M = 768) and at the decoder's (M = 51, through the
backend's call-site wrappers, fused epilogues included). Each call site is captured 4 x 18 times in one
hipGraph, cycling 18 weight matrices (so the weights stream from HBM as in the model), and the
median over 20 replays is printed per call.

Ours include their epilogues (residual, bias, GELU, GeGLU); the vendor calls include the
residual (addmm, beta = 1) but not the bias / activation, and the gated FFN's vendor form is one
GEMM over the concatenated gate / up weights without the GeGLU.

    python3 flash-vla_amd/probes/vendor_gemm.py
"""
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(HERE)]

import torch  # noqa: E402

from flash_vla_amd.arena import ScratchPool  # noqa: E402
from flash_vla_amd.backends.hip import _abi  # noqa: E402
from flash_vla_amd.backends.hip import wrappers as W  # noqa: E402

LAYERS = 18


def time_graph(run):
    """Median microseconds per call of run(i), captured LAYERS x 4 times in one graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(LAYERS):
            run(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(LAYERS * 4):
            run(i)
    ts = []
    for _ in range(20):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b) * 1000 / (LAYERS * 4))
    return statistics.median(ts)


def weights(K, N, scale=0.02):
    return [(torch.randn(K, N, device="cuda") * scale).to(torch.bfloat16) for _ in range(LAYERS)]


def row(name, M, K, N, ours, vendor):
    flops = 2 * M * K * N
    print(f"| {name} | {M} x {K} x {N} | {ours:.1f} | {flops / ours / 1e6:.0f} | {vendor:.1f} | "
          f"{flops / vendor / 1e6:.0f} |", flush=True)


def main():
    torch.manual_seed(0)
    print("| call site | M x K x N | ours us | ours TFLOP/s | vendor us | vendor TFLOP/s |")
    print("|---|---|---:|---:|---:|---:|")
    with W.use_pool(ScratchPool()):
        M = 768
        # encoder ffn-down + residual (split-K 4 + reduce) and o-proj + residual
        for name, K, N, splitk in (("encoder ffn-down + residual", 16384, 2048, 4),
                                   ("encoder o-proj + residual", 2048, 2048, 1)):
            x = (torch.randn(M, K, device="cuda")).to(torch.bfloat16)
            ws_t = weights(K, N)
            out = torch.randn(M, N, device="cuda").to(torch.bfloat16)
            packed = [W.packed_weight_ptr(w, 32) for w in ws_t]
            nbytes = _abi.lib().pi0hip_tile_workspace_bytes(M, N, splitk)
            ws = W.scratch(f"probe_ws_{name}", (max(nbytes, 1),), torch.uint8, x.device)
            ours = time_graph(lambda i: _abi.call(
                "pi0hip_tile_linear_residual", x.data_ptr(), K, packed[i % LAYERS], out.data_ptr(), N,
                M, N, K, splitk, ws.data_ptr() if nbytes else None, nbytes, W._stream()))
            vendor = time_graph(lambda i: torch.addmm(out, x, ws_t[i % LAYERS], out=out))
            row(name, M, K, N, ours, vendor)
        # encoder QKV shape as a plain GEMM (ours: the tile kernel without its RoPE epilogue)
        K, N = 2048, 2560
        x = (torch.randn(M, K, device="cuda")).to(torch.bfloat16)
        ws_t = weights(K, N)
        out = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        packed = [W.packed_weight_ptr(w, 32) for w in ws_t]
        ours = time_graph(lambda i: _abi.call("pi0hip_tile_linear", x.data_ptr(), K, packed[i % LAYERS],
                                              None, out.data_ptr(), N, M, N, K, W._stream()))
        vendor = time_graph(lambda i: torch.mm(x, ws_t[i % LAYERS], out=out))
        row("encoder QKV shape (plain)", M, K, N, ours, vendor)
        # encoder gated FFN: ours with GeGLU; vendor one GEMM over [gate | up]
        K, N = 2048, 16384
        x = (torch.randn(M, K, device="cuda")).to(torch.bfloat16)
        wg, wu = weights(K, N), weights(K, N)
        wcat = [torch.cat([g, u], dim=1) for g, u in zip(wg, wu)]
        out = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        out2 = torch.empty(M, 2 * N, device="cuda", dtype=torch.bfloat16)
        pg = [W.packed_weight_ptr(w, 32) for w in wg]
        pu = [W.packed_weight_ptr(w, 32) for w in wu]
        ours = time_graph(lambda i: _abi.call("pi0hip_tile_gated_ffn", x.data_ptr(), K, pg[i % LAYERS],
                                              pu[i % LAYERS], out.data_ptr(), N, M, N, K, W._stream()))
        vendor = time_graph(lambda i: torch.mm(x, wcat[i % LAYERS], out=out2))
        row("encoder gate / up (+ GeGLU for ours)", M, K, 2 * N, ours, vendor)
        # vision FFN-down + bias + residual, FFN-up + bias + GELU, o-proj + bias + residual
        for name, K, N, K_pad, N_pad, kind in (
                ("vision FFN-down + bias + residual", 4304, 1152, 4352, 1152, "res"),
                ("vision FFN-up + bias + GELU", 1152, 4304, 1152, 4352, "gelu"),
                ("vision o-proj + bias + residual", 1152, 1152, 1152, 1152, "res")):
            x = (torch.randn(M, K_pad, device="cuda")).to(torch.bfloat16)
            ws_t = weights(K, N)
            b = (torch.randn(N, device="cuda") * 0.1).to(torch.bfloat16)
            out = torch.randn(M, N, device="cuda").to(torch.bfloat16)
            packed = [W.packed_weight_ptr(w, 32, (K_pad, N_pad)) for w in ws_t]
            if kind == "res":
                ours = time_graph(lambda i: _abi.call(
                    "pi0hip_tile_linear_bias_res", x.data_ptr(), K_pad, packed[i % LAYERS], b.data_ptr(),
                    out.data_ptr(), N, 0, out.data_ptr(), N, M, N, K, N_pad, K_pad, W._stream()))
                vendor = time_graph(lambda i: torch.addmm(out, x[:, :K], ws_t[i % LAYERS], out=out))
            else:
                ours = time_graph(lambda i: _abi.call(
                    "pi0hip_tile_linear_bias_gelu", x.data_ptr(), K_pad, packed[i % LAYERS], b.data_ptr(),
                    out.data_ptr(), N, M, N, K, N_pad, K_pad, W._stream()))
                vendor = time_graph(lambda i: torch.mm(x[:, :K], ws_t[i % LAYERS], out=out))
            row(name, M, K, N, ours, vendor)
        # decoder call sites at M = 51 (config 2): ours fused (RMS factor, RoPE, GeGLU, residual)
        M = 51
        x = (torch.randn(M, 1024, device="cuda")).to(torch.bfloat16)
        wq = weights(1024, 2560)
        rope = torch.ones(M, 256, device="cuda", dtype=torch.bfloat16)
        q = torch.empty(M * 8, 256, device="cuda", dtype=torch.bfloat16)
        kc = torch.empty(M, 256, device="cuda", dtype=torch.bfloat16)
        vc = torch.empty(M, 256, device="cuda", dtype=torch.bfloat16)
        nf = torch.empty(M, device="cuda", dtype=torch.bfloat16)
        outq = torch.empty(M, 2560, device="cuda", dtype=torch.bfloat16)
        ours = time_graph(lambda i: W.decoder_norm_qkv_rope(x, wq[i % LAYERS], rope, q, kc, vc, nf))
        vendor = time_graph(lambda i: torch.mm(x, wq[i % LAYERS], out=outq))
        row("decoder norm + QKV + RoPE", M, 1024, 2560, ours, vendor)
        wg, wu = weights(1024, 4096), weights(1024, 4096)
        wcat = [torch.cat([g, u], dim=1) for g, u in zip(wg, wu)]
        hid = torch.empty(M, 4096, device="cuda", dtype=torch.bfloat16)
        hid2 = torch.empty(M, 8192, device="cuda", dtype=torch.bfloat16)
        ours = time_graph(lambda i: W.decoder_norm_gated_ffn(x, wg[i % LAYERS], wu[i % LAYERS], hid, None))
        vendor = time_graph(lambda i: torch.mm(x, wcat[i % LAYERS], out=hid2))
        row("decoder norm + gate / up + GeGLU", M, 1024, 8192, ours, vendor)
        for name, K in (("decoder o-proj + residual", 2048), ("decoder ffn-down + residual", 4096)):
            xa = (torch.randn(M, K, device="cuda")).to(torch.bfloat16)
            wr = weights(K, 1024)
            res = torch.randn(M, 1024, device="cuda").to(torch.bfloat16)
            ours = time_graph(lambda i: W.decoder_out_proj_residual(xa, wr[i % LAYERS], res))
            vendor = time_graph(lambda i: torch.addmm(res, xa, wr[i % LAYERS], out=res))
            row(name, M, K, 1024, ours, vendor)
        # attention against torch's scaled_dot_product_attention (one KV head, expanded)
        import flash_vla_amd.backends.hip.encoder_wrappers as EW
        F = torch.nn.functional
        print("\n| attention | shape | ours us | vendor us |\n|---|---|---:|---:|")
        q = (torch.randn(408, 256, device="cuda")).to(torch.bfloat16)
        k = (torch.randn(819, 256, device="cuda")).to(torch.bfloat16)
        v = (torch.randn(819, 256, device="cuda")).to(torch.bfloat16)
        o = torch.empty_like(q)
        mask = torch.ones(408, 819, dtype=torch.bool, device="cuda")
        mask[:8, 769:] = False                         # the state token's rows see the prefix + itself
        q4 = q.view(51, 8, 256).transpose(0, 1).unsqueeze(0)
        k4, v4 = k.view(1, 1, 819, 256).expand(1, 8, 819, 256), v.view(1, 1, 819, 256).expand(1, 8, 819, 256)
        m4 = mask.view(51, 8, 819).transpose(0, 1).unsqueeze(0)
        ours = time_graph(lambda i: W.decoder_attention(q, k, v, None, o, 768))
        vendor = time_graph(lambda i: F.scaled_dot_product_attention(q4, k4, v4, attn_mask=m4))
        print(f"| decoder (merge launch included, no prefetch) | 51 tokens x 8 heads, 819 keys | {ours:.1f} | {vendor:.1f} |")
        q = (torch.randn(6144, 256, device="cuda")).to(torch.bfloat16)
        k = (torch.randn(768, 256, device="cuda")).to(torch.bfloat16)
        v = (torch.randn(768, 256, device="cuda")).to(torch.bfloat16)
        q4 = q.view(768, 8, 256).transpose(0, 1).unsqueeze(0)
        k4, v4 = k.view(1, 1, 768, 256).expand(1, 8, 768, 256), v.view(1, 1, 768, 256).expand(1, 8, 768, 256)
        ours = time_graph(lambda i: EW.encoder_attention(q, k, v, 256 ** -0.5))
        vendor = time_graph(lambda i: F.scaled_dot_product_attention(q4, k4, v4))
        print(f"| encoder (K / V fragment pre-pass included) | 768 tokens x 8 heads, 768 keys | {ours:.1f} | {vendor:.1f} |")


if __name__ == "__main__":
    main()
