"""Engines: static buffers + one hipGraph for the Pi0 denoising loop.

`Pi0DecoderEngine` mirrors the capture discipline of the reference's
`Pi0Inference` (`hardware/nvidia/h100/pi0/engine.py:26-86`): allocate every
buffer up front, copy weights in, warm up (which also fills the scratch pool
and the packed-weight cache), freeze the pool, capture one graph on a side
stream; `forward` copies the inputs into their static buffers and replays.
The prefix KV cache (the encoder's output) is supplied by the caller through
`load_prefix`; the vision and prefix-encoder stages are not part of this
engine. `Pi0EncoderEngine` is the same discipline for the prefix encoder
(`pipeline.py:57-89`): its input is the [M, 2048] encoder activation, its
output the K/V cache rows the decoder attends over.
"""
from __future__ import annotations

import torch

from . import pipeline
from .arena import ScratchPool
from .backends import BACKENDS
from .buffers import allocate_decoder_buffers, allocate_encoder_buffers, allocate_static_buffers
from .ops import op_table
from .spec import DECODER_WEIGHT_NAMES, decoder_weight_shapes, weight_shapes


def _attention_prefetch(backend, ops, enabled: bool):
    """The backend's prefetching form of the table's decoder_attention, if it has one
    (the table entry itself is left untouched, so a plan that routes decoder_attention
    elsewhere gets no prefetch)."""
    pick = getattr(backend, "attention_prefetch_for", None)
    return pick(ops.decoder_attention) if enabled and pick is not None else None


def _refresh(backend, pinned=None, weights=None) -> int:
    """Re-derive the backend's prepared (packed) weight copies from the engine's weights
    after they were updated in place; the captured graph reads the copies at fixed
    addresses, so its next replay uses the new values. Packed copies are not refreshed
    during replay: weights are frozen between refreshes. A weight replaced by another
    tensor (not updated in place) is an error: the graph cannot see it."""
    check = getattr(backend, "check_pinned", None)
    if check is not None and pinned:
        check(pinned, weights)
    fn = getattr(backend, "repack_stale", None)
    return fn() if fn is not None else 0


def _hip_runtime():
    """The HIP runtime library this process already uses (the one torch loaded)."""
    import ctypes
    import re
    with open("/proc/self/maps") as f:
        paths = sorted(set(re.findall(r"(/\S*libamdhip64\.so\S*)", f.read())))
    if not paths:
        raise RuntimeError("the HIP runtime is not loaded")
    return ctypes.CDLL(paths[0])


_NODE_TYPES = {0: "kernel", 1: "memcpy", 2: "memset", 5: "empty"}


def graph_node_counts(graph) -> dict:
    """Nodes of a captured graph by type ({"kernel": n, "memcpy": n, ...}); `graph` must
    have been created with keep_graph=True. Every kernel and copy node is one dependent
    dispatch of the replay (the decoder graph is a single chain)."""
    import ctypes
    hip = _hip_runtime()
    g = ctypes.c_void_p(graph.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(g, None, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    nodes = (ctypes.c_void_p * n.value)()
    if hip.hipGraphGetNodes(g, nodes, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    counts: dict = {}
    for node in nodes:
        t = ctypes.c_int(-1)
        if hip.hipGraphNodeGetType(ctypes.c_void_p(node), ctypes.byref(t)) != 0:
            raise RuntimeError("hipGraphNodeGetType failed")
        name = _NODE_TYPES.get(t.value, f"type{t.value}")
        counts[name] = counts.get(name, 0) + 1
    return counts


def _pin(backend, weights) -> list:
    """Keep the packed copies a captured graph reads alive as long as the engine."""
    fn = getattr(backend, "pin_packed_weights", None)
    return fn(list(weights.values())) if fn is not None else []


class Pi0DecoderEngine:
    """The captured 10-step decoder loop against a caller-supplied prefix KV cache.

    steps and layers exist for bisection, as in the reference engine. With `prefetch`
    (default) and a backend that offers it, each layer's attention launch also pulls the
    layer's FFN weights into L2 (same results; see `backends.hip.attention_prefetch_for`).
    `batch` > 1 runs B independent requests through every GEMM at once (BASELINE config
    5's decoder; not in the reference): each request has its own prefix K/V cache, and the
    rows are stacked states first (the B state tokens, then the B x chunk action tokens).
    """

    def __init__(self, weights: dict, encoder_seq_len: int = 768, chunk_size: int = 50,
                 steps: int = 10, layers: int = 18, fused: bool = True, backend: str = "hip",
                 plan: dict | None = None, device: str = "cuda", capture: bool = True,
                 warmup: int = 3, fp32_euler: bool = True, prefetch: bool = True,
                 batch: int = 1):
        self.encoder_seq_len = encoder_seq_len
        self.batch = batch
        self.chunk_size = chunk_size
        self.steps = steps
        self.layers = layers
        self.ops = op_table(fused, backend=backend, plan=plan)
        self.backend = BACKENDS[backend]
        self.attention_prefetch = _attention_prefetch(self.backend, self.ops, prefetch)
        n_layers = weights["decoder_attn_qkv_w"].shape[0]
        if layers > n_layers:
            raise ValueError(f"layers={layers} but the checkpoint has {n_layers}")
        dims = _dims_from(weights)
        expected = decoder_weight_shapes(n_layers, **dims)
        self.weights = {}
        for name in DECODER_WEIGHT_NAMES:
            w = weights[name]
            if tuple(w.shape) != expected[name]:
                raise ValueError(f"{name}: shape {tuple(w.shape)}, expected {expected[name]}")
            self.weights[name] = torch.empty(expected[name], dtype=torch.bfloat16, device=device)
            self.weights[name].copy_(w)
        self.buffers = allocate_decoder_buffers(
            encoder_seq_len, chunk_size, device, layers=n_layers, width=dims["width"],
            ffn=dims["ffn"], heads=dims["heads"], head_dim=dims["head_dim"],
            action_dim=dims["action_dim"], batch=batch)
        if fp32_euler:
            # the Euler accumulator stays fp32 between steps; diffusion_noise (bf16) is the output
            self.buffers["diffusion_noise_f32"] = torch.zeros(
                batch * chunk_size, dims["action_dim"], dtype=torch.float32, device=device)
        self.pool = ScratchPool()
        self.graph = None
        self._pinned = []
        if hasattr(self.backend, "prepare_weights"):
            self.backend.prepare_weights(self.weights)
        if capture:
            self._capture(warmup)

    def _run(self):
        with self.backend.use_pool(self.pool):
            pipeline.transformer_decoder(self.ops, self.weights, self.buffers,
                                         self.encoder_seq_len, steps=self.steps,
                                         layers=self.layers,
                                         attention_prefetch=self.attention_prefetch)

    def _capture(self, warmup: int):
        saved = self.buffers["diffusion_noise"].clone()
        self._sync_master()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._run()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.pool.freeze()
        self.graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(self.graph):
            self._run()
        self.graph.instantiate()
        self._pinned = _pin(self.backend, self.weights)
        torch.cuda.synchronize()
        self.buffers["diffusion_noise"].copy_(saved)
        self._sync_master()

    def graph_nodes(self) -> dict:
        """Nodes of the captured loop by type (see `graph_node_counts`)."""
        return graph_node_counts(self.graph)

    def _sync_master(self):
        if "diffusion_noise_f32" in self.buffers:
            self.buffers["diffusion_noise_f32"].copy_(self.buffers["diffusion_noise"])

    def load_prefix(self, prefix_k: torch.Tensor, prefix_v: torch.Tensor) -> None:
        """Copy the prefix K/V ([layers, >= enc_len, head_dim]; batched: [B, layers, ...])
        into the static cache."""
        e = self.encoder_seq_len
        self.buffers["encoder_K"][..., :e, :].copy_(prefix_k[..., :e, :])
        self.buffers["encoder_V"][..., :e, :].copy_(prefix_v[..., :e, :])

    def forward(self, state: torch.Tensor, noise: torch.Tensor) -> torch.Tensor:
        """Denoise one action chunk; returns the static `diffusion_noise` buffer.

        Batched: state [B, 32] and noise [B, chunk, 32] or [B * chunk, 32]; the result
        is [B * chunk, 32], request b in rows b * chunk .. (b + 1) * chunk - 1."""
        self.buffers["observation_state_normalized"].copy_(
            state.reshape(self.buffers["observation_state_normalized"].shape))
        noise = noise.reshape(self.buffers["diffusion_noise"].shape)
        self.buffers["diffusion_noise"].copy_(noise)
        if "diffusion_noise_f32" in self.buffers:
            self.buffers["diffusion_noise_f32"].copy_(noise)
        if self.graph is not None:
            self.graph.replay()
        else:
            self._run()
        return self.buffers["diffusion_noise"]

    def replay(self) -> None:
        """Replay the captured loop on whatever the static buffers hold (benchmarks)."""
        self.graph.replay()

    def refresh_weights(self) -> int:
        """Call after updating `self.weights` in place (see `_refresh`)."""
        return _refresh(self.backend, self._pinned, self.weights.values())


class Pi0EncoderEngine:
    """The captured prefix encoder: [M, 2048] input rows -> K/V cache rows of every layer."""

    WEIGHTS = ("encoder_attn_qkv_w", "encoder_attn_o_w", "encoder_ffn_gate_w",
               "encoder_ffn_up_w", "encoder_ffn_down_w")

    def __init__(self, weights: dict, encoder_seq_len: int = 768, layers: int | None = None,
                 backend: str = "hip", plan: dict | None = None, device: str = "cuda",
                 capture: bool = True, warmup: int = 2, cache_len: int | None = None,
                 copy_weights: bool = True):
        self.encoder_seq_len = encoder_seq_len
        self.ops = op_table(True, backend=backend, plan=plan)
        self.backend = BACKENDS[backend]
        n_layers = weights["encoder_attn_qkv_w"].shape[0]
        self.layers = n_layers if layers is None else layers
        if self.layers > n_layers:
            raise ValueError(f"layers={layers} but the checkpoint has {n_layers}")
        self.weights = {}
        for name in self.WEIGHTS:
            w = weights[name]
            if copy_weights or w.device != torch.device(device) or w.dtype != torch.bfloat16:
                w = w.to(device=device, dtype=torch.bfloat16).contiguous()
            self.weights[name] = w
        qkv, o = self.weights["encoder_attn_qkv_w"], self.weights["encoder_attn_o_w"]
        head_dim = (qkv.shape[2] - o.shape[1]) // 2
        self.buffers = allocate_encoder_buffers(
            encoder_seq_len, device, layers=n_layers, width=qkv.shape[1],
            ffn=self.weights["encoder_ffn_gate_w"].shape[2], heads=o.shape[1] // head_dim,
            head_dim=head_dim, cache_len=cache_len)
        self.pool = ScratchPool()
        self.graph = None
        self._pinned = []
        if hasattr(self.backend, "prepare_weights"):
            self.backend.prepare_weights(self.weights)
        if capture:
            self._capture(warmup)

    def _run(self):
        with self.backend.use_pool(self.pool):
            pipeline.transformer_encoder(self.ops, self.weights, self.buffers,
                                         self.encoder_seq_len, layers=self.layers, project=False)

    def _capture(self, warmup: int):
        saved = self.buffers["encoder_x"].clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.buffers["encoder_x"].copy_(saved)
                self._run()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.pool.freeze()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._run()
        self._pinned = _pin(self.backend, self.weights)
        torch.cuda.synchronize()
        self.buffers["encoder_x"].copy_(saved)

    def forward(self, x: torch.Tensor):
        """Run the encoder on `x` ([M, width]); returns (encoder_K, encoder_V) static buffers."""
        self.buffers["encoder_x"].copy_(x)
        if self.graph is not None:
            self.graph.replay()
        else:
            self._run()
        return self.buffers["encoder_K"], self.buffers["encoder_V"]

    def replay(self) -> None:
        self.graph.replay()

    def refresh_weights(self) -> int:
        """Call after updating `self.weights` in place (see `_refresh`)."""
        return _refresh(self.backend, self._pinned, self.weights.values())


class Pi0Inference:
    """One captured Pi0 forward pass: vision tower, prefix encoder and the 10-step
    decoder loop in one hipGraph (`hardware/nvidia/h100/pi0/engine.py:26-86`).

    `steps` and `layers` (decoder), `vision_layers` and `encoder_layers` exist for
    bisection, as in the reference. With `fp32_euler` (default) the Euler
    accumulator is an fp32 copy of `diffusion_noise`, seeded inside the graph and
    rounded into the bf16 output once at the end.
    """

    def __init__(self, checkpoint: dict, num_views: int = 3, chunk_size: int = 50,
                 steps: int = 10, layers: int = 18, fused: bool = True, device: str = "cuda",
                 backend: str = "hip", plan: dict | None = None, fp32_euler: bool = True,
                 vision_layers: int | None = None, encoder_layers: int | None = None,
                 capture: bool = True, warmup: int = 3, batch: int = 1, prompt_tokens: int = 0,
                 prefetch: bool = True):
        """batch > 1 and prompt_tokens > 0 are the BASELINE config-5 profile (not in the
        reference, which is batch-1 with precomputed `language_embeds`): B independent
        requests share every GEMM, and each request's prompt is `prompt_tokens` token ids
        embedded from `checkpoint["embed_tokens"]` ([vocab, 2048]) and scaled by sqrt(2048)."""
        self.batch = batch
        self.prompt_tokens = prompt_tokens
        self.num_views = num_views
        self.chunk_size = chunk_size
        self.steps = steps
        self.layers = layers
        self.vision_layers = vision_layers
        self.encoder_layers = encoder_layers
        self.ops = op_table(fused, backend=backend, plan=plan)
        self.backend = BACKENDS[backend]
        self.attention_prefetch = _attention_prefetch(self.backend, self.ops, prefetch)
        self.prompt_len = prompt_tokens if prompt_tokens else len(checkpoint["language_embeds"])
        bf16 = torch.bfloat16
        shapes = weight_shapes(self.prompt_len)
        if prompt_tokens:
            shapes.pop("language_embeds")
            shapes["embed_tokens"] = tuple(checkpoint["embed_tokens"].shape)
        self.weights = {}
        for name, shape in shapes.items():
            src = checkpoint[name]
            got = tuple(src.shape)
            # per-layer stacks may hold fewer layers than the model (shallow test models)
            stacked = name.startswith(("vision_attn", "vision_ffn", "vision_pre", "encoder_attn",
                                       "encoder_ffn", "decoder_attn", "decoder_ffn"))
            ok = got == tuple(shape) or (stacked and got[1:] == tuple(shape[1:]) and got[0] >= 1)
            if not ok:
                raise ValueError(f"{name}: shape {got}, expected {tuple(shape)}")
            self.weights[name] = torch.empty(got, dtype=bf16, device=device)
            self.weights[name].copy_(src)
        self.layers = min(self.layers, self.weights["decoder_attn_qkv_w"].shape[0])
        self.buffers, self.encoder_seq_len = allocate_static_buffers(
            num_views, chunk_size, self.prompt_len, device, batch=batch)
        if prompt_tokens:
            self.buffers["prompt_token_ids"] = torch.zeros(batch, prompt_tokens, dtype=torch.int32,
                                                           device=device)
        if fp32_euler:
            self.buffers["diffusion_noise_f32"] = torch.zeros(
                batch * chunk_size, shapes["decoder_state_in_proj_w"][0], dtype=torch.float32,
                device=device)
        self.pool = ScratchPool()
        self.graph = None
        self._pinned = []
        if hasattr(self.backend, "prepare_weights"):
            self.backend.prepare_weights(self.weights)
        if capture:
            self._capture(warmup)

    def _run(self):
        """One full forward pass, in place on the static buffers (engine.py:58-65)."""
        b = self.buffers
        L, v0 = self.encoder_seq_len, self.num_views * 256
        if self.prompt_tokens:
            self.ops.embed_prompt(b["prompt_token_ids"], self.weights["embed_tokens"],
                                  b["encoder_x"], v0, L, float(self.weights["embed_tokens"].shape[1]) ** 0.5)
        elif self.prompt_len:
            for r in range(self.batch):
                b["encoder_x"][r * L + v0:(r + 1) * L].copy_(self.weights["language_embeds"])
        if "diffusion_noise_f32" in b:
            b["diffusion_noise_f32"].copy_(b["diffusion_noise"])
        with self.backend.use_pool(self.pool):
            pipeline.vision_encoder(self.ops, self.weights, b, self.num_views,
                                    layers=self.vision_layers)
            pipeline.transformer_encoder(self.ops, self.weights, b, self.encoder_seq_len,
                                         layers=self.encoder_layers)
            pipeline.transformer_decoder(self.ops, self.weights, b, self.encoder_seq_len,
                                         steps=self.steps, layers=self.layers,
                                         attention_prefetch=self.attention_prefetch)

    def _capture(self, warmup: int):
        saved = self.buffers["diffusion_noise"].clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.buffers["diffusion_noise"].copy_(saved)
                self._run()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.pool.freeze()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._run()
        self._pinned = _pin(self.backend, self.weights)
        torch.cuda.synchronize()
        self.buffers["diffusion_noise"].copy_(saved)

    def forward(self, images, state, noise, token_ids=None):
        """Copy inputs into the static buffers, replay, return the denoised chunk (engine.py:80-86).

        Batched: images [B, views, 224, 224, 3], state [B, 32], noise [B, chunk, 32] (the
        result is [B * chunk, 32]), token_ids [B, prompt_tokens] int32."""
        b = self.buffers
        b["observation_images_normalized"].copy_(images.reshape(b["observation_images_normalized"].shape))
        b["observation_state_normalized"].copy_(state.reshape(b["observation_state_normalized"].shape))
        b["diffusion_noise"].copy_(noise.reshape(b["diffusion_noise"].shape))
        if self.prompt_tokens:
            if token_ids is None:
                raise ValueError("this engine embeds its prompt from token ids: pass token_ids")
            b["prompt_token_ids"].copy_(token_ids.reshape(b["prompt_token_ids"].shape))
        if self.graph is not None:
            self.graph.replay()
        else:
            self._run()
        return self.buffers["diffusion_noise"]

    def refresh_weights(self) -> int:
        """Call after updating `self.weights` in place (see `_refresh`)."""
        return _refresh(self.backend, self._pinned, self.weights.values())


def _dims_from(weights: dict) -> dict:
    qkv = weights["decoder_attn_qkv_w"]
    o = weights["decoder_attn_o_w"]
    width = qkv.shape[1]
    qkv_n = qkv.shape[2]
    q_dim = o.shape[1]
    head_dim = (qkv_n - q_dim) // 2
    return dict(width=width, ffn=weights["decoder_ffn_gate_w"].shape[2], heads=q_dim // head_dim,
                head_dim=head_dim, action_dim=weights["decoder_state_in_proj_w"].shape[0],
                steps=weights["decoder_action_fused_time_biases"].shape[0])
