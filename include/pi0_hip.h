/*
 * C ABI of libpi0hip.so: hand-written gfx950 (MI355X) kernels for the Pi0
 * action-expert denoising loop.
 *
 * Every entry point takes plain device pointers, element counts / leading
 * dimensions (in elements), an optional workspace and a hipStream_t. All
 * tensors are bf16 row-major unless stated. Launches are asynchronous, never
 * synchronise and never allocate, so they can be recorded into a hipGraph.
 * Return value: 0 on success, a negative PI0HIP_ERR_* for a rejected
 * argument (nothing launched), or a positive hipError_t from the launch.
 *
 * Weights named `*_packed` are in the B-fragment layout written by
 * pi0hip_pack_weight (one-time, outside the hot loop).
 *
 * Each entry point replaces the reference call site named in its comment
 * (paths relative to src/flash_vla/hardware/nvidia/h100/pi0/backends/tilelang/).
 */
#ifndef PI0_HIP_H
#define PI0_HIP_H

#include <stddef.h>
#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PI0HIP_ERR_ARG (-1)        /* null pointer, non-positive size, bad enum */
#define PI0HIP_ERR_SHAPE (-2)      /* shape the kernels do not support         */
#define PI0HIP_ERR_WORKSPACE (-3)  /* workspace missing or too small           */

/* Library version. */
int pi0hip_version(void);

/* W[batch][K][N] -> B-fragment packed copy of the same size. K % 32 == 0, N % 16 == 0.
 * Replaces nothing in the reference (TileLang reads the [K, N] weights through
 * TMA); this is the one-time relayout that makes the weight stream coalesced. */
int pi0hip_pack_weight(const void* w, void* packed, int K, int N, int batch, hipStream_t s);

/* Workspace for the split-K GEMMs (0 when splitk == 1): fp32 partial tiles
 * written by the GEMM launch and summed by its second (reduce) launch. */
size_t pi0hip_gemm_workspace_bytes(int M, int N, int splitk, int dual);

/* out[m, n] = act(x[m, :K] @ w[K, N] + bias[n]); act 0 = identity, 1 = silu.
 * Unpacked w; K must be 32, N and ldo multiples of 8.
 * decoder_state_proj     wrappers.py:108-112 (tl_matmul_bias, kernels/base.py:158-192)
 * decoder_action_in_proj wrappers.py:115-120 (tl_matmul_bias_silu, kernels/base.py:304-335) */
int pi0hip_small_linear(const void* x, int ldx, const void* w, const void* bias, void* out,
                        int ldo, int M, int N, int K, int act, hipStream_t s);

/* pi0hip_small_linear with an fp32 x (the fp32 Euler accumulator as the
 * action_in_proj input). Same reference call site. */
int pi0hip_small_linear_f32x(const void* x, int ldx, const void* w, const void* bias, void* out,
                             int ldo, int M, int N, int K, int act, hipStream_t s);

/* The skinny GEMMs below (pi0hip_linear_bias, pi0hip_linear_residual,
 * pi0hip_rms_linear_bias_residual[_f32], pi0hip_norm_qkv_rope[_batched],
 * pi0hip_norm_gated_ffn) read x rows 16 bytes at a time and store four outputs
 * at a time: x 16-byte aligned with ldx % 8 == 0 and ldx >= K; out (and K / V)
 * 8-byte aligned (16 for the fp32 accumulator) with ldo (ldkv) % 4 == 0;
 * otherwise PI0HIP_ERR_SHAPE. */

/* out = x @ W + bias, fp32 accumulation, M <= 64 per 64-row block.
 * decoder_action_mlp wrappers.py:123-128 (tl_matmul_bias, kernels/base.py:158-192) */
int pi0hip_linear_bias(const void* x, int ldx, const void* w_packed, const void* bias, void* out,
                       int ldo, int M, int N, int K, int splitk, void* ws, size_t ws_bytes,
                       hipStream_t s);

/* out += x @ W (in place, one bf16 rounding).
 * decoder_out_proj_residual wrappers.py:176-181, decoder_ffn_down_residual
 * wrappers.py:184-189 (tl_matmul_res, kernels/base.py:115-154) */
int pi0hip_linear_residual(const void* x, int ldx, const void* w_packed, void* out, int ldo,
                           int M, int N, int K, int splitk, void* ws, size_t ws_bytes,
                           hipStream_t s);

/* out += bias + f * (x @ W), f[m] = bf16(rsqrt(mean(x[m]^2) + 1e-6)).
 * decoder_action_out_proj fused_wrappers.py:57-67 (tl_fused_rms_matmul_bias_res,
 * kernels/fused_norm.py:81-125) */
int pi0hip_rms_linear_bias_residual(const void* x, int ldx, const void* w_packed,
                                    const void* bias, void* out, int ldo, int M, int N, int K,
                                    int splitk, void* ws, size_t ws_bytes, hipStream_t s);

/* pi0hip_rms_linear_bias_residual with an fp32 residual / destination (the
 * Euler accumulator kept in fp32 between steps; ldo % 4 == 0). Same call site. */
int pi0hip_rms_linear_bias_residual_f32(const void* x, int ldx, const void* w_packed,
                                        const void* bias, float* out, int ldo, int M, int N, int K,
                                        int splitk, void* ws, size_t ws_bytes, hipStream_t s);

/* acc = f * (x @ Wqkv), RoPE on adjacent pairs of the first (heads+1)*head_dim
 * columns with rope[m] = interleaved bf16 (cos, sin); scatter to
 * q [M, heads*head_dim], k/v rows [M, ldkv]; norm_factor[m] = f (optional, may be NULL).
 * decoder_norm_qkv_rope wrappers.py:131-144 (tl_rms_factor + tl_qkv_gemm_rope,
 * kernels/base.py:344-370, 607-669) */
int pi0hip_norm_qkv_rope(const void* x, int ldx, const void* w_packed, const void* rope, void* q,
                         void* k, void* v, int ldkv, void* norm_factor, int M, int K, int heads,
                         int head_dim, hipStream_t s);

/* out = gelu_tanh(f * (x @ Wg)) * (f * (x @ Wu)), f from x in-kernel.
 * decoder_norm_gated_ffn fused_wrappers.py:45-54 (tl_fused_rms_gate,
 * kernels/fused_norm.py:26-78) */
int pi0hip_norm_gated_ffn(const void* x, int ldx, const void* gate_packed, const void* up_packed,
                          void* out, int ldo, int M, int N, int K, hipStream_t s);

/* Workspace for pi0hip_attention. */
size_t pi0hip_attention_workspace_bytes(int rows, int keys);

/* pi0hip_norm_qkv_rope for a batch of `batch` requests (the
 * reference is batch-1 only): the M = batch x (T + 1) rows are ordered "states
 * first" (the batch's state tokens, then each request's T action tokens); token t
 * of request b uses RoPE row t, writes Q row b (T + 1) + t (request-major) and K / V
 * row t of request b's cache at k / v + b * kv_bstride. batch = 1 is
 * pi0hip_norm_qkv_rope. decoder_norm_qkv_rope wrappers.py:131-144 (batched). */
int pi0hip_norm_qkv_rope_batched(const void* x, int ldx, const void* w_packed, const void* rope,
                                 void* q, void* k, void* v, int ldkv, long long kv_bstride,
                                 void* norm_factor, int M, int K, int heads, int head_dim,
                                 int batch, hipStream_t s);

/* Workspace of pi0hip_attention_batched (rows and keys per request). */
size_t pi0hip_attention_batched_workspace_bytes(int rows, int keys, int batch);

/* pi0hip_attention over `batch` requests: request b's `rows` request-major query rows
 * start at q + b * rows * ldq and read its own cache at k / v + b * kv_bstride; the
 * output rows are written back in the "states first" token order of
 * pi0hip_norm_qkv_rope_batched (rows % heads == 0 when batch > 1). batch = 1 is
 * pi0hip_attention. decoder_attention fused_wrappers.py:88-115 (batched). */
int pi0hip_attention_batched(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             long long kv_bstride, void* out, int ldo, int rows, int keys,
                             int enc_len, int heads, int head_dim, int batch, void* ws,
                             size_t ws_bytes, hipStream_t s);

/* pi0hip_attention (one request) plus an L2 prefetch for the launches that follow it:
 * spare workgroups (filling the chip to two per CU next to the attention's) touch
 * every 128-byte line of up to four regions, region r being pfr_slices equal slices
 * of pfr_bytes in all, where slice s is what workgroup s of the consuming launch reads
 * (workgroup s runs on XCD s % 8, so the slice lands in that XCD's L2). A null region
 * is skipped; pfr_bytes / pfr_slices must be a multiple of 128, pfr 4-byte aligned.
 * Loads only: `out` is bitwise that of pi0hip_attention. No reference counterpart
 * (the reference's decoder_attention, fused_wrappers.py:88-115, launches no prefetch);
 * the decoder engine passes the layer's gate, up and down weights in regions 0-2
 * (their launches read slice s on XCD s % 8) and leaves region 3 null. */
int pi0hip_attention_prefetch(const void* q, int ldq, const void* k, const void* v, int ldkv,
                              void* out, int ldo, int rows, int keys, int enc_len, int heads,
                              int head_dim, void* ws, size_t ws_bytes, const void* pf0,
                              size_t pf0_bytes, int pf0_slices, const void* pf1, size_t pf1_bytes,
                              int pf1_slices, const void* pf2, size_t pf2_bytes, int pf2_slices,
                              const void* pf3, size_t pf3_bytes, int pf3_slices, hipStream_t s);

/* out = softmax(mask(q k^T / sqrt(head_dim))) v over `keys` cache rows; flat
 * query row r = token * heads + head; rows r < heads keep keys j <= enc_len.
 * `out` may alias `q`. head_dim must be 256, keys <= 2048.
 * decoder_attention fused_wrappers.py:88-115 (tl_fd_flat_split + tl_fd_flat_combine,
 * kernels/base.py:801-923) */
int pi0hip_attention(const void* q, int ldq, const void* k, const void* v, int ldkv, void* out,
                     int ldo, int rows, int keys, int enc_len, int heads, int head_dim,
                     void* ws, size_t ws_bytes, hipStream_t s);

/* out[M, N] += x[M, K] @ w[K, N] in one launch: 16-row x 16-column workgroups over the
 * whole K (no split-K partials, no reduce launch). Packed w; K in {512, 1024, 2048, 4096},
 * N % 16 == 0, x 16-byte aligned with ldx % 8 == 0.
 * decoder_out_proj_residual wrappers.py:176-181, decoder_ffn_down_residual
 * wrappers.py:184-189 (tl_matmul_res, kernels/base.py:115-154) */
int pi0hip_linear_residual_rows(const void* x, int ldx, const void* w_packed, void* out, int ldo,
                                int M, int N, int K, hipStream_t s);


/* ---- unfused decoder call sites (op_table(fused=False)) ------------------------
 * The reference's two-kernel decoder path, kept for its rounding points: the RMS
 * factor is a separate pass that stores bf16 f, and x * f is rounded to bf16 per
 * element before the GEMM; the attention materialises the bf16 score matrix and the
 * bf16 probabilities. */

/* f[m] = bf16(rsqrt(mean_k x[m, k]^2 + 1e-6)); K % 8 == 0, x 16-byte aligned.
 * _rms_factor wrappers.py:101-105 (tl_rms_factor, kernels/base.py:344-370) */
int pi0hip_rms_factor(const void* x, int ldx, void* f, int M, int K, hipStream_t s);

/* out = bf16(gelu_tanh(a @ gate) * (a @ up)) with a = bf16(x * f[row]) per element;
 * packed gate / up; same operand rules as pi0hip_norm_gated_ffn.
 * decoder_norm_gated_ffn wrappers.py:192-198 (tl_scaled_gate, kernels/base.py:453-505) */
int pi0hip_scaled_gated_ffn(const void* x, int ldx, const void* f, const void* gate_packed,
                            const void* up_packed, void* out, int ldo, int M, int N, int K,
                            hipStream_t s);

/* out += bias + bf16(x * f[row]) @ w (bf16 out), split-K as pi0hip_linear_bias.
 * decoder_action_out_proj wrappers.py:201-208 (tl_scaled_matmul_bias_res,
 * kernels/base.py:552-596) */
int pi0hip_scaled_linear_bias_residual(const void* x, int ldx, const void* f,
                                       const void* w_packed, const void* bias, void* out, int ldo,
                                       int M, int N, int K, int splitk, void* ws, size_t ws_bytes,
                                       hipStream_t s);

/* The same into an fp32 destination / residual (the fp32 Euler accumulator).
 * Same reference call site. */
int pi0hip_scaled_linear_bias_residual_f32(const void* x, int ldx, const void* f,
                                           const void* w_packed, const void* bias, float* out,
                                           int ldo, int M, int N, int K, int splitk, void* ws,
                                           size_t ws_bytes, hipStream_t s);

/* Three launches: scores = bf16((q k^T) / sqrt(head_dim)) [rows, keys];
 * probs = bf16(softmax(mask(scores))) with masked keys filled with -3e38 (flat rows
 * r < heads keep keys j <= enc_len); out = bf16(probs @ v). `out` may alias `q`;
 * `scores` and `probs` must not alias. head_dim must be 256, keys <= 2048.
 * decoder_attention wrappers.py:147-173 (tl_matmul_abT_scale, tl_softmax_mask0,
 * tl_matmul: kernels/base.py:737-798, 84-111) */
int pi0hip_attention_unfused(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             void* scores, int ld_scores, void* probs, int ld_probs, void* out,
                             int ldo, int rows, int keys, int enc_len, int heads, int head_dim,
                             hipStream_t s);

/* pi0hip_attention without a workspace argument and without any allocation: the
 * partial outputs live in a static per-device array of pi0hip_attention_noalloc_streams()
 * (4) slots of pi0hip_attention_noalloc_max_bytes() (8 MiB) each, enough for
 * pi0hip_attention_workspace_bytes(rows, keys) up to e.g. 408 rows x 2048 keys; larger
 * shapes return PI0HIP_ERR_WORKSPACE without launching. Each stream takes its own slot on
 * its first call on a device and keeps it until the process ends, so calls on different
 * streams do not share scratch; a fifth stream on one device is rejected with
 * PI0HIP_ERR_WORKSPACE. Calls on one stream run in stream order and reuse its slot.
 * No counterpart in the reference: for callers that cannot allocate device memory
 * (code under graph capture that may not call hipMalloc, tight serving loops). */
size_t pi0hip_attention_noalloc_max_bytes(void);
int pi0hip_attention_noalloc_streams(void);
int pi0hip_attention_noalloc(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             void* out, int ldo, int rows, int keys, int enc_len, int heads,
                             int head_dim, hipStream_t s);

/* ---- prefix encoder (M = 768..816 token rows, width 2048) --------------------
 * LDS-tiled MFMA GEMMs for the MFMA-bound encoder shapes (32x32x16 MFMAs);
 * weights packed by pi0hip_pack_weight32, K % 128 == 0; activation / output rows
 * 16-byte aligned (pointers 16-byte aligned, leading dimensions % 8 == 0). */

/* W[batch][K][N] -> the 32x32x16 B-fragment layout of the encoder GEMMs: tile
 * (nt, kt) of 16 k x 32 n is 64 lanes x 8 bf16, lane = (k%16/8)*32 + n%32,
 * element k%8, tiles ordered [nt][kt]. K % 16 == 0, N % 32 == 0. One-time
 * relayout, like pi0hip_pack_weight (no reference counterpart). */
int pi0hip_pack_weight32(const void* w, void* packed, int K, int N, int batch, hipStream_t s);

/* pi0hip_pack_weight32 into a K_pad x N_pad packed block (K_pad % 16 == 0,
 * N_pad % 32 == 0), zero outside the K x N source: lets GEMMs with ragged K / N
 * (the vision FFN's 4304, the 588-wide patches) run on whole tiles. */
int pi0hip_pack_weight32_padded(const void* w, void* packed, int K, int N, int K_pad, int N_pad,
                                int batch, hipStream_t s);

/* out = bf16(x * rsqrt(mean(x^2) + 1e-6)), one row per wave; K in {1024, 2048}.
 * tl_rms_norm, kernels/base.py:373-403 (encoder_norm_qkv_rope / encoder_norm_gated_ffn,
 * wrappers.py:347-381) */
int pi0hip_rms_norm(const void* x, int ldx, void* out, int ldo, int M, int K, hipStream_t s);

/* fp32 split-K partials of pi0hip_tile_linear_residual (0 when splitk == 1). */
size_t pi0hip_tile_workspace_bytes(int M, int N, int splitk);

/* out = x @ W (+ bias[n] when bias != NULL); N % 128 == 0, K % 128 == 0.
 * encoder_projector GEMM, wrappers.py:336-344 (tl_matmul_bias, kernels/base.py:158-192) */
int pi0hip_tile_linear(const void* x, int ldx, const void* w_packed, const void* bias, void* out,
                       int ldo, int M, int N, int K, hipStream_t s);

/* out += x @ W in place, one bf16 rounding; splitk > 1 sums fp32 partials in a
 * second launch (K / 64 divisible by splitk). N % 128 == 0.
 * encoder_out_proj_residual wrappers.py:366-371, encoder_ffn_down_residual
 * wrappers.py:383-392 (tl_matmul_res_ws, kernels/base.py:115-155) */
int pi0hip_tile_linear_residual(const void* x, int ldx, const void* w_packed, void* out, int ldo,
                                int M, int N, int K, int splitk, void* ws, size_t ws_bytes,
                                hipStream_t s);

/* out = bf16(gelu_tanh(x @ Wg) * (x @ Wu)) on fp32 accumulators; N % 128 == 0.
 * encoder_norm_gated_ffn GEMM, wrappers.py:374-380 (tl_matmul_gate, kernels/base.py:508-549) */
int pi0hip_tile_gated_ffn(const void* x, int ldx, const void* gate_packed, const void* up_packed,
                          void* out, int ldo, int M, int N, int K, hipStream_t s);

/* out = bf16(gelu_tanh(f * x @ Wg) * (f * x @ Wu)) with the decoder's fused RMS pre-norm
 * f = bf16(rsqrt(mean_k x^2 + 1e-6)) per row of the raw input x; packed weights in the
 * 16 k x 32 n (pi0hip_pack_weight32) order; K % 128 == 0, N % 128 == 0. The batched
 * decoder's gated FFN (M > 64 rows): decoder_norm_gated_ffn, fused_wrappers.py:45-54
 * (tl_fused_rms_gate, kernels/fused_norm.py:26-78). */
int pi0hip_tile_norm_gated_ffn(const void* x, int ldx, const void* gate_packed,
                               const void* up_packed, void* out, int ldo, int M, int N, int K,
                               hipStream_t s);

/* proj = bf16(x @ W), W = [K, (heads + 2) * head_dim]; RoPE (interleaved pairs,
 * table rope[M, head_dim]) on the rounded Q and K columns, then scatter to
 * q [M, heads*head_dim], k / v rows [M, ldkv].
 * encoder_norm_qkv_rope GEMM + scatter, wrappers.py:347-363 (tl_matmul_ws +
 * tl_rope_scatter_bf16, kernels/base.py:112, 672-726) */
int pi0hip_tile_qkv_rope(const void* x, int ldx, const void* w_packed, const void* rope, void* q,
                         void* k, void* v, int ldkv, int M, int K, int heads, int head_dim,
                         hipStream_t s);

/* out = bf16((x - mean) * rsqrt(var + eps) * w + b), var = E[x^2] - mean^2 in fp32;
 * K % 8 == 0, K <= 2048.
 * encoder_projector's vision final norm, wrappers.py:336-344 (tl_layer_norm,
 * kernels/base.py:405-447) */
int pi0hip_layer_norm(const void* x, int ldx, const void* w, const void* b, void* out, int ldo,
                      int M, int K, float eps, hipStream_t s);

/* pi0hip_tile_qkv_rope over requests of `rows_per_batch` prefix rows each: row r is
 * position r % rows_per_batch of request r / rows_per_batch, whose K / V cache starts at
 * k / v + request * kv_bstride. encoder_norm_qkv_rope (batched, config 5). */
int pi0hip_tile_qkv_rope_batched(const void* x, int ldx, const void* w_packed, const void* rope,
                                 void* q, void* k, void* v, int ldkv, long long kv_bstride,
                                 int rows_per_batch, int M, int K, int heads, int head_dim,
                                 hipStream_t s);

/* Workspace of pi0hip_encoder_attention_batched. */
size_t pi0hip_encoder_attention_batched_workspace_bytes(int keys, int batch);

/* pi0hip_encoder_attention over `batch` requests: request b's `rows` query / output rows
 * follow request b - 1's, its K / V start at k / v + b * kv_bstride.
 * encoder_attention (batched, config 5). */
int pi0hip_encoder_attention_batched(const void* q, int ldq, const void* k, const void* v,
                                     int ldkv, long long kv_bstride, void* out, int ldo, int rows,
                                     int keys, int head_dim, float scale, int batch, void* ws,
                                     size_t ws_bytes, hipStream_t s);

/* Prompt embedding: out[b * rows_per_batch + row0 + j] = bf16(table[ids[b * n_tok + j]] *
 * scale) for a [vocab, dim] bf16 table and int32 ids (clamped to the vocabulary).
 * No reference counterpart (it takes precomputed language_embeds, spec.py:46,
 * engine.py:60); BASELINE config 5's 48-token prompt, scale sqrt(2048). */
int pi0hip_embed_tokens(const int* ids, int n_tok, int batch, const void* table, int vocab, int dim,
                        float scale, void* out, int ldo, int row0, int rows_per_batch,
                        hipStream_t s);

/* Workspace of pi0hip_encoder_attention: the transposed V (256 x keys rounded up to 64). */
size_t pi0hip_encoder_attention_workspace_bytes(int keys);

/* out = softmax(scale * bf16(q k^T)) v, every flat query row over every key
 * (one shared KV head, no mask); head_dim must be 256. `out` must not alias q.
 * Two launches: V -> V^T into the workspace, then the attention.
 * encoder_attention, kernels/attention.py:29-34 */
int pi0hip_encoder_attention(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             void* out, int ldo, int rows, int keys, int head_dim, float scale,
                             void* ws, size_t ws_bytes, hipStream_t s);

/* ---- SigLIP vision tower (M = views x 256 rows, width 1152, 16 heads of 72) ---- */

/* out = x @ W + bias + res[r], r = row % res_mod (res_mod > 0) or row; `res` may
 * alias `out`. W packed by pi0hip_pack_weight32_padded to K_pad x N_pad (N_pad %
 * 128 == 0, K_pad % 128 == 0); only the N valid columns are stored (N % 8 == 0).
 * vision_out_proj_residual / vision_ffn_down_residual / vision_patch_embed
 * (wrappers.py:252-313; tl_matmul_bias_res / _mod, kernels/base.py:197-270) */
int pi0hip_tile_linear_bias_res(const void* x, int ldx, const void* w_packed, const void* bias,
                                const void* res, int ldres, int res_mod, void* out, int ldo, int M,
                                int N, int K, int N_pad, int K_pad, hipStream_t s);

/* out = gelu_tanh(x @ W + bias), same padding rules.
 * vision_norm_ffn_up GEMM (wrappers.py:292-299; tl_matmul_bias_gelu, kernels/base.py:273-300) */
int pi0hip_tile_linear_bias_gelu(const void* x, int ldx, const void* w_packed, const void* bias,
                                 void* out, int ldo, int M, int N, int K, int N_pad, int K_pad,
                                 hipStream_t s);

/* images [views][224][224][3] -> patch rows [views*256][ldo] (14 x 14 x 3 features in
 * (iy, ix, c) order, zero-filled from column 588 to ldo); ldo % 8 == 0, ldo >= 588.
 * The patchify of vision_patch_embed (wrappers.py:257-269). */
int pi0hip_im2col_patches(const void* images, int views, void* out, int ldo, hipStream_t s);

/* Workspace of pi0hip_vision_attention: per-head transposed V. */
size_t pi0hip_vision_attention_workspace_bytes(int views, int heads);

/* Per view and head: out = softmax(scale * q k^T) v over the view's 256 tokens, q / k / v
 * read from the packed QKV rows [views*256][ldqkv] (q | k | v, heads x 72 each); out
 * [views*256][ldo] in head-major columns. tokens must be 256, head_dim 72.
 * vision_attention, kernels/attention.py:20-26 */
int pi0hip_vision_attention(const void* qkv, int ldqkv, void* out, int ldo, int views, int tokens,
                            int heads, int head_dim, float scale, void* ws, size_t ws_bytes,
                            hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif /* PI0_HIP_H */
