// Prefix-encoder kernels for gfx950: M = 768..816 token rows at width 2048.
//
// At these shapes the GEMMs are MFMA-bound (2 * 768 * 2048 * 32768 flops for the
// gated FFN alone), so the design is the classic LDS-tiled one:
//   * tile_gemm_kernel<BM, BN, EPI, DUAL>: 4 waves in a 2 x 2 grid, BM x BN
//     output block, K consumed 64 at a time through two LDS stages. Both
//     operands are kept in LDS in MFMA fragment order (one 1 KB slot per
//     16 x 32 fragment: lane-contiguous 16-byte reads, free of bank conflicts):
//     A (row-major activations) is loaded one fragment per instruction straight
//     from global memory, B is the packed weight stream, already in that order.
//     While a stage is multiplied, the next stage's fragments are in flight in
//     registers; one barrier per 64-deep step.
//   * tiles are assigned so that the workgroups dispatched to one XCD (the
//     hardware deals workgroups round-robin over the 8 XCDs) cover consecutive
//     tiles -- all row blocks of a weight column block -- so each weight block
//     is read into one XCD's L2 once.
//   * split-K (ffn-down, K = 16384) writes fp32 partials and a second launch
//     sums them in split order and applies the residual epilogue.
// Epilogues (reference file:line, backends/tilelang/):
//   TE_STORE     C                      plain projection
//   TE_BIAS      C + b                  encoder_projector GEMM (wrappers.py:336-344)
//   TE_RES       out += C               encoder o-proj / ffn-down (wrappers.py:366-392)
//   TE_GATE      gelu(C_g) * C_u        encoder gated FFN (kernels/base.py:508-549)
//   TE_QKV_ROPE  bf16(C), RoPE on the rounded values, scatter Q / K / V
//                                       (kernels/base.py:672-726)
//   TE_PARTIAL   fp32 split-K partial
//   TE_BIAS_RES  C + b + R               vision o-proj / ffn-down / patch embedding
//                                       (kernels/base.py:197-270)
//   TE_BIAS_GELU gelu_tanh(C + b)        vision ffn-up (kernels/base.py:273-300)
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

enum TileEpi {
  TE_STORE = 0, TE_BIAS = 1, TE_RES = 2, TE_GATE = 3, TE_QKV_ROPE = 4, TE_PARTIAL = 5,
  TE_BIAS_RES = 6,    // C + b + R[row % res_mod or row]   (vision residual GEMMs, patch embedding)
  TE_BIAS_GELU = 7    // gelu_tanh(C + b)                   (vision FFN up)
};

struct TileArgs {
  const __bf16* a; int lda;
  const __bf16* w0; const __bf16* w1;   // packed B fragments ([nt][kt] tiles of 32 k x 16 n)
  const __bf16* bias;
  __bf16* out; int ldo;
  __bf16* out_k; __bf16* out_v; int ldkv;
  const __bf16* rope;
  float* part;                          // TE_PARTIAL: [splitk][M][N] fp32
  const __bf16* res; int ldres, res_mod;  // TE_BIAS_RES residual (may alias out); res_mod 0 = row
  int n_valid;                          // output columns stored (<= N; the rest is padding)
  int rows_per_batch;                   // TE_QKV_ROPE: prefix rows per request (RoPE position
  long long kv_bstride;                 //   = row % rows_per_batch), cache stride per request
  int M, N, K;                          // N, K = the packed (padded) weight's shape
  int tiles_m, tiles_n, splitk, ksteps; // ksteps = 64-deep steps per split
  int heads, head_dim;
  int xcd_remap;
};


__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_bf16 is used because one wave per SIMD sustains ~90% of the
// MFMA peak with it (the 16x16x32 form stalls near 55-60% at this occupancy).
// Fragment layouts (lane l, j = 0..7, e = 0..15):
//   A (32 rows x 16 k): A[l % 32][8 (l / 32) + j]
//   B (16 k x 32 cols): B[8 (l / 32) + j][l % 32]      (pi0hip_pack_weight32 order)
//   C (32 x 32):        C[8 (e / 4) + 4 (l / 32) + e % 4][l % 32]
//
// Workgroup = 4 waves side by side along N; each wave owns all BM rows of the
// block and WN of its B columns. Both operands run D 64-deep steps ahead:
//   * A (activations, shared by the 4 waves) goes global -> LDS directly
//     (buffer_load ... lds, 16 bytes per lane, one MFMA fragment per
//     instruction) into a D-slot ring; the buffer resource ends at row M so the
//     rows of a ragged last block load as zeros;
//   * B (the packed weight stream, private to the wave) goes global -> VGPRs
//     into a D-slot register ring, so no weight byte passes through LDS.
// The step count is a multiple of D (the host checks), so the ring unrolls with
// static slots; every step issues the same number of loads (steps past the end
// re-load the last step into the free slot), so "A of step s has landed" is the
// fixed count vmcnt <= LB + (D - 2) * (LA + LB) of loads issued after it; a plain
// s_barrier (no fence: the fence would wait for every prefetch) then publishes it.
//
// RMS = 1 fuses the decoder's RMS pre-norm for its batched gated FFN (fused_norm.py:26-78):
// the block sees every k of its rows, so each row's sum of squares is accumulated from
// the A fragments it already reads (v_dot2 on bf16 pairs; row tile i by wave i % 4),
// f = bf16(rsqrt(mean(x^2) + 1e-6)) goes to LDS and the epilogue forms
// gelu(f * x@Wg) * (f * x@Wu) from the fp32 accumulators.
template <int BM, int WN, int D, int EPI, bool DUAL, int OCC, int RMS = 0>
__global__ __launch_bounds__(256, OCC) void tile_gemm_kernel(TileArgs a) {
  constexpr int BN = 4 * WN;               // B columns per workgroup
  constexpr int FM = BM / 32;              // 32-row fragments (every wave holds all rows)
  constexpr int FN = WN / 32;              // 32-column B tiles per wave
  constexpr int TA = FM * 4;               // A fragments per 64-deep step (4 x k16)
  constexpr int LA = TA / 4;               // ... loaded by each wave
  constexpr int LB = FN * 4;               // B fragments per wave per step
  constexpr int AWAIT = LB + (D - 2) * (LA + LB);
  constexpr int PF = 3;                    // A-fragment register ring
  static_assert(BM % 32 == 0 && WN % 32 == 0 && (!DUAL || WN % 64 == 0), "tile shape");
  static_assert(D >= 2 && AWAIT < 64, "pipeline depth");
  constexpr int OUTC = DUAL ? BN / 2 : BN;           // output columns of the block
  constexpr int CP = OUTC + 4;                       // fp32 pitch of the parked tile
  constexpr int RING = D * TA * 64;                  // 16-byte slots of the operand ring
  constexpr int PARK = (BM * CP * 4 + 15) / 16;
  __shared__ bf16x8 lds[RING > PARK ? RING : PARK];
  __shared__ float rms_f[RMS ? BM : 1];

  PI0_PROBE(0);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  float ssr[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) ssr[i] = 0.f;
  int id = blockIdx.x;
  if (a.xcd_remap) id = (id & 7) * (gridDim.x >> 3) + (id >> 3);
  const int mt = id % a.tiles_m;
  id /= a.tiles_m;
  const int ntile = id % a.tiles_n, ks = id / a.tiles_n;
  const int m0 = mt * BM;
  const int KT = a.K >> 4;                 // 16-deep k tiles
  const int step0 = ks * a.ksteps, nsteps = a.ksteps;

  const int arows = max(min(BM, a.M - m0), 0);
  const __amdgpu_buffer_rsrc_t ar =
      rows_rsrc_sgpr(a.a + (size_t)m0 * a.lda, arows * a.lda * (int)sizeof(__bf16));
  int aoff[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int q = i * 4 + wave, rt = q >> 2, kq = q & 3;   // A fragment q = rt * 4 + kq
    aoff[i] = ((rt * 32 + (lane & 31)) * a.lda + kq * 16 + (lane >> 5) * 8) * (int)sizeof(__bf16);
  }
  // this wave's 32-column B tiles: for the gated FFN, FN / 2 gate tiles then FN / 2 up tiles
  const __bf16* bptr[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    if constexpr (DUAL) {
      const int half = FN / 2, jj = j < half ? j : j - half;
      const int ntg = ntile * (BN / 64) + wave * half + jj;
      bptr[j] = (j < half ? a.w0 : a.w1) + (size_t)ntg * KT * 512 + lane * 8;
    } else {
      const int ntg = ntile * (BN / 32) + wave * FN + j;
      bptr[j] = a.w0 + (size_t)ntg * KT * 512 + lane * 8;
    }
  }

  // the epilogue's bias / residual pieces (8 columns of a row per thread and pass) do not
  // depend on the product: they are loaded right after the ring's first steps are issued
  // and land while the k loop runs
  constexpr int C8 = OUTC / 8, NEP = (BM * C8 + 255) / 256;
  constexpr bool EB = EPI == TE_BIAS || EPI == TE_BIAS_RES || EPI == TE_BIAS_GELU;
  constexpr bool ER = EPI == TE_RES || EPI == TE_BIAS_RES;
  bf16x8 epb[EB ? NEP : 1], epr[ER ? NEP : 1];
  bf16x8 breg[D][FN][4];
  auto issue = [&](int s, int slot) {
    const int st = min(s, nsteps - 1) + step0;   // past the end: a harmless re-load
    const int abase = st * 64 * (int)sizeof(__bf16);
#pragma unroll
    for (int i = 0; i < LA; ++i)
      buf_load16_lds(ar, &lds[(slot * TA + i * 4 + wave) * 64], aoff[i] + abase);
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) breg[slot][j][kq] = load8(bptr[j] + ((size_t)st * 4 + kq) * 512);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

#pragma unroll
  for (int u = 0; u < D - 1; ++u) issue(u, u);
  if constexpr (EB || ER) {
    // unconditional loads through bounded resources (pieces past the end read as zeros and
    // are never stored), so no divergent branch makes the compiler wait on the ring above
    const __amdgpu_buffer_rsrc_t br = rows_rsrc_sgpr(a.bias, EB ? a.n_valid * (int)sizeof(__bf16) : 0);
    const int rrows = EPI == TE_RES ? a.M : (a.res_mod ? a.res_mod : a.M);
    const int rld = EPI == TE_RES ? a.ldo : a.ldres;
    const __amdgpu_buffer_rsrc_t rr =
        rows_rsrc_sgpr(EPI == TE_RES ? (const void*)a.out : (const void*)a.res,
                       ER ? rrows * rld * (int)sizeof(__bf16) : 0);
#pragma unroll
    for (int k = 0; k < NEP; ++k) {
      const int idx = t + 256 * k, row = idx / C8, c = (idx - row * C8) * 8;
      const int grow = m0 + row, col = ntile * OUTC + c;
      const bool in = idx < BM * C8;
      if constexpr (EB) epb[k] = buf_load8(br, in ? col * (int)sizeof(__bf16) : INT_MAX - 64);
      if constexpr (ER) {
        const int rrow = EPI == TE_BIAS_RES && a.res_mod ? grow % a.res_mod : grow;
        epr[k] = buf_load8(rr, in && rrow < rrows ? (rrow * rld + col) * (int)sizeof(__bf16) : INT_MAX - 64);
      }
    }
  }

  PI0_PROBE(1);

  for (int s0 = 0; s0 < nsteps; s0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int s = s0 + u;
      __builtin_amdgcn_s_waitcnt(PI0_VMCNT(AWAIT));
      __builtin_amdgcn_s_barrier();
      PI0_PROBE(8 + s);
      issue(s + D - 1, (u + D - 1) % D);
      // A fragments through a PF-deep register ring (f = kq * FM + i): the read of
      // fragment f + PF - 1 is issued before the MFMAs of fragment f.
      const bf16x8* st = lds + u * TA * 64;
      bf16x8 ap[PF];
#pragma unroll
      for (int p = 0; p < PF - 1; ++p) ap[p] = st[((p % FM) * 4 + p / FM) * 64 + lane];
#pragma unroll
      for (int f = 0; f < 4 * FM; ++f) {
        const int kq = f / FM, i = f % FM;
        if (f + PF - 1 < 4 * FM) {
          const int fn = f + PF - 1;
          ap[(f + PF - 1) % PF] = st[((fn % FM) * 4 + fn / FM) * 64 + lane];
        }
        __builtin_amdgcn_sched_barrier(0);   // keep the prefetch ahead of these MFMAs
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32(ap[f % PF], breg[u][j][kq], acc[i][j]);
        if constexpr (RMS) {
          if (wave == (i & 3)) {
            typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
            const bf16x8 v = ap[f % PF];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
              const bf16x2_t q = {v[2 * p], v[2 * p + 1]};
              ssr[i] = __builtin_amdgcn_fdot2_f32_bf16(q, q, ssr[i], false);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  PI0_PROBE(2);
  __builtin_amdgcn_s_waitcnt(PI0_VMCNT(0));   // drain the dummy tail loads before exit
  if constexpr (RMS) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (wave != (i & 3)) continue;
      const float ss = ssr[i] + __shfl_xor(ssr[i], 32);    // the two k halves of row lane % 32
      if (lane < 32) rms_f[i * 32 + lane] = round_bf(rsqrtf(ss / (float)a.K + 1e-6f));
    }
  }

  // ---- epilogue through LDS (the ring is free now): the waves park their fp32 tiles
  // row-major, then every thread finishes 8 consecutive output columns of a row with
  // 16-byte loads and stores (residual, RoPE table, outputs, split-K partials).
  // Lane holds C[8 (e / 4) + 4 (lane / 32) + e % 4][lane % 32] of each fragment.
  __syncthreads();
  float* cs = reinterpret_cast<float*>(lds);
  {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if constexpr (DUAL) {
          const float fr = RMS ? rms_f[row] : 1.f;
#pragma unroll
          for (int j = 0; j < FN / 2; ++j)
            cs[row * CP + (wave * (FN / 2) + j) * 32 + r] =
                gelu_tanh(fr * acc[i][j][e]) * (fr * acc[i][FN / 2 + j][e]);
        } else {
#pragma unroll
          for (int j = 0; j < FN; ++j) cs[row * CP + (wave * FN + j) * 32 + r] = acc[i][j][e];
        }
      }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NEP; ++k) {
    const int idx = t + 256 * k;
    if (idx >= BM * C8) continue;
    const int row = idx / C8, c = (idx - row * C8) * 8;
    const int grow = m0 + row;
    if (grow >= a.M) continue;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(&cs[row * CP + c]);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(&cs[row * CP + c + 4]);
    float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const int col = ntile * OUTC + c;
    if (col >= a.n_valid) continue;            // padded weight columns
    if constexpr (EPI == TE_PARTIAL) {
      float* dst = a.part + ((size_t)ks * a.M + grow) * a.N + col;
      *reinterpret_cast<f32x4*>(dst) = lo;
      *reinterpret_cast<f32x4*>(dst + 4) = hi;
      continue;
    }
    __bf16* dst;
    if constexpr (EPI == TE_QKV_ROPE) {
      const int hd = a.head_dim, qdim = a.heads * hd;
      const int bq = grow / a.rows_per_batch, tq = grow - bq * a.rows_per_batch;
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = round_bf(v[q]);
      if (col < qdim + hd) {          // rotate the rounded pairs (2p, 2p + 1)
        const bf16x8 rp = load8(a.rope + (size_t)tq * hd + (col % hd));
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float cs_ = bf2f(rp[2 * p]), sn = bf2f(rp[2 * p + 1]);
          const float x0 = v[2 * p], x1 = v[2 * p + 1];
          v[2 * p] = x0 * cs_ - x1 * sn;
          v[2 * p + 1] = x1 * cs_ + x0 * sn;
        }
      }
      const size_t kv = (size_t)bq * a.kv_bstride + (size_t)tq * a.ldkv;
      if (col < qdim) dst = a.out + (size_t)grow * qdim + col;
      else if (col < qdim + hd) dst = a.out_k + kv + (col - qdim);
      else dst = a.out_v + kv + (col - qdim - hd);
    } else {
      dst = a.out + (size_t)grow * a.ldo + col;
      if constexpr (EPI == TE_BIAS) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] += bf2f(epb[k][q]);
      }
      if constexpr (EPI == TE_RES) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] += bf2f(epr[k][q]);
      }
      if constexpr (EPI == TE_BIAS_RES || EPI == TE_BIAS_GELU) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] += bf2f(epb[k][q]);
      }
      if constexpr (EPI == TE_BIAS_RES) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] += bf2f(epr[k][q]);
      }
      if constexpr (EPI == TE_BIAS_GELU) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = gelu_tanh(v[q]);
      }
    }
    bf16x8 o;
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = f2bf(v[q]);
    *reinterpret_cast<bf16x8*>(dst) = o;
  }
  PI0_PROBE(3);
}

// ---- gated FFN on a wave grid, both operands staged in LDS ---------------------------
// Workgroup = NW waves as (NW / 2) x 2: BM rows x 256 packed B columns (128 gate + the
// matching 128 up), i.e. 128 output columns; wave (wm, wn) owns BM / (NW / 2) rows and
// output columns wn * 64 .. + 64 (gate tiles 2 wn, 2 wn + 1 and the same up tiles). Per
// 64-deep step a 384-row block loads 384 + 256 rows of 128 bytes for 384 x 256 x 64 MACs,
// against 2 x (128 + 256) rows for 2 x 128 x 256 x 64 in the two-per-CU strip kernel
// above, whose weight stream into VGPRs saturates the per-CU load path. Both operands go
// global -> LDS directly (buffer_load ... lds, one 1 KB fragment per instruction) into a
// D-slot ring of KS k16 slices per step, and every wave reads its A and B fragments from
// there. One workgroup per CU (BM = 384, KS = 4: 80 KB per slot, two slots = all 160 KB
// of LDS; 8 waves of 192 accumulators). Accumulation order per output element is the
// strip kernel's (k16 fragments in k order), so the two kernels give bitwise-equal results.
template <int BM, int D, int NW, int KS>
__global__ __launch_bounds__(64 * NW, 1) void tile2_gated_kernel(TileArgs a) {
  constexpr int WMR = NW / 2;              // wave rows (2 wave columns)
  constexpr int FM = BM / (32 * WMR);      // 32-row fragments per wave
  constexpr int FN = 4;                    // 2 gate + 2 up 32-column tiles per wave
  constexpr int TA = (BM / 32) * KS;       // A fragments per step (KS k16 slices deep)
  constexpr int TB = 8 * KS;               // B fragments per step (8 tiles x KS k16)
  constexpr int CPW = NW / KS;             // tiles covered by one copy index
  constexpr int LA = TA / NW, LB = TB / NW;  // ... issued by each wave
  constexpr int SLOT = (TA + TB) * 64;     // 16-byte LDS words per ring slot
  constexpr int OUTC = 128, OP = OUTC + 8; // output columns, bf16 pitch of the parked tile
  constexpr int PARK = (BM * OP * 2 + 15) / 16;
  static_assert(BM % (32 * WMR) == 0 && TA % NW == 0 && TB % NW == 0 && D >= 2, "tile shape");
  static_assert(NW % KS == 0 && 4 % CPW == 0, "copy assignment");
  __shared__ bf16x8 lds[D * SLOT > PARK ? D * SLOT : PARK];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int id = blockIdx.x;
  if (a.xcd_remap) id = (id & 7) * (gridDim.x >> 3) + (id >> 3);
  const int mt = id % a.tiles_m, ntile = id / a.tiles_m;
  const int m0 = mt * BM;
  const int KT = a.K >> 4;
  const int nsteps = a.ksteps;

  const int arows = max(min(BM, a.M - m0), 0);
  const __amdgpu_buffer_rsrc_t ar =
      rows_rsrc_sgpr(a.a + (size_t)m0 * a.lda, arows * a.lda * (int)sizeof(__bf16));
  // gate tiles ntile * 4 + c and up tiles likewise; one resource per weight, starting at
  // this block's first tile (its 4 tiles are contiguous: [nt][kt] order)
  const int wbytes = 4 * KT * 512 * (int)sizeof(__bf16);
  const __amdgpu_buffer_rsrc_t gr = rows_rsrc_sgpr(a.w0 + (size_t)ntile * 4 * KT * 512, wbytes);
  const __amdgpu_buffer_rsrc_t ur = rows_rsrc_sgpr(a.w1 + (size_t)ntile * 4 * KT * 512, wbytes);
  // copy i of wave w is fragment q = i * NW + w of each operand (q = tile * KS + slice,
  // slice w % KS, tile i * CPW + w / KS); the i-dependent parts of the offsets are
  // wave-uniform (scalar), so each operand needs one lane offset
  const int avoff = (((wave / KS) * 32 + (lane & 31)) * a.lda + (wave % KS) * 16 + (lane >> 5) * 8) *
                    (int)sizeof(__bf16);
  const int btile = KT * 512 * (int)sizeof(__bf16);
  const int bvoff = ((wave % KS) * 512 + lane * 8) * (int)sizeof(__bf16) + (wave / KS) * btile;
  const int arow_step = CPW * 32 * a.lda * (int)sizeof(__bf16);

  auto issue = [&](int s, int slot) {
    const int abase = s * KS * 16 * (int)sizeof(__bf16);
    const int bbase = s * KS * 512 * (int)sizeof(__bf16);
    bf16x8* dst = lds + slot * SLOT;
#pragma unroll
    for (int i = 0; i < LA; ++i)
      buf_load16_lds_s(ar, &dst[(i * NW + wave) * 64], avoff, abase + i * arow_step);
#pragma unroll
    for (int i = 0; i < LB; ++i)     // tiles 0-3 gate, 4-7 up
      buf_load16_lds_s(i * CPW < 4 ? gr : ur, &dst[(TA + i * NW + wave) * 64], bvoff,
                       bbase + ((i * CPW) & 3) * btile);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

#pragma unroll
  for (int u = 0; u < D - 1; ++u) issue(u, u);

  for (int s0 = 0; s0 < nsteps; s0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int s = s0 + u;
      // every copy of step s has landed (the D - 2 later steps may still be in flight)
      __builtin_amdgcn_s_waitcnt(PI0_VMCNT((D - 2) * (LA + LB)));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // past the end a harmless re-load of the last step keeps the count per step fixed
      issue(min(s + D - 1, nsteps - 1), (u + D - 1) % D);
      __builtin_amdgcn_sched_barrier(0);
      const bf16x8* st = lds + u * SLOT;
#pragma unroll
      for (int kq = 0; kq < KS; ++kq) {
        bf16x8 bf[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int tile = (j < 2 ? 0 : 4) + wn * 2 + (j & 1);
          bf[j] = st[(TA + tile * KS + kq) * 64 + lane];
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const bf16x8 af = st[((wm * FM + i) * KS + kq) * 64 + lane];
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] = mfma32(af, bf[j], acc[i][j]);
        }
        __builtin_amdgcn_sched_barrier(0);   // bound the fragments held: 384 accumulators
      }
    }
  }

  // ---- epilogue: GeGLU in registers, parked as bf16 row-major, stored 16 bytes a lane
  __builtin_amdgcn_s_waitcnt(PI0_VMCNT(0));
  __syncthreads();
  __bf16* cs = reinterpret_cast<__bf16*>(lds);
  {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = (wm * FM + i) * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          cs[row * OP + wn * 64 + j * 32 + r] = f2bf(gelu_tanh(acc[i][j][e]) * acc[i][2 + j][e]);
      }
  }
  __syncthreads();
  constexpr int C8 = OUTC / 8;
  for (int idx = t; idx < BM * C8; idx += 64 * NW) {
    const int row = idx / C8, c = (idx - row * C8) * 8;
    const int grow = m0 + row, col = ntile * OUTC + c;
    if (grow >= a.M || col >= a.n_valid) continue;
    *reinterpret_cast<bf16x8*>(a.out + (size_t)grow * a.ldo + col) =
        *reinterpret_cast<const bf16x8*>(&cs[row * OP + c]);
  }
}

// W[batch][K][N] -> 32x32x16 B fragments: tile (nt, kt) of 16 k x 32 n is 64 lanes x 8 bf16,
// lane = (k % 16 / 8) * 32 + n % 32, element k % 8; tiles ordered [nt][kt].
// K_pad x N_pad (multiples of 16 / 32) with zeros outside the K x N source.
__global__ void pack_weight32_kernel(const __bf16* __restrict__ w, __bf16* __restrict__ p,
                                     int K, int N, int K_pad, int N_pad, long long total_frags) {
  const long long f = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= total_frags) return;
  const long long per = (long long)(K_pad / 16) * (N_pad / 32) * 64;
  const long long b = f / per;
  long long rem = f - b * per;
  const int lane = (int)(rem & 63);
  rem >>= 6;
  const int KT = K_pad / 16;
  const int kt = (int)(rem % KT), nt = (int)(rem / KT);
  const int n = nt * 32 + (lane & 31);
  const int k0 = kt * 16 + (lane >> 5) * 8;
  const __bf16* src = w + b * (long long)K * N + (long long)k0 * N + n;
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (n < N && k0 + j < K) ? src[(long long)j * N] : __bf16(0.f);
  *reinterpret_cast<bf16x8*>(p + f * 8) = v;
}

// Split-K second pass: sum the partials in split order, add the residual, round once.
__global__ __launch_bounds__(256) void tile_reduce_res_kernel(TileArgs a) {
  const int id = blockIdx.x * 256 + threadIdx.x;
  const int per_row = a.N >> 2;
  const int row = id / per_row, col = (id - row * per_row) * 4;
  if (row >= a.M) return;
  f32x4 s = zero4();
  for (int k = 0; k < a.splitk; ++k)
    s += *reinterpret_cast<const f32x4*>(a.part + ((size_t)k * a.M + row) * a.N + col);
  __bf16* dst = a.out + (size_t)row * a.ldo + col;
  const bf16x4 rv = *reinterpret_cast<const bf16x4*>(dst);
  const bf16x4 o = {f2bf(s[0] + bf2f(rv[0])), f2bf(s[1] + bf2f(rv[1])),
                    f2bf(s[2] + bf2f(rv[2])), f2bf(s[3] + bf2f(rv[3]))};
  *reinterpret_cast<bf16x4*>(dst) = o;
}

// ---- encoder RMSNorm: out = bf16(x * rsqrt(mean(x^2) + 1e-6)), one wave per row
// (kernels/base.py:373-403; the Gemma 1 + w weight is folded into the next GEMM).
template <int CPL>   // 16-byte chunks per lane: K = CPL * 512
__global__ __launch_bounds__(256) void rms_norm_kernel(const __bf16* __restrict__ x, int ldx,
                                                       __bf16* __restrict__ out, int ldo, int M,
                                                       int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const __bf16* xr = x + (size_t)row * ldx;
  bf16x8 v[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) v[c] = load8(xr + (c * 64 + lane) * 8);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) { const float f = bf2f(v[c][j]); ss += f * f; }
  ss = warp_sum(ss);
  const float f = rsqrtf(ss / (float)K + 1e-6f);
  __bf16* orow = out + (size_t)row * ldo;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f2bf(bf2f(v[c][j]) * f);
    *reinterpret_cast<bf16x8*>(orow + (c * 64 + lane) * 8) = o;
  }
}

// ---- LayerNorm: out = bf16((x - mean) * rsqrt(E[x^2] - mean^2 + eps) * w + b), one wave
// per row, statistics in fp32 (kernels/base.py:405-447; the vision tower's final norm in
// encoder_projector, wrappers.py:336-344). K % 8 == 0, K <= 2048.
__global__ __launch_bounds__(256) void layer_norm_kernel(const __bf16* __restrict__ x, int ldx,
                                                         const __bf16* __restrict__ w,
                                                         const __bf16* __restrict__ b,
                                                         __bf16* __restrict__ out, int ldo, int M,
                                                         int K, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int chunks = K >> 3;
  const __bf16* xr = x + (size_t)row * ldx;
  bf16x8 v[4], wv[4], bv[4];
  // the row and the affine parameters are requested together: one memory round trip
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int ch = c * 64 + lane;
    v[c] = ch < chunks ? load8(xr + ch * 8) : zero8();
    wv[c] = ch < chunks ? load8(w + ch * 8) : zero8();
    bv[c] = ch < chunks ? load8(b + ch * 8) : zero8();
  }
  float s = 0.f, ss = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) { const float f = bf2f(v[c][j]); s += f; ss += f * f; }
  }
  s = warp_sum(s);
  ss = warp_sum(ss);
  const float mean = s / (float)K;
  const float inv = rsqrtf(ss / (float)K - mean * mean + eps);
  __bf16* orow = out + (size_t)row * ldo;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int ch = c * 64 + lane;
    if (ch >= chunks) continue;
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      o[j] = f2bf((bf2f(v[c][j]) - mean) * inv * bf2f(wv[c][j]) + bf2f(bv[c][j]));
    *reinterpret_cast<bf16x8*>(orow + ch * 8) = o;
  }
}

// ---- encoder multi-query attention (attention.py:29-34): every flat query row
// (token * heads + head) attends over all keys of the one KV head, no mask.
//
// Workgroup = 32 query rows; wave w takes the 32-key blocks b with b % 4 == w, so
// each K / V byte is read once per workgroup, straight from L2 into registers
// (no LDS staging, no barriers in the key loop). Per block, with 32x32x16 MFMAs:
//   S^T[32 keys][32 q] = K Q^T      A = K rows (16 B loads), B = Q^T (held all along)
//   online softmax per query in the log2 domain (the logits are rounded to bf16
//   first, as the reference's bf16 matmul output is); each lane owns one query
//   and 16 of its keys, the other 16 sit in lane ^ 32;
//   O^T[256 d][32 q] += V^T P^T     A = V^T (rows of the transposed V, pre-pass
//   below), B = P^T, which is exactly the S^T accumulator's layout once the key
//   slots of V^T are permuted the same way -- P never moves between lanes and
//   the per-query rescale is lane-local.
// The 4 waves' partial (m, l, O^T) are merged through LDS at the end.
constexpr int EA_HD = 256;

struct EncAttnArgs {
  const __bf16* q; int ldq;
  const __bf16* kp;                     // K in fragment order (see pack_kv_kernel)
  const __bf16* vp;                     // V^T in fragment order
  int ldvt;                             // keys zero-padded to a multiple of 64
  __bf16* out; int ldo;
  int rows, keys;                       // per request (grid.y = requests)
  float scale_log2;
  long long kv_bstride;                 // elements between two requests' K
};

// Attention pre-pass: K and V of one request in the order enc_attn_kernel's MFMA fragments
// read them, so every fragment load of the attention is one contiguous 1 KB per wave (from
// row-major K / V^T each 16-byte fragment sits on its own cache line). For 32-key block b:
//   kp[((b * 16 + kk) * 64 + l) * 8 ..]          = K[32 b + l % 32][16 kk + 8 (l / 32) ..]
//   vp[(((b * 8 + dt) * 2 + c) * 64 + l) * 8 ..] = V^T[32 dt + l % 32][slots 32 b + 16 c + 8 (l / 32) ..]
// where V^T's key slots follow, inside every 16-key chunk, the order the P^T operand uses,
// {0-3, 8-11, 4-7, 12-15}. Keys past `keys` (up to ldvt, a multiple of 64) are zero.
// One workgroup: a 64-key x 64-dim tile of K (copied) and of V (transposed through LDS).
__global__ __launch_bounds__(256) void pack_kv_kernel(const __bf16* __restrict__ k,
                                                      const __bf16* __restrict__ v, int ldkv,
                                                      __bf16* __restrict__ kp, __bf16* __restrict__ vp,
                                                      int ldvt, int keys, long long kv_bstride) {
  __shared__ __attribute__((aligned(16))) __bf16 tile[64][72];
  const int k0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  k += (size_t)blockIdx.z * kv_bstride;
  v += (size_t)blockIdx.z * kv_bstride;
  kp += (size_t)blockIdx.z * EA_HD * ldvt;
  vp += (size_t)blockIdx.z * EA_HD * ldvt;
  const int t = threadIdx.x;
  // 16-byte loads: key row kr, dims d0 + 8 c .. + 7 (keys past the end read as zeros)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = t + 256 * j, kr = i >> 3, c = (i & 7) * 8, key = k0 + kr, d = d0 + c;
    const bool in = key < keys;
    const bf16x8 kx = in ? load8(k + (size_t)key * ldkv + d) : zero8();
    const bf16x8 vx = in ? load8(v + (size_t)key * ldkv + d) : zero8();
    const int l = ((d & 15) >> 3) * 32 + (key & 31);
    *reinterpret_cast<bf16x8*>(kp + (((size_t)(key >> 5) * 16 + (d >> 4)) * 64 + l) * 8) = kx;
    *reinterpret_cast<bf16x8*>(&tile[kr][c]) = vx;
  }
  __syncthreads();
  // V^T row d, storage slots s .. s + 7 (each slot's key permuted into the P^T order)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = t + 256 * j, dr = i >> 3, c = (i & 7) * 8;
    bf16x8 o;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int kc = c + q, sl = kc & 15;
      const int key = (kc & ~15) + ((sl & 4) ? 8 : 0) + ((sl & 8) ? 4 : 0) + (sl & 3);
      o[q] = tile[key][dr];
    }
    const int d = d0 + dr, sl0 = k0 + c;                       // slot of o[0]
    const int l = ((sl0 & 15) >> 3) * 32 + (d & 31);
    const size_t frag = ((size_t)(sl0 >> 5) * 8 + (d >> 5)) * 2 + ((sl0 & 31) >> 4);
    *reinterpret_cast<bf16x8*>(vp + (frag * 64 + l) * 8) = o;
  }
}

__global__ __launch_bounds__(256, 1) void enc_attn_kernel(EncAttnArgs a) {
  constexpr int DP = EA_HD + 4;                        // fp32 pitch of a parked O row
  __shared__ __attribute__((aligned(16))) float ob[4][32][DP];   // per wave: O[q][d]; first Q^T
  __shared__ float ml[4][2][32];                       // per wave: m and l of each query

  PI0_PROBE(0);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int q0 = blockIdx.x * 32;
  {                                     // request blockIdx.y: its rows, K and V^T
    const int bq = blockIdx.y;
    a.q += (size_t)bq * a.rows * a.ldq;
    a.out += (size_t)bq * a.rows * a.ldo;
    a.kp += (size_t)bq * EA_HD * a.ldvt;
    a.vp += (size_t)bq * EA_HD * a.ldvt;
  }

  const int nblk = (a.keys + 31) / 32;
  const int mine = nblk > wave ? (nblk - wave + 3) / 4 : 0;     // blocks b = wave + 4 i
  // Staggered single buffers: V^T of block i is requested before its S^T MFMAs, and
  // K of block i + 1 right after them (into the registers they just consumed), so
  // each load has the other phase's 16 MFMAs to land.
  bf16x8 kf[16], vf[8][2];
  auto blk = [&](int i) { return wave + 4 * min(i, mine - 1); };   // past the end: re-load
  // fragment-ordered K / V^T: each fragment is one contiguous 1 KB wave load
  auto load_k = [&](int i) {
    const __bf16* src = a.kp + ((size_t)blk(i) * 16 * 64 + lane) * 8;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) kf[kk] = load8(src + kk * 64 * 8);
  };
  auto load_v = [&](int i) {
    const __bf16* src = a.vp + ((size_t)blk(i) * 16 * 64 + lane) * 8;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c) vf[dt][c] = load8(src + (dt * 2 + c) * 64 * 8);
  };
  if (mine > 0) load_k(0);                  // block 0's K is in flight during the Q staging

  // Q^T fragments (B operand, 16 d each; lane holds Q[q0 + r][16 kk + 8 h .. + 7]) are
  // shared by the 4 waves: staged once in LDS (in the merge buffer's space)
  bf16x8* qs = reinterpret_cast<bf16x8*>(&ob[0][0][0]);    // [16 kk][64 lanes]
  {
    const __amdgpu_buffer_rsrc_t qr =
        rows_rsrc_sgpr(a.q + (size_t)q0 * a.ldq, max(min(32, a.rows - q0), 0) * a.ldq * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kk = wave * 4 + i;
      qs[kk * 64 + lane] = buf_load8(qr, (r * a.ldq + kk * 16 + h * 8) * 2);
    }
  }
  __syncthreads();
  PI0_PROBE(1);

  float m_run = -1.0e30f, l_run = 0.f;
  f32x16 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;

  for (int i = 0; i < mine; ++i) {
    const int key0 = (wave + 4 * i) * 32;
    PI0_PROBE(8 + i);
    load_v(i);
    bf16x8 qv[16];
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) qv[kk] = qs[kk * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);     // keep the V^T and Q requests ahead of the S^T MFMAs
    f32x16 st;
#pragma unroll
    for (int e = 0; e < 16; ++e) st[e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) st = mfma32(kf[kk], qv[kk], st);
    __builtin_amdgcn_sched_barrier(0);
    load_k(i + 1);
    __builtin_amdgcn_sched_barrier(0);     // and the next K requests ahead of the softmax
    // lane holds S^T[key 8 (e / 4) + 4 h + e % 4][query r]
    float sv[16], mx = -1.0e30f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = key0 + 8 * (e >> 2) + 4 * h + (e & 3);
      sv[e] = key < a.keys ? round_bf(st[e]) * a.scale_log2 : -1.0e30f;
      mx = fmaxf(mx, sv[e]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, PI0_WAVE));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    float ps = 0.f;
    bf16x8 pf[2];                                      // P^T for chunk c = e / 8
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pv = fast_exp2(sv[e] - m_new);
      ps += pv;
      pf[e >> 3][e & 7] = f2bf(pv);
    }
    ps += __shfl_xor(ps, 32, PI0_WAVE);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      f32x16 acc = o[dt] * alpha;
#pragma unroll
      for (int c = 0; c < 2; ++c) acc = mfma32(vf[dt][c], pf[c], acc);
      o[dt] = acc;
    }
  }
  PI0_PROBE(2);
  __syncthreads();                                     // every wave is done with qs

  // ---- merge the 4 waves' partials: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w.
  // Every wave parks its O rows (lane: query r, 4 consecutive d per 16-byte store), then
  // wave w finishes head dims 64 w .. 64 w + 63 of all 32 rows, summing the waves in order.
  if (h == 0) { ml[wave][0][r] = m_run; ml[wave][1][r] = l_run; }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const f32x4 v4 = {o[dt][e4 * 4], o[dt][e4 * 4 + 1], o[dt][e4 * 4 + 2], o[dt][e4 * 4 + 3]};
      *reinterpret_cast<f32x4*>(&ob[wave][r][dt * 32 + 8 * e4 + 4 * h]) = v4;
    }
  __syncthreads();
  float M = -1.0e30f;
#pragma unroll
  for (int w = 0; w < 4; ++w) M = fmaxf(M, ml[w][0][r]);
  float wgt[4], L = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    wgt[w] = fast_exp2(ml[w][0][r] - M);     // 0 for a wave that saw no key
    L += wgt[w] * ml[w][1][r];
  }
  const float inv = __builtin_amdgcn_rcpf(L);
  const int row = q0 + r;
  if (row >= a.rows) return;
  __bf16* orow = a.out + (size_t)row * a.ldo;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {           // 4 consecutive d per load and store
      const int d0 = (2 * wave + j) * 32 + 8 * e4 + 4 * h;
      f32x4 v = *reinterpret_cast<const f32x4*>(&ob[0][r][d0]) * wgt[0];
#pragma unroll
      for (int w = 1; w < 4; ++w) v += *reinterpret_cast<const f32x4*>(&ob[w][r][d0]) * wgt[w];
      const bf16x4 pk = {f2bf(v[0] * inv), f2bf(v[1] * inv), f2bf(v[2] * inv), f2bf(v[3] * inv)};
      *reinterpret_cast<bf16x4*>(orow + d0) = pk;
    }
  PI0_PROBE(3);
}


// ---- SigLIP vision tower pieces (pipeline.py:21-54) -----------------------------

// images [views][224][224][3] -> patch rows [views * 256][ldo]: row = view * 256 + py * 16 + px,
// column (iy * 14 + ix) * 3 + c for the 14 x 14 x 3 patch, zero for columns 588 .. ldo - 1
// (the patchify of vision_patch_embed, wrappers.py:257-269).
__global__ __launch_bounds__(256) void im2col_patches_kernel(const __bf16* __restrict__ img,
                                                             __bf16* __restrict__ out, int ldo,
                                                             int rows) {
  const int id = blockIdx.x * 256 + threadIdx.x;
  const int chunks = ldo >> 3;
  const int row = id / chunks, c0 = (id - row * chunks) * 8;
  if (row >= rows) return;
  const int view = row >> 8, py = (row >> 4) & 15, px = row & 15;
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = c0 + j;
    __bf16 x = __bf16(0.f);
    if (k < 588) {
      const int iy = k / 42, r = k - iy * 42;           // 42 = 14 columns x 3 channels
      x = img[(((size_t)view * 224 + py * 14 + iy) * 224 + px * 14) * 3 + r];
    }
    v[j] = x;
  }
  *reinterpret_cast<bf16x8*>(out + (size_t)row * ldo + c0) = v;
}

// Multi-head vision attention (attention.py:20-26, SDPA over each view's 256 tokens,
// 16 heads of 72). V of every (view, head) is first transposed into
// vt[view][head][96 d][tokens] (d >= 72 zero; keys of every 16-key chunk in the P^T
// slot order, as for the encoder), then one wave per (view, head, 32 queries) runs
// S^T = K Q^T / O^T = V^T P^T on 32x32x16 MFMAs over the 8 key blocks (head_dim
// zero-padded to 80 for the k16 steps), softmax in fp32 with P rounded to bf16.
constexpr int VA_TOK = 256, VA_HD = 72, VA_HDP = 96;

__global__ __launch_bounds__(256) void vision_vt_kernel(const __bf16* __restrict__ qkv, int ldqkv,
                                                        __bf16* __restrict__ vt, int heads,
                                                        int dim) {
  __shared__ __attribute__((aligned(16))) __bf16 tile[64][VA_HD + 8];
  const int kc = blockIdx.x, head = blockIdx.y, view = blockIdx.z;
  const int t = threadIdx.x;
  const __bf16* src = qkv + ((size_t)view * VA_TOK + kc * 64) * ldqkv + 2 * dim + head * VA_HD;
  // 16-byte loads: 64 key rows x 9 chunks of 8 head dims
  for (int i = t; i < 64 * 9; i += 256) {
    const int kr = i / 9, c = (i - kr * 9) * 8;
    *reinterpret_cast<bf16x8*>(&tile[kr][c]) = load8(src + (size_t)kr * ldqkv + c);
  }
  __syncthreads();
  // 16-byte stores: 96 padded dims x 8 chunks of 8 storage slots (keys in P^T slot order)
  __bf16* dst = vt + (((size_t)view * heads + head) * VA_HDP) * VA_TOK + kc * 64;
  for (int i = t; i < VA_HDP * 8; i += 256) {
    const int d = i >> 3, c = (i & 7) * 8;
    bf16x8 o;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int slot = c + q, sl = slot & 15;
      const int key = (slot & ~15) + ((sl & 4) ? 8 : 0) + ((sl & 8) ? 4 : 0) + (sl & 3);
      o[q] = d < VA_HD ? tile[key][d] : __bf16(0.f);
    }
    *reinterpret_cast<bf16x8*>(dst + (size_t)d * VA_TOK + c) = o;
  }
}

struct VisAttnArgs {
  const __bf16* qkv; int ldqkv;
  const __bf16* vt;
  __bf16* out; int ldo;
  int heads, dim;
  float scale_log2;
};

// One wave per 32 queries of a (view, head); a workgroup holds NWQ consecutive query tiles
// of the same (view, head), whose waves read the same K / V^T fragments.
template <int NWQ>
__global__ __launch_bounds__(64 * NWQ, 1) void vision_attn_kernel(VisAttnArgs a) {
  PI0_PROBE(0);
  const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  const int qt = blockIdx.x * NWQ + (threadIdx.x >> 6), head = blockIdx.y, view = blockIdx.z;
  const size_t row0 = (size_t)view * VA_TOK;
  const int q = qt * 32 + r;
  // Q^T fragments: lane holds Q[q][16 kk + 8 h .. + 7] (zero past d = 72)
  bf16x8 qf[5];
#pragma unroll
  for (int kk = 0; kk < 5; ++kk) {
    const int d = kk * 16 + h * 8;
    qf[kk] = d < VA_HD ? load8(a.qkv + (row0 + q) * a.ldqkv + head * VA_HD + d) : zero8();
  }
  float m_run = -1.0e30f, l_run = 0.f;
  f32x16 o[3];
#pragma unroll
  for (int dt = 0; dt < 3; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  const __bf16* vt = a.vt + (((size_t)view * a.heads + head) * VA_HDP) * VA_TOK;
  // A three-slot register ring over the 8 key blocks: block kb + 3 is requested as soon
  // as block kb has consumed its slot, so two blocks are always in flight.
  constexpr int NB = VA_TOK / 32, RS = 3;
  bf16x8 kf[RS][5], vf[RS][3][2];
  auto load_blk = [&](int kb) {
    const int sl = kb % RS;
    // columns 72..79 of the padded head are read unmasked (the next head's K, or for the
    // last head the first V columns of the same row): Q^T is zero there, so they add 0
#pragma unroll
    for (int kk = 0; kk < 5; ++kk)
      kf[sl][kk] = load8(a.qkv + (row0 + kb * 32 + r) * a.ldqkv + a.dim + head * VA_HD + kk * 16 + h * 8);
#pragma unroll
    for (int dt = 0; dt < 3; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        vf[sl][dt][c] = load8(vt + (size_t)(dt * 32 + r) * VA_TOK + kb * 32 + 16 * c + 8 * h);
  };
#pragma unroll
  for (int kb = 0; kb < RS; ++kb) load_blk(kb);
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    const int sl = kb % RS;
    PI0_PROBE(8 + kb);
    f32x16 st;
#pragma unroll
    for (int e = 0; e < 16; ++e) st[e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 5; ++kk) st = mfma32(kf[sl][kk], qf[kk], st);
    float mx = -1.0e30f;
#pragma unroll
    for (int e = 0; e < 16; ++e) { st[e] *= a.scale_log2; mx = fmaxf(mx, st[e]); }
    mx = fmaxf(mx, __shfl_xor(mx, 32, PI0_WAVE));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    float ps = 0.f;
    bf16x8 pf[2];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pv = fast_exp2(st[e] - m_new);
      ps += pv;
      pf[e >> 3][e & 7] = f2bf(pv);
    }
    ps += __shfl_xor(ps, 32, PI0_WAVE);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 3; ++dt) {
      f32x16 acc = o[dt] * alpha;
#pragma unroll
      for (int c = 0; c < 2; ++c) acc = mfma32(vf[sl][dt][c], pf[c], acc);
      o[dt] = acc;
    }
    if (kb + RS < NB) load_blk(kb + RS);
    __builtin_amdgcn_sched_barrier(0);                 // keep each refill in its iteration
  }
  PI0_PROBE(2);
  // lane holds O^T[d = 32 dt + 8 (e / 4) + 4 h + e % 4][query r]
  const float inv = __builtin_amdgcn_rcpf(l_run);
  __bf16* orow = a.out + (row0 + q) * a.ldo + head * VA_HD;
#pragma unroll
  for (int dt = 0; dt < 3; ++dt)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const int d = dt * 32 + 8 * e4 + 4 * h;
      if (d < VA_HD) {
        const bf16x4 pk = {f2bf(o[dt][e4 * 4] * inv), f2bf(o[dt][e4 * 4 + 1] * inv),
                           f2bf(o[dt][e4 * 4 + 2] * inv), f2bf(o[dt][e4 * 4 + 3] * inv)};
        *reinterpret_cast<bf16x4*>(orow + d) = pk;
      }
    }
  PI0_PROBE(3);
}


// Prompt embedding (the reference takes precomputed embeddings,
// spec.py:46): out[b * rows_per_batch + row0 + j] = bf16(table[ids[b][j]] * scale).
__global__ __launch_bounds__(256) void embed_tokens_kernel(const int* __restrict__ ids, int n_tok,
                                                           const __bf16* __restrict__ table,
                                                           int vocab, int dim, float scale,
                                                           __bf16* __restrict__ out, int ldo,
                                                           int row0, int rows_per_batch,
                                                           int total) {
  const int per_row = dim >> 3;
  const int id = blockIdx.x * 256 + threadIdx.x;
  if (id >= total * per_row) return;
  const int tok = id / per_row, c = (id - tok * per_row) * 8;
  const int b = tok / n_tok, j = tok - b * n_tok;
  const int v = min(max(ids[tok], 0), vocab - 1);      // out-of-range ids clamp (checked on host)
  const bf16x8 e = load8(table + (size_t)v * dim + c);
  bf16x8 o;
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] = f2bf(bf2f(e[q]) * scale);
  *reinterpret_cast<bf16x8*>(out + ((size_t)b * rows_per_batch + row0 + j) * ldo + c) = o;
}

}  // namespace pi0

using namespace pi0;

// ---- host-side launch helpers ----------------------------------------------------

template <int BM, int WN, int D, int EPI, bool DUAL, int OCC, int RMS = 0>
static int launch_tile(TileArgs a, hipStream_t s) {
  a.tiles_m = (a.M + BM - 1) / BM;
  const int bn_out = DUAL ? 2 * WN : 4 * WN;
  if (a.N % bn_out) return PI0HIP_ERR_SHAPE;
  a.tiles_n = a.N / bn_out;
  const int steps = a.K / 64;
  if (a.K % 64 || steps % a.splitk || (steps / a.splitk) % D) return PI0HIP_ERR_SHAPE;
  a.ksteps = steps / a.splitk;
  const int grid = a.tiles_m * a.tiles_n * a.splitk;
  // XCD-contiguous tile order needs a grid divisible by the 8 XCDs
  a.xcd_remap = (grid % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL((tile_gemm_kernel<BM, WN, D, EPI, DUAL, OCC, RMS>), dim3(grid), dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

// Pipeline depth: the deepest even ring (<= DMAX) whose depth divides the per-split step count.
template <int BM, int WN, int DMAX, int EPI, bool DUAL, int OCC = 1, int RMS = 0>
static int launch_tile_auto(TileArgs a, hipStream_t s) {
  if (a.K % 64 || a.splitk < 1 || (a.K / 64) % a.splitk) return PI0HIP_ERR_SHAPE;
  const int steps = a.K / 64 / a.splitk;
  if (DMAX >= 8 && steps % 8 == 0) return launch_tile<BM, WN, (DMAX >= 8 ? 8 : 2), EPI, DUAL, OCC, RMS>(a, s);
  if (DMAX >= 6 && steps % 6 == 0) return launch_tile<BM, WN, (DMAX >= 6 ? 6 : 2), EPI, DUAL, OCC, RMS>(a, s);
  if (DMAX >= 4 && steps % 4 == 0) return launch_tile<BM, WN, (DMAX >= 4 ? 4 : 2), EPI, DUAL, OCC, RMS>(a, s);
  if (steps % 2 == 0) return launch_tile<BM, WN, 2, EPI, DUAL, OCC, RMS>(a, s);
  return PI0HIP_ERR_SHAPE;
}

// Pipeline depth preferring 4 (measured faster than 8 at K = 2048, M = 768), then 3
// (at K = 1152, 18 steps, the projector takes 9.4 us with 3 against 10.6 with 6) and 6.
template <int BM, int WN, int EPI, bool DUAL, int OCC = 1>
static int launch_tile_d4(TileArgs a, hipStream_t s) {
  if (a.K % 64 || a.splitk < 1 || (a.K / 64) % a.splitk) return PI0HIP_ERR_SHAPE;
  const int steps = a.K / 64 / a.splitk;
  if (steps % 4 == 0) return launch_tile<BM, WN, 4, EPI, DUAL, OCC>(a, s);
  if (steps % 3 == 0) return launch_tile<BM, WN, 3, EPI, DUAL, OCC>(a, s);
  if (steps % 6 == 0) return launch_tile<BM, WN, 6, EPI, DUAL, OCC>(a, s);
  if (steps % 2 == 0) return launch_tile<BM, WN, 2, EPI, DUAL, OCC>(a, s);
  return PI0HIP_ERR_SHAPE;
}

// Gated FFN on tile2_gated_kernel: BM-row x 128-output-column blocks, D-slot ring.
template <int BM, int D, int NW, int KS>
static int launch_tile2_gated(TileArgs a, hipStream_t s) {
  const int kstep = KS * 16;
  if (a.K % kstep || a.N % 128 || (a.K / kstep) % D) return PI0HIP_ERR_SHAPE;
  if ((long long)a.K * 128 * (long long)sizeof(__bf16) > INT_MAX ||
      (long long)BM * a.lda * (long long)sizeof(__bf16) > INT_MAX)
    return PI0HIP_ERR_SHAPE;                 // 32-bit buffer offsets
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = a.N / 128;
  a.splitk = 1;
  a.ksteps = a.K / kstep;
  const int grid = a.tiles_m * a.tiles_n;
  a.xcd_remap = (grid % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL((tile2_gated_kernel<BM, D, NW, KS>), dim3(grid), dim3(64 * NW), 0, s, a);
  return (int)hipGetLastError();
}

static TileArgs tile_args(const void* x, int ldx, const void* w, void* out, int ldo, int M, int N,
                          int K) {
  TileArgs a = {};
  a.a = (const __bf16*)x; a.lda = ldx; a.w0 = (const __bf16*)w;
  a.out = (__bf16*)out; a.ldo = ldo;
  a.M = M; a.N = N; a.K = K; a.splitk = 1; a.n_valid = N; a.rows_per_batch = M;
  return a;
}

static bool bad_dims(int M, int N, int K) { return M <= 0 || N <= 0 || K <= 0; }
// 16-byte vector access in the staging loads and the epilogues: row starts must be
// 16-byte aligned (leading dimension a multiple of 8 bf16, pointer 16-byte aligned).
static bool misaligned(const void* p, int ld) {
  return (reinterpret_cast<uintptr_t>(p) & 15) != 0 || (ld & 7) != 0;
}

extern "C" {

int pi0hip_pack_weight32(const void* w, void* packed, int K, int N, int batch, hipStream_t s) {
  if (K % 16 || N % 32) return (K <= 0 || N <= 0) ? PI0HIP_ERR_ARG : PI0HIP_ERR_SHAPE;
  return pi0hip_pack_weight32_padded(w, packed, K, N, K, N, batch, s);
}

int pi0hip_pack_weight32_padded(const void* w, void* packed, int K, int N, int K_pad, int N_pad,
                                int batch, hipStream_t s) {
  if (!w || !packed || K <= 0 || N <= 0 || batch <= 0) return PI0HIP_ERR_ARG;
  if (K_pad % 16 || N_pad % 32 || K_pad < K || N_pad < N) return PI0HIP_ERR_SHAPE;
  const long long frags = (long long)batch * (K_pad / 16) * (N_pad / 32) * 64;
  const long long blocks = (frags + 255) / 256;
  hipLaunchKernelGGL(pack_weight32_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     (const __bf16*)w, (__bf16*)packed, K, N, K_pad, N_pad, frags);
  return (int)hipGetLastError();
}

int pi0hip_rms_norm(const void* x, int ldx, void* out, int ldo, int M, int K, hipStream_t s) {
  if (!x || !out || M <= 0 || K <= 0) return PI0HIP_ERR_ARG;
  const dim3 grid((M + 3) / 4);
  switch (K) {
    case 1024: hipLaunchKernelGGL(rms_norm_kernel<2>, grid, dim3(256), 0, s, (const __bf16*)x, ldx, (__bf16*)out, ldo, M, K); break;
    case 2048: hipLaunchKernelGGL(rms_norm_kernel<4>, grid, dim3(256), 0, s, (const __bf16*)x, ldx, (__bf16*)out, ldo, M, K); break;
    default: return PI0HIP_ERR_SHAPE;
  }
  return (int)hipGetLastError();
}

size_t pi0hip_tile_workspace_bytes(int M, int N, int splitk) {
  if (M <= 0 || N <= 0 || splitk <= 1) return 0;
  return (size_t)splitk * M * N * sizeof(float);
}

int pi0hip_tile_linear(const void* x, int ldx, const void* w_packed, const void* bias, void* out,
                       int ldo, int M, int N, int K, hipStream_t s) {
  if (!x || !w_packed || !out || bad_dims(M, N, K)) return PI0HIP_ERR_ARG;
  if (misaligned(x, ldx) || misaligned(out, ldo) || misaligned(bias, 0)) return PI0HIP_ERR_SHAPE;
  TileArgs a = tile_args(x, ldx, w_packed, out, ldo, M, N, K);
  a.bias = (const __bf16*)bias;
  // 64-row tiles unless they overflow one round of the 256 CUs while 96-row tiles fit in
  // one (vision QKV: 324 -> 216 workgroups at M = 768), or M is large (M >= 2048: the
  // batched profile, where the taller tiles win by moving fewer bytes per flop).
  const int steps = K / 64;
  if (N % 128 == 0 && K % 64 == 0 && steps % 3 == 0 &&
      ((((M + 63) / 64) * (N / 128) > 256 && ((M + 95) / 96) * (N / 128) <= 256) || M >= 2048))
    return bias ? launch_tile<96, 32, 3, TE_BIAS, false, 2>(a, s)
                : launch_tile<96, 32, 3, TE_STORE, false, 2>(a, s);
  return bias ? launch_tile_d4<64, 32, TE_BIAS, false>(a, s)
              : launch_tile_d4<64, 32, TE_STORE, false>(a, s);
}

int pi0hip_tile_linear_residual(const void* x, int ldx, const void* w_packed, void* out, int ldo,
                                int M, int N, int K, int splitk, void* ws, size_t ws_bytes,
                                hipStream_t s) {
  if (!x || !w_packed || !out || bad_dims(M, N, K) || splitk < 1) return PI0HIP_ERR_ARG;
  if (misaligned(x, ldx) || misaligned(out, ldo)) return PI0HIP_ERR_SHAPE;
  TileArgs a = tile_args(x, ldx, w_packed, out, ldo, M, N, K);
  a.splitk = splitk;
  if (splitk == 1) {
    // large M (>= 2048 rows): 128 x 256 tiles fill the chip without splitting K
    if (M >= 2048 && N % 256 == 0) return launch_tile_d4<128, 64, TE_RES, false>(a, s);
    return launch_tile_d4<64, 32, TE_RES, false>(a, s);
  }
  if (N % 4 || ldo % 4) return PI0HIP_ERR_SHAPE;
  if (!ws || ws_bytes < pi0hip_tile_workspace_bytes(M, N, splitk)) return PI0HIP_ERR_WORKSPACE;
  a.part = (float*)ws;
  // small M (the batched decoder, 204 rows): 32-row tiles, two workgroups per CU
  if (int e = M <= 256 ? launch_tile_auto<32, 32, 4, TE_PARTIAL, false, 2>(a, s)
                       : launch_tile_auto<192, 32, 4, TE_PARTIAL, false>(a, s))
    return e;
  hipLaunchKernelGGL(tile_reduce_res_kernel, dim3((M * (N / 4) + 255) / 256), dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

int pi0hip_tile_gated_ffn(const void* x, int ldx, const void* gate_packed, const void* up_packed,
                          void* out, int ldo, int M, int N, int K, hipStream_t s) {
  if (!x || !gate_packed || !up_packed || !out || bad_dims(M, N, K)) return PI0HIP_ERR_ARG;
  if (misaligned(x, ldx) || misaligned(out, ldo)) return PI0HIP_ERR_SHAPE;
  TileArgs a = tile_args(x, ldx, gate_packed, out, ldo, M, N, K);
  a.w1 = (const __bf16*)up_packed;
  // From 512 rows (the prefix encoder: 768, batched 3264) the 8-wave 384-row blocks with
  // both operands in LDS (768 rows: 115 -> 103 us with cold weights, bitwise equal); below,
  // where 384-row blocks would be mostly padding, the two-per-CU strip kernel.
  if (M >= 512) {
    const int e = launch_tile2_gated<384, 2, 8, 4>(a, s);
    if (e != PI0HIP_ERR_SHAPE) return e;
  }
  return launch_tile_auto<128, 64, 2, TE_GATE, true, 2>(a, s);
}

int pi0hip_tile_norm_gated_ffn(const void* x, int ldx, const void* gate_packed,
                               const void* up_packed, void* out, int ldo, int M, int N, int K,
                               hipStream_t s) {
  if (!x || !gate_packed || !up_packed || !out || bad_dims(M, N, K)) return PI0HIP_ERR_ARG;
  if (misaligned(x, ldx) || misaligned(out, ldo) || K % 128) return PI0HIP_ERR_SHAPE;
  TileArgs a = tile_args(x, ldx, gate_packed, out, ldo, M, N, K);
  a.w1 = (const __bf16*)up_packed;
  return launch_tile_auto<32, 64, 2, TE_GATE, true, 1, 1>(a, s);
}

int pi0hip_tile_qkv_rope(const void* x, int ldx, const void* w_packed, const void* rope, void* q,
                         void* k, void* v, int ldkv, int M, int K, int heads, int head_dim,
                         hipStream_t s) {
  return pi0hip_tile_qkv_rope_batched(x, ldx, w_packed, rope, q, k, v, ldkv, 0, M, M, K, heads,
                                      head_dim, s);
}

int pi0hip_tile_qkv_rope_batched(const void* x, int ldx, const void* w_packed, const void* rope,
                                 void* q, void* k, void* v, int ldkv, long long kv_bstride,
                                 int rows_per_batch, int M, int K, int heads, int head_dim,
                                 hipStream_t s) {
  if (!x || !w_packed || !rope || !q || !k || !v || M <= 0 || K <= 0 || heads <= 0 ||
      rows_per_batch <= 0)
    return PI0HIP_ERR_ARG;
  if (M % rows_per_batch || (kv_bstride & 7)) return PI0HIP_ERR_SHAPE;
  if (head_dim % 16 || misaligned(x, ldx) || misaligned(q, 0) || misaligned(k, ldkv) ||
      misaligned(v, ldkv) || misaligned(rope, head_dim))
    return PI0HIP_ERR_SHAPE;
  TileArgs a = tile_args(x, ldx, w_packed, q, heads * head_dim, M, (heads + 2) * head_dim, K);
  a.out_k = (__bf16*)k; a.out_v = (__bf16*)v; a.ldkv = ldkv;
  a.rope = (const __bf16*)rope; a.heads = heads; a.head_dim = head_dim;
  a.rows_per_batch = rows_per_batch; a.kv_bstride = kv_bstride;
  if (M >= 2048 && a.N % 256 == 0) return launch_tile_d4<64, 64, TE_QKV_ROPE, false>(a, s);
  return launch_tile_d4<64, 32, TE_QKV_ROPE, false>(a, s);
}

int pi0hip_layer_norm(const void* x, int ldx, const void* w, const void* b, void* out, int ldo,
                      int M, int K, float eps, hipStream_t s) {
  if (!x || !w || !b || !out || M <= 0 || K <= 0) return PI0HIP_ERR_ARG;
  if (K % 8 || K > 2048) return PI0HIP_ERR_SHAPE;
  hipLaunchKernelGGL(layer_norm_kernel, dim3((M + 3) / 4), dim3(256), 0, s, (const __bf16*)x, ldx,
                     (const __bf16*)w, (const __bf16*)b, (__bf16*)out, ldo, M, K, eps);
  return (int)hipGetLastError();
}

static inline size_t round256_(size_t v) { return (v + 255) / 256 * 256; }

size_t pi0hip_encoder_attention_batched_workspace_bytes(int keys, int batch) {
  if (keys <= 0 || batch <= 0) return 0;
  const size_t ldvt = (size_t)(keys + 63) / 64 * 64;
  return 2 * round256_((size_t)batch * EA_HD * ldvt * sizeof(__bf16));   // packed K, packed V^T
}

size_t pi0hip_encoder_attention_workspace_bytes(int keys) {
  return pi0hip_encoder_attention_batched_workspace_bytes(keys, 1);
}

int pi0hip_encoder_attention(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             void* out, int ldo, int rows, int keys, int head_dim, float scale,
                             void* ws, size_t ws_bytes, hipStream_t s) {
  return pi0hip_encoder_attention_batched(q, ldq, k, v, ldkv, 0, out, ldo, rows, keys, head_dim,
                                          scale, 1, ws, ws_bytes, s);
}

int pi0hip_encoder_attention_batched(const void* q, int ldq, const void* k, const void* v,
                                     int ldkv, long long kv_bstride, void* out, int ldo, int rows,
                                     int keys, int head_dim, float scale, int batch, void* ws,
                                     size_t ws_bytes, hipStream_t s) {
  if (!q || !k || !v || !out || rows <= 0 || keys <= 0 || batch <= 0) return PI0HIP_ERR_ARG;
  if (head_dim != EA_HD || misaligned(q, ldq) || misaligned(k, ldkv) || misaligned(v, ldkv) ||
      (ldo & 3) ||
      (reinterpret_cast<uintptr_t>(out) & 7) || (kv_bstride & 7))
    return PI0HIP_ERR_SHAPE;
  if (!ws || ws_bytes < pi0hip_encoder_attention_batched_workspace_bytes(keys, batch))
    return PI0HIP_ERR_WORKSPACE;
  const int ldvt = (keys + 63) / 64 * 64;
  __bf16* kp = reinterpret_cast<__bf16*>(ws);
  __bf16* vp = kp + round256_((size_t)batch * EA_HD * ldvt * sizeof(__bf16)) / sizeof(__bf16);
  hipLaunchKernelGGL(pack_kv_kernel, dim3(ldvt / 64, EA_HD / 64, batch), dim3(256), 0, s,
                     (const __bf16*)k, (const __bf16*)v, ldkv, kp, vp, ldvt, keys, kv_bstride);
  if (hipError_t e = hipGetLastError()) return (int)e;
  EncAttnArgs a = {};
  a.q = (const __bf16*)q; a.ldq = ldq;
  a.kp = kp; a.vp = vp; a.ldvt = ldvt;
  a.out = (__bf16*)out; a.ldo = ldo;
  a.rows = rows; a.keys = keys;
  a.scale_log2 = 1.4426950408889634f * scale;
  a.kv_bstride = kv_bstride;
  hipLaunchKernelGGL(enc_attn_kernel, dim3((rows + 31) / 32, batch), dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

int pi0hip_tile_linear_bias_res(const void* x, int ldx, const void* w_packed, const void* bias,
                                const void* res, int ldres, int res_mod, void* out, int ldo, int M,
                                int N, int K, int N_pad, int K_pad, hipStream_t s) {
  if (!x || !w_packed || !bias || !res || !out || bad_dims(M, N, K) || res_mod < 0)
    return PI0HIP_ERR_ARG;
  if (N_pad < N || K_pad < K || N % 8 || misaligned(x, ldx) || misaligned(out, ldo) ||
      misaligned(res, ldres) || misaligned(bias, 0))
    return PI0HIP_ERR_SHAPE;
  TileArgs a = tile_args(x, ldx, w_packed, out, ldo, M, N_pad, K_pad);
  a.n_valid = N;
  a.bias = (const __bf16*)bias;
  a.res = (const __bf16*)res; a.ldres = ldres; a.res_mod = res_mod;
  // vision o-proj (K = 1152, 18 steps): a 3-deep ring, 7.1 us against 7.8-8.0 with 6 at
  // M = 768, 17.3 against 19.2 at M = 3072
  const bool d3 = (K_pad / 64) % 3 == 0 && (K_pad / 64) % 4 != 0;
  if (M >= 2048)
    return d3 ? launch_tile<128, 32, 3, TE_BIAS_RES, false, 1>(a, s)
              : launch_tile_auto<128, 32, 8, TE_BIAS_RES, false>(a, s);
  return d3 ? launch_tile<32, 32, 3, TE_BIAS_RES, false, 1>(a, s)
            : launch_tile_auto<32, 32, 8, TE_BIAS_RES, false>(a, s);
}

int pi0hip_tile_linear_bias_gelu(const void* x, int ldx, const void* w_packed, const void* bias,
                                 void* out, int ldo, int M, int N, int K, int N_pad, int K_pad,
                                 hipStream_t s) {
  if (!x || !w_packed || !bias || !out || bad_dims(M, N, K)) return PI0HIP_ERR_ARG;
  if (N_pad < N || K_pad < K || N % 8 || misaligned(x, ldx) || misaligned(out, ldo) ||
      misaligned(bias, 0))
    return PI0HIP_ERR_SHAPE;
  TileArgs a = tile_args(x, ldx, w_packed, out, ldo, M, N_pad, K_pad);
  a.n_valid = N;
  a.bias = (const __bf16*)bias;
  // vision FFN up (K = 1152, N = 4352), two workgroups per CU: 128-column tiles at
  // M = 768 (408 workgroups; 18.1 us against 18.7 with 256 columns), 256-column
  // tiles from 2048 rows (M = 3072: 51 us against 58)
  if (M < 2048 && N_pad % 128 == 0 && K_pad % 192 == 0)
    return launch_tile<64, 32, 3, TE_BIAS_GELU, false, 2>(a, s);
  if (N_pad % 256 == 0 && K_pad % 192 == 0)
    return launch_tile<64, 64, 3, TE_BIAS_GELU, false, 2>(a, s);
  return launch_tile_auto<64, 32, 8, TE_BIAS_GELU, false>(a, s);
}

int pi0hip_im2col_patches(const void* images, int views, void* out, int ldo, hipStream_t s) {
  if (!images || !out || views <= 0) return PI0HIP_ERR_ARG;
  if (ldo < 588 || ldo % 8 || misaligned(out, ldo)) return PI0HIP_ERR_SHAPE;
  const int rows = views * 256;
  const int threads = rows * (ldo / 8);
  hipLaunchKernelGGL(im2col_patches_kernel, dim3((threads + 255) / 256), dim3(256), 0, s,
                     (const __bf16*)images, (__bf16*)out, ldo, rows);
  return (int)hipGetLastError();
}

size_t pi0hip_vision_attention_workspace_bytes(int views, int heads) {
  if (views <= 0 || heads <= 0) return 0;
  return round256_((size_t)views * heads * VA_HDP * VA_TOK * sizeof(__bf16));
}

int pi0hip_vision_attention(const void* qkv, int ldqkv, void* out, int ldo, int views, int tokens,
                            int heads, int head_dim, float scale, void* ws, size_t ws_bytes,
                            hipStream_t s) {
  if (!qkv || !out || views <= 0 || heads <= 0) return PI0HIP_ERR_ARG;
  const int dim = heads * head_dim;
  if (tokens != VA_TOK || head_dim != VA_HD || ldqkv < 3 * dim || ldo < dim ||
      misaligned(qkv, ldqkv) || (ldo & 3) || (reinterpret_cast<uintptr_t>(out) & 7))
    return PI0HIP_ERR_SHAPE;
  if (!ws || ws_bytes < pi0hip_vision_attention_workspace_bytes(views, heads))
    return PI0HIP_ERR_WORKSPACE;
  hipLaunchKernelGGL(vision_vt_kernel, dim3(VA_TOK / 64, heads, views), dim3(256), 0, s,
                     (const __bf16*)qkv, ldqkv, (__bf16*)ws, heads, dim);
  if (hipError_t e = hipGetLastError()) return (int)e;
  VisAttnArgs a = {};
  a.qkv = (const __bf16*)qkv; a.ldqkv = ldqkv;
  a.vt = (const __bf16*)ws;
  a.out = (__bf16*)out; a.ldo = ldo;
  a.heads = heads; a.dim = dim;
  a.scale_log2 = 1.4426950408889634f * scale;
  // two 32-query tiles of one (view, head) per workgroup: their identical K / V^T fragment
  // loads meet in one CU's L1 (3 views: 14.5 -> 13.8 us with the V^T pass, 12 views:
  // 37.9 -> 35.8; four tiles: 17.9 / 35.3)
  hipLaunchKernelGGL(vision_attn_kernel<2>, dim3(VA_TOK / 64, heads, views), dim3(128), 0, s, a);
  return (int)hipGetLastError();
}

int pi0hip_embed_tokens(const int* ids, int n_tok, int batch, const void* table, int vocab, int dim,
                        float scale, void* out, int ldo, int row0, int rows_per_batch,
                        hipStream_t s) {
  if (!ids || !table || !out || n_tok <= 0 || batch <= 0 || vocab <= 0 || dim <= 0)
    return PI0HIP_ERR_ARG;
  if (dim % 8 || misaligned(out, ldo) || misaligned(table, dim) || row0 + n_tok > rows_per_batch)
    return PI0HIP_ERR_SHAPE;
  const int total = n_tok * batch;
  hipLaunchKernelGGL(embed_tokens_kernel, dim3((total * (dim / 8) + 255) / 256), dim3(256), 0, s,
                     ids, n_tok, (const __bf16*)table, vocab, dim, scale, (__bf16*)out, ldo, row0,
                     rows_per_batch, total);
  return (int)hipGetLastError();
}

}  // extern "C"
