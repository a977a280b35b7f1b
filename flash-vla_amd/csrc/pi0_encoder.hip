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
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

enum TileEpi { TE_STORE = 0, TE_BIAS = 1, TE_RES = 2, TE_GATE = 3, TE_QKV_ROPE = 4, TE_PARTIAL = 5 };

struct TileArgs {
  const __bf16* a; int lda;
  const __bf16* w0; const __bf16* w1;   // packed B fragments ([nt][kt] tiles of 32 k x 16 n)
  const __bf16* bias;
  __bf16* out; int ldo;
  __bf16* out_k; __bf16* out_v; int ldkv;
  const __bf16* rope;
  float* part;                          // TE_PARTIAL: [splitk][M][N] fp32
  int M, N, K;                          // N = output columns
  int tiles_m, tiles_n, splitk, ksteps; // ksteps = 64-deep steps per split
  int heads, head_dim;
  int xcd_remap;
};

// vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and 15:14).
#define PI0_VMCNT(n) (((n) & 0xF) | (0x7 << 4) | (0xF << 8) | (((n) >> 4) << 14))

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
template <int BM, int WN, int D, int EPI, bool DUAL, int OCC>
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
  __shared__ bf16x8 lds[D * TA * 64];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
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

  for (int s0 = 0; s0 < nsteps; s0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int s = s0 + u;
      __builtin_amdgcn_s_waitcnt(PI0_VMCNT(AWAIT));
      __builtin_amdgcn_s_barrier();
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
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(PI0_VMCNT(0));   // drain the dummy tail loads before exit

  // ---- epilogue: lane holds C[8 (e / 4) + 4 (lane / 32) + e % 4][lane % 32] per fragment
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = m0 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
      const bool live = row < a.M;
      if constexpr (EPI == TE_GATE) {
#pragma unroll
        for (int j = 0; j < FN / 2; ++j) {
          const int col = (ntile * (BN / 64) + wave * (FN / 2) + j) * 32 + r;
          const float v = gelu_tanh(acc[i][j][e]) * acc[i][FN / 2 + j][e];
          if (live) a.out[(size_t)row * a.ldo + col] = f2bf(v);
        }
      } else if constexpr (EPI == TE_QKV_ROPE) {
        const int hd = a.head_dim, qdim = a.heads * hd;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int col = (ntile * (BN / 32) + wave * FN + j) * 32 + r;
          const float v = round_bf(acc[i][j][e]);
          const float p = __shfl_xor(v, 1, PI0_WAVE);   // the other column of the RoPE pair
          float o = v;
          if (col < qdim + hd && live) {
            const __bf16* rp = a.rope + (size_t)row * hd + ((col % hd) & ~1);
            const float cs = bf2f(rp[0]), sn = bf2f(rp[1]);
            o = (col & 1) ? v * cs + p * sn : v * cs - p * sn;
          }
          if (live) {
            __bf16* dst;
            if (col < qdim) dst = a.out + (size_t)row * qdim + col;
            else if (col < qdim + hd) dst = a.out_k + (size_t)row * a.ldkv + (col - qdim);
            else dst = a.out_v + (size_t)row * a.ldkv + (col - qdim - hd);
            *dst = f2bf(o);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int col = (ntile * (BN / 32) + wave * FN + j) * 32 + r;
          float v = acc[i][j][e];
          if (!live) continue;
          if constexpr (EPI == TE_PARTIAL) {
            a.part[((size_t)ks * a.M + row) * a.N + col] = v;
            continue;
          }
          __bf16* dst = a.out + (size_t)row * a.ldo + col;
          if constexpr (EPI == TE_BIAS) v += bf2f(a.bias[col]);
          if constexpr (EPI == TE_RES) v += bf2f(*dst);
          *dst = f2bf(v);
        }
      }
    }
  }
}

// W[batch][K][N] -> 32x32x16 B fragments: tile (nt, kt) of 16 k x 32 n is 64 lanes x 8 bf16,
// lane = (k % 16 / 8) * 32 + n % 32, element k % 8; tiles ordered [nt][kt].
__global__ void pack_weight32_kernel(const __bf16* __restrict__ w, __bf16* __restrict__ p,
                                     int K, int N, long long total_frags) {
  const long long f = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= total_frags) return;
  const long long per = (long long)(K / 16) * (N / 32) * 64;
  const long long b = f / per;
  long long rem = f - b * per;
  const int lane = (int)(rem & 63);
  rem >>= 6;
  const int KT = K / 16;
  const int kt = (int)(rem % KT), nt = (int)(rem / KT);
  const int n = nt * 32 + (lane & 31);
  const int k0 = kt * 16 + (lane >> 5) * 8;
  const __bf16* src = w + b * (long long)K * N + (long long)k0 * N + n;
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = src[(long long)j * N];
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
  bf16x8 v[4];
  float s = 0.f, ss = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int ch = c * 64 + lane;
    v[c] = ch < chunks ? load8(xr + ch * 8) : zero8();
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
    const bf16x8 wv = load8(w + ch * 8), bv = load8(b + ch * 8);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f2bf((bf2f(v[c][j]) - mean) * inv * bf2f(wv[j]) + bf2f(bv[j]));
    *reinterpret_cast<bf16x8*>(orow + ch * 8) = o;
  }
}

// ---- encoder multi-query attention (attention.py:29-34): every flat query row
// (token * heads + head) attends over all keys of the one KV head, no mask.
// Workgroup = 32 query rows; wave w takes row tile w & 1 and key half w >> 1 of
// each 64-key block. K / V blocks are staged through LDS; per wave an online
// (flash) softmax in the log2 domain with S^T = K Q^T, so the probabilities are
// already the A operand of P @ V (same key-slot permutation as the decoder
// kernel). The logits are rounded to bf16 as the reference's bf16 matmul does.
constexpr int EA_HD = 256;
constexpr int EA_KB = 64;                 // keys per block (32 per key half)
constexpr int EA_P = EA_HD + 8;           // bf16 pitch of staged rows
constexpr int EA_OP = EA_HD + 4;          // fp32 pitch of the merge buffer

struct EncAttnArgs {
  const __bf16* q; int ldq;
  const __bf16* k; const __bf16* v; int ldkv;
  __bf16* out; int ldo;
  int rows, keys;
  float scale_log2;
};

__global__ __launch_bounds__(256, 1) void enc_attn_kernel(EncAttnArgs a) {
  __shared__ __attribute__((aligned(16))) __bf16 ks_[EA_KB][EA_P];   // also the merge buffer
  __shared__ __attribute__((aligned(16))) __bf16 vs_[EA_KB][EA_P];
  __shared__ float mrg_m[2][16], mrg_l[2][16];   // [row tile][row] of key half 1

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int rt = wave & 1, half = wave >> 1;
  const int q0 = blockIdx.x * 32 + rt * 16;

  // Q^T fragments of this wave's 16 rows (B operand), straight from global memory
  bf16x8 qf[8];
  {
    const __amdgpu_buffer_rsrc_t qr =
        rows_rsrc(a.q + (size_t)q0 * a.ldq, max(min(16, a.rows - q0), 0) * a.ldq * 2);
#pragma unroll
    for (int kq = 0; kq < 8; ++kq) qf[kq] = buf_load8(qr, (r * a.ldq + kq * 32 + g * 8) * 2);
  }

  const __amdgpu_buffer_rsrc_t kr = rows_rsrc(a.k, a.keys * a.ldkv * 2);
  const __amdgpu_buffer_rsrc_t vr = rows_rsrc(a.v, a.keys * a.ldkv * 2);
  const int srow = t >> 5, sch = t & 31;     // staging: 8 rows x 32 chunks per pass
  bf16x8 kv[8], vv[8];
  auto issue = [&](int kb) {
    const int off = ((kb * EA_KB + srow) * a.ldkv + sch * 8) * 2;
    const int step = 8 * a.ldkv * 2;
#pragma unroll
    for (int j = 0; j < 8; ++j) kv[j] = buf_load8(kr, off + j * step);
#pragma unroll
    for (int j = 0; j < 8; ++j) vv[j] = buf_load8(vr, off + j * step);
  };

  float m_run = -1.0e30f, l_run = 0.f;     // per query row r (replicated over g)
  f32x4 o[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) o[dt] = zero4();

  const int nblk = (a.keys + EA_KB - 1) / EA_KB;
  issue(0);
  for (int kb = 0; kb < nblk; ++kb) {
    __syncthreads();                           // previous block fully consumed
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      *reinterpret_cast<bf16x8*>(&ks_[srow + 8 * j][sch * 8]) = kv[j];
      *reinterpret_cast<bf16x8*>(&vs_[srow + 8 * j][sch * 8]) = vv[j];
    }
    __syncthreads();
    if (kb + 1 < nblk) issue(kb + 1);

    const int kw = half * 32;
    f32x4 st[2] = {zero4(), zero4()};
#pragma unroll
    for (int kq = 0; kq < 8; ++kq) {
      const bf16x8 k0f = *reinterpret_cast<const bf16x8*>(&ks_[kw + r][kq * 32 + g * 8]);
      const bf16x8 k1f = *reinterpret_cast<const bf16x8*>(&ks_[kw + 16 + r][kq * 32 + g * 8]);
      st[0] = mfma16(k0f, qf[kq], st[0]);
      st[1] = mfma16(k1f, qf[kq], st[1]);
    }
    float s[8], mx = -1.0e30f;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = kb * EA_KB + kw + nt * 16 + g * 4 + e;
        const float v = key < a.keys ? round_bf(st[nt][e]) * a.scale_log2 : -1.0e30f;
        s[nt * 4 + e] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, PI0_WAVE));
    mx = fmaxf(mx, __shfl_xor(mx, 32, PI0_WAVE));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    float ps = 0.f;
    bf16x8 pf;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = fast_exp2(s[j] - m_new);
      ps += p;
      pf[j] = f2bf(p);
    }
    ps += __shfl_xor(ps, 16, PI0_WAVE);
    ps += __shfl_xor(ps, 32, PI0_WAVE);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    // O rows are 4g + e: fetch those rows' rescale factors
    float al[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) al[e] = __shfl(alpha, g * 4 + e, PI0_WAVE);
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const int col = dt * 16 + r;
      bf16x8 vf;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vf[j] = vs_[kw + g * 4 + j][col];
        vf[4 + j] = vs_[kw + 16 + g * 4 + j][col];
      }
      f32x4 sc;
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[e] = o[dt][e] * al[e];
      o[dt] = mfma16(pf, vf, sc);
    }
  }

  // ---- merge the two key halves of each row tile through LDS
  __syncthreads();
  if (half == 1 && g == 0) { mrg_m[rt][r] = m_run; mrg_l[rt][r] = l_run; }
  float* ob = reinterpret_cast<float*>(&ks_[0][0]);     // [2 row tiles][16][EA_OP], half 1 only
  if (half == 1) {
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) ob[(rt * 16 + g * 4 + e) * EA_OP + dt * 16 + r] = o[dt][e];
  }
  __syncthreads();
  if (half == 1) return;
  // wave rt (key half 0) merges with wave rt + 2 (key half 1) of the same row tile
  float w0[4], w1[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int rr = g * 4 + e;
    const float ma = __shfl(m_run, rr, PI0_WAVE), la = __shfl(l_run, rr, PI0_WAVE);
    const float mb = mrg_m[rt][rr], lb = mrg_l[rt][rr];
    const float M = fmaxf(ma, mb);
    const float ea = fast_exp2(ma - M), eb = fast_exp2(mb - M);
    const float inv = __builtin_amdgcn_rcpf(la * ea + lb * eb);
    w0[e] = ea * inv;
    w1[e] = eb * inv;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = q0 + g * 4 + e;
    if (row >= a.rows) continue;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const float v = o[dt][e] * w0[e] + ob[(rt * 16 + g * 4 + e) * EA_OP + dt * 16 + r] * w1[e];
      a.out[(size_t)row * a.ldo + dt * 16 + r] = f2bf(v);
    }
  }
}

}  // namespace pi0

using namespace pi0;

// ---- host-side launch helpers ----------------------------------------------------

template <int BM, int WN, int D, int EPI, bool DUAL, int OCC>
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
  hipLaunchKernelGGL((tile_gemm_kernel<BM, WN, D, EPI, DUAL, OCC>), dim3(grid), dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

// Pipeline depth: the deepest even ring (<= DMAX) whose depth divides the per-split step count.
template <int BM, int WN, int DMAX, int EPI, bool DUAL, int OCC = 1>
static int launch_tile_auto(TileArgs a, hipStream_t s) {
  if (a.K % 64 || a.splitk < 1 || (a.K / 64) % a.splitk) return PI0HIP_ERR_SHAPE;
  const int steps = a.K / 64 / a.splitk;
  if (DMAX >= 8 && steps % 8 == 0) return launch_tile<BM, WN, (DMAX >= 8 ? 8 : 2), EPI, DUAL, OCC>(a, s);
  if (DMAX >= 6 && steps % 6 == 0) return launch_tile<BM, WN, (DMAX >= 6 ? 6 : 2), EPI, DUAL, OCC>(a, s);
  if (DMAX >= 4 && steps % 4 == 0) return launch_tile<BM, WN, (DMAX >= 4 ? 4 : 2), EPI, DUAL, OCC>(a, s);
  if (steps % 2 == 0) return launch_tile<BM, WN, 2, EPI, DUAL, OCC>(a, s);
  return PI0HIP_ERR_SHAPE;
}

static TileArgs tile_args(const void* x, int ldx, const void* w, void* out, int ldo, int M, int N,
                          int K) {
  TileArgs a = {};
  a.a = (const __bf16*)x; a.lda = ldx; a.w0 = (const __bf16*)w;
  a.out = (__bf16*)out; a.ldo = ldo;
  a.M = M; a.N = N; a.K = K; a.splitk = 1;
  return a;
}

static bool bad_dims(int M, int N, int K) { return M <= 0 || N <= 0 || K <= 0; }

extern "C" {

int pi0hip_pack_weight32(const void* w, void* packed, int K, int N, int batch, hipStream_t s) {
  if (!w || !packed || K <= 0 || N <= 0 || batch <= 0) return PI0HIP_ERR_ARG;
  if (K % 16 || N % 32) return PI0HIP_ERR_SHAPE;
  const long long frags = (long long)batch * (K / 16) * (N / 32) * 64;
  const long long blocks = (frags + 255) / 256;
  hipLaunchKernelGGL(pack_weight32_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     (const __bf16*)w, (__bf16*)packed, K, N, frags);
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
  TileArgs a = tile_args(x, ldx, w_packed, out, ldo, M, N, K);
  a.bias = (const __bf16*)bias;
  return bias ? launch_tile_auto<64, 32, 8, TE_BIAS, false>(a, s)
              : launch_tile_auto<64, 32, 8, TE_STORE, false>(a, s);
}

int pi0hip_tile_linear_residual(const void* x, int ldx, const void* w_packed, void* out, int ldo,
                                int M, int N, int K, int splitk, void* ws, size_t ws_bytes,
                                hipStream_t s) {
  if (!x || !w_packed || !out || bad_dims(M, N, K) || splitk < 1) return PI0HIP_ERR_ARG;
  TileArgs a = tile_args(x, ldx, w_packed, out, ldo, M, N, K);
  a.splitk = splitk;
  if (splitk == 1) return launch_tile_auto<64, 32, 8, TE_RES, false>(a, s);
  if (N % 4 || ldo % 4) return PI0HIP_ERR_SHAPE;
  if (!ws || ws_bytes < pi0hip_tile_workspace_bytes(M, N, splitk)) return PI0HIP_ERR_WORKSPACE;
  a.part = (float*)ws;
  if (int e = launch_tile_auto<192, 32, 4, TE_PARTIAL, false>(a, s)) return e;
  hipLaunchKernelGGL(tile_reduce_res_kernel, dim3((M * (N / 4) + 255) / 256), dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

int pi0hip_tile_gated_ffn(const void* x, int ldx, const void* gate_packed, const void* up_packed,
                          void* out, int ldo, int M, int N, int K, hipStream_t s) {
  if (!x || !gate_packed || !up_packed || !out || bad_dims(M, N, K)) return PI0HIP_ERR_ARG;
  TileArgs a = tile_args(x, ldx, gate_packed, out, ldo, M, N, K);
  a.w1 = (const __bf16*)up_packed;
  return launch_tile_auto<96, 64, 2, TE_GATE, true, 2>(a, s);
}

int pi0hip_tile_qkv_rope(const void* x, int ldx, const void* w_packed, const void* rope, void* q,
                         void* k, void* v, int ldkv, int M, int K, int heads, int head_dim,
                         hipStream_t s) {
  if (!x || !w_packed || !rope || !q || !k || !v || M <= 0 || K <= 0 || heads <= 0)
    return PI0HIP_ERR_ARG;
  if (head_dim % 16) return PI0HIP_ERR_SHAPE;
  TileArgs a = tile_args(x, ldx, w_packed, q, heads * head_dim, M, (heads + 2) * head_dim, K);
  a.out_k = (__bf16*)k; a.out_v = (__bf16*)v; a.ldkv = ldkv;
  a.rope = (const __bf16*)rope; a.heads = heads; a.head_dim = head_dim;
  return launch_tile_auto<64, 32, 8, TE_QKV_ROPE, false>(a, s);
}

int pi0hip_layer_norm(const void* x, int ldx, const void* w, const void* b, void* out, int ldo,
                      int M, int K, float eps, hipStream_t s) {
  if (!x || !w || !b || !out || M <= 0 || K <= 0) return PI0HIP_ERR_ARG;
  if (K % 8 || K > 2048) return PI0HIP_ERR_SHAPE;
  hipLaunchKernelGGL(layer_norm_kernel, dim3((M + 3) / 4), dim3(256), 0, s, (const __bf16*)x, ldx,
                     (const __bf16*)w, (const __bf16*)b, (__bf16*)out, ldo, M, K, eps);
  return (int)hipGetLastError();
}

int pi0hip_encoder_attention(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             void* out, int ldo, int rows, int keys, int head_dim, float scale,
                             hipStream_t s) {
  if (!q || !k || !v || !out || rows <= 0 || keys <= 0) return PI0HIP_ERR_ARG;
  if (head_dim != EA_HD) return PI0HIP_ERR_SHAPE;
  EncAttnArgs a = {};
  a.q = (const __bf16*)q; a.ldq = ldq;
  a.k = (const __bf16*)k; a.v = (const __bf16*)v; a.ldkv = ldkv;
  a.out = (__bf16*)out; a.ldo = ldo;
  a.rows = rows; a.keys = keys;
  a.scale_log2 = 1.4426950408889634f * scale;
  hipLaunchKernelGGL(enc_attn_kernel, dim3((rows + 31) / 32), dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

}  // extern "C"
