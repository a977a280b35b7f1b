// Skinny bf16 MFMA GEMMs for the Pi0 decoder (M <= 64 rows per block).
//
// Every decoder projection is C[M, N] = x[M, K] @ W[K, N] with M = 50 or 51:
// the cost is streaming W from HBM once. One workgroup (4 waves) owns a
// 16-column tile of W and a K range; each wave issues all of its loads before
// the first MFMA so that the whole slice is in flight at once: its activation
// rows go from L2 straight into LDS (buffer loads with the LDS destination) in
// 64-column k-blocks, each followed by that k-block's weight fragments (16 bytes
// per lane, one contiguous 1 KB packed fragment per instruction), and the MFMAs
// of a k-block wait only for the loads issued up to it. Waves split K; their
// accumulators are summed in LDS. When the column tiles alone cannot fill the
// chip (N = 1024), K is also split across workgroups: they store fp32 partial
// tiles and a second launch (splitk_reduce_kernel) sums them in split order --
// deterministic -- and runs the epilogue.
//
// The epilogues are the decoder's fused call sites (reference file:line):
//   EPI_BIAS        x@W + b                    decoder_action_mlp  (wrappers.py:123-128)
//   EPI_RES         out += x@W                 o-proj / ffn-down   (wrappers.py:176-189)
//   EPI_RMS_BIAS_RES out += b + f * x@W        action out-proj     (fused_norm.py:81-125)
//   EPI_QKV_ROPE    f * x@W, RoPE, scatter     qkv + rope          (base.py:607-669)
//   EPI_GATE        gelu(f x@Wg) * (f x@Wu)    gated FFN           (fused_norm.py:26-78)
// with f = bf16(rsqrt(mean_k x^2 + 1e-6)) computed from the same A fragments.
// The unfused call sites (op_table(fused=False)) take f from a prior rms-factor pass
// and round x * f to bf16 per element before the MFMA, as the reference's two-kernel
// path does:
//   EPI_GATE_PRE         gelu(bf16(x f)@Wg) * (bf16(x f)@Wu)   (base.py:453-505)
//   EPI_RMS_BIAS_RES_PRE out += b + bf16(x f)@W              (base.py:552-596)
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

constexpr int MAX_SPLITK = 8;
// split-K second pass: threads per workgroup (4 per output row of a 16-column tile, so
// 16 rows; one wave spreads the pass over 4x the CUs of a 64-row workgroup)
constexpr int RED_THREADS = 64;

enum Epi { EPI_BIAS = 0, EPI_RES = 1, EPI_RMS_BIAS_RES = 2, EPI_QKV_ROPE = 3, EPI_GATE = 4,
           EPI_GATE_PRE = 5, EPI_RMS_BIAS_RES_PRE = 6 };

struct GemmArgs {
  const __bf16* x; int ldx;
  const __bf16* w0; const __bf16* w1;
  const __bf16* bias;
  __bf16* out; int ldo;
  __bf16* out_k; __bf16* out_v; int ldkv;
  const __bf16* rope;
  __bf16* norm_factor;
  float* ws;
  int M, N, K, splitk, heads, head_dim;
  int batch;              // EPI_QKV_ROPE: requests stacked "states first" (see gemm_epilogue)
  long long kv_bstride;   // EPI_QKV_ROPE: elements between two requests' K / V caches
  float* out_f32;  // EPI_RMS_BIAS_RES(_PRE): fp32 residual / destination instead of `out`
  const __bf16* prescale;  // *_PRE: per-row bf16 factor applied to x before the MFMA
};

constexpr bool uses_rms(int epi) {
  return epi == EPI_RMS_BIAS_RES || epi == EPI_QKV_ROPE || epi == EPI_GATE;
}
constexpr bool uses_prescale(int epi) { return epi == EPI_GATE_PRE || epi == EPI_RMS_BIAS_RES_PRE; }

// Per-tile scratch layout inside the workspace: [mb][nt][ks][64 rows][16 * ND] fp32,
// then [mb][nt][ks][64] fp32 sums of squares. Counters live in a separate int array.
__host__ __device__ inline size_t part_floats(int tiles, int splitk, int nd) {
  return (size_t)tiles * splitk * 64 * 16 * nd;
}

// RoPE position of output row `row` (EPI_QKV_ROPE). Row order of a batch of B requests:
// the B state tokens first, then the B x T action tokens request by request (for B = 1:
// state, actions). Token t of request b takes RoPE position t, Q row b (T + 1) + t
// (request-major) and cache row t of request b.
__device__ __forceinline__ void qkv_token(const GemmArgs& a, int row, int& b, int& t) {
  const int T = a.M / a.batch - 1;
  b = 0; t = row;
  if (a.batch > 1) {
    if (row < a.batch) { b = row; t = 0; }
    else { b = (row - a.batch) / T; t = 1 + (row - a.batch) - b * T; }
  }
}

// EPI_QKV_ROPE: the (cos, sin) pairs of one 4-column piece, read before the product is
// known (the caller issues this ahead of its operand loads). Unconditional: a resource
// bounded to the table makes rows past M and the V columns read zeros (never used).
__device__ __forceinline__ bf16x4 qkv_rope_piece(const GemmArgs& a, int row, int nt, int c4) {
  const int hd = a.head_dim, qdim = a.heads * hd, n = nt * 16 + c4;
  int b, t;
  qkv_token(a, row, b, t);
  const int npos = a.M / a.batch;
  const __amdgpu_buffer_rsrc_t rr = rows_rsrc_sgpr(a.rope, npos * hd * (int)sizeof(__bf16));
  const int off = row < a.M && n < qdim + hd ? (t * hd + n % hd) * (int)sizeof(__bf16) : INT_MAX - 64;
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(rr, off, 0, 0));
}

// Epilogue of one 4-column piece of output row `row` (columns nt*16 + c4 ..+3) from
// the fp32 accumulators v0 (and v1 for the dual gate/up GEMM) and, for the RMS
// call sites, the row's sum of squares over the full K; rope4 holds the piece's RoPE
// table entries (EPI_QKV_ROPE, read early by the caller).
template <int EPI, bool DUAL>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& a, int row, int nt, int c4,
                                              bool nf_writer, const float* v0, const float* v1,
                                              float ss, bf16x4 rope4 = {}) {
  constexpr bool RMS = uses_rms(EPI);
  if (row >= a.M) return;
  const int n = nt * 16 + c4;
  float f = 1.f;
  if constexpr (RMS) f = round_bf(rsqrtf(ss / (float)a.K + 1e-6f));

  float o[4];
  if constexpr (EPI == EPI_BIAS) {
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = v0[c] + bf2f(a.bias[n + c]);
  } else if constexpr (EPI == EPI_RES) {
    const __bf16* rp = a.out + (size_t)row * a.ldo + n;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = v0[c] + bf2f(rp[c]);
  } else if constexpr (EPI == EPI_RMS_BIAS_RES || EPI == EPI_RMS_BIAS_RES_PRE) {
    if (a.out_f32) {            // fp32 Euler accumulator: read, update and store in fp32
      float* rp = a.out_f32 + (size_t)row * a.ldo + n;
      const f32x4 r4 = *reinterpret_cast<const f32x4*>(rp);
      f32x4 o4;
#pragma unroll
      for (int c = 0; c < 4; ++c) o4[c] = v0[c] * f + bf2f(a.bias[n + c]) + r4[c];
      *reinterpret_cast<f32x4*>(rp) = o4;
      return;
    }
    const __bf16* rp = a.out + (size_t)row * a.ldo + n;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = v0[c] * f + bf2f(a.bias[n + c]) + bf2f(rp[c]);
  } else if constexpr (EPI == EPI_GATE || EPI == EPI_GATE_PRE) {
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = gelu_tanh(v0[c] * f) * (v1[c] * f);
  } else if constexpr (EPI == EPI_QKV_ROPE) {
    const int hd = a.head_dim, qdim = a.heads * hd;
    const int T = a.M / a.batch - 1;
    int b, t;
    qkv_token(a, row, b, t);
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = v0[c] * f;
    if (n < qdim + hd) {
#pragma unroll
      for (int p = 0; p < 4; p += 2) {
        const float cs = bf2f(rope4[p]), sn = bf2f(rope4[p + 1]);
        const float x0 = o[p], x1 = o[p + 1];
        // explicit fused forms: the rounding does not depend on the compiler's contraction
        o[p] = fmaf(x0, cs, -(x1 * sn));
        o[p + 1] = fmaf(x1, cs, x0 * sn);
      }
    }
    __bf16* dst;
    const size_t kv = (size_t)b * a.kv_bstride + (size_t)t * a.ldkv;
    if (n < qdim) dst = a.out + ((size_t)b * (T + 1) + t) * qdim + n;
    else if (n < qdim + hd) dst = a.out_k + kv + (n - qdim);
    else dst = a.out_v + kv + (n - qdim - hd);
    bf16x4 pk = {f2bf(o[0]), f2bf(o[1]), f2bf(o[2]), f2bf(o[3])};
    *reinterpret_cast<bf16x4*>(dst) = pk;
    if (a.norm_factor && nt == 0 && nf_writer) a.norm_factor[row] = f2bf(f);
    return;
  }
  bf16x4 pk = {f2bf(o[0]), f2bf(o[1]), f2bf(o[2]), f2bf(o[3])};
  *reinterpret_cast<bf16x4*>(a.out + (size_t)row * a.ldo + n) = pk;
}

// Issue sequence of the staging loads: with WL < 0 each k-block's x rows then its
// weights; with WL >= 0 the weights of k-block s, then the x rows of k-block s - WL.
// ops_after(kb) = vector-memory ops issued after both halves of k-block kb.
template <int NKB, int WL, int XOPS, int WOPS>
constexpr int ops_after(int kb) {
  int pos = 0, done_x = -1, done_w = -1;
  const int steps = WL < 0 ? NKB : NKB + WL;
  for (int st = 0; st < steps; ++st) {
    if (WL < 0) {
      pos += XOPS; if (st == kb) done_x = pos;
      pos += WOPS; if (st == kb) done_w = pos;
    } else {
      if (st < NKB) { pos += WOPS; if (st == kb) done_w = pos; }
      if (st >= WL) { pos += XOPS; if (st - WL == kb) done_x = pos; }
    }
  }
  return pos - (done_x > done_w ? done_x : done_w);
}

template <int EPI, bool DUAL, int KTW, int NW, int WL = -1, int XR = 64>
__global__ __launch_bounds__(NW * 64, 1) void skinny_gemm_kernel(GemmArgs a) {
  constexpr int ND = DUAL ? 2 : 1;
  constexpr bool RMS = uses_rms(EPI);
  constexpr int KW = KTW * 32;            // k columns per wave
  // x staging: k-blocks of KB k-tiles, k-block-major in LDS ([kb][64 rows][KB * 32])
  constexpr int KB = KTW >= 2 ? 2 : 1;    // k-tiles per k-block
  constexpr int NKB = KTW / KB;
  constexpr int BCH = KB * 4;             // 16-byte chunks per row of a k-block
  constexpr int XIB = BCH;                // load instructions per k-block (64 rows x 16 B x BCH)
  constexpr int BRPI = PI0_WAVE / BCH;    // rows per load instruction
  constexpr int OPS = XIB + KB * ND;      // vector-memory ops issued per k-block
  static_assert(NKB <= 4 && 3 * OPS <= 63, "k-block waits");
  constexpr int XIS = XR / BRPI;          // x load instructions issued per k-block
  static_assert(XIS * BRPI == XR && XIS <= XIB, "staged rows");   // XR: x rows staged
  constexpr size_t X_BYTES = NW * 64 * KW * 2;
  constexpr size_t R_BYTES = (ND * NW * 4 * 4 * PI0_WAVE + NW * 4 * PI0_WAVE) * 4;
  __shared__ __attribute__((aligned(16))) char smem[X_BYTES > R_BYTES ? X_BYTES : R_BYTES];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int splitk = a.splitk;
  const int ntiles = a.N >> 4;
  const int nt = blockIdx.x / splitk, ks = blockIdx.x - nt * splitk;
  const int mb = blockIdx.y, m0 = mb * 64;
  const int rows = min(64, a.M - m0);
  const int KT = a.K >> 5;
  const int kt0 = ks * (KT / splitk) + wave * KTW;

  // 16-byte chunk c of row `row` of a k-block sits at chunk c ^ swz(row): the fragment
  // reads of 8 consecutive rows then hit distinct banks
  auto swz = [](int row) { return BCH == 8 ? (row & 7) : ((row >> 1) & 3); };
  __bf16* xs = reinterpret_cast<__bf16*>(smem) + wave * 64 * KW;
  bf16x8 b0[KTW], b1[KTW];
  // *_PRE: this lane's row factors (rows mt*16 + lane%16), loaded before the staging
  // loads so that every k-block wait below also covers them
  float fpre[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (uses_prescale(EPI)) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) fpre[mt] = bf2f(a.prescale[m0 + min(mt * 16 + (lane & 15), rows - 1)]);
  }
  // EPI_QKV_ROPE: this thread's epilogue piece (row t / 4, columns 4 (t % 4)..) needs four
  // RoPE table entries; issued first, they are the oldest load under every k-block wait
  bf16x4 rope4 = {};
  if constexpr (EPI == EPI_QKV_ROPE) rope4 = qkv_rope_piece(a, m0 + (t >> 2), nt, (t & 3) * 4);
  __builtin_amdgcn_sched_barrier(0);
  PI0_PROBE(0);
  // ---- issue: this wave's x slice [64 x KW] goes straight from L2 into LDS (buffer
  // loads with the LDS destination), one k-block at a time, each followed by the
  // weight fragments of its k-tiles (cold, 16 bytes per lane, 1 KB per instruction), or
  // with WL >= 0 the weight fragments WL k-blocks ahead of the x rows.
  // The scheduling barriers keep this order, which the k-block waits below count on.
  // The buffer resource ends after row `rows`: rows past M arrive as zeros (XR < 64: rows
  // XR..63 are not loaded at all).
  {
    const __amdgpu_buffer_rsrc_t xr =
        rows_rsrc(a.x + (size_t)m0 * a.ldx, rows * a.ldx * (int)sizeof(__bf16));
    const int lrow0 = lane / BCH, lp = lane % BCH;
    const __bf16* wp = a.w0 + ((size_t)nt * KT + kt0) * 512 + lane * 8;
    const __bf16* wq = a.w1 + ((size_t)nt * KT + kt0) * 512 + lane * 8;
    auto issue_x = [&](int kb) {
#pragma unroll
      for (int q = 0; q < XIS; ++q) {
        const int row = q * BRPI + lrow0, c = lp ^ swz(row);
        buf_load16_lds(xr, xs + kb * 64 * KB * 32 + q * 512,
                       (row * a.ldx + (kt0 + kb * KB) * 32 + c * 8) * (int)sizeof(__bf16));
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    auto issue_w = [&](int kb) {
#pragma unroll
      for (int k2 = 0; k2 < KB; ++k2) {
        b0[kb * KB + k2] = load8(wp + (kb * KB + k2) * 512);
        if constexpr (DUAL) b1[kb * KB + k2] = load8(wq + (kb * KB + k2) * 512);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (WL < 0) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) { issue_x(kb); issue_w(kb); }
    } else {
#pragma unroll
      for (int st = 0; st < NKB + WL; ++st) {
        if (st < NKB) issue_w(st);
        if (st >= WL) issue_x(st - WL);
      }
    }
  }
  PI0_PROBE(3);
  // (each wave reads only the rows it staged itself: no workgroup barrier needed)

  const int r = lane & 15, g = lane >> 4;
  f32x4 acc0[4], acc1[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) { acc0[mt] = zero4(); acc1[mt] = zero4(); }
  float ssl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KTW; ++i) {
    if (i % KB == 0) {
      // k-block i / KB: memory operations complete in issue order, so once at most the
      // operations issued after both of its halves are outstanding, its x chunks are in
      // LDS and its weight fragments in registers
      __builtin_amdgcn_sched_barrier(0);
      constexpr int WOPS = KB * ND;
      switch (i / KB) {   // folds to one s_waitcnt once the loop is unrolled
        case 0: __builtin_amdgcn_s_waitcnt(PI0_VMCNT((ops_after<NKB, WL, XIS, WOPS>(0)))); break;
        case 1: __builtin_amdgcn_s_waitcnt(PI0_VMCNT((ops_after<NKB, WL, XIS, WOPS>(1)))); break;
        case 2: __builtin_amdgcn_s_waitcnt(PI0_VMCNT((ops_after<NKB, WL, XIS, WOPS>(2)))); break;
        default: __builtin_amdgcn_s_waitcnt(PI0_VMCNT((ops_after<NKB, WL, XIS, WOPS>(3)))); break;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int xrow = mt * 16 + r;
      bf16x8 av = *reinterpret_cast<const bf16x8*>(
          xs + (i / KB) * 64 * KB * 32 + xrow * KB * 32 + ((((i % KB) * 4 + g) ^ swz(xrow)) * 8));
      if constexpr (uses_prescale(EPI)) {
#pragma unroll
        for (int j = 0; j < 8; ++j) av[j] = f2bf(bf2f(av[j]) * fpre[mt]);
      }
      acc0[mt] = mfma16(av, b0[i], acc0[mt]);
      if constexpr (DUAL) acc1[mt] = mfma16(av, b1[i], acc1[mt]);
      if constexpr (RMS) {       // sum of squares with v_dot2 (two bf16 products per op)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x2 q = {av[2 * j], av[2 * j + 1]};
          ssl[mt] = __builtin_amdgcn_fdot2_f32_bf16(q, q, ssl[mt], false);
        }
      }
    }
  }
  PI0_PROBE(4);
  __syncthreads();                        // x staging area becomes the reduction area

  // ---- intra-workgroup reduction over the NW waves' K ranges
  typedef float RedT[NW][4][4][PI0_WAVE];  // [wave][mt][i][lane]
  RedT* red = reinterpret_cast<RedT*>(smem);
  float (*ssred)[4][PI0_WAVE] = reinterpret_cast<float (*)[4][PI0_WAVE]>(
      smem + ND * sizeof(RedT));
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[0][wave][mt][i][lane] = acc0[mt][i];
      if constexpr (DUAL) red[ND - 1][wave][mt][i][lane] = acc1[mt][i];
    }
    if constexpr (RMS) ssred[wave][mt][lane] = ssl[mt];
  }
  __syncthreads();

  PI0_PROBE(5);
  // thread t < 256 owns row t/4 (of 64) and columns 4*(t%4) .. +3 of the tile
  if (NW > 4 && t >= 256) return;
  const int lrow = t >> 2, c4 = (t & 3) * 4;
  const int mt = lrow >> 4, r16 = lrow & 15, ii = r16 & 3, gg = r16 >> 2;
  float v0[4], v1[4], ss = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      s0 += red[0][w][mt][ii][gg * 16 + c4 + c];
      if constexpr (DUAL) s1 += red[ND - 1][w][mt][ii][gg * 16 + c4 + c];
    }
    v0[c] = s0; v1[c] = s1;
  }
  if constexpr (RMS) {
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int q = 0; q < 4; ++q) ss += ssred[w][mt][q * 16 + r16];
  }

  // ---- split-K across workgroups: publish the fp32 partial tile (plain stores; the
  // kernel boundary orders them before splitk_reduce_kernel, which sums the splits
  // in order -- deterministic -- and runs the epilogue)
  if (splitk > 1) {
    const int tile = mb * ntiles + nt;
    const size_t tiles = (size_t)gridDim.y * ntiles;
    float* p = a.ws + (((size_t)tile * splitk + ks) * 64 + lrow) * 16 * ND + c4;
    *reinterpret_cast<f32x4*>(p) = f32x4{v0[0], v0[1], v0[2], v0[3]};
    if constexpr (DUAL) *reinterpret_cast<f32x4*>(p + 16) = f32x4{v1[0], v1[1], v1[2], v1[3]};
    if (RMS && (t & 3) == 0)
      a.ws[part_floats((int)tiles, splitk, ND) + ((size_t)tile * splitk + ks) * 64 + lrow] = ss;
    return;
  }
  gemm_epilogue<EPI, DUAL>(a, m0 + lrow, nt, c4, (t & 3) == 0, v0, v1, ss, rope4);
  PI0_PROBE(6);
}


// Second pass of split-K: one workgroup per 64 x 16 output tile; thread t owns row
// t/4, columns 4*(t%4)..; sums the splits in split order, then the epilogue. SK is the
// split count when it is known at compile time (exactly SK partial loads), 0 for any
// count up to MAX_SPLITK. The residual of the EPI_RES call sites is loaded together
// with the partials, so the kernel pays one memory round trip, not two.
template <int EPI, bool DUAL, int SK>
__global__ __launch_bounds__(RED_THREADS) void splitk_reduce_kernel(GemmArgs a) {
  constexpr int ND = DUAL ? 2 : 1;
  constexpr bool RMS = uses_rms(EPI);
  constexpr int NL = SK > 0 ? SK : MAX_SPLITK;
  constexpr int QUARTERS = 256 / RED_THREADS;             // workgroups per 64-row tile
  const int mb = blockIdx.y / QUARTERS;
  const int t = threadIdx.x, lrow = (blockIdx.y % QUARTERS) * RED_THREADS / 4 + (t >> 2);
  const int c4 = (t & 3) * 4;
  const int nt = blockIdx.x, ntiles = gridDim.x;
  const int tile = mb * ntiles + nt, splitk = SK > 0 ? SK : a.splitk;
  const size_t tiles = (size_t)(gridDim.y / QUARTERS) * ntiles;
  const int row = mb * 64 + lrow;
  if (mb * 64 + (blockIdx.y % QUARTERS) * RED_THREADS / 4 >= a.M) return;   // padding rows only
  bf16x4 res4 = {};
  if constexpr (EPI == EPI_RES) {
    if (row < a.M) res4 = *reinterpret_cast<const bf16x4*>(a.out + (size_t)row * a.ldo + nt * 16 + c4);
  }
  f32x4 q0[NL], q1[NL];
  float qs[NL];
#pragma unroll
  for (int k = 0; k < NL; ++k) {     // unconditional loads; extra ones (SK = 0) are ignored
    const int kk = SK > 0 ? k : min(k, splitk - 1);
    const float* p = a.ws + (((size_t)tile * splitk + kk) * 64 + lrow) * 16 * ND + c4;
    q0[k] = *reinterpret_cast<const f32x4*>(p);
    if constexpr (DUAL) q1[k] = *reinterpret_cast<const f32x4*>(p + 16);
    if constexpr (RMS) qs[k] = a.ws[part_floats((int)tiles, splitk, ND) + ((size_t)tile * splitk + kk) * 64 + lrow];
  }
  float v0[4] = {0.f, 0.f, 0.f, 0.f}, v1[4] = {0.f, 0.f, 0.f, 0.f}, ss = 0.f;
#pragma unroll
  for (int k = 0; k < NL; ++k) {
    if (SK > 0 || k < splitk) {
#pragma unroll
      for (int c = 0; c < 4; ++c) v0[c] += q0[k][c];
      if constexpr (DUAL) {
#pragma unroll
        for (int c = 0; c < 4; ++c) v1[c] += q1[k][c];
      }
      if constexpr (RMS) ss += qs[k];
    }
  }
  if constexpr (EPI == EPI_RES) {
    if (row >= a.M) return;
    const bf16x4 pk = {f2bf(v0[0] + bf2f(res4[0])), f2bf(v0[1] + bf2f(res4[1])),
                       f2bf(v0[2] + bf2f(res4[2])), f2bf(v0[3] + bf2f(res4[3]))};
    *reinterpret_cast<bf16x4*>(a.out + (size_t)row * a.ldo + nt * 16 + c4) = pk;
    return;
  }
  bf16x4 rope4 = {};
  if constexpr (EPI == EPI_QKV_ROPE) rope4 = qkv_rope_piece(a, row, nt, c4);
  gemm_epilogue<EPI, DUAL>(a, row, nt, c4, (t & 3) == 0, v0, v1, ss, rope4);
}

// x rows are read (and copied into LDS) 16 bytes at a time; outputs are stored four
// elements at a time (8 bytes, 16 for the fp32 Euler accumulator)
static bool bad_alignment(const GemmArgs& a) {
  const auto off = [](const void* p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & m) != 0; };
  if (off(a.x, 15) || (a.ldx & 7) || a.ldx < a.K || (a.ldo & 3)) return true;
  if (a.out_f32 ? off(a.out_f32, 15) : off(a.out, 7)) return true;
  if (a.out_k && (off(a.out_k, 7) || off(a.out_v, 7) || (a.ldkv & 3))) return true;
  return false;
}

template <int EPI, bool DUAL>
static int launch_gemm(const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0) return PI0HIP_ERR_ARG;
  if (a.K % 32 || a.N % 16 || a.splitk < 1 || a.splitk > MAX_SPLITK) return PI0HIP_ERR_SHAPE;
  if (bad_alignment(a)) return PI0HIP_ERR_SHAPE;
  const int KT = a.K / 32;
  if (KT % (4 * a.splitk)) return PI0HIP_ERR_SHAPE;
  if (a.splitk > 1 && !a.ws) return PI0HIP_ERR_WORKSPACE;
  // 4 waves split the workgroup's K range (8 or 16 waves with fewer loads each measured
  // slower: the cross-wave reduction grows with the wave count)
  constexpr int nw = 4;
  const int kts = KT / a.splitk;
  const int ktw = kts / nw;
  dim3 grid((a.N / 16) * a.splitk, (a.M + 63) / 64);
#define PI0_SKINNY(KTW_, NW_) skinny_gemm_kernel<EPI, DUAL, KTW_, NW_><<<grid, NW_ * 64, 0, s>>>(a)
  if (ktw == 1) PI0_SKINNY(1, 4);
  else if (ktw == 2) PI0_SKINNY(2, 4);
  else if (ktw == 4) PI0_SKINNY(4, 4);
  else if (ktw == 8) {
    // QKV: all weight fragments before the x rows. Inside the decoder loop x comes from the
    // previous launch's freshly written rows while the weights stream cold from HBM, so the
    // weights go first: 0.055 ms per chunk. The gate measured 6% slower alone that way.
    // one row block of at most 56 rows (the decoder's 51): the last x load instruction of
    // each k-block (rows 56-63) is not issued. Those LDS rows keep stale values; each
    // product row depends only on its own x row and rows past M are not stored.
    // Cold gate 6.71 -> 6.57 us, loop 5.881 -> 5.870 ms per chunk.
    const bool x56 = grid.y == 1 && a.M <= 56;
    if constexpr (EPI == EPI_QKV_ROPE) {
      if (x56) skinny_gemm_kernel<EPI, DUAL, 8, 4, 4, 56><<<grid, 256, 0, s>>>(a);
      else skinny_gemm_kernel<EPI, DUAL, 8, 4, 4><<<grid, 256, 0, s>>>(a);
    } else if constexpr (EPI == EPI_GATE) {
      if (x56) skinny_gemm_kernel<EPI, DUAL, 8, 4, -1, 56><<<grid, 256, 0, s>>>(a);
      else PI0_SKINNY(8, 4);
    } else PI0_SKINNY(8, 4);
  }
  else return PI0HIP_ERR_SHAPE;
#undef PI0_SKINNY
  if (a.splitk > 1) {
    if (hipError_t e = hipGetLastError()) return (int)e;
    const dim3 rgrid(a.N / 16, (a.M + 63) / 64 * (256 / RED_THREADS));
    const dim3 rblock(RED_THREADS);
    switch (a.splitk) {
      case 2: hipLaunchKernelGGL((splitk_reduce_kernel<EPI, DUAL, 2>), rgrid, rblock, 0, s, a); break;
      case 4: hipLaunchKernelGGL((splitk_reduce_kernel<EPI, DUAL, 4>), rgrid, rblock, 0, s, a); break;
      case 8: hipLaunchKernelGGL((splitk_reduce_kernel<EPI, DUAL, 8>), rgrid, rblock, 0, s, a); break;
      default: hipLaunchKernelGGL((splitk_reduce_kernel<EPI, DUAL, 0>), rgrid, rblock, 0, s, a); break;
    }
  }
  return (int)hipGetLastError();
}


// Row-split GEMM: out[M, N] (+)= x[M, K] @ W[K, N] (+ epilogue) in one launch, no split-K.
// Workgroup = 16 rows x 16 columns over the whole K; its NW waves split K and are summed
// through LDS. With M = 51 and N = 1024 that is 4 row blocks x 64 column tiles = 256
// workgroups, so the chip fills without fp32 partials and without a second (reduce)
// launch. Each wave copies its x slice (16 rows x K / NW) from L2 straight into LDS with
// loads that each read whole contiguous row segments (a load whose 16 lanes sit on 16
// rows 2-8 KB apart is ~2x slower), 16-byte chunks XOR-swizzled by row so the A-fragment
// reads are free of bank conflicts; the packed B fragments go to registers. The 4 row
// blocks of a column tile are placed on one XCD (workgroup b runs on XCD b % 8), so its
// weight tile crosses HBM once and the other three read it from that XCD's L2.
template <int EPI, int KTW, int NW>
__global__ __launch_bounds__(NW * 64, 1) void rows16_kernel(GemmArgs a, int nrb, int xcd_map) {
  constexpr int KW = KTW * 32;                 // k per wave
  constexpr int CPR = KW / 8;                  // 16-byte chunks per row of the wave's slice
  constexpr int RPI = PI0_WAVE / CPR;          // rows per load instruction
  constexpr int XI = 16 / RPI;                 // load instructions per wave
  constexpr int SWM = (CPR < 16 ? CPR : 16) - 1;
  constexpr bool RMS = uses_rms(EPI), PRE = uses_prescale(EPI);
  static_assert(RPI >= 1 && RPI * CPR == PI0_WAVE && XI * RPI == 16, "slice shape");
  static_assert(EPI == EPI_RES || EPI == EPI_BIAS || EPI == EPI_RMS_BIAS_RES ||
                EPI == EPI_RMS_BIAS_RES_PRE, "row-split epilogues");
  // (EPI_BIAS and the Euler out-projection epilogues were measured on the small per-step
  // projections too: 0.02 ms per chunk, below box-to-box noise, so only EPI_RES ships)
  constexpr size_t X_BYTES = (size_t)NW * 16 * KW * 2;
  __shared__ __attribute__((aligned(16))) char smem[X_BYTES];
  __shared__ float ssw[NW][16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int KT = a.K >> 5;
  int nt, rb;
  if (xcd_map) {            // column tiles congruent to the XCD index, all row blocks each
    const int b = blockIdx.x, xcd = b & 7, j = b >> 3;
    nt = (j / nrb) * 8 + xcd;
    rb = j - (j / nrb) * nrb;
  } else {
    nt = blockIdx.x / nrb;
    rb = blockIdx.x - nt * nrb;
  }
  const int m0 = rb * 16, rows = min(16, a.M - m0);
  const int kt0 = wave * KTW;
  const int r = lane & 15, g = lane >> 4;
  float fpre = 1.f;
  if constexpr (PRE) fpre = bf2f(a.prescale[m0 + min(r, rows - 1)]);
  // bounded resource over this row block: rows past M read as zeros
  const __amdgpu_buffer_rsrc_t xr =
      rows_rsrc_sgpr(a.x + (size_t)m0 * a.ldx, rows * a.ldx * (int)sizeof(__bf16));
  char* xs = smem + (size_t)wave * 16 * KW * 2;
  {
    const int lrow = lane / CPR, c = lane % CPR;
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int row = i * RPI + lrow;
      // LDS slot (row, c) receives global chunk c ^ swz(row)
      buf_load16_lds(xr, xs + i * 1024,
                     (row * a.ldx + kt0 * 32 + ((c ^ (row & SWM)) * 8)) * (int)sizeof(__bf16));
    }
  }
  const __bf16* wq = a.w0 + ((size_t)nt * KT + kt0) * 512 + lane * 8;
  bf16x8 bv[KTW];
#pragma unroll
  for (int i = 0; i < KTW; ++i) bv[i] = load8(wq + i * 512);
  // EPI_RES: the residual element this thread finishes (row t / 16, column t % 16) does not
  // depend on the product, so it is read now, under the same wait as the operands (an
  // unconditional load through a resource bounded to the row block: out of range reads 0)
  float resv = 0.f;
  if constexpr (EPI == EPI_RES) {
    const __amdgpu_buffer_rsrc_t orr =
        rows_rsrc_sgpr(a.out + (size_t)m0 * a.ldo, rows * a.ldo * (int)sizeof(__bf16));
    const int off = t < 256 ? ((t >> 4) * a.ldo + nt * 16 + (t & 15)) * (int)sizeof(__bf16)
                            : INT_MAX - 64;
    resv = bf2f(__builtin_bit_cast(__bf16, __builtin_amdgcn_raw_buffer_load_b16(orr, off, 0, 0)));
  }
  __builtin_amdgcn_s_waitcnt(PI0_VMCNT(0));    // this wave's LDS copies and fragments
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc = zero4();
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < KTW; ++i) {
    const int ch = (i * 4 + g) ^ (r & SWM);
    bf16x8 av = *reinterpret_cast<const bf16x8*>(xs + (r * CPR + ch) * 16);
    if constexpr (RMS) {     // the row's sum of squares from the same fragments
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bf16x2 q = {av[2 * e], av[2 * e + 1]};
        ss = __builtin_amdgcn_fdot2_f32_bf16(q, q, ss, false);
      }
    }
    if constexpr (PRE) {
#pragma unroll
      for (int e = 0; e < 8; ++e) av[e] = f2bf(bf2f(av[e]) * fpre);
    }
    acc = mfma16(av, bv[i], acc);
  }
  if constexpr (RMS) {
    ss += __shfl_xor(ss, 16, PI0_WAVE);
    ss += __shfl_xor(ss, 32, PI0_WAVE);
    if (g == 0) ssw[wave][r] = ss;
  }
  __syncthreads();                             // every wave is done with its x slice
  float (*red)[4][PI0_WAVE] = reinterpret_cast<float (*)[4][PI0_WAVE]>(smem);
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][i][lane] = acc[i];
  __syncthreads();
  // thread t: row t / 16, column t % 16; C lane (row / 4) * 16 + col holds element row % 4
  const int row = t >> 4, col = t & 15;
  if (t >= 256 || row >= rows) return;
  const int l = (row >> 2) * 16 + col, i = row & 3;
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) v += red[w][i][l];
  const int n = nt * 16 + col;
  const size_t o = (size_t)(m0 + row) * a.ldo + n;
  if constexpr (EPI == EPI_RES) {
    a.out[o] = f2bf(v + resv);
  } else if constexpr (EPI == EPI_BIAS) {
    a.out[o] = f2bf(v + bf2f(a.bias[n]));
  } else {
    float f = 1.f;
    if constexpr (RMS) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum += ssw[w][row];
      f = round_bf(rsqrtf(sum / (float)a.K + 1e-6f));
    }
    if (a.out_f32) a.out_f32[o] += v * f + bf2f(a.bias[n]);   // fp32 Euler accumulator
    else a.out[o] = f2bf(v * f + bf2f(a.bias[n]) + bf2f(a.out[o]));
  }
}

// W[batch][K][N] row-major -> packed B fragments, one thread per 16-byte fragment row.
__global__ void pack_weight_kernel(const __bf16* __restrict__ w, __bf16* __restrict__ p,
                                   int K, int N, long long total_frags) {
  const long long f = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= total_frags) return;
  const long long per = (long long)(K / 32) * (N / 16) * 64;
  const long long b = f / per;
  long long rem = f - b * per;
  const int lane = (int)(rem & 63);
  rem >>= 6;
  const int KT = K / 32;
  const int kt = (int)(rem % KT), nt = (int)(rem / KT);
  const int n = nt * 16 + (lane & 15);
  const int k0 = kt * 32 + (lane >> 4) * 8;
  const __bf16* src = w + b * (long long)K * N + (long long)k0 * N + n;
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = src[(long long)j * N];
  *reinterpret_cast<bf16x8*>(p + f * 8) = v;
}

}  // namespace pi0

using namespace pi0;


static inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

template <int EPI>
static int launch_rows(const GemmArgs& a, hipStream_t s) {
  if (!a.x || !a.w0 || !(a.out || a.out_f32) || a.M <= 0 || a.N <= 0 || a.K <= 0)
    return PI0HIP_ERR_ARG;
  if (a.N % 16 || a.ldx < a.K || (a.ldx & 7) || (reinterpret_cast<uintptr_t>(a.x) & 15))
    return PI0HIP_ERR_SHAPE;
  const int nrb = (a.M + 15) / 16, ntiles = a.N / 16;
  const int grid = nrb * ntiles;
  const int xcd_map = ntiles % 8 == 0;
  // 8 waves split K (at most 16 fragments of W in registers per wave). (Spare workgroups
  // prefetching the ffn-down weights from this launch measured slower: it is bound by its
  // CUs' load path.)
  switch (a.K) {
    case 512: rows16_kernel<EPI, 2, 8><<<grid, 512, 0, s>>>(a, nrb, xcd_map); break;
    case 1024: rows16_kernel<EPI, 4, 8><<<grid, 512, 0, s>>>(a, nrb, xcd_map); break;
    case 2048: rows16_kernel<EPI, 8, 8><<<grid, 512, 0, s>>>(a, nrb, xcd_map); break;
    case 4096: rows16_kernel<EPI, 16, 8><<<grid, 512, 0, s>>>(a, nrb, xcd_map); break;
    default: return PI0HIP_ERR_SHAPE;
  }
  return (int)hipGetLastError();
}

extern "C" {

size_t pi0hip_gemm_workspace_bytes(int M, int N, int splitk, int dual) {
  if (splitk <= 1) return 0;
  const size_t tiles = (size_t)((M + 63) / 64) * (N / 16);
  const int nd = dual ? 2 : 1;
  const size_t floats = part_floats((int)tiles, splitk, nd) + tiles * splitk * 64;
  return floats * sizeof(float);
}

static int setup_ws(GemmArgs& a, void* ws, size_t ws_bytes, int dual) {
  if (a.splitk <= 1) { a.ws = nullptr; return 0; }
  const size_t need = pi0hip_gemm_workspace_bytes(a.M, a.N, a.splitk, dual);
  if (!ws || ws_bytes < need) return PI0HIP_ERR_WORKSPACE;
  a.ws = reinterpret_cast<float*>(ws);
  return 0;
}

static GemmArgs base_args(const void* x, int ldx, const void* w, void* out, int ldo,
                          int M, int N, int K, int splitk) {
  GemmArgs a = {};
  a.batch = 1;
  a.x = (const __bf16*)x; a.ldx = ldx; a.w0 = (const __bf16*)w;
  a.out = (__bf16*)out; a.ldo = ldo;
  a.M = M; a.N = N; a.K = K; a.splitk = splitk;
  return a;
}

int pi0hip_pack_weight(const void* w, void* packed, int K, int N, int batch, hipStream_t s) {
  if (!w || !packed || K <= 0 || N <= 0 || batch <= 0) return PI0HIP_ERR_ARG;
  if (K % 32 || N % 16) return PI0HIP_ERR_SHAPE;
  const long long frags = (long long)batch * (K / 32) * (N / 16) * 64;
  const int threads = 256;
  const long long blocks = (frags + threads - 1) / threads;
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)blocks), dim3(threads), 0, s,
                     (const __bf16*)w, (__bf16*)packed, K, N, frags);
  return (int)hipGetLastError();
}

int pi0hip_linear_bias(const void* x, int ldx, const void* wp, const void* bias, void* out,
                       int ldo, int M, int N, int K, int splitk, void* ws, size_t ws_bytes,
                       hipStream_t s) {
  if (!x || !wp || !bias || !out) return PI0HIP_ERR_ARG;
  GemmArgs a = base_args(x, ldx, wp, out, ldo, M, N, K, splitk);
  a.bias = (const __bf16*)bias;
  if (int e = setup_ws(a, ws, ws_bytes, 0)) return e;
  return launch_gemm<EPI_BIAS, false>(a, s);
}

int pi0hip_linear_residual(const void* x, int ldx, const void* wp, void* out, int ldo,
                           int M, int N, int K, int splitk, void* ws, size_t ws_bytes,
                           hipStream_t s) {
  if (!x || !wp || !out) return PI0HIP_ERR_ARG;
  GemmArgs a = base_args(x, ldx, wp, out, ldo, M, N, K, splitk);
  if (int e = setup_ws(a, ws, ws_bytes, 0)) return e;
  return launch_gemm<EPI_RES, false>(a, s);
}

int pi0hip_linear_residual_rows(const void* x, int ldx, const void* wp, void* out, int ldo,
                                int M, int N, int K, hipStream_t s) {
  return launch_rows<EPI_RES>(base_args(x, ldx, wp, out, ldo, M, N, K, 1), s);
}

int pi0hip_rms_linear_bias_residual(const void* x, int ldx, const void* wp, const void* bias,
                                    void* out, int ldo, int M, int N, int K, int splitk,
                                    void* ws, size_t ws_bytes, hipStream_t s) {
  if (!x || !wp || !bias || !out) return PI0HIP_ERR_ARG;
  GemmArgs a = base_args(x, ldx, wp, out, ldo, M, N, K, splitk);
  a.bias = (const __bf16*)bias;
  if (int e = setup_ws(a, ws, ws_bytes, 0)) return e;
  return launch_gemm<EPI_RMS_BIAS_RES, false>(a, s);
}

int pi0hip_rms_linear_bias_residual_f32(const void* x, int ldx, const void* wp, const void* bias,
                                        float* out, int ldo, int M, int N, int K, int splitk,
                                        void* ws, size_t ws_bytes, hipStream_t s) {
  if (!x || !wp || !bias || !out) return PI0HIP_ERR_ARG;
  if (ldo % 4) return PI0HIP_ERR_SHAPE;
  GemmArgs a = base_args(x, ldx, wp, nullptr, ldo, M, N, K, splitk);
  a.bias = (const __bf16*)bias;
  a.out_f32 = out;
  if (int e = setup_ws(a, ws, ws_bytes, 0)) return e;
  return launch_gemm<EPI_RMS_BIAS_RES, false>(a, s);
}

int pi0hip_norm_qkv_rope_batched(const void* x, int ldx, const void* wp, const void* rope, void* q,
                                 void* k, void* v, int ldkv, long long kv_bstride,
                                 void* norm_factor, int M, int K, int heads, int head_dim,
                                 int batch, hipStream_t s) {
  if (!x || !wp || !rope || !q || !k || !v || batch <= 0 || M <= 0) return PI0HIP_ERR_ARG;
  if (head_dim % 16 || heads <= 0 || M % batch || M / batch < 2) return PI0HIP_ERR_SHAPE;
  GemmArgs a = base_args(x, ldx, wp, q, heads * head_dim, M, (heads + 2) * head_dim, K, 1);
  a.out_k = (__bf16*)k; a.out_v = (__bf16*)v; a.ldkv = ldkv;
  a.rope = (const __bf16*)rope; a.norm_factor = (__bf16*)norm_factor;
  a.heads = heads; a.head_dim = head_dim;
  a.batch = batch; a.kv_bstride = kv_bstride;
  return launch_gemm<EPI_QKV_ROPE, false>(a, s);
}

int pi0hip_norm_qkv_rope(const void* x, int ldx, const void* wp, const void* rope, void* q,
                         void* k, void* v, int ldkv, void* norm_factor, int M, int K,
                         int heads, int head_dim, hipStream_t s) {
  if (M == 1) {     // a lone state token: one request of one row
    if (!x || !wp || !rope || !q || !k || !v) return PI0HIP_ERR_ARG;
    if (head_dim % 16 || heads <= 0) return PI0HIP_ERR_SHAPE;
    GemmArgs a = base_args(x, ldx, wp, q, heads * head_dim, M, (heads + 2) * head_dim, K, 1);
    a.out_k = (__bf16*)k; a.out_v = (__bf16*)v; a.ldkv = ldkv;
    a.rope = (const __bf16*)rope; a.norm_factor = (__bf16*)norm_factor;
    a.heads = heads; a.head_dim = head_dim;
    return launch_gemm<EPI_QKV_ROPE, false>(a, s);
  }
  return pi0hip_norm_qkv_rope_batched(x, ldx, wp, rope, q, k, v, ldkv, 0, norm_factor, M, K, heads,
                                      head_dim, 1, s);
}

int pi0hip_scaled_gated_ffn(const void* x, int ldx, const void* f, const void* gate_p,
                            const void* up_p, void* out, int ldo, int M, int N, int K,
                            hipStream_t s) {
  if (!x || !f || !gate_p || !up_p || !out) return PI0HIP_ERR_ARG;
  GemmArgs a = base_args(x, ldx, gate_p, out, ldo, M, N, K, 1);
  a.w1 = (const __bf16*)up_p;
  a.prescale = (const __bf16*)f;
  return launch_gemm<EPI_GATE_PRE, true>(a, s);
}

int pi0hip_scaled_linear_bias_residual(const void* x, int ldx, const void* f, const void* wp,
                                       const void* bias, void* out, int ldo, int M, int N, int K,
                                       int splitk, void* ws, size_t ws_bytes, hipStream_t s) {
  if (!x || !f || !wp || !bias || !out) return PI0HIP_ERR_ARG;
  GemmArgs a = base_args(x, ldx, wp, out, ldo, M, N, K, splitk);
  a.bias = (const __bf16*)bias;
  a.prescale = (const __bf16*)f;
  if (int e = setup_ws(a, ws, ws_bytes, 0)) return e;
  return launch_gemm<EPI_RMS_BIAS_RES_PRE, false>(a, s);
}

int pi0hip_scaled_linear_bias_residual_f32(const void* x, int ldx, const void* f, const void* wp,
                                           const void* bias, float* out, int ldo, int M, int N,
                                           int K, int splitk, void* ws, size_t ws_bytes,
                                           hipStream_t s) {
  if (!x || !f || !wp || !bias || !out) return PI0HIP_ERR_ARG;
  if (ldo % 4) return PI0HIP_ERR_SHAPE;
  GemmArgs a = base_args(x, ldx, wp, nullptr, ldo, M, N, K, splitk);
  a.bias = (const __bf16*)bias;
  a.out_f32 = out;
  a.prescale = (const __bf16*)f;
  if (int e = setup_ws(a, ws, ws_bytes, 0)) return e;
  return launch_gemm<EPI_RMS_BIAS_RES_PRE, false>(a, s);
}

int pi0hip_norm_gated_ffn(const void* x, int ldx, const void* gate_p, const void* up_p,
                          void* out, int ldo, int M, int N, int K, hipStream_t s) {
  if (!x || !gate_p || !up_p || !out) return PI0HIP_ERR_ARG;
  GemmArgs a = base_args(x, ldx, gate_p, out, ldo, M, N, K, 1);
  a.w1 = (const __bf16*)up_p;
  return launch_gemm<EPI_GATE, true>(a, s);
}

}  // extern "C"
