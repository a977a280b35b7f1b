// Decoder attention: single KV head, flat (token * heads + head) query rows.
//
// Reference semantics (fused_wrappers.py:88-115, base.py:801-923):
//   o = softmax(mask(Q K^T / sqrt(256))) V, where flat rows < heads (the state
//   token) keep keys j <= enc_len and every other row keeps all keys.
//
// Split kernel: one workgroup per (64 query rows, 64 keys). The 4 waves split
// the 256-wide head dimension for S = Q K^T (A = Q rows, B = K rows, both read
// straight from global as MFMA fragments, nothing replicated), the partial S
// tiles are summed through LDS, each thread then owns one row quarter for the
// log2-domain softmax (row max / sum with lane shuffles). P is rounded to bf16
// in LDS, as the reference does before P @ V. For P @ V each wave owns 64
// output columns; its V slice is transposed into LDS on the way in so that a
// B fragment (8 consecutive keys of one column) is a single 16-byte LDS read.
// Output: per-chunk normalised partial O (fp32) and its log2-sum-exp.
// Combine kernel: per row, weights exp2(lse_c - max) / sum over chunks.
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

constexpr int ATT_HD = 256;
constexpr int ATT_QT = 64;    // query rows per workgroup
constexpr int ATT_CH = 64;    // keys per workgroup
constexpr int P_LD = ATT_CH + 8;    // bf16 row pitch of P in LDS
constexpr int VT_LD = ATT_CH + 8;   // bf16 row pitch of the transposed V slice
constexpr float NEG_BIG = -1.0e30f;

struct AttnArgs {
  const __bf16* q; int ldq;
  const __bf16* k; const __bf16* v; int ldkv;
  __bf16* out; int ldo;
  float* part; float* lse;
  int rows, keys, enc_len, heads, nchunks;
  float scale_log2;
};

__global__ __launch_bounds__(256, 1) void attn_split_kernel(AttnArgs a) {
  __shared__ float sred[4][4][4][4][PI0_WAVE];          // [wave][mt][nt][i][lane]
  __shared__ __attribute__((aligned(16))) __bf16 pl[ATT_QT][P_LD];
  __shared__ __attribute__((aligned(16))) __bf16 vt[4][64][VT_LD];   // [wave][d][key]
  __shared__ float lrow[ATT_QT];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int q0 = blockIdx.x * ATT_QT, c = blockIdx.y, k0 = c * ATT_CH;
  const int r = lane & 15, g = lane >> 4;

  // ---- V slice of this wave (64 keys x 64 columns) -> registers (issued first)
  bf16x8 vreg[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int key = k0 + p * 8 + (lane >> 3);
    const int d = wave * 64 + (lane & 7) * 8;
    vreg[p] = key < a.keys ? load8(a.v + (size_t)key * a.ldkv + d) : zero8();
  }
  // ---- S partial over this wave's 64-wide slice of the head dimension
  bf16x8 qa[4][2], kb[4][2];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int row = q0 + mt * 16 + r;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      qa[mt][ks] = row < a.rows ? load8(a.q + (size_t)row * a.ldq + wave * 64 + ks * 32 + g * 8)
                                : zero8();
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int key = k0 + nt * 16 + r;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      kb[nt][ks] = key < a.keys ? load8(a.k + (size_t)key * a.ldkv + wave * 64 + ks * 32 + g * 8)
                                : zero8();
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      f32x4 acc = zero4();
      acc = mfma16(qa[mt][0], kb[nt][0], acc);
      acc = mfma16(qa[mt][1], kb[nt][1], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) sred[wave][mt][nt][i][lane] = acc[i];
    }
  }
  // transpose this wave's V slice into LDS: vt[wave][d][key]
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int key = p * 8 + (lane >> 3);
    const int d = (lane & 7) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) vt[wave][d + j][key] = vreg[p][j];
  }
  __syncthreads();

  // ---- softmax: thread t owns query row t/4, keys 16*(t%4) .. +15
  {
    const int qr = t >> 2, kq = t & 3;
    const int mt = qr >> 4, r16 = qr & 15, ii = r16 & 3, gg = r16 >> 2;
    const int grow = q0 + qr;
    const bool state_row = grow < a.heads;
    float s[16];
    float mx = NEG_BIG;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) v += sred[w][mt][kq][ii][gg * 16 + j];
      const int key = k0 + kq * 16 + j;
      const bool keep = key < a.keys && (!state_row || key <= a.enc_len);
      v = keep ? v * a.scale_log2 : NEG_BIG;
      s[j] = v;
      mx = fmaxf(mx, v);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, PI0_WAVE));
    mx = fmaxf(mx, __shfl_xor(mx, 2, PI0_WAVE));
    const bool empty = mx <= 0.5f * NEG_BIG;
    float sum = 0.f;
    __attribute__((aligned(16))) __bf16 pb[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float p = empty ? 0.f : fast_exp2(s[j] - mx);
      sum += p;
      pb[j] = f2bf(p);
    }
    sum += __shfl_xor(sum, 1, PI0_WAVE);
    sum += __shfl_xor(sum, 2, PI0_WAVE);
    *reinterpret_cast<bf16x8*>(&pl[qr][kq * 16]) = *reinterpret_cast<bf16x8*>(&pb[0]);
    *reinterpret_cast<bf16x8*>(&pl[qr][kq * 16 + 8]) = *reinterpret_cast<bf16x8*>(&pb[8]);
    if (kq == 0) {
      lrow[qr] = sum;
      if (grow < a.rows)
        a.lse[(size_t)c * a.rows + grow] = (empty || sum <= 0.f) ? NEG_BIG : mx + log2f(sum);
    }
  }
  __syncthreads();

  // ---- O = P V for this wave's 64 columns
  f32x4 o[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) o[mt][nt] = zero4();
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    bf16x8 pa[4], vb[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      pa[mt] = *reinterpret_cast<const bf16x8*>(&pl[mt * 16 + r][ks * 32 + g * 8]);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
      vb[nt] = *reinterpret_cast<const bf16x8*>(&vt[wave][nt * 16 + r][ks * 32 + g * 8]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) o[mt][nt] = mfma16(pa[mt], vb[nt], o[mt][nt]);
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qr = mt * 16 + g * 4 + i;
      const int grow = q0 + qr;
      if (grow >= a.rows) continue;
      const float l = lrow[qr];
      const float inv = l > 0.f ? 1.0f / l : 0.f;
      float* dst = a.part + ((size_t)c * a.rows + grow) * ATT_HD + wave * 64 + r;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) dst[nt * 16] = o[mt][nt][i] * inv;
    }
  }
}

__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const int t = threadIdx.x;
  const int row = blockIdx.x * 4 + (t >> 6);
  if (row >= a.rows) return;
  const int d = (t & 63) * 4;
  float mx = NEG_BIG;
  for (int c = 0; c < a.nchunks; ++c) mx = fmaxf(mx, a.lse[(size_t)c * a.rows + row]);
  float wsum = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < a.nchunks; ++c) {
    const float l = a.lse[(size_t)c * a.rows + row];
    const float w = l <= 0.5f * NEG_BIG ? 0.f : fast_exp2(l - mx);
    wsum += w;
    const f32x4 p = *reinterpret_cast<const f32x4*>(a.part + ((size_t)c * a.rows + row) * ATT_HD + d);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] += w * p[j];
  }
  const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
  bf16x4 pk = {f2bf(acc[0] * inv), f2bf(acc[1] * inv), f2bf(acc[2] * inv), f2bf(acc[3] * inv)};
  *reinterpret_cast<bf16x4*>(a.out + (size_t)row * a.ldo + d) = pk;
}

}  // namespace pi0

using namespace pi0;

extern "C" {

size_t pi0hip_attention_workspace_bytes(int rows, int keys) {
  const size_t nch = (size_t)(keys + ATT_CH - 1) / ATT_CH;
  return nch * rows * ATT_HD * sizeof(float) + ((nch * rows * sizeof(float) + 255) / 256) * 256;
}

int pi0hip_attention(const void* q, int ldq, const void* k, const void* v, int ldkv, void* out,
                     int ldo, int rows, int keys, int enc_len, int heads, int head_dim,
                     void* ws, size_t ws_bytes, hipStream_t s) {
  if (!q || !k || !v || !out || rows <= 0 || keys <= 0) return PI0HIP_ERR_ARG;
  if (head_dim != ATT_HD) return PI0HIP_ERR_SHAPE;
  if (!ws || ws_bytes < pi0hip_attention_workspace_bytes(rows, keys)) return PI0HIP_ERR_WORKSPACE;
  AttnArgs a = {};
  a.q = (const __bf16*)q; a.ldq = ldq;
  a.k = (const __bf16*)k; a.v = (const __bf16*)v; a.ldkv = ldkv;
  a.out = (__bf16*)out; a.ldo = ldo;
  a.rows = rows; a.keys = keys; a.enc_len = enc_len; a.heads = heads;
  a.nchunks = (keys + ATT_CH - 1) / ATT_CH;
  const size_t lse_floats = (size_t)a.nchunks * rows;
  a.lse = reinterpret_cast<float*>(ws);
  a.part = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + ((lse_floats * 4 + 255) / 256) * 256);
  a.scale_log2 = 1.4426950408889634f / sqrtf((float)head_dim);
  dim3 g1((rows + ATT_QT - 1) / ATT_QT, a.nchunks);
  hipLaunchKernelGGL(attn_split_kernel, g1, dim3(256), 0, s, a);
  if (hipError_t e = hipGetLastError()) return (int)e;
  hipLaunchKernelGGL(attn_combine_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

}  // extern "C"
