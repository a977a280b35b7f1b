// Decoder attention: single KV head, flat (token * heads + head) query rows.
//
// Reference semantics (fused_wrappers.py:88-115, base.py:801-923):
//   o = softmax(mask(Q K^T / sqrt(256))) V, where flat rows < heads (the state
//   token) keep keys j <= enc_len and every other row keeps all keys.
//
// One kernel. Workgroup = 16 query rows x 128 keys; its 4 waves take 32 keys
// each (flash-decoding inside the workgroup):
//   * S^T = K Q^T with K rows as the MFMA A operand and Q rows as B, both read
//     straight from global memory in fragment order. In the S^T accumulator a
//     lane holds, for one query row, keys {4g..4g+3} of each 16-key tile --
//     exactly the A-operand layout P @ V needs once the MFMA's key slots are
//     permuted the same way in the V fragment, so P never leaves registers.
//   * V (row-major, 256 columns per key) is transposed into LDS on the way in
//     so that the B fragment (4 + 4 keys of one column) is two 8-byte reads.
//   * log2-domain softmax per wave, merged across the 4 waves through LDS,
//     P rounded to bf16 before P @ V as in the reference.
// When the keys span several chunks, each workgroup writes its normalised
// partial O and log2-sum-exp with device-scope stores; the last workgroup of
// a query tile (arrival counter) merges them in chunk order and writes O.
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

constexpr int ATT_HD = 256;
constexpr int ATT_QT = 16;     // query rows per workgroup
constexpr int ATT_CH = 128;    // keys per workgroup (32 per wave)
constexpr int VT_P = 40;       // bf16 pitch of a transposed-V row (32 keys + pad)
constexpr float NEG_BIG = -1.0e30f;

struct AttnArgs {
  const __bf16* q; int ldq;
  const __bf16* k; const __bf16* v; int ldkv;
  __bf16* out; int ldo;
  float* part; float* lse; int* counters;
  int rows, keys, enc_len, heads, nchunks, rows_pad;
  float scale_log2;
};

__global__ __launch_bounds__(256, 1) void attn_kernel(AttnArgs a) {
  // vt: per-wave transposed V slice; reused as the per-wave O buffer after P @ V.
  __shared__ __attribute__((aligned(16))) __bf16 vt[4][ATT_HD][VT_P];
  __shared__ float sm[4][ATT_QT], sl[4][ATT_QT];
  __shared__ int s_last;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int qt = blockIdx.x, c = blockIdx.y;
  const int q0 = qt * ATT_QT;
  const int kw0 = c * ATT_CH + wave * 32;            // first key of this wave

  // ---- issue global loads: V slice (for LDS), K fragments (A), Q fragments (B)
  bf16x8 vreg[16];
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int key = kw0 + (lane & 31);
    const int d = (p * 2 + (lane >> 5)) * 8;
    vreg[p] = key < a.keys ? load8(a.v + (size_t)key * a.ldkv + d) : zero8();
  }
  bf16x8 kf[2][8], qf[8];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int key = kw0 + nt * 16 + r;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      kf[nt][ks] = key < a.keys ? load8(a.k + (size_t)key * a.ldkv + ks * 32 + g * 8) : zero8();
  }
  {
    const int row = q0 + r;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      qf[ks] = row < a.rows ? load8(a.q + (size_t)row * a.ldq + ks * 32 + g * 8) : zero8();
  }

  // ---- S^T tiles: lane holds query row q0+r, keys kw0 + nt*16 + 4g + i
  f32x4 st[2] = {zero4(), zero4()};
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    st[0] = mfma16(kf[0][ks], qf[ks], st[0]);
    st[1] = mfma16(kf[1][ks], qf[ks], st[1]);
  }

  // ---- V -> LDS, transposed (vt[wave][d][key])
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int kk = lane & 31;
    const int d = (p * 2 + (lane >> 5)) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) vt[wave][d + j][kk] = vreg[p][j];
  }

  // ---- masked log2-domain softmax of this wave's 32 keys
  const int qrow = q0 + r;
  const bool state_row = qrow < a.heads;
  float s[8];
  float mx = NEG_BIG;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kw0 + nt * 16 + g * 4 + i;
      const bool keep = key < a.keys && (!state_row || key <= a.enc_len);
      const float v = keep ? st[nt][i] * a.scale_log2 : NEG_BIG;
      s[nt * 4 + i] = v;
      mx = fmaxf(mx, v);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, PI0_WAVE));
  mx = fmaxf(mx, __shfl_xor(mx, 32, PI0_WAVE));
  const bool empty = mx <= 0.5f * NEG_BIG;
  float lsum = 0.f;
  bf16x8 pf;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p = empty ? 0.f : fast_exp2(s[j] - mx);
    lsum += p;
    pf[j] = f2bf(p);
  }
  lsum += __shfl_xor(lsum, 16, PI0_WAVE);
  lsum += __shfl_xor(lsum, 32, PI0_WAVE);
  if (g == 0) { sm[wave][r] = mx; sl[wave][r] = lsum; }
  __syncthreads();

  // ---- O_w = P V_w : lane holds column dt*16 + r, query rows 4g + i
  f32x4 o[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) {
    const __bf16* vp = &vt[wave][dt * 16 + r][0];
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vp + g * 4);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vp + 16 + g * 4);
    const bf16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    o[dt] = mfma16(pf, vf, zero4());
  }

  // ---- merge the 4 waves: O = sum_w 2^(m_w - M) O_w, L = sum_w 2^(m_w - M) l_w
  float alpha[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int qr = g * 4 + i;
    float M = NEG_BIG;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][qr]);
    const float mw = sm[wave][qr];
    alpha[i] = (mw <= 0.5f * NEG_BIG) ? 0.f : fast_exp2(mw - M);
  }
  __syncthreads();                                   // all waves done reading vt
  float* ob = reinterpret_cast<float*>(&vt[0][0][0]);   // [4][16][256] fp32 = 64 KB
#pragma unroll
  for (int dt = 0; dt < 16; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ob[(wave * ATT_QT + g * 4 + i) * ATT_HD + dt * 16 + r] = o[dt][i] * alpha[i];
  __syncthreads();

  // thread t: query row t/16, columns 16*(t%16) .. +15
  const int orow = t >> 4, oc = (t & 15) * 16;
  float M = NEG_BIG;
#pragma unroll
  for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][orow]);
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float mw = sm[w][orow];
    if (mw > 0.5f * NEG_BIG) L += fast_exp2(mw - M) * sl[w][orow];
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) v += ob[(w * ATT_QT + orow) * ATT_HD + oc + j];
    acc[j] = v * inv;
  }
  const int grow = q0 + orow;

  if (a.nchunks == 1) {
    if (grow < a.rows) {
      bf16x8 lo, hi;
#pragma unroll
      for (int j = 0; j < 8; ++j) { lo[j] = f2bf(acc[j]); hi[j] = f2bf(acc[8 + j]); }
      *reinterpret_cast<bf16x8*>(a.out + (size_t)grow * a.ldo + oc) = lo;
      *reinterpret_cast<bf16x8*>(a.out + (size_t)grow * a.ldo + oc + 8) = hi;
    }
    return;
  }

  // ---- several chunks: publish this chunk's partial, last arrival merges
  {
    float* pp = a.part + ((size_t)c * a.rows_pad + grow) * ATT_HD + oc;
#pragma unroll
    for (int j = 0; j < 16; j += 4) store_dev4(pp + j, f32x4{acc[j], acc[j + 1], acc[j + 2], acc[j + 3]});
    if ((t & 15) == 0)
      store_dev1(a.lse + (size_t)c * a.rows_pad + grow,
                 (L > 0.f) ? M + log2f(L) : NEG_BIG);
  }
  if (!arrive_last(a.counters + qt, a.nchunks, &s_last)) return;

  float lmax = NEG_BIG;
  for (int cc = 0; cc < a.nchunks; ++cc) lmax = fmaxf(lmax, load_dev1(a.lse + (size_t)cc * a.rows_pad + grow));
  float wsum = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  for (int cc = 0; cc < a.nchunks; ++cc) {
    const float l = load_dev1(a.lse + (size_t)cc * a.rows_pad + grow);
    const float w = (l <= 0.5f * NEG_BIG) ? 0.f : fast_exp2(l - lmax);
    wsum += w;
    const float* pp = a.part + ((size_t)cc * a.rows_pad + grow) * ATT_HD + oc;
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
      const f32x4 pv = load_dev4(pp + j);
      acc[j] += w * pv[0]; acc[j + 1] += w * pv[1]; acc[j + 2] += w * pv[2]; acc[j + 3] += w * pv[3];
    }
  }
  if (grow < a.rows) {
    const float winv = wsum > 0.f ? 1.0f / wsum : 0.f;
    bf16x8 lo, hi;
#pragma unroll
    for (int j = 0; j < 8; ++j) { lo[j] = f2bf(acc[j] * winv); hi[j] = f2bf(acc[8 + j] * winv); }
    *reinterpret_cast<bf16x8*>(a.out + (size_t)grow * a.ldo + oc) = lo;
    *reinterpret_cast<bf16x8*>(a.out + (size_t)grow * a.ldo + oc + 8) = hi;
  }
}

}  // namespace pi0

using namespace pi0;

static inline size_t round256(size_t v) { return (v + 255) / 256 * 256; }

extern "C" {

size_t pi0hip_attention_workspace_bytes(int rows, int keys) {
  if (rows <= 0 || keys <= 0) return 0;
  const size_t nch = (size_t)(keys + ATT_CH - 1) / ATT_CH;
  const size_t nqt = (size_t)(rows + ATT_QT - 1) / ATT_QT;
  const size_t rows_pad = nqt * ATT_QT;
  return round256(nqt * sizeof(int)) + round256(nch * rows_pad * sizeof(float)) +
         nch * rows_pad * ATT_HD * sizeof(float);
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
  const int nqt = (rows + ATT_QT - 1) / ATT_QT;
  a.rows_pad = nqt * ATT_QT;
  char* base = reinterpret_cast<char*>(ws);
  a.counters = reinterpret_cast<int*>(base);
  base += round256((size_t)nqt * sizeof(int));
  a.lse = reinterpret_cast<float*>(base);
  base += round256((size_t)a.nchunks * a.rows_pad * sizeof(float));
  a.part = reinterpret_cast<float*>(base);
  a.scale_log2 = 1.4426950408889634f / sqrtf((float)head_dim);
  hipLaunchKernelGGL(attn_kernel, dim3(nqt, a.nchunks), dim3(256), 0, s, a);
  return (int)hipGetLastError();
}

}  // extern "C"
