// The decoder's unfused call sites (op_table(fused=False)): the reference's two-kernel
// forms, kept for their rounding points rather than their speed.
//
//   rms_factor_kernel   f[m] = bf16(rsqrt(mean_k x^2 + 1e-6))      tl_rms_factor (base.py:344-370)
//   scores_kernel       S = bf16((Q K^T) * scale)                  tl_matmul_abT_scale (base.py:737-762)
//   softmax_mask_kernel P = bf16(softmax(mask(S)))                 tl_softmax_mask0 (base.py:765-798)
//   pv_kernel           O = bf16(P V)                              tl_matmul (base.py:84-111)
//
// The prescaled GEMMs that consume f live with the other skinny GEMMs (pi0_gemm.hip,
// EPI_GATE_PRE / EPI_RMS_BIAS_RES_PRE).
//
// The score and P V products are small (408 x 819 x 256 MACs each at BASELINE config 2);
// they run as one dot product per thread over K / V rows staged in LDS, with fp32
// accumulation, which is all the reference's rounding contract fixes.
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

constexpr float UNFUSED_NEG = -3.0e38f;   // tl_softmax_mask0's masked-score fill (base.py:780)

// One wave per row; K % 8 == 0.
__global__ __launch_bounds__(256) void rms_factor_kernel(const __bf16* __restrict__ x, int ldx,
                                                          __bf16* __restrict__ f, int M, int K) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const __bf16* p = x + (size_t)row * ldx;
  float ss = 0.f;
  for (int k = lane * 8; k < K; k += 64 * 8) {
    const bf16x8 v = load8(p + k);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += bf2f(v[j]) * bf2f(v[j]);
  }
  ss = warp_sum(ss);
  if (lane == 0) f[row] = f2bf(rsqrtf(ss / (float)K + 1e-6f));
}

// S[r][j] = bf16(dot(Q[r], K[j]) * scale). Workgroup: 16 query rows (in LDS) x 256 keys,
// one key per thread.
constexpr int SC_ROWS = 16;
constexpr int SC_HD = 256;
__global__ __launch_bounds__(256) void scores_kernel(const __bf16* __restrict__ q, int ldq,
                                                     const __bf16* __restrict__ k, int ldk,
                                                     __bf16* __restrict__ s, int lds, int rows,
                                                     int keys, float scale) {
  __shared__ float qs[SC_ROWS][SC_HD];
  const int r0 = blockIdx.y * SC_ROWS, t = threadIdx.x;
  for (int i = t; i < SC_ROWS * SC_HD; i += 256) {
    const int r = i / SC_HD, d = i % SC_HD;
    qs[r][d] = r0 + r < rows ? bf2f(q[(size_t)(r0 + r) * ldq + d]) : 0.f;
  }
  __syncthreads();
  const int j = blockIdx.x * 256 + t;
  if (j >= keys) return;
  float acc[SC_ROWS];
#pragma unroll
  for (int r = 0; r < SC_ROWS; ++r) acc[r] = 0.f;
  const __bf16* kp = k + (size_t)j * ldk;
  for (int d0 = 0; d0 < SC_HD; d0 += 8) {
    const bf16x8 kv = load8(kp + d0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float kf = bf2f(kv[e]);
#pragma unroll
      for (int r = 0; r < SC_ROWS; ++r) acc[r] += qs[r][d0 + e] * kf;
    }
  }
#pragma unroll
  for (int r = 0; r < SC_ROWS; ++r)
    if (r0 + r < rows) s[(size_t)(r0 + r) * lds + j] = f2bf(acc[r] * scale);
}

// One wave per row: keep key j when j < keys and (row >= heads or j <= enc_len); masked
// scores read as UNFUSED_NEG; P = bf16(exp(s - max) / sum). keys <= 2048 (32 per lane).
constexpr int SM_PER_LANE = 32;
__global__ __launch_bounds__(256) void softmax_mask_kernel(const __bf16* __restrict__ s, int lds,
                                                           __bf16* __restrict__ p, int ldp,
                                                           int rows, int keys, int enc_len,
                                                           int heads) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  float v[SM_PER_LANE];
  float mx = UNFUSED_NEG;
#pragma unroll
  for (int i = 0; i < SM_PER_LANE; ++i) {
    const int j = lane + 64 * i;
    const bool keep = j < keys && (row >= heads || j <= enc_len);
    v[i] = keep ? bf2f(s[(size_t)row * lds + j]) : UNFUSED_NEG;
    mx = fmaxf(mx, v[i]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, PI0_WAVE));
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < SM_PER_LANE; ++i) {
    v[i] = __expf(v[i] - mx);
    sum += v[i];
  }
  sum = warp_sum(sum);
#pragma unroll
  for (int i = 0; i < SM_PER_LANE; ++i) {
    const int j = lane + 64 * i;
    if (j < keys) p[(size_t)row * ldp + j] = f2bf(v[i] / sum);
  }
}

// O[r][d] = bf16(sum_j P[r][j] V[j][d]). Workgroup: 4 query rows x 256 columns (one column
// per thread, 4 rows each); P rows staged in LDS 256 keys at a time.
constexpr int PV_ROWS = 4;
constexpr int PV_KB = 256;
__global__ __launch_bounds__(256) void pv_kernel(const __bf16* __restrict__ p, int ldp,
                                                 const __bf16* __restrict__ v, int ldv,
                                                 __bf16* __restrict__ out, int ldo, int rows,
                                                 int keys) {
  __shared__ float ps[PV_ROWS][PV_KB];
  const int r0 = blockIdx.x * PV_ROWS, d = threadIdx.x;
  float acc[PV_ROWS] = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < keys; j0 += PV_KB) {
    __syncthreads();
    for (int i = d; i < PV_ROWS * PV_KB; i += 256) {
      const int r = i / PV_KB, j = j0 + i % PV_KB;
      ps[r][i % PV_KB] = (r0 + r < rows && j < keys) ? bf2f(p[(size_t)(r0 + r) * ldp + j]) : 0.f;
    }
    __syncthreads();
    const int n = min(PV_KB, keys - j0);
    for (int jj = 0; jj < n; ++jj) {
      const float vf = bf2f(v[(size_t)(j0 + jj) * ldv + d]);
#pragma unroll
      for (int r = 0; r < PV_ROWS; ++r) acc[r] += ps[r][jj] * vf;
    }
  }
#pragma unroll
  for (int r = 0; r < PV_ROWS; ++r)
    if (r0 + r < rows) out[(size_t)(r0 + r) * ldo + d] = f2bf(acc[r]);
}

}  // namespace pi0

using namespace pi0;

extern "C" {

int pi0hip_rms_factor(const void* x, int ldx, void* f, int M, int K, hipStream_t s) {
  if (!x || !f || M <= 0 || K <= 0) return PI0HIP_ERR_ARG;
  if (K % 8 || ldx < K || ldx % 8 || (reinterpret_cast<uintptr_t>(x) & 15)) return PI0HIP_ERR_SHAPE;
  hipLaunchKernelGGL(rms_factor_kernel, dim3((M + 3) / 4), dim3(256), 0, s, (const __bf16*)x, ldx,
                     (__bf16*)f, M, K);
  return (int)hipGetLastError();
}

int pi0hip_attention_unfused(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             void* scores, int ld_scores, void* probs, int ld_probs, void* out,
                             int ldo, int rows, int keys, int enc_len, int heads, int head_dim,
                             hipStream_t s) {
  if (!q || !k || !v || !scores || !probs || !out || rows <= 0 || keys <= 0 || heads <= 0)
    return PI0HIP_ERR_ARG;
  if (head_dim != SC_HD || keys > 64 * SM_PER_LANE || ld_scores < keys || ld_probs < keys ||
      (ldkv % 8) || (reinterpret_cast<uintptr_t>(k) & 15))
    return PI0HIP_ERR_SHAPE;
  if (scores == probs) return PI0HIP_ERR_ARG;
  const float scale = 1.0f / sqrtf((float)head_dim);
  hipLaunchKernelGGL(scores_kernel, dim3((keys + 255) / 256, (rows + SC_ROWS - 1) / SC_ROWS),
                     dim3(256), 0, s, (const __bf16*)q, ldq, (const __bf16*)k, ldkv,
                     (__bf16*)scores, ld_scores, rows, keys, scale);
  if (hipError_t e = hipGetLastError()) return (int)e;
  hipLaunchKernelGGL(softmax_mask_kernel, dim3((rows + 3) / 4), dim3(256), 0, s,
                     (const __bf16*)scores, ld_scores, (__bf16*)probs, ld_probs, rows, keys,
                     enc_len, heads);
  if (hipError_t e = hipGetLastError()) return (int)e;
  hipLaunchKernelGGL(pv_kernel, dim3((rows + PV_ROWS - 1) / PV_ROWS), dim3(256), 0, s,
                     (const __bf16*)probs, ld_probs, (const __bf16*)v, ldkv, (__bf16*)out, ldo,
                     rows, keys);
  return (int)hipGetLastError();
}

}  // extern "C"
