// Projections from the 32-wide action/state space (K = 32): far too small for
// MFMA tiling to matter. One thread computes 8 adjacent outputs of one row in
// fp32 from 16-byte weight loads, all K rows of loads in flight at once.
//   decoder_state_proj      out = x @ W + b          (wrappers.py:108-112)
//   decoder_action_in_proj  out = silu(x @ W + b)    (wrappers.py:115-120)
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

template <int K, typename XT>
__global__ __launch_bounds__(256) void small_k_linear_kernel(
    const XT* __restrict__ x, int ldx, const __bf16* __restrict__ w,
    const __bf16* __restrict__ bias, __bf16* __restrict__ out, int ldo, int M, int N, int act) {
  const int groups = N / 8;
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= M * groups) return;
  const int m = id / groups, n = (id - m * groups) * 8;
  bf16x8 wv[K];
#pragma unroll
  for (int k = 0; k < K; ++k) wv[k] = load8(w + (size_t)k * N + n);
  float xv[K];
#pragma unroll
  for (int k = 0; k < K; ++k) xv[k] = static_cast<float>(x[(size_t)m * ldx + k]);
  const bf16x8 bv = load8(bias + n);
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) acc += xv[k] * bf2f(wv[k][j]);
    acc += bf2f(bv[j]);
    if (act == 1) acc = silu(acc);
    o[j] = f2bf(acc);
  }
  *reinterpret_cast<bf16x8*>(out + (size_t)m * ldo + n) = o;
}

}  // namespace pi0

template <typename XT>
static int launch_small(const void* x, int ldx, const void* w, const void* bias, void* out, int ldo,
                        int M, int N, int K, int act, hipStream_t s) {
  if (!x || !w || !bias || !out || M <= 0 || N <= 0 || K <= 0) return PI0HIP_ERR_ARG;
  if (act != 0 && act != 1) return PI0HIP_ERR_ARG;
  if (N % 8 || K != 32 || ldo % 8) return PI0HIP_ERR_SHAPE;
  const int threads = M * (N / 8);
  hipLaunchKernelGGL((pi0::small_k_linear_kernel<32, XT>), dim3((threads + 255) / 256), dim3(256),
                     0, s, (const XT*)x, ldx, (const __bf16*)w, (const __bf16*)bias, (__bf16*)out,
                     ldo, M, N, act);
  return (int)hipGetLastError();
}

extern "C" int pi0hip_small_linear(const void* x, int ldx, const void* w, const void* bias,
                                   void* out, int ldo, int M, int N, int K, int act,
                                   hipStream_t s) {
  return launch_small<__bf16>(x, ldx, w, bias, out, ldo, M, N, K, act, s);
}

extern "C" int pi0hip_small_linear_f32x(const void* x, int ldx, const void* w, const void* bias,
                                        void* out, int ldo, int M, int N, int K, int act,
                                        hipStream_t s) {
  return launch_small<float>(x, ldx, w, bias, out, ldo, M, N, K, act, s);
}
