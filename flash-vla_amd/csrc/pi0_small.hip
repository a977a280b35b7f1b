// Projections from the 32-wide action/state space (K = 32): far too small for
// MFMA tiling to matter, so one thread computes one output element in fp32.
//   decoder_state_proj      out = x @ W + b          (wrappers.py:108-112)
//   decoder_action_in_proj  out = silu(x @ W + b)    (wrappers.py:115-120)
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

__global__ __launch_bounds__(256) void small_k_linear_kernel(
    const __bf16* __restrict__ x, int ldx, const __bf16* __restrict__ w,
    const __bf16* __restrict__ bias, __bf16* __restrict__ out, int ldo, int M, int N, int K,
    int act) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N || m >= M) return;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) acc += bf2f(x[(size_t)m * ldx + k]) * bf2f(w[(size_t)k * N + n]);
  acc += bf2f(bias[n]);
  if (act == 1) acc = silu(acc);
  out[(size_t)m * ldo + n] = f2bf(acc);
}

}  // namespace pi0

extern "C" int pi0hip_small_linear(const void* x, int ldx, const void* w, const void* bias,
                                   void* out, int ldo, int M, int N, int K, int act,
                                   hipStream_t s) {
  if (!x || !w || !bias || !out || M <= 0 || N <= 0 || K <= 0) return PI0HIP_ERR_ARG;
  if (act != 0 && act != 1) return PI0HIP_ERR_ARG;
  dim3 grid((N + 255) / 256, M);
  hipLaunchKernelGGL(pi0::small_k_linear_kernel, grid, dim3(256), 0, s, (const __bf16*)x, ldx,
                     (const __bf16*)w, (const __bf16*)bias, (__bf16*)out, ldo, M, N, K, act);
  return (int)hipGetLastError();
}
