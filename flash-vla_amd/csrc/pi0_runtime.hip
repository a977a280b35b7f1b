// Library-level state: version and the one-time check of the workgroup -> XCD
// dispatch order that the XCD-local partial exchanges rely on.
#include <stdlib.h>
#include <string.h>
#include "pi0_common.h"
#include "pi0_hip.h"

namespace pi0 {

constexpr int MAX_DEVICES = 64;
static int g_xcd_ok[MAX_DEVICES];   // 0 unknown or not round-robin, 1 verified, 2 verified but off

__global__ void xcd_probe_kernel(int* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcd_id();
}

}  // namespace pi0

extern "C" {

int pi0hip_version(void) { return 2; }

int pi0hip_init(void) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= pi0::MAX_DEVICES) return PI0HIP_ERR_ARG;
  const char* env = getenv("PI0HIP_XCD_LOCAL");
  if (env && strcmp(env, "0") == 0) { pi0::g_xcd_ok[dev] = 0; return 0; }
  constexpr int n = 1024;
  int* d = nullptr;
  if ((e = hipMalloc(&d, n * sizeof(int))) != hipSuccess) return (int)e;
  hipLaunchKernelGGL(pi0::xcd_probe_kernel, dim3(n), dim3(64), 0, 0, d);
  int h[n];
  e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost);
  hipFree(d);
  if (e != hipSuccess) return (int)e;
  int ok = 1;
  for (int i = 0; i < n; ++i) ok &= (h[i] == i % pi0::NUM_XCD);
  pi0::g_xcd_ok[dev] = ok;
  return 0;
}

int pi0hip_set_xcd_local(int enable) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= pi0::MAX_DEVICES) return PI0HIP_ERR_ARG;
  if (enable) {
    const int ok = pi0::g_xcd_ok[dev];
    if (ok != 1 && ok != 2) return PI0HIP_ERR_ARG;   // only re-enable after pi0hip_init verified it
    pi0::g_xcd_ok[dev] = 1;
  } else if (pi0::g_xcd_ok[dev] == 1) {
    pi0::g_xcd_ok[dev] = 2;                           // verified but switched off
  }
  return 0;
}

int pi0hip_xcd_dispatch_ok(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= pi0::MAX_DEVICES) return 0;
  return pi0::g_xcd_ok[dev] == 1;
}

}  // extern "C"
