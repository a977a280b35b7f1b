// Shared device helpers for the gfx950 Pi0 decoder kernels.
//
// Conventions used by every kernel in this library:
//  * activations are bf16, row-major, with an explicit leading dimension;
//  * weights are consumed in a "B-fragment" packed layout produced once by
//    pi0hip_pack_weight (see pi0_gemm.hip): for W[K][N] the tile (kt, nt) of
//    32 k x 16 n is 64 lanes x 8 bf16, lane = (k%32/8)*16 + n%16, element k%8,
//    tiles ordered [nt][kt] so that one column tile is a contiguous stream;
//  * the MFMA is v_mfma_f32_16x16x32_bf16: A lane l holds A[l%16][8*(l/16)+j],
//    B lane l holds B[8*(l/16)+j][l%16], C lane l holds C[4*(l/16)+i][l%16].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define PI0_WAVE 64

// Timing probes for kernel tuning: compiled out unless PI0_PROBE_ENABLED is defined
// (an instrumented build then records a shader-clock stamp per probe point).
#ifndef PI0_PROBE
#define PI0_PROBE(i) ((void)0)
#endif

// s_waitcnt immediate: vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14).
#define PI0_VMCNT(n) (((n) & 0xF) | (0x7 << 4) | (0xF << 8) | (((n) >> 4) << 14))

namespace pi0 {

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf2f(__bf16 v) { return static_cast<float>(v); }
__device__ __forceinline__ __bf16 f2bf(float v) { return static_cast<__bf16>(v); }
// Round an fp32 value to the nearest bf16 and return it as fp32.
__device__ __forceinline__ float round_bf(float v) { return bf2f(f2bf(v)); }

__device__ __forceinline__ bf16x8 load8(const __bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
__device__ __forceinline__ bf16x8 zero8() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(bf16x8, z);
}
__device__ __forceinline__ f32x4 zero4() {
  f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return z;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Gemma tanh-GELU written as v * sigmoid(2*sqrt(2/pi) * (v + 0.044715 v^3)).
__device__ __forceinline__ float gelu_tanh(float v) {
  const float c0 = 1.5957691216057308f, c1 = 0.044715f;
  return v / (1.0f + __expf(-(c0 * v * (1.0f + c1 * v * v))));
}
__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// ---- bounds-checked row loads ---------------------------------------------------
// A buffer resource covering exactly `nbytes` makes every load past the end return
// zeros without faulting, so staging loops need no clamping or branches and their
// offsets stay 32-bit (row * pitch + column, plus per-iteration immediates).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, 0x00020000);
}
// The same resource built from readfirstlane'd values: provably wave-uniform, so it
// lives in SGPRs (instructions that take it need no per-lane waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc_sgpr(const void* base, int nbytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
  void* q = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(q, 0, __builtin_amdgcn_readfirstlane(nbytes), 0x00020000);
}
// 16 bytes per lane from a buffer resource straight into LDS: lane l writes
// lds_base + 16 l (lds_base must be wave-uniform). Completion is counted by vmcnt.
__device__ __forceinline__ void buf_load16_lds(__amdgpu_buffer_rsrc_t r, void* lds_base, int off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base,
                                           16, off, 0, 0, 0);
}
// The same with a wave-uniform byte offset `soff` (an SGPR) added to the lane offset.
__device__ __forceinline__ void buf_load16_lds_s(__amdgpu_buffer_rsrc_t r, void* lds_base, int off,
                                                 int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base,
                                           16, off, __builtin_amdgcn_readfirstlane(soff), 0, 0);
}
__device__ __forceinline__ bf16x8 buf_load8(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, PI0_WAVE);
  return v;
}

// ---- L2 prefetch by spare workgroups ------------------------------------------------
// A launch may carry extra workgroups (blockIdx.x >= work_grid) that only touch one dword
// of every 128-byte line of up to PF_REGIONS regions, so that a later launch finds those
// lines in L2. Region r is nslices[r] equal slices of slice_words[r] dwords; slice s is
// what workgroup s of the consuming launch reads, and workgroup s of a launch runs on XCD
// s % 8, so slice s is touched by a spare workgroup on XCD s % 8. Loads only.
constexpr int PF_REGIONS = 4;
struct L2Prefetch {
  int work_grid, workgroups, n;
  const unsigned* base[PF_REGIONS];
  int slice_words[PF_REGIONS], nslices[PF_REGIONS];
};

__device__ __forceinline__ void prefetch_slices(const L2Prefetch& a) {
  const int p = blockIdx.x, x = p & 7, t = threadIdx.x;
  const int k0 = (x - a.work_grid % 8 + 8) % 8;          // first spare workgroup on XCD x
  if (a.workgroups <= k0) return;
  const int j = (p - a.work_grid - k0) / 8;             // its index there ...
  const int per_xcd = (a.workgroups - k0 + 7) / 8;      // ... and their number
  unsigned acc = 0;
#pragma unroll
  for (int r = 0; r < PF_REGIONS; ++r) {  // constant indices: the argument arrays stay in SGPRs
    if (r >= a.n) break;
    const int lines = a.slice_words[r] / 32;
    const int items = (a.nslices[r] - x + 7) / 8 * lines;
    const unsigned* base = a.base[r];
    for (int it = j * (int)blockDim.x + t; it < items; it += per_xcd * (int)blockDim.x) {
      const int sl = x + 8 * (it / lines), l = it - (it / lines) * lines;
      acc += base[(size_t)sl * a.slice_words[r] + l * 32];
    }
  }
  asm volatile("" ::"v"(acc));
}

// Host side: fill `pf` from up to PF_REGIONS (pointer, bytes, slices) triples; null
// pointers are skipped. Returns false for a region that is not whole 128-byte lines per
// slice or not 4-byte aligned.
inline bool make_l2_prefetch(L2Prefetch& pf, int work_grid, int spare, int n,
                             const void* const* ptr, const size_t* bytes, const int* slices) {
  pf = L2Prefetch{};
  pf.work_grid = work_grid;
  for (int r = 0; r < n && r < PF_REGIONS; ++r) {
    if (!ptr[r]) continue;
    const size_t b = bytes[r];
    const int ns = slices[r];
    if (ns <= 0 || b == 0 || b % ns || (b / ns) % 128 || b / ns / 4 > (size_t)INT32_MAX ||
        (reinterpret_cast<uintptr_t>(ptr[r]) & 3))
      return false;
    pf.base[pf.n] = static_cast<const unsigned*>(ptr[r]);
    pf.slice_words[pf.n] = static_cast<int>(b / ns / 4);
    pf.nslices[pf.n] = ns;
    ++pf.n;
  }
  pf.workgroups = pf.n ? spare : 0;
  return true;
}

// CUs of the current device (cached per device).
inline int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace pi0
