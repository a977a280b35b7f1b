// Measurement probe (not part of the library): the decoder layer's four GEMM phases --
// RMS-norm + QKV, o-proj + residual, RMS-norm + gated FFN, ffn-down + residual -- for 18
// layers in ONE persistent cooperative launch (one 4-wave workgroup per CU), with a grid
// barrier between phases instead of a kernel boundary. It answers one question: does a
// persistent decoder beat the captured graph of per-phase kernels on this GPU once the next
// phase's weight stream is overlapped with the barrier?
//
// Shapes are those of the Pi0 decoder at M = 51 rows (width 1024, FFN 4096, 8 x 256 query
// + 2 x 256 KV columns), weights in the library's packed B-fragment layout (one 32k x 16n
// tile = 64 lanes x 16 bytes, tiles [nt][kt]), bf16 activations, fp32 accumulation:
//   QKV    K 1024, N 2560: 160 column tiles x all 64 rows (workgroups >= 160 idle)
//   o-proj K 2048, N 1024: 64 column tiles x 4 row blocks of 16 (row-split, as the library)
//   gate   K 1024, N 4096 gate + 4096 up: 256 column tiles x all 64 rows
//   down   K 4096, N 1024: 64 column tiles x 4 row blocks of 16
// Each wave takes a quarter of K, stages its x slice into LDS with direct buffer->LDS loads
// (16-byte chunks XOR-swizzled by row) and keeps its weight fragments in registers; the 4
// waves are summed through LDS. Activations cross XCDs inside the launch, so every
// activation store and load is device-coherent (SC1 cache policy), and a workgroup arrives
// at the barrier only after its stores are acknowledged. The workgroup that owns an x tile
// in the o-proj owns the same tile in the down projection, so the residual stays in its
// registers. Variants (runtime): the next phase's weight loads issued right after this
// workgroup's arrival (overlapping the wait) or after the release; and no barriers at all
// (a timing floor only: the phases then race and the values are meaningless).
// Compile-time: -DSTORE_POLICY=18 (SC1 + non-temporal stores).
//
// Barrier: epoch-numbered arrival flags set by atomic exchange; workgroup 0 polls them all
// and then publishes the epoch in a release flag that every workgroup polls. Every spin is
// bounded; a timeout sets an error word and every workgroup leaves its loop, so the grid
// always drains. The launch is cooperative, so it fails rather than hangs if the 256
// workgroups cannot all be resident.
//
// Build and run (one MI355X):
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       -o /tmp/persistent_chain flash-vla_amd/probes/persistent_chain.hip
//   /tmp/persistent_chain
// The graph it is compared with: python3 flash-vla_amd/probes/graph_chain.py
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>

#define SC1 16            // device-coherent cache policy (a macro: the builtins take an immediate)
#ifndef STORE_POLICY
#define STORE_POLICY 16   // SC1: device-coherent
#endif

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

namespace {


constexpr int SPIN_MAX = 1 << 18;
constexpr int ROWS_M = 51;
constexpr int LAYERS = 18;
constexpr int NWG = 256;
constexpr int PROBE_LAYER = 5;
constexpr int RELEASE_FLAG = 1024;

#define CHECK(call)                                                                   \
  do {                                                                                \
    hipError_t e_ = (call);                                                           \
    if (e_ != hipSuccess) {                                                           \
      std::fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));          \
      std::exit(1);                                                                   \
    }                                                                                 \
  } while (0)

struct Args {
  const __bf16* w_qkv; const __bf16* w_o; const __bf16* w_gate; const __bf16* w_up;
  const __bf16* w_down;
  __bf16* x;      // [64][1024] residual stream
  __bf16* attn;   // [64][2048] attention output (input of the o-proj)
  __bf16* qkv;    // [64][2560]
  __bf16* hid;    // [64][4096]
  unsigned* flags; unsigned* err;
  unsigned long long* stamps;   // [4 phases][6] real-time stamps of workgroup 0, one layer
  int barriers;
};

enum Kind { QKV = 0, OPROJ = 1, GATE = 2, DOWN = 3 };
template <int KIND> struct Shape;
template <> struct Shape<QKV> { static constexpr int K = 1024, N = 2560, RT = 4; static constexpr bool DUAL = false; };
template <> struct Shape<OPROJ> { static constexpr int K = 2048, N = 1024, RT = 1; static constexpr bool DUAL = false; };
template <> struct Shape<GATE> { static constexpr int K = 1024, N = 4096, RT = 4; static constexpr bool DUAL = true; };
template <> struct Shape<DOWN> { static constexpr int K = 4096, N = 1024, RT = 1; static constexpr bool DUAL = false; };

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, 0x00020000);
}
// 16 bytes per lane, device-coherent, straight into LDS: lane l writes lds + 16 l.
__device__ __forceinline__ void load16_lds_coherent(__amdgpu_buffer_rsrc_t r, void* lds, int off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off,
                                           0, 0, SC1);
}
__device__ __forceinline__ unsigned load_agent(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float gelu_tanh(float v) {
  return v / (1.0f + __expf(-(1.5957691216057308f * v * (1.0f + 0.044715f * v * v))));
}
__device__ __forceinline__ void stamp(const Args& a, int layer, int kind, int point) {
  if (layer == PROBE_LAYER && blockIdx.x == 0 && threadIdx.x == 0)
    a.stamps[kind * 6 + point] = __builtin_amdgcn_s_memrealtime();
}

// Output tile of workgroup b: 64-row phases take column tile b; 16-row phases place the 4
// row blocks of column tile nt on one XCD (workgroup b runs on XCD b % 8).
template <int KIND>
__device__ __forceinline__ bool tile_of(int b, int& nt, int& rb) {
  if constexpr (Shape<KIND>::RT == 4) {
    nt = b; rb = 0;
    return b < Shape<KIND>::N / 16;
  } else {
    const int xcd = b & 7, j = b >> 3;
    nt = (j / 4) * 8 + xcd; rb = j % 4;
    return true;
  }
}

// Issue this wave's weight fragments of phase KIND, layer `layer`, into registers.
template <int KIND>
__device__ __forceinline__ void load_weights(const Args& a, int layer, bf16x8 (&w)[32]) {
  using S = Shape<KIND>;
  constexpr int KT = S::K / 32, KTW = KT / 4;
  int nt, rb;
  if (!tile_of<KIND>(blockIdx.x, nt, rb)) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const __bf16* base = KIND == QKV ? a.w_qkv : KIND == OPROJ ? a.w_o : KIND == GATE ? a.w_gate : a.w_down;
  const size_t layer_elems = (size_t)S::K * S::N;
  const size_t off = layer * layer_elems + ((size_t)nt * KT + wave * KTW) * 512 + lane * 8;
#pragma unroll
  for (int i = 0; i < KTW; ++i) w[i] = *reinterpret_cast<const bf16x8*>(base + off + i * 512);
  if constexpr (S::DUAL) {
#pragma unroll
    for (int i = 0; i < KTW; ++i) w[KTW + i] = *reinterpret_cast<const bf16x8*>(a.w_up + off + i * 512);
  }
}

__device__ __forceinline__ void arrive(const Args& a, unsigned epoch) {
  if (threadIdx.x == 0)
    __hip_atomic_exchange(&a.flags[blockIdx.x], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ bool wait_release(const Args& a, unsigned epoch) {
  const int t = threadIdx.x;
  if (blockIdx.x == 0 && t < 64) {
    bool ok = true;
    for (int spins = 0;; ++spins) {
      bool done = true;
      for (int j = 0; j < NWG / 64; ++j)
        if ((int)(load_agent(&a.flags[j * 64 + t]) - epoch) < 0) done = false;
      if (__all(done)) break;
      if (spins > SPIN_MAX || load_agent(a.err)) { ok = false; break; }
    }
    if (!ok && t == 0) atomicAdd(a.err, 1u);
    if (t == 0)
      __hip_atomic_exchange(&a.flags[RELEASE_FLAG], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (t == 0) {
    for (int spins = 0; (int)(load_agent(&a.flags[RELEASE_FLAG]) - epoch) < 0; ++spins)
      if (spins > SPIN_MAX || load_agent(a.err)) { atomicAdd(a.err, 1u); break; }
  }
  __builtin_amdgcn_s_barrier();
  return load_agent(a.err) == 0;
}

template <int KIND>
__device__ void run_phase(const Args& a, int layer, bf16x8 (&w)[32], char* smem, float (&xres)[4]) {
  using S = Shape<KIND>;
  constexpr int KT = S::K / 32, KTW = KT / 4, KW = KTW * 32, RT = S::RT, ROWS = RT * 16;
  constexpr int CPR = KW / 8;                 // 16-byte chunks per row of a wave's x slice
  constexpr int LOADS = ROWS * CPR / 64;      // buffer->LDS instructions per wave
  constexpr int SWM = (CPR < 16 ? CPR : 16) - 1;
  constexpr bool RMS = KIND == QKV || KIND == GATE;
  constexpr int ND = S::DUAL ? 2 : 1;
  constexpr int LDX = S::K;                   // x row pitch
  stamp(a, layer, KIND, 0);
  int nt, rb;
  const bool active = tile_of<KIND>(blockIdx.x, nt, rb);
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const __bf16* xin = KIND == OPROJ ? a.attn : KIND == DOWN ? a.hid : a.x;
  const int m0 = rb * 16, rows = min(ROWS, ROWS_M - m0);
  char* xs = smem + (size_t)wave * ROWS * KW * 2;
  f32x4 acc[RT], acc1[RT];
  float ss[RT];
  if (active) {
    const auto xr = rsrc(xin + (size_t)m0 * S::K, rows * S::K * 2);   // rows past M read 0
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int id = i * 64 + lane, row = id / CPR, c = id % CPR;
      load16_lds_coherent(xr, xs + i * 1024, (row * LDX + wave * KW + ((c ^ (row & SWM)) * 8)) * 2);
    }
    __builtin_amdgcn_s_waitcnt(0);            // x slice and weight fragments have landed
    stamp(a, layer, KIND, 1);
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc1[rt] = acc[rt];
      ss[rt] = 0.f;
      const int row = rt * 16 + r;
#pragma unroll
      for (int i = 0; i < KTW; ++i) {
        const int ch = (i * 4 + g) ^ (row & SWM);
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(xs + (row * CPR + ch) * 16);
        if constexpr (RMS) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bf16x2 q = {av[2 * e], av[2 * e + 1]};
            ss[rt] = __builtin_amdgcn_fdot2_f32_bf16(q, q, ss[rt], false);
          }
        }
        acc[rt] = mfma16(av, w[i], acc[rt]);
        if constexpr (S::DUAL) acc1[rt] = mfma16(av, w[KTW + i], acc1[rt]);
      }
    }
  }
  stamp(a, layer, KIND, 2);
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);          // [wave][rt][nd][4][64]
  float* ssr = red + 4 * RT * ND * 4 * 64;              // [wave][rt][16]
  if (active) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        red[(((wave * RT + rt) * ND) * 4 + i) * 64 + lane] = acc[rt][i];
        if constexpr (S::DUAL) red[(((wave * RT + rt) * ND + 1) * 4 + i) * 64 + lane] = acc1[rt][i];
      }
      if constexpr (RMS) {
        float s = ss[rt];
        s += __shfl_xor(s, 16, 64);
        s += __shfl_xor(s, 32, 64);
        if (lane < 16) ssr[(wave * RT + rt) * 16 + lane] = s;
      }
    }
  }
  __syncthreads();
  stamp(a, layer, KIND, 3);
  if (!active) return;
  // epilogue: 4 consecutive columns of one row per thread, one 8-byte device-coherent store
  for (int idx = t; idx < ROWS * 4; idx += 256) {
    const int lr = idx >> 2, c0 = (idx & 3) * 4;
    if (lr >= rows) continue;
    const int rt = lr >> 4, rr = lr & 15, i = rr & 3;
    float f = 1.f;
    if constexpr (RMS) {
      float s = 0.f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) s += ssr[(wv * RT + rt) * 16 + rr];
      f = (float)(__bf16)rsqrtf(s / (float)S::K + 1e-6f);
    }
    float o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int l = (rr >> 2) * 16 + c0 + c;
      float v0 = 0.f, v1 = 0.f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) {
        v0 += red[(((wv * RT + rt) * ND) * 4 + i) * 64 + l];
        if constexpr (S::DUAL) v1 += red[(((wv * RT + rt) * ND + 1) * 4 + i) * 64 + l];
      }
      if constexpr (KIND == QKV) o[c] = v0 * f;
      else if constexpr (KIND == GATE) o[c] = gelu_tanh(v0 * f) * (v1 * f);
      else { o[c] = v0 + xres[c]; xres[c] = (float)(__bf16)o[c]; }   // residual kept in registers
    }
    const int n = nt * 16 + c0, grow = m0 + lr;
    __bf16* dst = KIND == QKV ? a.qkv + (size_t)grow * 2560 + n
                : KIND == GATE ? a.hid + (size_t)grow * 4096 + n : a.x + (size_t)grow * 1024 + n;
    const bf16x4 pk = {(__bf16)o[0], (__bf16)o[1], (__bf16)o[2], (__bf16)o[3]};
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, pk), rsrc(dst, 8), 0, 0, STORE_POLICY);
  }
}

// One phase, then the grid barrier; the next phase's weights are issued after this
// workgroup's arrival (PREFETCH) or after the release.
template <bool PREFETCH, int KIND, int NEXT>
__device__ bool step(const Args& a, int layer, int next_layer, bf16x8 (&w)[32], char* smem,
                     unsigned& epoch, float (&xres)[4]) {
  run_phase<KIND>(a, layer, w, smem, xres);
  __builtin_amdgcn_s_waitcnt(0);              // this wave's stores are acknowledged
  stamp(a, layer, KIND, 4);
  if (!a.barriers) {
    load_weights<NEXT>(a, next_layer, w);
    return true;
  }
  __syncthreads();
  arrive(a, ++epoch);
  if constexpr (PREFETCH) load_weights<NEXT>(a, next_layer, w);
  asm volatile("" ::: "memory");              // keep the weight loads ahead of the polling
  const bool ok = wait_release(a, epoch);
  asm volatile("" ::: "memory");
  if constexpr (!PREFETCH) load_weights<NEXT>(a, next_layer, w);
  stamp(a, layer, KIND, 5);
  return ok;
}

template <bool PREFETCH>
__global__ __launch_bounds__(256, 1) void persistent_chain(Args a) {
  __shared__ __attribute__((aligned(16))) char smem[128 * 1024 + 4096];
  bf16x8 w[32];
  float xres[4] = {0.f, 0.f, 0.f, 0.f};
  unsigned epoch = 0;
  {   // the x tile this workgroup owns in the residual phases (16 x 16, 4 per thread)
    int nt, rb;
    tile_of<OPROJ>(blockIdx.x, nt, rb);
    const int t = threadIdx.x, grow = rb * 16 + (t >> 2);
    if (t < 64 && grow < ROWS_M) {
      const auto v = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(
          rsrc(a.x + (size_t)grow * 1024 + nt * 16 + (t & 3) * 4, 8), 0, 0, SC1));
      for (int c = 0; c < 4; ++c) xres[c] = (float)v[c];
    }
  }
  load_weights<QKV>(a, 0, w);
  for (int layer = 0; layer < LAYERS; ++layer) {
    const int next = layer + 1 < LAYERS ? layer + 1 : 0;
    if (!step<PREFETCH, QKV, OPROJ>(a, layer, layer, w, smem, epoch, xres)) break;
    if (!step<PREFETCH, OPROJ, GATE>(a, layer, layer, w, smem, epoch, xres)) break;
    if (!step<PREFETCH, GATE, DOWN>(a, layer, layer, w, smem, epoch, xres)) break;
    if (!step<PREFETCH, DOWN, QKV>(a, layer, next, w, smem, epoch, xres)) break;
  }
  if (threadIdx.x == 0) atomicAdd(a.err + 1, 1u);      // workgroups that finished
}

__global__ void fill(__bf16* p, size_t n, unsigned seed) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    unsigned h = (unsigned)i * 2654435761u ^ seed;
    h ^= h >> 13; h *= 0x5bd1e995u; h ^= h >> 15;
    p[i] = (__bf16)(((int)(h & 1023) - 512) * (0.02f / 512.f));
  }
}

__bf16* filled(size_t n, unsigned seed) {
  __bf16* p = nullptr;
  CHECK(hipMalloc(&p, n * sizeof(__bf16)));
  hipLaunchKernelGGL(fill, dim3(1024), dim3(256), 0, 0, p, n, seed);
  CHECK(hipGetLastError());
  return p;
}

}  // namespace

int main() {
  int dev = 0, cus = 0, coop = 0, per_cu = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
  CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, persistent_chain<true>, 256, 0));
  std::printf("CUs %d, cooperative launch %d, resident workgroups per CU %d\n", cus, coop, per_cu);
  if (cus != NWG || per_cu != 1 || !coop) {
    std::printf("this probe expects 256 CUs, one resident workgroup per CU and cooperative launch\n");
    return 1;
  }
  Args a = {};
  a.w_qkv = filled((size_t)LAYERS * 1024 * 2560, 1);
  a.w_o = filled((size_t)LAYERS * 2048 * 1024, 2);
  a.w_gate = filled((size_t)LAYERS * 1024 * 4096, 3);
  a.w_up = filled((size_t)LAYERS * 1024 * 4096, 4);
  a.w_down = filled((size_t)LAYERS * 4096 * 1024, 5);
  a.x = filled(64 * 1024, 6);
  a.attn = filled(64 * 2048, 7);
  a.qkv = filled(64 * 2560, 8);
  a.hid = filled(64 * 4096, 9);
  CHECK(hipMalloc(&a.flags, 8192));
  CHECK(hipMalloc(&a.err, 64));
  CHECK(hipMalloc(&a.stamps, 24 * sizeof(unsigned long long)));
  CHECK(hipDeviceSynchronize());
  struct Variant { bool prefetch; int barriers; const char* name; };
  const Variant variants[] = {{true, 1, "barriers, next weights issued at arrival"},
                              {false, 1, "barriers, next weights issued after release"},
                              {true, 0, "no barriers (timing floor; values race)"}};
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (const Variant& v : variants) {
    for (int rep = 0; rep < 3; ++rep) {     // the first launch of each variant is cold
      CHECK(hipMemset(a.flags, 0, 8192));
      CHECK(hipMemset(a.err, 0, 64));
      a.barriers = v.barriers;
      void* kargs[] = {&a};
      CHECK(hipEventRecord(e0));
      CHECK(hipLaunchCooperativeKernel(v.prefetch ? (const void*)persistent_chain<true>
                                                  : (const void*)persistent_chain<false>,
                                       dim3(NWG), dim3(256), kargs, 0, 0));
      CHECK(hipEventRecord(e1));
      CHECK(hipEventSynchronize(e1));
      float ms = 0.f;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      unsigned err[2];
      CHECK(hipMemcpy(err, a.err, sizeof err, hipMemcpyDeviceToHost));
      std::printf("%-46s %8.2f us per layer (4 phases)  timeouts %u  finished %u\n", v.name,
                  ms * 1000.f / LAYERS, err[0], err[1]);
      if (err[0]) return 2;
      if (rep == 2) {
        unsigned long long s[24];
        CHECK(hipMemcpy(s, a.stamps, sizeof s, hipMemcpyDeviceToHost));
        std::printf("  workgroup 0, layer %d, us from the QKV phase start "
                    "(x+weights landed / MFMA done / reduced / stores acked / released):\n",
                    PROBE_LAYER);
        const char* names[] = {"qkv", "o-proj", "gate", "down"};
        for (int k = 0; k < 4; ++k) {
          std::printf("    %-7s", names[k]);
          for (int j = 0; j < (v.barriers ? 6 : 5); ++j)
            std::printf(" %7.2f", (double)(long long)(s[k * 6 + j] - s[0]) / 100.0);
          std::printf("\n");
        }
      }
    }
  }
  return 0;
}
