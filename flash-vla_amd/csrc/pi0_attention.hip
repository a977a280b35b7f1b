// Decoder attention: single KV head, flat (token * heads + head) query rows.
//
// Reference semantics (fused_wrappers.py:88-115, base.py:801-923):
//   o = softmax(mask(Q K^T / sqrt(256))) V, where flat rows < heads (the state
//   token) keep keys j <= enc_len and every other row keeps all keys.
//
// One kernel. Workgroup = 16 query rows x 128 keys:
//   * K, V (128 rows) and Q (16 rows) are staged in LDS with coalesced
//     16-byte loads (row pitch padded by 16 bytes so fragment reads are free
//     of bank conflicts);
//   * each of the 4 waves takes 32 keys (flash-decoding inside the
//     workgroup): S^T = K Q^T with K rows as the MFMA A operand and Q rows as
//     B. In the S^T accumulator a lane holds, for one query row, keys
//     {4g..4g+3} of each 16-key tile -- the A-operand layout P @ V needs once
//     the MFMA's key slots are permuted the same way in the V fragment, so P
//     never leaves registers;
//   * log2-domain softmax per wave (lane shuffles), merged across the 4 waves
//     through LDS; P is rounded to bf16 before P @ V as in the reference.
// When the keys span several chunks, each workgroup writes its normalised
// partial O and log2-sum-exp, and attn_combine_kernel (second launch) merges
// them per row in chunk order. (A merge by the last-arriving workgroup through
// device-scope traffic measured ~1.2 us slower than the kernel boundary.)
#include "pi0_common.h"
#include "pi0_hip.h"

#include <mutex>

namespace pi0 {

constexpr int ATT_HD = 256;
constexpr int ATT_QT = 16;          // query rows per workgroup
constexpr int ATT_CH = 128;         // keys per workgroup (32 per wave)
constexpr int KP = ATT_HD + 8;      // bf16 pitch of staged K / Q rows
constexpr int VP = ATT_HD + 16;     // bf16 pitch of staged V rows (544 B: 4 rows hit 4 bank groups)
constexpr int OBP = ATT_HD + 4;     // fp32 pitch of the per-wave O buffer
constexpr float NEG_BIG = -1.0e30f;
constexpr int MAX_CHUNKS = 16;      // keys <= 2048 (prompts up to 1229 tokens with 3 views)
constexpr int PF_MAX = PF_REGIONS;  // prefetch regions

struct AttnArgs {
  const __bf16* q; int ldq;
  const __bf16* k; const __bf16* v; int ldkv;
  __bf16* out; int ldo;
  float* part; float* lse;
  int rows, keys, enc_len, heads, nchunks, rows_pad, nqt;   // rows / keys per request
  float scale_log2;
  int batch;                 // requests (grid.y); request b reads K / V at b * kv_bstride
  long long kv_bstride;
  L2Prefetch pf;              // optional L2 prefetch by spare workgroups (batch 1)
};

// Output row of local flat row lr (= token * heads + head) of request b: the tokens of a
// batch are stored "states first" (B state tokens, then B x T action tokens), the order
// the decoder's residual stream uses; for one request this is the identity.
__device__ __forceinline__ int out_row(const AttnArgs& a, int b, int lr) {
  const int t = lr / a.heads, head = lr - t * a.heads;
  const int T = a.rows / a.heads - 1;
  const int tok = t == 0 ? b : a.batch + b * T + (t - 1);
  return tok * a.heads + head;
}

// Merge of one 16-byte output piece (row, columns col..col+3) over the key chunks, in chunk
// order: O = sum_c 2^(lse_c - max) O_c / sum_c 2^(lse_c - max).
template <int MAXC>     // MAXC >= nchunks: the loads are unrolled MAXC deep
__device__ __forceinline__ bf16x4 merge_piece(__amdgpu_buffer_rsrc_t pr, __amdgpu_buffer_rsrc_t lr,
                                              int nchunks, int rows_pad, int row, int col) {
  float lse_c[MAXC];
  f32x4 pv[MAXC];
#pragma unroll
  for (int cc = 0; cc < MAXC; ++cc) {
    const int ci = min(cc, nchunks - 1);
    lse_c[cc] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              lr, (ci * rows_pad + row) * 4, 0, 0));
    pv[cc] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           pr, ((ci * rows_pad + row) * ATT_HD + col) * 4, 0, 0));
  }
  float lmax = NEG_BIG;
#pragma unroll
  for (int cc = 0; cc < MAXC; ++cc) {
    lse_c[cc] = cc < nchunks ? lse_c[cc] : NEG_BIG;
    lmax = fmaxf(lmax, lse_c[cc]);
  }
  float wsum = 0.f;
  f32x4 o4 = zero4();
#pragma unroll
  for (int cc = 0; cc < MAXC; ++cc) {
    const float w = cc < nchunks ? fast_exp2(lse_c[cc] - lmax) : 0.f;
    wsum += w;
    o4 += w * pv[cc];
  }
  const float winv = wsum > 0.f ? __builtin_amdgcn_rcpf(wsum) : 0.f;
  return bf16x4{f2bf(o4[0] * winv), f2bf(o4[1] * winv), f2bf(o4[2] * winv), f2bf(o4[3] * winv)};
}

// NWV waves: 4 key groups of 32 keys x NWV / 4 slices of the head dimension for P @ V
// (with 8 waves each S is computed twice, and every wave issues half the staging loads).
template <int NWV>
__global__ __launch_bounds__(NWV * 64, 2) void attn_kernel(AttnArgs a) {
  constexpr int NT = NWV * 64;              // threads
  constexpr int RP = NT / 32;               // staged rows per pass (32 16-byte chunks per row)
  constexpr int KPASS = ATT_CH / RP, QPASS = ATT_QT / RP > 0 ? ATT_QT / RP : 1;
  constexpr int NDH = NWV / 4, DTW = 16 / NDH;   // head-dim slices, 16-column tiles per wave
  // One LDS area holds K (pitch KP) for S, then V (pitch VP) for P @ V, then the fp32
  // per-wave O buffer: ~79 KB in all, so two workgroups fit on a CU (batched requests).
  __shared__ __attribute__((aligned(16))) __bf16 kv_[ATT_CH * VP];
  __shared__ __attribute__((aligned(16))) __bf16 qs_[ATT_QT][KP];
  auto ks_ = reinterpret_cast<__bf16 (*)[KP]>(kv_);
  auto vs_ = reinterpret_cast<__bf16 (*)[VP]>(kv_);
  static_assert(4 * ATT_QT * OBP * sizeof(float) <= sizeof(kv_), "O buffer");
  __shared__ float sm[4][ATT_QT], sl[4][ATT_QT];

  if ((int)blockIdx.x >= a.pf.work_grid) {
    prefetch_slices(a.pf);
    return;
  }
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int kg = wave & 3, dh = wave >> 2;  // key group, head-dim slice
  const int qt = blockIdx.x % a.nqt, c = blockIdx.x / a.nqt;
  const int q0 = qt * ATT_QT, k0 = c * ATT_CH;
  const int bq = blockIdx.y;
  a.q += (size_t)bq * a.rows * a.ldq;                       // request-major Q rows
  a.k += (size_t)bq * a.kv_bstride;
  a.v += (size_t)bq * a.kv_bstride;
  a.part += (size_t)bq * a.nchunks * a.rows_pad * ATT_HD;
  a.lse += (size_t)bq * a.nchunks * a.rows_pad;

  PI0_PROBE(0);
  // ---- stage K, V, Q with coalesced loads. The buffer resources end at the last
  // key / query row: rows past the end load as zeros (such keys are masked out
  // below, such query rows are never stored).
  bf16x8 vv[KPASS];
  const int row0 = t >> 5, ch = t & 31;                    // RP rows x 32 chunks per pass
  {
    const int kbytes = max(a.keys - k0, 0) * a.ldkv * (int)sizeof(__bf16);
    const __amdgpu_buffer_rsrc_t kr = rows_rsrc(a.k + (size_t)k0 * a.ldkv, kbytes);
    const __amdgpu_buffer_rsrc_t vr = rows_rsrc(a.v + (size_t)k0 * a.ldkv, kbytes);
    const __amdgpu_buffer_rsrc_t qr =
        rows_rsrc(a.q + (size_t)q0 * a.ldq, max(a.rows - q0, 0) * a.ldq * (int)sizeof(__bf16));
    const int koff = (row0 * a.ldkv + ch * 8) * (int)sizeof(__bf16);
    const int kstep = RP * a.ldkv * (int)sizeof(__bf16);
    const int qoff = (row0 * a.ldq + ch * 8) * (int)sizeof(__bf16);
    const int qstep = RP * a.ldq * (int)sizeof(__bf16);
    bf16x8 kv[KPASS], qv[QPASS];
    // issue order = order of use: Q, K, then V (loads return in order). Q and K are
    // published first; V lands while S = K Q^T and the softmax run.
#pragma unroll
    for (int j = 0; j < QPASS; ++j) qv[j] = buf_load8(qr, qoff + j * qstep);
#pragma unroll
    for (int j = 0; j < KPASS; ++j) kv[j] = buf_load8(kr, koff + j * kstep);
#pragma unroll
    for (int j = 0; j < KPASS; ++j) vv[j] = buf_load8(vr, koff + j * kstep);
#pragma unroll
    for (int j = 0; j < QPASS; ++j) *reinterpret_cast<bf16x8*>(&qs_[row0 + RP * j][ch * 8]) = qv[j];
#pragma unroll
    for (int j = 0; j < KPASS; ++j) *reinterpret_cast<bf16x8*>(&ks_[row0 + RP * j][ch * 8]) = kv[j];
  }
  __syncthreads();
  PI0_PROBE(1);

  // ---- S^T tiles of this wave: lane holds query row q0+r, keys kw + nt*16 + 4g + i
  const int kw = kg * 32;
  f32x4 st[2] = {zero4(), zero4()};
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const bf16x8 qf = *reinterpret_cast<const bf16x8*>(&qs_[r][ks * 32 + g * 8]);
    const bf16x8 k0f = *reinterpret_cast<const bf16x8*>(&ks_[kw + r][ks * 32 + g * 8]);
    const bf16x8 k1f = *reinterpret_cast<const bf16x8*>(&ks_[kw + 16 + r][ks * 32 + g * 8]);
    st[0] = mfma16(k0f, qf, st[0]);
    st[1] = mfma16(k1f, qf, st[1]);
  }

  // ---- masked log2-domain softmax of this wave's 32 keys
  const bool state_row = q0 + r < a.heads;
  float s[8];
  float mx = NEG_BIG;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = k0 + kw + nt * 16 + g * 4 + i;
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
  if (g == 0 && dh == 0) { sm[kg][r] = mx; sl[kg][r] = lsum; }

  __syncthreads();          // every wave is done reading K: V takes its place
  // ---- publish V (its loads were in flight during S and the softmax)
#pragma unroll
  for (int j = 0; j < KPASS; ++j) *reinterpret_cast<bf16x8*>(&vs_[row0 + RP * j][ch * 8]) = vv[j];
  __syncthreads();
  PI0_PROBE(2);
  // ---- O_w = P V_w : B fragment = V[keys kw + {4g..4g+3, 16+4g..16+4g+3}][column].
  // Each half comes from one transposing LDS read: within a 16-lane group, lane j slot
  // k receives element j % 4 of the 8 bytes at lane 4k + j / 4's address, so lane
  // 4k + c points at V[kw + 4g + k][16 dt + 4c .. +3] and lane r (column 16 dt + r)
  // gets keys 4g .. 4g + 3 of its column.
  f32x4 o[DTW];
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const int vkey = kw + 4 * g + (r >> 2), vcol = dh * DTW * 16 + (r & 3) * 4;
#pragma unroll
  for (int dt = 0; dt < DTW; ++dt) {
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4*)&vs_[vkey][dt * 16 + vcol]);
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4*)&vs_[vkey + 16][dt * 16 + vcol]);
    const bf16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    o[dt] = mfma16(pf, vf, zero4());
  }
  PI0_PROBE(3);
  __syncthreads();          // every wave is done reading V

  // ---- merge the 4 waves: O = sum_w 2^(m_w - M) O_w (rows 4g+i of this lane)
  float alpha[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int qr = g * 4 + i;
    float M = NEG_BIG;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][qr]);
    alpha[i] = fast_exp2(sm[kg][qr] - M);     // 0 for an empty wave next to a non-empty one
  }
  float* ob = reinterpret_cast<float*>(kv_);             // [4][16][OBP] fp32
#pragma unroll
  for (int dt = 0; dt < DTW; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ob[(kg * ATT_QT + g * 4 + i) * OBP + (dh * DTW + dt) * 16 + r] = o[dt][i] * alpha[i];
  // the merged rows' 1 / L and log2-sum-exp, once per row (threads 0..15)
  __shared__ float rinv[ATT_QT], rlse[ATT_QT];
  if (t < ATT_QT) {
    float M = NEG_BIG;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][t]);
    // branch-free: an empty wave has m_w = NEG_BIG and l_w = 0, so its term is 0
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) L += fast_exp2(sm[w][t] - M) * sl[w][t];
    rinv[t] = L > 0.f ? __builtin_amdgcn_rcpf(L) : 0.f;
    rlse[t] = L > 0.f ? M + __builtin_amdgcn_logf(L) : NEG_BIG;
  }
  __syncthreads();

  PI0_PROBE(4);
  // thread t owns PPT 16-byte pieces: piece id = t + NT j -> row id/64, columns 4*(id%64)..
  constexpr int PPT = ATT_QT * 64 / NT;
  f32x4 acc[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int id = t + NT * j, row = id >> 6, col = (id & 63) * 4;
    f32x4 v = zero4();
#pragma unroll
    for (int w = 0; w < 4; ++w) v += *reinterpret_cast<const f32x4*>(&ob[(w * ATT_QT + row) * OBP + col]);
    acc[j] = v * rinv[row];
  }

  if (a.nchunks == 1) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int id = t + NT * j, grow = q0 + (id >> 6), col = (id & 63) * 4;
      if (grow < a.rows) {
        const bf16x4 pk = {f2bf(acc[j][0]), f2bf(acc[j][1]), f2bf(acc[j][2]), f2bf(acc[j][3])};
        *reinterpret_cast<bf16x4*>(a.out + (size_t)out_row(a, bq, grow) * a.ldo + col) = pk;
      }
    }
    return;
  }

  // ---- several chunks: publish this chunk's normalised partial and log2-sum-exp
  // (plain stores; the kernel boundary orders them before attn_combine_kernel)
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int id = t + NT * j, prow = q0 + (id >> 6), col = (id & 63) * 4;
    *reinterpret_cast<f32x4*>(a.part + ((size_t)c * a.rows_pad + prow) * ATT_HD + col) = acc[j];
    if ((id & 63) == 0) a.lse[(size_t)c * a.rows_pad + prow] = rlse[id >> 6];
  }
}

// Second pass (several chunks): workgroup = one output row (64 threads x 16-byte pieces of
// its 256 columns), merged over the chunks in chunk order. The row index is the block
// index, so the buffer resources are provably uniform and live in SGPRs; the loads are
// unrolled to the smallest of 8 / MAX_CHUNKS that covers nchunks.
constexpr int CMB_THREADS = 64;     // one row per workgroup (408 workgroups at config 2)
static_assert(CMB_THREADS * 4 == ATT_HD, "one row per workgroup");
template <int MAXC>
__global__ __launch_bounds__(CMB_THREADS) void attn_combine_kernel(AttnArgs a) {
  const int grow = blockIdx.x, col = threadIdx.x * 4;
  const int bq = grow / a.rows, row = grow - bq * a.rows;
  a.part += (size_t)bq * a.nchunks * a.rows_pad * ATT_HD;
  a.lse += (size_t)bq * a.nchunks * a.rows_pad;
  const __amdgpu_buffer_rsrc_t pr =
      rows_rsrc_sgpr(a.part, a.nchunks * a.rows_pad * ATT_HD * (int)sizeof(float));
  const __amdgpu_buffer_rsrc_t lr = rows_rsrc_sgpr(a.lse, a.nchunks * a.rows_pad * (int)sizeof(float));
  const bf16x4 pk = merge_piece<MAXC>(pr, lr, a.nchunks, a.rows_pad, row, col);
  *reinterpret_cast<bf16x4*>(a.out + (size_t)out_row(a, bq, row) * a.ldo + col) = pk;
}

}  // namespace pi0

using namespace pi0;

static inline size_t round256(size_t v) { return (v + 255) / 256 * 256; }


extern "C" size_t pi0hip_attention_batched_workspace_bytes(int rows, int keys, int batch);

static int attention_launch(const void* q, int ldq, const void* k, const void* v, int ldkv,
                            long long kv_bstride, void* out, int ldo, int rows, int keys,
                            int enc_len, int heads, int head_dim, int batch, void* ws,
                            size_t ws_bytes, int npf, const void* const* pf_ptr,
                            const size_t* pf_bytes, const int* pf_slices, hipStream_t s) {
  if (!q || !k || !v || !out || rows <= 0 || keys <= 0 || batch <= 0 || heads <= 0)
    return PI0HIP_ERR_ARG;
  if (head_dim != ATT_HD || keys > MAX_CHUNKS * ATT_CH || (batch > 1 && rows % heads))
    return PI0HIP_ERR_SHAPE;
  if (!ws || ws_bytes < pi0hip_attention_batched_workspace_bytes(rows, keys, batch))
    return PI0HIP_ERR_WORKSPACE;
  // with one key chunk the output is stored by the split launch itself, which must not
  // overwrite query rows that other workgroups of a multi-request batch still read
  if (batch > 1 && keys <= ATT_CH && out == q) return PI0HIP_ERR_ARG;
  AttnArgs a = {};
  a.batch = batch; a.kv_bstride = kv_bstride;
  a.q = (const __bf16*)q; a.ldq = ldq;
  a.k = (const __bf16*)k; a.v = (const __bf16*)v; a.ldkv = ldkv;
  a.out = (__bf16*)out; a.ldo = ldo;
  a.rows = rows; a.keys = keys; a.enc_len = enc_len; a.heads = heads;
  a.nchunks = (keys + ATT_CH - 1) / ATT_CH;
  const int nqt = (rows + ATT_QT - 1) / ATT_QT;
  a.rows_pad = nqt * ATT_QT;
  a.nqt = nqt;
  const int grid = nqt * a.nchunks;
  // spare workgroups fill the chip to two per CU, the attention kernel's occupancy
  if (!make_l2_prefetch(a.pf, grid, max(0, 2 * device_cus() - grid), npf, pf_ptr, pf_bytes,
                        pf_slices))
    return PI0HIP_ERR_SHAPE;
  char* base = reinterpret_cast<char*>(ws);
  a.lse = reinterpret_cast<float*>(base);
  base += round256((size_t)batch * a.nchunks * a.rows_pad * sizeof(float));
  a.part = reinterpret_cast<float*>(base);
  a.scale_log2 = 1.4426950408889634f / sqrtf((float)head_dim);
  // (8 waves, each with half the head dimension of P @ V, measured slower in the loop)
  hipLaunchKernelGGL(attn_kernel<4>, dim3(grid + a.pf.workgroups, batch), dim3(256), 0, s, a);
  if (a.nchunks > 1) {
    if (hipError_t e = hipGetLastError()) return (int)e;
    if (a.nchunks <= 8)
      hipLaunchKernelGGL(attn_combine_kernel<8>, dim3(batch * rows), dim3(CMB_THREADS), 0, s, a);
    else
      hipLaunchKernelGGL(attn_combine_kernel<MAX_CHUNKS>, dim3(batch * rows), dim3(CMB_THREADS), 0,
                         s, a);
  }
  return (int)hipGetLastError();
}

extern "C" {

size_t pi0hip_attention_batched_workspace_bytes(int rows, int keys, int batch) {
  if (rows <= 0 || keys <= 0 || batch <= 0) return 0;
  const size_t nch = (size_t)(keys + ATT_CH - 1) / ATT_CH;
  const size_t nqt = (size_t)(rows + ATT_QT - 1) / ATT_QT;
  const size_t rows_pad = nqt * ATT_QT;
  return round256((size_t)batch * nch * rows_pad * sizeof(float)) +
         (size_t)batch * nch * rows_pad * ATT_HD * sizeof(float);
}

size_t pi0hip_attention_workspace_bytes(int rows, int keys) {
  return pi0hip_attention_batched_workspace_bytes(rows, keys, 1);
}

int pi0hip_attention_batched(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             long long kv_bstride, void* out, int ldo, int rows, int keys,
                             int enc_len, int heads, int head_dim, int batch, void* ws,
                             size_t ws_bytes, hipStream_t s) {
  return attention_launch(q, ldq, k, v, ldkv, kv_bstride, out, ldo, rows, keys, enc_len, heads,
                          head_dim, batch, ws, ws_bytes, 0, nullptr, nullptr, nullptr, s);
}

int pi0hip_attention_prefetch(const void* q, int ldq, const void* k, const void* v, int ldkv,
                              void* out, int ldo, int rows, int keys, int enc_len, int heads,
                              int head_dim, void* ws, size_t ws_bytes, const void* pf0,
                              size_t pf0_bytes, int pf0_slices, const void* pf1, size_t pf1_bytes,
                              int pf1_slices, const void* pf2, size_t pf2_bytes, int pf2_slices,
                              const void* pf3, size_t pf3_bytes, int pf3_slices, hipStream_t s) {
  const void* ptr[PF_MAX] = {pf0, pf1, pf2, pf3};
  const size_t bytes[PF_MAX] = {pf0_bytes, pf1_bytes, pf2_bytes, pf3_bytes};
  const int slices[PF_MAX] = {pf0_slices, pf1_slices, pf2_slices, pf3_slices};
  return attention_launch(q, ldq, k, v, ldkv, 0, out, ldo, rows, keys, enc_len, heads, head_dim,
                          1, ws, ws_bytes, PF_MAX, ptr, bytes, slices, s);
}

int pi0hip_attention(const void* q, int ldq, const void* k, const void* v, int ldkv, void* out,
                     int ldo, int rows, int keys, int enc_len, int heads, int head_dim,
                     void* ws, size_t ws_bytes, hipStream_t s) {
  return pi0hip_attention_batched(q, ldq, k, v, ldkv, 0, out, ldo, rows, keys, enc_len, heads,
                                  head_dim, 1, ws, ws_bytes, s);
}

}  // extern "C"

// ---- allocation-free variant --------------------------------------------------------
// The attention's workspace (per-chunk partial outputs and log2-sum-exps) lives in a
// file-scope device array; every GPU the library runs on holds its own copy until the
// process ends. Host code must not use the array's name as a device address: its address
// on the current device comes from hipGetSymbolAddress, fetched once per device and cached.
// The array holds NOALLOC_SLOTS slots of ATT_NOALLOC_SCRATCH_BYTES. A stream takes a slot
// on its first call on a device and keeps it for the process, so calls on different
// streams never share scratch; calls on one stream are ordered by the stream. A stream
// beyond the slots is rejected (PI0HIP_ERR_WORKSPACE) rather than given a shared slot.
constexpr size_t ATT_NOALLOC_SCRATCH_BYTES = size_t(8) << 20;
constexpr int NOALLOC_SLOTS = 4;
static __device__ __align__(256) char scratch[NOALLOC_SLOTS * ATT_NOALLOC_SCRATCH_BYTES];

static constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static char* g_scratch_ptr[MAX_DEVICES];
static hipStream_t g_slot_stream[MAX_DEVICES][NOALLOC_SLOTS];
static int g_slots_used[MAX_DEVICES];

// Scratch slot of stream `s` on the current device.
static int scratch_slot(hipStream_t s, void** out) {
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev)) return (int)e;
  if (dev < 0 || dev >= MAX_DEVICES) return PI0HIP_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) return (int)e;
    if (!p) return PI0HIP_ERR_WORKSPACE;
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  int slot = -1;
  for (int i = 0; i < g_slots_used[dev]; ++i)
    if (g_slot_stream[dev][i] == s) slot = i;
  if (slot < 0) {
    if (g_slots_used[dev] == NOALLOC_SLOTS) return PI0HIP_ERR_WORKSPACE;
    slot = g_slots_used[dev]++;
    g_slot_stream[dev][slot] = s;
  }
  *out = g_scratch_ptr[dev] + (size_t)slot * ATT_NOALLOC_SCRATCH_BYTES;
  return 0;
}

extern "C" {

size_t pi0hip_attention_noalloc_max_bytes(void) { return ATT_NOALLOC_SCRATCH_BYTES; }
int pi0hip_attention_noalloc_streams(void) { return NOALLOC_SLOTS; }

int pi0hip_attention_noalloc(const void* q, int ldq, const void* k, const void* v, int ldkv,
                             void* out, int ldo, int rows, int keys, int enc_len, int heads,
                             int head_dim, hipStream_t s) {
  if (rows <= 0 || keys <= 0) return PI0HIP_ERR_ARG;
  const size_t need = pi0hip_attention_batched_workspace_bytes(rows, keys, 1);
  if (need > ATT_NOALLOC_SCRATCH_BYTES) return PI0HIP_ERR_WORKSPACE;
  void* ws = nullptr;
  if (int e = scratch_slot(s, &ws)) return e;
  // every byte the kernels read from the workspace is written earlier in the same call, so
  // nothing needs clearing; the contents left by the stream's previous call are overwritten
  return attention_launch(q, ldq, k, v, ldkv, 0, out, ldo, rows, keys, enc_len, heads, head_dim,
                          1, ws, ATT_NOALLOC_SCRATCH_BYTES, 0, nullptr, nullptr, nullptr, s);
}

}  // extern "C"
