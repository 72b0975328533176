// Multi-row sparse NF4 linears, slot-table gathers and synthetic NF4 data.
//
//   output linear : gate/up over the active slots of each row
//                   (TSM:1340-1375 triton_sparse_output_linear_4bit, with the
//                   row-major payload its runtime callers pass, RT:4630-4660)
//   input linear  : down over the active slots of each row
//                   (TSM:1303-1337 triton_sparse_input_linear_4bit, RT:5651-5675)
//   silu * up     : TSM:1577-1578
//   gathers       : gate/up row blocks (RT:4530-4578, RT:2722-2786) and down
//                   column blocks (RT:4455-4528, RT:2619-2720)
//   synthetic     : counter-based normal samples and an NF4 quantiser that
//                   restates the bitsandbytes nf4 rule (nearest code by
//                   midpoint thresholds, element 2i in the high nibble).
#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kThreads = 256;

// ----------------------------------------------------------- output linear
template <int LPR>
__global__ void __launch_bounds__(kThreads) k_out_partial(LinearArgs a) {
  constexpr int kStep = kThreads / LPR;  // rows per pass
  constexpr int NR = 32 / kStep;         // rows per thread
  static_assert(NR >= 1, "lanes per row must be >= 8");
  const int s = blockIdx.x;
  const int task = blockIdx.y;  // t * kk + i
  const int t = task / a.kk;
  const int slot = a.active_idx[task];
  if (slot < 0 || slot >= a.A) return;
  const int tid = threadIdx.x;
  __shared__ float lut[16];
  if (tid < 16) lut[tid] = a.code[tid];
  const int cc = tid % LPR;
  const int r0 = tid / LPR;
  const int col = s * a.cs + cc * 32;
  const long long row_bytes = a.in_dim / 2;
  const long long row_abs = a.in_dim / a.qbs;
  uint4 w[NR];
  float am[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const long long r = (long long)slot * 32 + r0 + i * kStep;
    w[i] = *reinterpret_cast<const uint4*>(a.packed + r * row_bytes + (col >> 1));
    am[i] = a.absmax[r * row_abs + col / a.qbs];
  }
  float xf[32];
  const uint16_t* xr = a.x + (long long)t * a.in_dim + col;
#pragma unroll
  for (int e = 0; e < 32; ++e) xf[e] = h2f(xr[e]);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    float acc = nf4_dot32_f32(w[i], xf, lut) * am[i];
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, kWave);
    if (cc == 0) a.part[((long long)task * a.splits + s) * 32 + r0 + i * kStep] = acc;
  }
}

__global__ void __launch_bounds__(kThreads) k_out_finish(LinearArgs a) {
  const int idx = blockIdx.x * kThreads + threadIdx.x;  // task * 32 + r
  if (idx >= a.rows * a.kk * 32) return;
  const int task = idx / 32, r = idx % 32;
  const int t = task / a.kk;
  const int slot = a.active_idx[task];
  if (slot < 0 || slot >= a.A) return;
  float acc = 0.0f;
  for (int s = 0; s < a.splits; ++s) acc += a.part[((long long)task * a.splits + s) * 32 + r];
  const long long n = (long long)slot * 32 + r;
  if (a.bias != nullptr) acc += h2f(a.bias[n]);
  uint16_t y = f2h(acc);
  if (a.mask != nullptr) y = f2h(h2f(y) * h2f(a.mask[(long long)t * a.A * 32 + n]));
  a.out[(long long)t * a.A * 32 + n] = y;
}

// ------------------------------------------------------------ input linear
constexpr int kInBatch = 16;

__global__ void __launch_bounds__(kThreads) k_in_linear(LinearArgs a) {
  const int o = blockIdx.x * kThreads + threadIdx.x;
  const int t = blockIdx.y;
  const int tid = threadIdx.x;
  __shared__ float lut[16];
  __shared__ float xs[kInBatch][32];
  __shared__ int slots[kInBatch];
  if (tid < 16) lut[tid] = a.code[tid];
  const bool live = o < a.out_dim;
  const long long row_bytes = a.in_dim / 2;
  const long long row_abs = a.in_dim / a.qbs;
  float acc = 0.0f;
  // active block e / bm contributes its 32-column slot e % bm
  const int n = a.kk * a.bm;
  for (int ib = 0; ib < n; ib += kInBatch) {
    __syncthreads();
    if (tid < kInBatch) {
      const int e = ib + tid;
      const int blk = e < n ? a.active_idx[(long long)t * a.kk + e / a.bm] : -1;
      const long long sl = (long long)blk * a.bm + e % a.bm;
      slots[tid] = (blk >= 0 && sl * 32 < a.in_dim) ? (int)sl : -1;
    }
    __syncthreads();
    for (int e = tid; e < kInBatch * 32; e += kThreads) {
      int i = e / 32, c = e % 32;
      int sl = slots[i];
      xs[i][c] = sl >= 0 ? h2f(a.x[(long long)t * a.in_dim + (long long)sl * 32 + c]) : 0.0f;
    }
    __syncthreads();
    uint4 w[kInBatch];
    float am[kInBatch];
#pragma unroll
    for (int i = 0; i < kInBatch; ++i) {
      const int sl = slots[i];
      w[i] = make_uint4(0, 0, 0, 0);
      am[i] = 0.0f;
      if (sl >= 0 && live) {
        w[i] = *reinterpret_cast<const uint4*>(a.packed + (long long)o * row_bytes + (long long)sl * 16);
        am[i] = a.absmax[(long long)o * row_abs + ((long long)sl * 32) / a.qbs];
      }
    }
#pragma unroll
    for (int i = 0; i < kInBatch; ++i)
      if (slots[i] >= 0) acc += nf4_dot32_f32(w[i], xs[i], lut) * am[i];
  }
  if (live) {
    if (a.bias != nullptr) acc += h2f(a.bias[o]);
    a.out[(long long)t * a.out_dim + o] = f2h(acc);
  }
}

__global__ void k_zero_u32(uint32_t* p, long long n) {
  long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Status hand-over: the workspace's status word is ORed into dst and
// cleared, in stream order (a kernel, not a memset, so it may sit in a
// captured graph).  dst may be pinned host memory: its accesses are
// system-scope, and it is read only when there is something to add.
__global__ void k_take_status(int* status, int* dst) {
  if (threadIdx.x == 0) {
    const int v = *status;
    *status = 0;
    if (v != 0 && dst != nullptr) {
      const int old = __hip_atomic_load(dst, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(dst, old | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

// Block counts [2] of a workspace added to dst [2] (int64) and cleared.
__global__ void k_take_counts(uint32_t* counts, long long* dst) {
  if (threadIdx.x < 2) {
    const uint32_t v = counts[threadIdx.x];
    counts[threadIdx.x] = 0;
    if (v != 0) {
      long long* d = dst + threadIdx.x;
      const long long old = __hip_atomic_load(d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(d, old + (long long)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

__global__ void k_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, long long n) {
  long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = f2h(silu_mul(h2f(g[i]), h2f(u[i])));
}

// ----------------------------------------------------------------- gathers
template <typename AbsT>
__global__ void k_gather_rows(const uint8_t* src, const AbsT* src_abs, const int32_t* blocks, int src_blocks,
                              long long bpb, long long apb, uint8_t* dst, AbsT* dst_abs) {
  const int i = blockIdx.y;
  const long long b = blocks[i];
  if (b < 0 || b >= src_blocks) return;  // out-of-range id: the destination block is left untouched
  const long long n16 = bpb / 16;
  for (long long v = (long long)blockIdx.x * kThreads + threadIdx.x; v < n16; v += (long long)gridDim.x * kThreads)
    reinterpret_cast<uint4*>(dst + i * bpb)[v] = reinterpret_cast<const uint4*>(src + b * bpb)[v];
  for (long long v = (long long)blockIdx.x * kThreads + threadIdx.x; v < apb; v += (long long)gridDim.x * kThreads)
    dst_abs[i * apb + v] = src_abs[b * apb + v];
}

// u8 absmax codes of row blocks into the slot layout [n][16][A][2] (A =
// entries per row): byte (r, c) of block i goes to ((r >> 1) A + c) 2 + (r & 1).
__global__ void k_gather_rows_q8(const uint8_t* src, const int32_t* blocks, int src_blocks, int A, uint8_t* dst) {
  const int i = blockIdx.y;
  const long long b = blocks[i];
  if (b < 0 || b >= src_blocks) return;
  const long long apb = 32LL * A;
  for (long long v = (long long)blockIdx.x * kThreads + threadIdx.x; v < apb; v += (long long)gridDim.x * kThreads) {
    const long long r = v / A, c = v % A;
    dst[i * apb + ((r >> 1) * A + c) * 2 + (r & 1)] = src[b * apb + v];
  }
}

template <typename AbsT>
__global__ void k_gather_down(const uint8_t* src, const AbsT* src_abs, const int32_t* blocks, int n, int out_f,
                              int in_f, int qbs, int layout, uint8_t* dst, AbsT* dst_abs) {
  const long long idx = (long long)blockIdx.x * kThreads + threadIdx.x;  // o * n + i
  if (idx >= (long long)out_f * n) return;
  const long long o = idx / n;
  const long long i = idx % n;
  const long long b = blocks[i];
  if (b < 0 || b >= in_f / 32) return;  // out-of-range id: the destination is left untouched
  const uint4 v = *reinterpret_cast<const uint4*>(src + o * (in_f / 2) + b * 16);
  const AbsT am = src_abs[o * (in_f / qbs) + (b * 32) / qbs];
  const long long d = layout == NSMLP_DOWN_BLOCK_MAJOR ? i * out_f + o : o * n + i;
  reinterpret_cast<uint4*>(dst)[d] = v;
  dst_abs[d] = am;
}

// ------------------------------------------------------- double-quantised absmax
// One workgroup of kDqThreads per block of dq_block absmax (dq_block a power
// of two in [1, 4096]; each thread handles dq_block / kDqThreads entries or
// one).  The same fp32 operations as the restated bitsandbytes quantiser:
// a = absmax - offset, absmax2 = max |a|, v = a * fp32(1 / absmax2), nearest
// code2 entry (ties: lower index).
constexpr int kDqThreads = 256;

__device__ __forceinline__ uint32_t nearest_code2(const float* c2, float v) {
  // c2 ascending: lo = number of entries < v; the nearest is lo - 1 or lo,
  // then the lowest index of equal computed distance
  int lo = 0, hi = 256;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (c2[mid] < v) lo = mid + 1; else hi = mid;
  }
  int best;
  if (lo == 256) best = 255;
  else if (lo == 0) best = 0;
  else best = fabsf(c2[lo - 1] - v) <= fabsf(c2[lo] - v) ? lo - 1 : lo;
  const float d = fabsf(c2[best] - v);
  while (best > 0 && fabsf(c2[best - 1] - v) == d) --best;
  return (uint32_t)best;
}

__global__ void __launch_bounds__(kDqThreads) k_absmax_dq(const float* absmax, long long n, int dq_block,
                                                          const float* code2, float offset, uint8_t* q,
                                                          float* absmax2) {
  __shared__ float c2[256];
  __shared__ float wmax[kDqThreads / kWave];
  const int tid = threadIdx.x;
  c2[tid] = code2[tid];
  const long long lo = (long long)blockIdx.x * dq_block;
  const long long hi = lo + dq_block < n ? lo + dq_block : n;
  float m = 0.0f;
  for (long long i = lo + tid; i < hi; i += kDqThreads) m = fmaxf(m, fabsf(__fsub_rn(absmax[i], offset)));
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, kWave));
  if ((tid & (kWave - 1)) == 0) wmax[tid / kWave] = m;
  __syncthreads();
  float amax = 0.0f;
#pragma unroll
  for (int w = 0; w < kDqThreads / kWave; ++w) amax = fmaxf(amax, wmax[w]);
  const float inv = amax > 0.0f ? __frcp_rn(amax) : 0.0f;
  if (tid == 0) absmax2[blockIdx.x] = amax;
  for (long long i = lo + tid; i < hi; i += kDqThreads)
    q[i] = (uint8_t)nearest_code2(c2, __fmul_rn(__fsub_rn(absmax[i], offset), inv));
}

__global__ void k_absmax_undq(const uint8_t* q, long long n, int dq_shift, const float* code2, const float* absmax2,
                              float offset, float* out) {
  const long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = dq_absmax(code2[q[i]], absmax2[i >> dq_shift], offset);
}

// ---------------------------------------------------------------- synthetic
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Standard normal sample for element i of stream `seed` (Box-Muller).
__device__ __forceinline__ float synth_normal(uint64_t seed, uint64_t i) {
  uint64_t h = mix64(seed * 0xD1B54A32D192ED03ull + mix64(i));
  float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
  float u2 = (float)(h & 0xFFFFFFull) * (1.0f / 16777216.0f);
  return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

__constant__ float c_nf4_mid[15];

__device__ __forceinline__ uint32_t nf4_nearest(float v) {
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < 15; ++i) c += v > c_nf4_mid[i];
  return c;
}

template <bool kSynth>
__global__ void __launch_bounds__(kThreads) k_nf4_quant(const float* w, uint64_t seed, float std, long long nblk,
                                                        int qbs, uint8_t* packed, float* absmax) {
  const long long blk = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (blk >= nblk) return;
  const long long e0 = blk * qbs;
  float amax = 0.0f;
  for (int i = 0; i < qbs; ++i) {
    float v = kSynth ? std * synth_normal(seed, e0 + i) : w[e0 + i];
    amax = fmaxf(amax, fabsf(v));
  }
  absmax[blk] = amax;
  const float inv = amax > 0.0f ? __frcp_rn(amax) : 0.0f;
  for (int i = 0; i < qbs; i += 8) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = kSynth ? std * synth_normal(seed, e0 + i + e) : w[e0 + i + e];
      uint32_t c = amax > 0.0f ? nf4_nearest(v * inv) : 7u;
      // byte e/2: even element -> high nibble
      word |= c << (8 * (e >> 1) + ((e & 1) ? 0 : 4));
    }
    *reinterpret_cast<uint32_t*>(packed + (e0 + i) / 2) = word;
  }
}

__global__ void k_synth_normal_f16(uint64_t seed, long long n, float std, uint16_t* out) {
  long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = f2h(std * synth_normal(seed, i));
}

__global__ void k_synth_normal_f32(uint64_t seed, long long n, float std, float* out) {
  long long i = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = std * synth_normal(seed, i);
}

unsigned grid_for(long long n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

void launch_output_linear(const LinearArgs& a, hipStream_t s) {
  dim3 grid(a.splits, a.rows * a.kk);
  switch (a.cs / 32) {
    case 8: hipLaunchKernelGGL(k_out_partial<8>, grid, dim3(kThreads), 0, s, a); break;
    case 16: hipLaunchKernelGGL(k_out_partial<16>, grid, dim3(kThreads), 0, s, a); break;
    case 32: hipLaunchKernelGGL(k_out_partial<32>, grid, dim3(kThreads), 0, s, a); break;
    default: hipLaunchKernelGGL(k_out_partial<64>, grid, dim3(kThreads), 0, s, a); break;
  }
  hipLaunchKernelGGL(k_out_finish, dim3(grid_for((long long)a.rows * a.kk * 32)), dim3(kThreads), 0, s, a);
}

void launch_input_linear(const LinearArgs& a, hipStream_t s) {
  dim3 grid(grid_for(a.out_dim), a.rows);
  hipLaunchKernelGGL(k_in_linear, grid, dim3(kThreads), 0, s, a);
}

void launch_zero_u32(uint32_t* p, long long n, hipStream_t s) {
  hipLaunchKernelGGL(k_zero_u32, dim3(grid_for(n)), dim3(kThreads), 0, s, p, n);
}

void launch_take_status(int* status, int* dst, hipStream_t s) {
  hipLaunchKernelGGL(k_take_status, dim3(1), dim3(64), 0, s, status, dst);
}

void launch_take_counts(uint32_t* counts, long long* dst, hipStream_t s) {
  hipLaunchKernelGGL(k_take_counts, dim3(1), dim3(64), 0, s, counts, dst);
}

void launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, long long n, hipStream_t s) {
  hipLaunchKernelGGL(k_silu_mul, dim3(grid_for(n)), dim3(kThreads), 0, s, g, u, out, n);
}

template <typename AbsT>
void launch_gather_rows(const uint8_t* src, const AbsT* src_abs, const int32_t* blocks, int src_blocks, int n,
                        long long bpb, long long apb, uint8_t* dst, AbsT* dst_abs, hipStream_t s) {
  long long per = (bpb / 16 > apb ? bpb / 16 : apb);
  unsigned gx = (unsigned)((per + kThreads - 1) / kThreads);
  if (gx > 64) gx = 64;
  k_gather_rows<AbsT><<<dim3(gx, n), dim3(kThreads), 0, s>>>(src, src_abs, blocks, src_blocks, bpb, apb, dst, dst_abs);
}
template void launch_gather_rows<float>(const uint8_t*, const float*, const int32_t*, int, int, long long, long long,
                                        uint8_t*, float*, hipStream_t);

void launch_gather_rows_q8(const uint8_t* src_packed, const uint8_t* src_q, const int32_t* blocks, int src_blocks,
                           int n, long long bpb, int A, uint8_t* dst_packed, uint8_t* dst_q, hipStream_t s) {
  const long long apb = 32LL * A;
  unsigned gx = (unsigned)((apb + kThreads - 1) / kThreads);
  if (gx > 64) gx = 64;
  k_gather_rows_q8<<<dim3(gx, n), dim3(kThreads), 0, s>>>(src_q, blocks, src_blocks, A, dst_q);
  if (src_packed != nullptr) {
    unsigned gp = (unsigned)((bpb / 16 + kThreads - 1) / kThreads);
    if (gp > 64) gp = 64;
    // packed bytes only (absmax count 0)
    k_gather_rows<uint8_t><<<dim3(gp, n), dim3(kThreads), 0, s>>>(src_packed, nullptr, blocks, src_blocks, bpb, 0,
                                                                  dst_packed, nullptr);
  }
}

template <typename AbsT>
void launch_gather_down(const uint8_t* src, const AbsT* src_abs, const int32_t* blocks, int n, int out_f, int in_f,
                        int qbs, int layout, uint8_t* dst, AbsT* dst_abs, hipStream_t s) {
  k_gather_down<AbsT><<<dim3(grid_for((long long)out_f * n)), dim3(kThreads), 0, s>>>(src, src_abs, blocks, n, out_f,
                                                                                      in_f, qbs, layout, dst, dst_abs);
}
template void launch_gather_down<float>(const uint8_t*, const float*, const int32_t*, int, int, int, int, int,
                                        uint8_t*, float*, hipStream_t);
template void launch_gather_down<uint8_t>(const uint8_t*, const uint8_t*, const int32_t*, int, int, int, int, int,
                                          uint8_t*, uint8_t*, hipStream_t);

void launch_absmax_dq(const float* absmax, long long n, int dq_block, const float* code2, float offset, uint8_t* q,
                      float* absmax2, hipStream_t s) {
  const long long nb = (n + dq_block - 1) / dq_block;
  k_absmax_dq<<<dim3((unsigned)nb), dim3(kDqThreads), 0, s>>>(absmax, n, dq_block, code2, offset, q, absmax2);
}

void launch_absmax_undq(const uint8_t* q, long long n, int dq_shift, const float* code2, const float* absmax2,
                        float offset, float* out, hipStream_t s) {
  k_absmax_undq<<<dim3(grid_for(n)), dim3(kThreads), 0, s>>>(q, n, dq_shift, code2, absmax2, offset, out);
}

void set_nf4_midpoints(const float* mid15) {
  (void)hipMemcpyToSymbol(HIP_SYMBOL(c_nf4_mid), mid15, 15 * sizeof(float));
}

void launch_nf4_quant(const float* w, uint64_t seed, float std, long long n, int qbs, bool synth, uint8_t* packed,
                      float* absmax, hipStream_t s) {
  long long nblk = n / qbs;
  if (synth)
    hipLaunchKernelGGL(k_nf4_quant<true>, dim3(grid_for(nblk)), dim3(kThreads), 0, s, w, seed, std, nblk, qbs, packed,
                       absmax);
  else
    hipLaunchKernelGGL(k_nf4_quant<false>, dim3(grid_for(nblk)), dim3(kThreads), 0, s, w, seed, std, nblk, qbs,
                       packed, absmax);
}

void launch_synth_normal_f16(uint64_t seed, long long n, float std, uint16_t* out, hipStream_t s) {
  hipLaunchKernelGGL(k_synth_normal_f16, dim3(grid_for(n)), dim3(kThreads), 0, s, seed, n, std, out);
}

void launch_synth_normal_f32(uint64_t seed, long long n, float std, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_synth_normal_f32, dim3(grid_for(n)), dim3(kThreads), 0, s, seed, n, std, out);
}

}  // namespace nsmlp
