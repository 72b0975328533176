// Fused blockwise-sparse NF4 MLP for one decode token (M = 1) on gfx950.
//
// Replaces the reference's gather + Triton/fallback dispatch for a decode
// token (RT:5104-5524; kernel semantics of TSM:807-914: fp32 dequant and
// accumulation, fp32 intermediate, one fp16 rounding of the output).
//
// Two kernels, no host round trip, deterministic (no float atomics):
//   k_gate_up : grid (splits, k).  Workgroup (s, j) streams columns
//               [s*cs, (s+1)*cs) of the 32 gate rows and 32 up rows of block
//               sel[j] straight from its slot (one 16-byte load per lane per
//               row, coalesced over the row), dots them with x, reduces over
//               the lanes of each row and writes 64 partial sums.  The last
//               workgroup of block j to finish (atomic counter) sums the
//               split partials in split order and stores
//               act[j] = silu(gate) * up (fp32).
//   k_down    : grid (row chunks, groups).  Each thread owns one output row
//               and streams the 16-byte row of every block in its group from
//               the block-major down slot; the partial per group goes to
//               outpart[group][row].  The last group to finish a row chunk
//               sums the groups in group order and writes the fp16 output.
// Counters live in the workspace and are reset by their last user.
#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kThreads = 256;
constexpr int kDownBatch = 16;  // down blocks whose loads are issued together

template <int LPR>
__global__ void __launch_bounds__(kThreads) k_gate_up(DecodeArgs a) {
  constexpr int kStep = kThreads / LPR;   // rows covered per pass
  constexpr int NR = 64 / kStep;          // rows per thread (half gate, half up)
  static_assert(NR >= 2 && NR % 2 == 0, "lanes per row must be in [8, 64]");
  const int s = blockIdx.x;
  const int j = blockIdx.y;
  const int tid = threadIdx.x;
  __shared__ float lut_g[16], lut_u[16];
  __shared__ int s_last;
  if (tid < 16) {
    lut_g[tid] = a.code[tid];
    lut_u[tid] = a.code_up[tid];
  }

  const BlockRef br = resolve_block(a, j);
  if (!br.ok && !br.silent && tid == 0 && s == 0) atomicOr(a.status, 1);
  const long long q = br.q;
  const ProjView& G = br.dev ? a.gate : a.host_gate;
  const ProjView& U = br.dev ? a.up : a.host_up;

  const int cc = tid % LPR;
  const int r0 = tid / LPR;
  const int col = s * a.cs + cc * 32;

  uint4 w[NR];
  float am[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const ProjView& P = (i < NR / 2) ? G : U;
    const int r = (r0 + i * kStep) & 31;
    w[i] = make_uint4(0, 0, 0, 0);
    am[i] = 0.0f;
    if (br.ok) {
      w[i] = *reinterpret_cast<const uint4*>(P.packed + q * P.blk_stride + (long long)r * P.row_stride + (col >> 1));
      am[i] = P.absmax[q * P.abs_blk_stride + (long long)r * P.abs_row_stride + col / a.qbs];
    }
  }
  float xf[32];
  {
    const uint4* xp = reinterpret_cast<const uint4*>(a.x + col);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      uint4 t = xp[v];
      const uint32_t ws[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xf[8 * v + 2 * e] = h2f((uint16_t)(ws[e] & 0xFFFFu));
        xf[8 * v + 2 * e + 1] = h2f((uint16_t)(ws[e] >> 16));
      }
    }
  }
  __syncthreads();  // lut
  float acc[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) acc[i] = nf4_dot32(w[i], xf, i < NR / 2 ? lut_g : lut_u) * am[i];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) acc[i] += __shfl_xor(acc[i], m, kWave);
  }
  float* part = a.part + ((long long)j * a.splits + s) * 64;
  if (cc == 0) {
#pragma unroll
    for (int i = 0; i < NR; ++i) part[r0 + i * kStep] = acc[i];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&a.blk_count[j], 1) == a.splits - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (tid < 32) {
    const float* pj = a.part + (long long)j * a.splits * 64;
    float g = 0.0f, u = 0.0f;
    for (int t = 0; t < a.splits; ++t) {
      g += pj[t * 64 + tid];
      u += pj[t * 64 + 32 + tid];
    }
    float act = 0.0f;
    if (br.ok) {
      const long long n = (long long)br.b * 32 + tid;
      if (a.gate_bias != nullptr) g += h2f(a.gate_bias[n]);
      if (a.up_bias != nullptr) u += h2f(a.up_bias[n]);
      if (a.mask != nullptr) {
        const float m = h2f(a.mask[n]);
        g *= m;
        u *= m;
      }
      act = silu_mul(g, u);
    }
    a.act[(long long)j * 32 + tid] = act;
  }
  if (tid == 0) atomicExch(&a.blk_count[j], 0);
}

__global__ void __launch_bounds__(kThreads) k_down(DecodeArgs a) {
  const int rc = blockIdx.x;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int per = (a.k + a.groups - 1) / a.groups;
  const int j0 = g * per;
  const int j1 = min(a.k, j0 + per);
  extern __shared__ float act[];  // [per][32]
  __shared__ float lut[16];
  __shared__ int s_last;
  if (tid < 16) lut[tid] = a.code_down[tid];
  for (int i = tid; i < (j1 - j0) * 32; i += kThreads) act[i] = a.act[(long long)j0 * 32 + i];
  __syncthreads();
  const int o = rc * a.rows_per_chunk + tid;
  const bool live = o < a.H;
  float acc = 0.0f;
  for (int jb = j0; jb < j1; jb += kDownBatch) {
    uint4 w[kDownBatch];
    float am[kDownBatch];
#pragma unroll
    for (int i = 0; i < kDownBatch; ++i) {
      const int j = jb + i;
      w[i] = make_uint4(0, 0, 0, 0);
      am[i] = 0.0f;
      if (j < j1) {
        const BlockRef br = resolve_block(a, j);
        const ProjView& P = br.dev ? a.down : a.host_down;
        if (live && br.ok) {
          w[i] = *reinterpret_cast<const uint4*>(P.packed + br.q * P.blk_stride + (long long)o * P.row_stride);
          am[i] = P.absmax[br.q * P.abs_blk_stride + (long long)o * P.abs_row_stride];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kDownBatch; ++i) {
      const int j = jb + i;
      if (j < j1) acc += nf4_dot32(w[i], act + (j - j0) * 32, lut) * am[i];
    }
  }
  if (live) a.outpart[(long long)g * a.H + o] = acc;
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&a.row_count[rc], 1) == a.groups - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (live) {
    float y = 0.0f;
    for (int t = 0; t < a.groups; ++t) y += a.outpart[(long long)t * a.H + o];
    if (a.out_f32 != nullptr) a.out_f32[o] = y;
    if (a.down_bias != nullptr) y += h2f(a.down_bias[o]);
    a.out[o] = f2h(y);
  }
  if (tid == 0) atomicExch(&a.row_count[rc], 0);
}

}  // namespace

void launch_decode_gate_up(const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.splits, a.k);
  switch (a.cs / 32) {
    case 8: hipLaunchKernelGGL(k_gate_up<8>, grid, dim3(kThreads), 0, s, a); break;
    case 16: hipLaunchKernelGGL(k_gate_up<16>, grid, dim3(kThreads), 0, s, a); break;
    case 32: hipLaunchKernelGGL(k_gate_up<32>, grid, dim3(kThreads), 0, s, a); break;
    default: hipLaunchKernelGGL(k_gate_up<64>, grid, dim3(kThreads), 0, s, a); break;
  }
}

void launch_decode_down(const DecodeArgs& a, hipStream_t s) {
  const int per = (a.k + a.groups - 1) / a.groups;
  dim3 grid((a.H + a.rows_per_chunk - 1) / a.rows_per_chunk, a.groups);
  hipLaunchKernelGGL(k_down, grid, dim3(kThreads), (size_t)per * 32 * sizeof(float), s, a);
}

}  // namespace nsmlp
