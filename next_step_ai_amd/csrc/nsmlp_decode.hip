// Fused blockwise-sparse NF4 MLP for one decode token (M = 1) on gfx950.
//
// Replaces the reference's gather + Triton/fallback dispatch for a decode
// token (RT:5104-5524; kernel semantics of TSM:807-914: fp32 accumulation,
// one fp16 rounding of the output).  Deterministic: no float atomics, every
// sum is taken in a fixed order.
//
// The streaming kernels for hidden sizes that are a multiple of 2048 live in
// nsmlp_stream.hip.
// Generic path (any hidden size that is a multiple of 256, any down layout):
// k_gate_up / k_down, the same arithmetic in two launches with a last-arriver
// hand-off.
#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kThreads = 256;
constexpr int kDownBatch = 16;  // down blocks whose loads are issued together

// Sum of 16 per-lane row partials over the 64 lanes of a wave: after the
// reduce-scatter every lane holds the total of row ((lane >> 2) & 15).
__device__ __forceinline__ float butterfly16(const float (&acc)[16], int lane) {
  float v8[8], v4[4], v2[2];
  const bool u5 = lane & 32, u4 = lane & 16, u3 = lane & 8, u2 = lane & 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float send = u5 ? acc[i] : acc[i + 8];
    float keep = u5 ? acc[i + 8] : acc[i];
    v8[i] = keep + __shfl_xor(send, 32, kWave);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float send = u4 ? v8[i] : v8[i + 4];
    float keep = u4 ? v8[i + 4] : v8[i];
    v4[i] = keep + __shfl_xor(send, 16, kWave);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float send = u3 ? v4[i] : v4[i + 2];
    float keep = u3 ? v4[i + 2] : v4[i];
    v2[i] = keep + __shfl_xor(send, 8, kWave);
  }
  float send = u2 ? v2[0] : v2[1];
  float v = (u2 ? v2[1] : v2[0]) + __shfl_xor(send, 4, kWave);
  v += __shfl_xor(v, 2, kWave);
  v += __shfl_xor(v, 1, kWave);
  return v;
}

struct DecodeSmem {
  __attribute__((aligned(16))) char lut_g[256];
  __attribute__((aligned(16))) char lut_u[256];
  __attribute__((aligned(16))) char lut_d[256];
  int s_last;
};

__device__ __forceinline__ void fill_luts(const DecodeArgs& a, DecodeSmem& sm, int tid) {
  lut_fill(sm.lut_g, a.code, tid);
  lut_fill(sm.lut_u, a.code_up, tid);
  lut_fill(sm.lut_d, a.code_down, tid);
}

// Gate/up work item (block position j, column split s).  The last split to
// finish block j computes act[j].
template <int LPR>
__device__ __forceinline__ void gate_up_task(const DecodeArgs& a, DecodeSmem& sm, int j, int s) {
  constexpr int kStep = kThreads / LPR;  // rows covered per pass
  constexpr int NR = 64 / kStep;         // rows per thread (half gate, half up)
  static_assert(NR >= 2 && NR % 2 == 0, "lanes per row must be in [8, 64]");
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);

  const BlockRef br = resolve_block(a, j);
  if (!br.ok && !br.silent && tid == 0 && s == 0) atomicOr(a.status, 1);
  if (br.ok && tid == 0 && s == 0 && a.served != nullptr) atomicAdd(a.served + (br.dev ? 0 : 1), 1u);
  const uint8_t* gbase = (br.dev ? a.gate.packed : a.host_gate.packed) + br.q * a.gate.blk_stride;
  const uint8_t* ubase = (br.dev ? a.up.packed : a.host_up.packed) + br.q * a.up.blk_stride;
  const float* gabs = (br.dev ? a.gate.absmax : a.host_gate.absmax) + br.q * a.gate.abs_blk_stride;
  const float* uabs = (br.dev ? a.up.absmax : a.host_up.absmax) + br.q * a.up.abs_blk_stride;
  const uint8_t* gq = (br.dev ? a.gate.qabsmax : a.host_gate.qabsmax) + br.q * a.gate.abs_blk_stride;
  const uint8_t* uq = (br.dev ? a.up.qabsmax : a.host_up.qabsmax) + br.q * a.up.abs_blk_stride;

  const int cc = tid % LPR;
  const int r0 = tid / LPR;
  const int col = s * a.cs + cc * 32;
  const uint32_t rs = (uint32_t)a.gate.row_stride;
  const uint32_t ars = (uint32_t)a.gate.abs_row_stride;
  const uint32_t off = (uint32_t)r0 * rs + (uint32_t)(col >> 1);
  const uint32_t aoff = (uint32_t)r0 * ars + (uint32_t)(col >> a.qbs_shift);

  uint4 w[NR];
  float am[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int ri = i % (NR / 2);
    const uint8_t* base = i < NR / 2 ? gbase : ubase;
    const float* abase = i < NR / 2 ? gabs : uabs;
    w[i] = make_uint4(0, 0, 0, 0);
    am[i] = 0.0f;
    if (br.ok) {
      w[i] = *reinterpret_cast<const uint4*>(base + off + (uint32_t)(ri * kStep) * rs);
      const uint32_t ai = aoff + (uint32_t)(ri * kStep) * ars;
      if (a.dq) {
        // u8 codes interleave row pairs: (r, c) at ((r >> 1) A + c) 2 + (r & 1)
        const ProjView& pv = i < NR / 2 ? a.gate : a.up;
        const uint32_t r = (uint32_t)(r0 + ri * kStep), c = (uint32_t)(col >> a.qbs_shift);
        const uint32_t qi = ((r >> 1) * ars + c) * 2u + (r & 1u);
        const long long f = ((long long)br.b * 32 + r) * ars + c;
        am[i] = dq_absmax(pv.code2[(i < NR / 2 ? gq : uq)[qi]], pv.absmax2[f >> a.dq_shift], pv.offset);
      } else {
        am[i] = abase[ai];
      }
    }
  }
  uint32_t xp[16];
  {
    const uint4* xv = reinterpret_cast<const uint4*>(a.x + col);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      uint4 t = xv[v];
      xp[4 * v] = t.x;
      xp[4 * v + 1] = t.y;
      xp[4 * v + 2] = t.z;
      xp[4 * v + 3] = t.w;
    }
  }
  float acc[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) acc[i] = nf4_dot32(w[i], xp, i < NR / 2 ? sm.lut_g : sm.lut_u) * am[i];

  float* part = a.part + ((long long)j * a.splits + s) * 64;
  if constexpr (LPR == 64) {
    const float v = butterfly16(acc, lane);
    if ((lane & 3) == 0) st_coherent(part + r0 + ((lane >> 2) & 15) * kStep, v);
  } else {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
#pragma unroll
      for (int m = LPR / 2; m >= 1; m >>= 1) acc[i] += __shfl_xor(acc[i], m, kWave);
    }
    if (cc == 0) {
#pragma unroll
      for (int i = 0; i < NR; ++i) st_coherent(part + r0 + i * kStep, acc[i]);
    }
  }
  wait_stores();
  __syncthreads();
  if (tid == 0) sm.s_last = atomicAdd(&a.blk_count[j], 1) == a.splits - 1;
  __syncthreads();
  if (!sm.s_last || tid >= kWave) return;
  // Last split of block j: act = silu(gate) * up, summed in split order.
  const float* pj = a.part + (long long)j * a.splits * 64;
  float act = 0.0f;
  if (lane < 32) {
    float g = 0.0f, u = 0.0f;
    for (int t = 0; t < a.splits; ++t) {
      g += ld_coherent(pj + t * 64 + lane);
      u += ld_coherent(pj + t * 64 + 32 + lane);
    }
    if (br.ok) {
      const long long n = (long long)br.b * 32 + lane;
      if (a.gate_bias != nullptr) g += h2f(a.gate_bias[n]);
      if (a.up_bias != nullptr) u += h2f(a.up_bias[n]);
      if (a.mask != nullptr) {
        const float m = h2f(a.mask[n]);
        g *= m;
        u *= m;
      }
      act = silu_mul(g, u);
    }
  }
  // fp16 storage scaled by a power of two so that max |act| lies in [0.5, 1).
  float mx = fabsf(act);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, kWave));
  int ex = 0;
  if (mx > 0.0f) frexpf(mx, &ex);
  const uint32_t h = f2h(ldexpf(act, -ex));
  const uint32_t hn = __shfl_xor(h, 1, kWave);
  if (lane < 32 && (lane & 1) == 0) st_coherent_u32(a.act + (long long)j * 16 + (lane >> 1), h | (hn << 16));
  if (lane == 0) st_coherent(a.act_scale + j, ldexpf(1.0f, ex));
  wait_stores();
  if (lane == 0) atomicExch(&a.blk_count[j], 0);
}

// Down work item (block group g, row chunk rc).
__device__ __forceinline__ void down_task(const DecodeArgs& a, DecodeSmem& sm, uint32_t* act, float* scale, int g,
                                          int rc) {
  const int tid = threadIdx.x;
  const int per = (a.k + a.groups - 1) / a.groups;
  const int j0 = g * per;
  const int j1 = min(a.k, j0 + per);
  for (int i = tid; i < (j1 - j0) * 16; i += kThreads) act[i] = ld_coherent_u32(a.act + (long long)j0 * 16 + i);
  for (int i = tid; i < j1 - j0; i += kThreads) scale[i] = ld_coherent(a.act_scale + j0 + i);
  __syncthreads();
  const int o = rc * a.rows_per_chunk + tid;
  const bool live = o < a.H;
  const uint32_t roff = (uint32_t)o * (uint32_t)a.down.row_stride;
  const uint32_t aroff = (uint32_t)o * (uint32_t)a.down.abs_row_stride;
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
        const uint8_t* base = (br.dev ? a.down.packed : a.host_down.packed) + br.q * a.down.blk_stride;
        const float* abase = (br.dev ? a.down.absmax : a.host_down.absmax) + br.q * a.down.abs_blk_stride;
        const uint8_t* qbase = (br.dev ? a.down.qabsmax : a.host_down.qabsmax) + br.q * a.down.abs_blk_stride;
        if (live && br.ok) {
          w[i] = *reinterpret_cast<const uint4*>(base + roff);
          if (a.dq) {
            const long long f = (long long)o * ((long long)a.NB * 32 >> a.qbs_shift) + ((br.b * 32) >> a.qbs_shift);
            am[i] = dq_absmax(a.down.code2[qbase[aroff]], a.down.absmax2[f >> a.dq_shift], a.down.offset);
          } else {
            am[i] = abase[aroff];
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kDownBatch; ++i) {
      const int j = jb + i;
      if (j < j1) acc += nf4_dot32(w[i], act + (j - j0) * 16, sm.lut_d) * (am[i] * scale[j - j0]);
    }
  }
  if (live) st_coherent(a.outpart + (long long)g * a.H + o, acc);
  wait_stores();
  __syncthreads();
  if (tid == 0) sm.s_last = atomicAdd(&a.row_count[rc], 1) == a.groups - 1;
  __syncthreads();
  if (!sm.s_last) return;
  if (live) {
    float y = 0.0f;
    for (int t = 0; t < a.groups; ++t) y += ld_coherent(a.outpart + (long long)t * a.H + o);
    a.out[o] = decode_out(a, o, y);
  }
  if (tid == 0) atomicExch(&a.row_count[rc], 0);
}

template <int LPR>
__global__ void __launch_bounds__(kThreads) k_gate_up(DecodeArgs a) {
  __shared__ DecodeSmem sm;
  fill_luts(a, sm, threadIdx.x);
  __syncthreads();
  gate_up_task<LPR>(a, sm, blockIdx.y, blockIdx.x);
}

__global__ void __launch_bounds__(kThreads) k_down(DecodeArgs a) {
  __shared__ DecodeSmem sm;
  extern __shared__ uint32_t dyn[];  // act [per][16] fp16 pairs, then scale [per]
  const int per = (a.k + a.groups - 1) / a.groups;
  fill_luts(a, sm, threadIdx.x);
  down_task(a, sm, dyn, reinterpret_cast<float*>(dyn + per * 16), blockIdx.y, blockIdx.x);
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
  hipLaunchKernelGGL(k_down, grid, dim3(kThreads), (size_t)per * (16 + 1) * sizeof(uint32_t), s, a);
}

}  // namespace nsmlp
