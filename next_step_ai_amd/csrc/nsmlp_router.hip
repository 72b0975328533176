// Learned-basis router of the blockwise-sparse MLP (the reference's
// _compute_sparse_basis_latent + _route_sparse_mlp, RT:4209-4238 and
// RT:4311-4352), as three gfx950 kernels:
//   1. latent partials : exact fp16 dot products of x with enc_w, split over
//                        many workgroups (the 2 MiB enc_w read is spread
//                        over the chip), accumulated with Exact3.
//   2. scores          : exact merge of the partials -> fp16 latent (+ the
//                        basis_top_k mask) -> exact score dots -> fp16,
//                        clamp, optional down_block_norm scaling.
//   3. select          : one workgroup per token; radix select of the k-th
//                        largest 32-bit key (fp16 order key << 16 | ~index),
//                        so ties resolve to the lowest block index, then an
//                        ordered compaction (ascending block ids) or a rank
//                        sort (score desc, index asc).
#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kLatThreads = 256;
constexpr int kScoreThreads = 256;
constexpr int kSelThreads = 1024;

template <bool kVec>
__global__ void __launch_bounds__(kLatThreads) k_latent_partial(RouteArgs a) {
  const int s = blockIdx.x;    // column split
  const int r = blockIdx.y;    // latent row
  const int row = blockIdx.z;  // token
  const int tid = threadIdx.x;
  const uint16_t* __restrict__ x = a.x + (long long)row * a.H;
  const uint16_t* __restrict__ w = a.enc_w + (long long)r * a.H;
  const int c0 = s * a.lat_cols + tid * 8;
  Exact3 acc = exact_zero();
  if (kVec) {
    if (c0 < a.H) {
      uint4 xv = *reinterpret_cast<const uint4*>(x + c0);
      uint4 wv = *reinterpret_cast<const uint4*>(w + c0);
      const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
      const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float p0 = h2f((uint16_t)(xs[q] & 0xFFFFu)) * h2f((uint16_t)(ws[q] & 0xFFFFu));
        float p1 = h2f((uint16_t)(xs[q] >> 16)) * h2f((uint16_t)(ws[q] >> 16));
        exact_add(acc, (double)p0);
        exact_add(acc, (double)p1);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int c = c0 + i;
      if (c < a.H) exact_add(acc, (double)(h2f(x[c]) * h2f(w[c])));
    }
  }
  if (s == 0 && tid == 0 && a.enc_b != nullptr) exact_add(acc, (double)h2f(a.enc_b[r]));
  acc = wave_sum_exact(acc);
  __shared__ double red[kLatThreads / kWave][3];
  const int wave = tid / kWave, lane = tid % kWave;
  if (lane == 0) {
    red[wave][0] = acc.a0;
    red[wave][1] = acc.a1;
    red[wave][2] = acc.a2;
  }
  __syncthreads();
  if (tid == 0) {
    Exact3 t = exact_zero();
    for (int wv = 0; wv < kLatThreads / kWave; ++wv) exact_merge(t, Exact3{red[wv][0], red[wv][1], red[wv][2]});
    double* dst = a.lat_part + (((long long)row * a.R + r) * a.lat_splits + s) * 3;
    dst[0] = t.a0;
    dst[1] = t.a1;
    dst[2] = t.a2;
  }
}

__global__ void __launch_bounds__(kScoreThreads) k_scores(RouteArgs a) {
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  extern __shared__ uint16_t lat16[];  // [R]
  // Latent: exact merge of the split partials, one fp16 rounding (RT:4221-4222).
  for (int r = tid; r < a.R; r += kScoreThreads) {
    const double* src = a.lat_part + ((long long)row * a.R + r) * a.lat_splits * 3;
    Exact3 e = exact_zero();
    for (int s = 0; s < a.lat_splits; ++s) exact_merge(e, Exact3{src[3 * s], src[3 * s + 1], src[3 * s + 2]});
    lat16[r] = exact_to_f16(e);
  }
  __syncthreads();
  // basis_top_k mask over |latent| (RT:4233-4238); ties keep the lower index.
  int btk = a.basis_top_k < 1 ? 1 : (a.basis_top_k > a.R ? a.R : a.basis_top_k);
  if (btk < a.R) {
    uint16_t keep_val[4];
    int nmine = 0;
    for (int r = tid; r < a.R; r += kScoreThreads) {
      uint32_t kr = f16_order_key((uint16_t)(lat16[r] & 0x7FFFu));
      int rank = 0;
      for (int q = 0; q < a.R; ++q) {
        uint32_t kq = f16_order_key((uint16_t)(lat16[q] & 0x7FFFu));
        rank += (kq > kr) || (kq == kr && q < r);
      }
      keep_val[nmine++] = rank < btk ? lat16[r] : (uint16_t)(lat16[r] & 0x8000u);
    }
    __syncthreads();
    nmine = 0;
    for (int r = tid; r < a.R; r += kScoreThreads) lat16[r] = keep_val[nmine++];
    __syncthreads();
  }
  if (blockIdx.x == 0 && a.latent_out != nullptr)
    for (int r = tid; r < a.R; r += kScoreThreads) a.latent_out[(long long)row * a.R + r] = lat16[r];
  const int j = blockIdx.x * kScoreThreads + tid;
  if (j >= a.NB) return;
  const uint16_t* __restrict__ w = a.score_w + (long long)j * a.R;
  Exact3 acc = exact_zero();
  const uint16_t amask = a.legacy_abs ? 0x7FFFu : 0xFFFFu;
  for (int r = 0; r < a.R; ++r) {
    float p = h2f((uint16_t)(lat16[r] & amask)) * h2f(w[r]);
    exact_add(acc, (double)p);
  }
  if (!a.legacy_abs && a.score_b != nullptr) exact_add(acc, (double)h2f(a.score_b[j]));
  uint16_t sc = exact_to_f16(acc);
  if (!a.legacy_abs && (sc & 0x8000u)) sc = 0;  // clamp_min(0) (RT:4331)
  if (a.dbn != nullptr) sc = f2h(h2f(sc) * h2f(a.dbn[j]));  // fp16 x fp16 is exact in fp32
  a.scores[(long long)row * a.NB + j] = sc;
  if (a.scores_out != nullptr) a.scores_out[(long long)row * a.NB + j] = sc;
}

__device__ __forceinline__ uint32_t sel_key(const uint16_t* sc, int i) {
  return (f16_order_key(sc[i]) << 16) | (uint32_t)(0xFFFFu - (uint32_t)i);
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    int o = __shfl_up(v, d, kWave);
    if (lane >= d) v += o;
  }
  return v;
}

__global__ void __launch_bounds__(kSelThreads) k_select(RouteArgs a) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid % kWave, wave = tid / kWave;
  const uint16_t* sc = a.scores + (long long)row * a.NB;
  const int NB = a.NB;
  const int k = a.k;
  __shared__ unsigned hist[256];
  __shared__ unsigned s_digit, s_above;
  __shared__ int wsum[kSelThreads / kWave];
  uint32_t prefix = 0, mask = 0;
  unsigned remaining = (unsigned)k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = tid; i < 256; i += kSelThreads) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < NB; i += kSelThreads) {
      uint32_t key = sel_key(sc, i);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 0xFFu], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      unsigned c[4];
      unsigned local = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        c[b] = hist[255 - 4 * lane - b];
        local += c[b];
      }
      unsigned incl = (unsigned)wave_incl_scan((int)local, lane);
      unsigned excl = incl - local;
      if (excl < remaining && remaining <= incl) {
        unsigned cum = excl;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (cum + c[b] >= remaining) {
            s_digit = 255u - 4u * lane - b;
            s_above = cum;
            break;
          }
          cum += c[b];
        }
      }
    }
    __syncthreads();
    prefix |= s_digit << shift;
    mask |= 0xFFu << shift;
    remaining -= s_above;
    __syncthreads();
  }
  const uint32_t T = prefix;  // the k-th largest key (keys are unique)
  // Ordered compaction: selected = keys >= T, ascending block index.
  const int per = (NB + kSelThreads - 1) / kSelThreads;
  const int i0 = tid * per;
  const int i1 = min(NB, i0 + per);
  int cnt = 0;
  for (int i = i0; i < i1; ++i) cnt += sel_key(sc, i) >= T;
  int incl = wave_incl_scan(cnt, lane);
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int v = lane < kSelThreads / kWave ? wsum[lane] : 0;
    int vi = wave_incl_scan(v, lane);
    if (lane < kSelThreads / kWave) wsum[lane] = vi - v;
  }
  __syncthreads();
  int pos = wsum[wave] + incl - cnt;
  int32_t* out = a.sel + (long long)row * k;
  if (!a.sorted) {
    for (int i = i0; i < i1; ++i)
      if (sel_key(sc, i) >= T && pos < k) out[pos++] = i;
    return;
  }
  extern __shared__ uint32_t selkeys[];  // [k]
  for (int i = i0; i < i1; ++i) {
    uint32_t key = sel_key(sc, i);
    if (key >= T && pos < k) selkeys[pos++] = key;
  }
  __syncthreads();
  for (int t = tid; t < k; t += kSelThreads) {
    uint32_t kt = selkeys[t];
    int rank = 0;
    for (int q = 0; q < k; ++q) rank += selkeys[q] > kt;
    if (rank < k) out[rank] = (int32_t)(0xFFFFu - (kt & 0xFFFFu));
  }
}

}  // namespace

void launch_route(const RouteArgs& a, hipStream_t s) {
  dim3 g1(a.lat_splits, a.R, a.rows);
  if (a.vec)
    hipLaunchKernelGGL(k_latent_partial<true>, g1, dim3(kLatThreads), 0, s, a);
  else
    hipLaunchKernelGGL(k_latent_partial<false>, g1, dim3(kLatThreads), 0, s, a);
  dim3 g2((a.NB + kScoreThreads - 1) / kScoreThreads, a.rows);
  hipLaunchKernelGGL(k_scores, g2, dim3(kScoreThreads), (size_t)a.R * sizeof(uint16_t), s, a);
  size_t lds = a.sorted ? (size_t)a.k * sizeof(uint32_t) : 0;
  hipLaunchKernelGGL(k_select, dim3(a.rows), dim3(kSelThreads), lds, s, a);
}

}  // namespace nsmlp
