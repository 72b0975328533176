// Learned-basis router of the blockwise-sparse MLP (the reference's
// _compute_sparse_basis_latent + _route_sparse_mlp, RT:4209-4238 and
// RT:4311-4352), as three gfx950 kernels:
//   1. latent          : one workgroup per latent row: exact fp16 dot product
//                        of x with the enc_w row (Exact3), one fp16 rounding;
//                        for fewer than 8 tokens one workgroup per 1/4 of a
//                        row (k_latent_part), the parts added and rounded by
//                        the scores kernel;
//                        from 8 tokens on, the sums on the matrix cores in
//                        fp64 with an error bound (k_latent_mf), exact
//                        sums only where the bound leaves the rounding open.
//   2. scores          : fp16 latent (+ the basis_top_k mask) -> exact score
//                        dots (8 lanes per block) -> fp16, clamp, optional
//                        down_block_norm scaling.
//   3. select          : one workgroup per token; two 8-bit histogram passes
//                        find the k-th largest score T, then an ordered
//                        compaction takes every score above T and the lowest
//                        block ids among the scores equal to T (the order of
//                        the unique key fp16 order key << 16 | ~index), in
//                        ascending block order or, sorted, by rank.
#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kLatThreads = 1024;
constexpr int kScoreThreads = 256;
constexpr int kSelThreads = 1024;

// One workgroup per (latent row, token): the exact dot product over the
// whole hidden size, rounded once to fp16 (RT:4221-4222).
template <bool kVec>
__global__ void __launch_bounds__(kLatThreads) k_latent(RouteArgs a) {
  const int r = blockIdx.x;    // latent row
  const int row = blockIdx.y;  // token
  const int tid = threadIdx.x;
  if (r == 0 && row == 0 && tid == 0 && a.sc_und_n != nullptr) *a.sc_und_n = 0;  // k_scores_mf appends after it
  const uint16_t* __restrict__ x = a.x + (long long)row * a.H;
  const uint16_t* __restrict__ w = a.enc_w + (long long)r * a.H;
  // the bias goes out with the first loads (an unconditional load: x[0]
  // stands in when there is no bias), not after the dot product
  const bool has_b = a.enc_b != nullptr;
  const uint16_t eb = (has_b ? a.enc_b : x)[has_b ? r : 0];
  Exact3 acc = exact_zero();
  if (kVec) {
#pragma unroll 8
    for (int c0 = tid * 8; c0 < a.H; c0 += kLatThreads * 8) {
      const uint4 xv = *reinterpret_cast<const uint4*>(x + c0);
      const uint4 wv = *reinterpret_cast<const uint4*>(w + c0);
      const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
      const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        exact_add(acc, (double)(h2f((uint16_t)(xs[q] & 0xFFFFu)) * h2f((uint16_t)(ws[q] & 0xFFFFu))));
        exact_add(acc, (double)(h2f((uint16_t)(xs[q] >> 16)) * h2f((uint16_t)(ws[q] >> 16))));
      }
    }
  } else {
    for (int c = tid; c < a.H; c += kLatThreads) exact_add(acc, (double)(h2f(x[c]) * h2f(w[c])));
  }
  if (tid == 0 && has_b) exact_add(acc, (double)h2f(eb));
  acc = wave_sum_exact(acc);
  __shared__ double red[kLatThreads / kWave][3];
  const int wave = tid / kWave, lane = tid % kWave;
  if (lane == 0) {
    red[wave][0] = acc.a0;
    red[wave][1] = acc.a1;
    red[wave][2] = acc.a2;
  }
  __syncthreads();
  if (wave == 0) {
    // the 16 wave sums meet in one wave (exact: any order gives the same sum)
    constexpr int kW = kLatThreads / kWave;
    Exact3 t = lane < kW ? Exact3{red[lane][0], red[lane][1], red[lane][2]} : exact_zero();
#pragma unroll
    for (int m = kW / 2; m >= 1; m >>= 1)
      exact_merge(t, Exact3{__shfl_xor(t.a0, m, kWave), __shfl_xor(t.a1, m, kWave), __shfl_xor(t.a2, m, kWave)});
    if (lane == 0) a.lat16[(long long)row * a.R + r] = exact_to_f16(t);
  }
}

// Many tokens (kLatSplitRows or more): the sums on the matrix cores.  A
// workgroup of 4 waves takes a 16-token x 16-latent-row tile and a range of
// the hidden size, a quarter of it per wave.  Per 32 columns lane l (i =
// l % 16, g = l / 16) loads columns 8 g .. 8 g + 7 of token t0 + i's x row
// and of latent row r0 + i's enc_w row and runs 8 steps of
// v_mfma_f64_16x16x4_f64 (every product of two fp16 values is exact in
// fp64; K slot g of step s is column 8 g + s) and the same steps on |x|, |w|
// in fp32 (v_mfma_f32_16x16x4_f32) for the error bound.  The waves' tiles
// meet in LDS in wave order and the workgroup writes range p of the sums.
// k_latent_mfin adds the ranges in order and the bias: a sum of n exact terms
// with any order of fp64 additions lies within n 2^-53 sum|t| of the exact
// sum, so where that interval (with a 2x margin on the fp32 magnitude sum,
// and 2^-49 for the bias add and the interval ends' own rounding) rounds to
// one fp16 value, that value is the exact sum's rounding (the common case).
// The other outputs (an exact sum near an fp16 rounding boundary, large
// cancelling terms, inf or nan) go to a list that k_latent_fix sums again in
// three parts (Exact3, exact for any fp16 inputs), one output per workgroup
// at a time, so the fp16 latent equals k_latent's.
typedef double mf_d4 __attribute__((ext_vector_type(4)));
typedef float mf_f4 __attribute__((ext_vector_type(4)));
constexpr int kMfThreads = 256;
constexpr int kFixThreads = 1024, kFixGroups = 64;

__global__ void __launch_bounds__(kMfThreads) k_latent_mf(RouteArgs a) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int RT = (a.R + 15) / 16;
  const int tile = (int)blockIdx.x, p = (int)blockIdx.y, P = (int)gridDim.y;
  const int r0 = (tile % RT) * 16, t0 = (tile / RT) * 16;
  if (tile == 0 && p == 0 && tid == 0) {
    *a.lat_und_n = 0;  // k_latent_mfin appends after this kernel
    if (a.sc_und_n != nullptr) *a.sc_und_n = 0;  // and k_scores_mf after that
  }
  const int i = lane & 15, g = lane >> 4;
  const int nt = min(16, a.rows - t0), nr = min(16, a.R - r0);
  // descriptors over the tile's rows only (every offset below fits 32 bits)
  const rsrc_t rx = make_rsrc(a.x + (long long)t0 * a.H, nt * a.H * 2);
  const rsrc_t rw = make_rsrc(a.enc_w + (long long)r0 * a.H, nr * a.H * 2);
  const uint32_t xo = i < nt ? ((uint32_t)i * (uint32_t)a.H + 8u * (uint32_t)g) * 2u : kOffNone;
  const uint32_t wo = i < nr ? ((uint32_t)i * (uint32_t)a.H + 8u * (uint32_t)g) * 2u : kOffNone;
  const int per = (a.H + 4 * P * 32 - 1) / (4 * P * 32) * 32;  // columns per wave
  const int k0 = (4 * p + wave) * per, k1 = min(a.H, k0 + per);
  // two fp64 accumulators (even and odd steps): two independent chains of
  // dependent MFMAs; added at the end (one more rounding per output)
  mf_d4 acc = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
  mf_f4 mag = {0.0f, 0.0f, 0.0f, 0.0f};
  // groups of 4 chunks of 32 columns, double-buffered in registers: a
  // group's loads are issued while the previous group is multiplied
  // (columns past the wave's range or H load zeros: H % 8 == 0, so a lane's
  // 8 columns are all inside or all past it)
  auto load = [&](uint4 (&xv)[4], uint4 (&wv)[4], int c0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = c0 + 32 * u;
      const bool in = c < k1 && c + 8 * g < a.H;
      xv[u] = buf_ld16c(rx, in ? xo : kOffNone, (uint32_t)c * 2u);
      wv[u] = buf_ld16c(rw, in ? wo : kOffNone, (uint32_t)c * 2u);
    }
  };
  auto mul = [&](const uint4 (&xv)[4], const uint4 (&wv)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t xs[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
      const uint32_t ws[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) {
        const float xf = h2f((uint16_t)(xs[s2 >> 1] >> (16 * (s2 & 1))));
        const float wf = h2f((uint16_t)(ws[s2 >> 1] >> (16 * (s2 & 1))));
        if (s2 & 1)
          acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)xf, (double)wf, acc1, 0, 0, 0);
        else
          acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)xf, (double)wf, acc, 0, 0, 0);
        mag = __builtin_amdgcn_mfma_f32_16x16x4f32(fabsf(xf), fabsf(wf), mag, 0, 0, 0);
      }
    }
  };
  uint4 xa[4], wa[4], xb[4], wb[4];
  load(xa, wa, k0);
  for (int c = k0; c < k1; c += 256) {
    load(xb, wb, c + 128);
    mul(xa, wa);
    load(xa, wa, c + 256);
    if (c + 128 < k1) mul(xb, wb);  // uniform
  }
  mfma_drain();
  acc += acc1;
  // C layouts (measured): f64 lane L element q = (token 4 q + L / 16, row
  // L % 16); f32 lane L element q = (token 4 (L / 16) + q, row L % 16)
  __shared__ double r64[4][256];
  __shared__ float r32[4][256];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    r64[wave][(4 * q + g) * 16 + i] = acc[q];
    r32[wave][(4 * g + q) * 16 + i] = mag[q];
  }
  __syncthreads();
  const int ot = tid >> 4, orr = tid & 15;  // thread tid: token t0 + ot, latent row r0 + orr
  if (ot < nt && orr < nr) {
    const double sv = ((r64[0][tid] + r64[1][tid]) + r64[2][tid]) + r64[3][tid];
    const float bv = ((r32[0][tid] + r32[1][tid]) + r32[2][tid]) + r32[3][tid];
    const long long o = ((long long)p * a.rows + (t0 + ot)) * a.R + (r0 + orr);
    a.lat_p64[o] = sv;
    a.lat_p32[o] = bv;
  }
}

// One thread per output: the ranges added in order, the bound, the write or
// the list of undecided outputs.
__global__ void __launch_bounds__(256) k_latent_mfin(RouteArgs a) {
  const long long n = (long long)a.rows * a.R;
  const long long o = (long long)blockIdx.x * 256 + threadIdx.x;
  if (o >= n) return;
  const int r = (int)(o % a.R);
  double sum1 = 0.0;
  float b = 0.0f;
  for (int p = 0; p < a.lat_nparts; ++p) {
    sum1 += a.lat_p64[p * n + o];
    b += a.lat_p32[p * n + o];
  }
  const double bias = a.enc_b != nullptr ? (double)h2f(a.enc_b[r]) : 0.0;
  const double sb = sum1 + bias;
  // (H + 64) 2^-53 (2 b): the sums' roundings (at most one per term, the
  // ranges' and the waves' additions; 2 b > sum|t|); 2^-49 (|sb| + |bias|):
  // the bias add and the interval ends' own rounding
  const double B = (double)(a.H + 64) * 1.1102230246251565e-16 * (2.0 * (double)b) +
                   1.7763568394002505e-15 * (fabs(sb) + fabs(bias));
  const uint16_t lo = exact_to_f16(Exact3{sb - B, 0.0, 0.0});
  const uint16_t hi = exact_to_f16(Exact3{sb + B, 0.0, 0.0});
  const bool ok = b < 3.0e38f && fabs(sb) < 1.0e300 && lo == hi;  // false for inf and nan
  if (ok) {
    a.lat16[o] = lo;
  } else {
    const int slot = atomicAdd(a.lat_und_n, 1);
    a.lat_und[slot] = (int)o;
  }
}

// The undecided outputs, exactly: workgroup w takes list entries w, w + G, ...
__global__ void __launch_bounds__(kFixThreads) k_latent_fix(RouteArgs a) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  __shared__ double xred[kFixThreads / kWave][3];
  const int cnt = *a.lat_und_n;
  for (int e = (int)blockIdx.x; e < cnt; e += (int)gridDim.x) {
    const int o = a.lat_und[e];
    const int t = o / a.R, r = o % a.R;
    const uint16_t* __restrict__ ux = a.x + (long long)t * a.H;
    const uint16_t* __restrict__ uw = a.enc_w + (long long)r * a.H;
    Exact3 ex = exact_zero();
    for (int c = tid; c < a.H; c += kFixThreads) exact_add(ex, (double)(h2f(ux[c]) * h2f(uw[c])));
    ex = wave_sum_exact(ex);
    if (lane == 0) {
      xred[wave][0] = ex.a0;
      xred[wave][1] = ex.a1;
      xred[wave][2] = ex.a2;
    }
    __syncthreads();
    if (tid == 0) {
      Exact3 sum = exact_zero();
#pragma unroll
      for (int v = 0; v < kFixThreads / kWave; ++v) exact_merge(sum, Exact3{xred[v][0], xred[v][1], xred[v][2]});
      if (a.enc_b != nullptr) exact_add(sum, (double)h2f(a.enc_b[r]));
      a.lat16[o] = exact_to_f16(sum);
    }
    __syncthreads();
  }
}

// Fewer than kLatSplitRows rows: one workgroup per (latent row, column range,
// token), kLatParts ranges per row, so a decode token's R rows fill the chip
// (R kLatParts workgroups).  Each writes the exact partial sum of its range
// (Exact3 parts; the bias goes into range 0); k_scores adds the parts (exact
// in any grouping) and rounds once, so the fp16 latent equals k_latent's.
constexpr int kLpThreads = 256;

template <bool kVec>
__global__ void __launch_bounds__(kLpThreads) k_latent_part(RouteArgs a) {
  kernarg_warm<sizeof(RouteArgs)>();
  const int r = blockIdx.x, p = blockIdx.y, row = blockIdx.z;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  if (a.clear_words != nullptr && (r | p | row) == 0 && tid < kClearWords) a.clear_words[tid] = 0;
  const uint16_t* __restrict__ x = a.x + (long long)row * a.H;
  const uint16_t* __restrict__ w = a.enc_w + (long long)r * a.H;
  const int span = (a.H + kLatParts * 8 - 1) / (kLatParts * 8) * 8;  // columns per range, a multiple of 8
  const int c_lo = p * span, c_hi = min(a.H, c_lo + span);
  // the bias goes out with the first loads (an unconditional load: x[0]
  // stands in when there is no bias)
  const bool has_b = a.enc_b != nullptr;
  const uint16_t eb = (has_b ? a.enc_b : x)[has_b ? r : 0];
  Exact3 acc = exact_zero();
  if (kVec) {
#pragma unroll 2
    for (int c0 = c_lo + tid * 8; c0 < c_hi; c0 += kLpThreads * 8) {
      const uint4 xv = *reinterpret_cast<const uint4*>(x + c0);
      const uint4 wv = *reinterpret_cast<const uint4*>(w + c0);
      const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
      const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        exact_add(acc, (double)(h2f((uint16_t)(xs[q] & 0xFFFFu)) * h2f((uint16_t)(ws[q] & 0xFFFFu))));
        exact_add(acc, (double)(h2f((uint16_t)(xs[q] >> 16)) * h2f((uint16_t)(ws[q] >> 16))));
      }
    }
  } else {
    for (int c = c_lo + tid; c < c_hi; c += kLpThreads) exact_add(acc, (double)(h2f(x[c]) * h2f(w[c])));
  }
  if (tid == 0 && has_b && p == 0) exact_add(acc, (double)h2f(eb));
  acc = wave_sum_exact(acc);
  __shared__ double red[kLpThreads / kWave][3];
  if (lane == 0) {
    red[wave][0] = acc.a0;
    red[wave][1] = acc.a1;
    red[wave][2] = acc.a2;
  }
  __syncthreads();
  if (tid < 3) {  // part tid of the Exact3 sum: the wave sums' parts add exactly
    double v = 0.0;
#pragma unroll
    for (int v4 = 0; v4 < kLpThreads / kWave; ++v4) v += red[v4][tid];
    a.lat_part[(((long long)row * a.R + r) * kLatParts + p) * 3 + tid] = v;
  }
}

void launch_latent(const RouteArgs& a, hipStream_t s) {
  if (a.vec && a.lat_p64 != nullptr) {
    const int tiles = ((a.rows + 15) / 16) * ((a.R + 15) / 16);
    hipLaunchKernelGGL(k_latent_mf, dim3(tiles, a.lat_nparts), dim3(kMfThreads), 0, s, a);
    const long long n = (long long)a.rows * a.R;
    hipLaunchKernelGGL(k_latent_mfin, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
    hipLaunchKernelGGL(k_latent_fix, dim3(kFixGroups), dim3(kFixThreads), 0, s, a);
    return;
  }
  if (a.lat_part != nullptr) {
    const dim3 g(a.R, kLatParts, a.rows);
    if (a.vec)
      hipLaunchKernelGGL(k_latent_part<true>, g, dim3(kLpThreads), 0, s, a);
    else
      hipLaunchKernelGGL(k_latent_part<false>, g, dim3(kLpThreads), 0, s, a);
    return;
  }
  const dim3 g1(a.R, a.rows);
  if (a.vec)
    hipLaunchKernelGGL(k_latent<true>, g1, dim3(kLatThreads), 0, s, a);
  else
    hipLaunchKernelGGL(k_latent<false>, g1, dim3(kLatThreads), 0, s, a);
}

// Scores: 8 lanes per block (kScoreLanes), each summing every 8th basis
// term exactly; the lane partials are merged exactly (plain fp64 adds of
// Exact3 parts) and rounded once.
constexpr int kScoreLanes = 8;
constexpr int kScoresPerWg = kScoreThreads / kScoreLanes;

// From 8 tokens on (and R <= 128), a workgroup scores 8 tokens with the same
// prefetched score_w terms (score_w is then read once per 8 tokens); the
// basis_top_k mask keeps at most 4 entries per thread (8 R <= 4 * 256).
constexpr int kScTok = 8;

__host__ __device__ inline int scores_tokens_per_wg(int rows, int R) {
  return rows >= kScTok && R * kScTok <= 4 * kScoreThreads ? kScTok : 1;
}

// Basis term r of prefetch slot i of a lane (lane `part` of a block's 8).
// kVecW: 16-byte score_w rows; the lane takes terms 8 part .. 8 part + 7 of
// each group of 64 (one 16-byte load per group).  Otherwise every 8th term.
// Either way the 8 lanes cover terms 0 .. 8 kPre - 1 once.
template <bool kVecW>
__device__ __forceinline__ int score_term(int part, int i) {
  return kVecW ? (i / 8) * 64 + part * 8 + (i % 8) : part + i * kScoreLanes;
}

template <bool kVecW>
__global__ void __launch_bounds__(kScoreThreads) k_scores(RouteArgs a) {
  kernarg_warm<sizeof(RouteArgs)>();
  const int tpw = scores_tokens_per_wg(a.rows, a.R);  // tokens of this workgroup
  const int row0 = (int)blockIdx.y * tpw;
  const int nrow = min(tpw, a.rows - row0);
  const int tid = threadIdx.x;
  extern __shared__ uint16_t lat16[];  // [tpw][R]
  // score_w terms of this lane (loaded before waiting for the latent)
  const int j = blockIdx.x * kScoresPerWg + tid / kScoreLanes;
  const int part = tid % kScoreLanes;
  const int jj = j < a.NB ? j : a.NB - 1;  // all lanes take part in the merge
  const uint16_t* __restrict__ w = a.score_w + (long long)jj * a.R;
  // bias and down_block_norm go out with the first loads (unconditional:
  // score_w stands in for an absent array), not after the dot products
  const bool has_b = !a.legacy_abs && a.score_b != nullptr, has_n = a.dbn != nullptr;
  const uint16_t sb = (has_b ? a.score_b : a.score_w)[has_b ? jj : 0];
  const uint16_t sn = (has_n ? a.dbn : a.score_w)[has_n ? jj : 0];
  // Every load is unconditional (clamped offsets, the value zeroed after the
  // load): a load under a condition would be waited for on its own.
  constexpr int kPre = 16;  // prefetched terms per lane (R <= 128)
  uint16_t wv[kPre];
  if constexpr (kVecW) {
#pragma unroll
    for (int g = 0; g < kPre / 8; ++g) {
      const int r0 = g * 64 + part * 8;  // R % 8 == 0: all 8 terms or none
      const uint4 t = *reinterpret_cast<const uint4*>(w + (r0 < a.R ? r0 : 0));
      const uint32_t tw[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int m = 0; m < 8; ++m) wv[8 * g + m] = r0 < a.R ? (uint16_t)(tw[m / 2] >> (16 * (m % 2))) : (uint16_t)0;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int r = part + i * kScoreLanes;
      const uint16_t t = w[r < a.R ? r : 0];
      wv[i] = r < a.R ? t : (uint16_t)0;
    }
  }
  if (a.lat_part != nullptr) {
    // the latent from its range parts: add them (exact) and round once;
    // workgroup 0 also keeps the fp16 latent in the workspace
    for (int i = tid; i < nrow * a.R; i += kScoreThreads) {
      const double* pp = a.lat_part + ((long long)row0 * a.R + i) * (kLatParts * 3);
      Exact3 e = exact_zero();
#pragma unroll
      for (int q = 0; q < kLatParts; ++q) exact_merge(e, Exact3{pp[3 * q], pp[3 * q + 1], pp[3 * q + 2]});
      const uint16_t v = exact_to_f16(e);
      lat16[i] = v;
      if (blockIdx.x == 0) a.lat16[(long long)row0 * a.R + i] = v;
    }
  } else {
    for (int i = tid; i < nrow * a.R; i += kScoreThreads) lat16[i] = a.lat16[(long long)row0 * a.R + i];
  }
  __syncthreads();
  // basis_top_k mask over |latent| per token (RT:4233-4238); ties keep the
  // lower index
  int btk = a.basis_top_k < 1 ? 1 : (a.basis_top_k > a.R ? a.R : a.basis_top_k);
  if (btk < a.R) {
    uint16_t keep_val[4];  // nrow * R <= 4 * kScoreThreads entries
    int nmine = 0;
    for (int i = tid; i < nrow * a.R; i += kScoreThreads) {
      const uint16_t* lt = lat16 + (i / a.R) * a.R;
      const int r = i % a.R;
      uint32_t kr = f16_order_key((uint16_t)(lt[r] & 0x7FFFu));
      int rank = 0;
      for (int q = 0; q < a.R; ++q) {
        uint32_t kq = f16_order_key((uint16_t)(lt[q] & 0x7FFFu));
        rank += (kq > kr) || (kq == kr && q < r);
      }
      keep_val[nmine++] = rank < btk ? lt[r] : (uint16_t)(lt[r] & 0x8000u);
    }
    __syncthreads();
    nmine = 0;
    for (int i = tid; i < nrow * a.R; i += kScoreThreads) lat16[i] = keep_val[nmine++];
    __syncthreads();
  }
  if (blockIdx.x == 0 && a.latent_out != nullptr)
    for (int i = tid; i < nrow * a.R; i += kScoreThreads) a.latent_out[(long long)row0 * a.R + i] = lat16[i];
  const uint16_t amask = a.legacy_abs ? 0x7FFFu : 0xFFFFu;
  for (int tt = 0; tt < nrow; ++tt) {
    const uint16_t* lt = lat16 + tt * a.R;
    Exact3 acc = exact_zero();
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int r = score_term<kVecW>(part, i);
      if (r < a.R) exact_add(acc, (double)(h2f((uint16_t)(lt[r] & amask)) * h2f(wv[i])));
    }
    for (int r = part + kPre * kScoreLanes; r < a.R; r += kScoreLanes) {
      const float p = h2f((uint16_t)(lt[r] & amask)) * h2f(w[r]);
      exact_add(acc, (double)p);
    }
#pragma unroll
    for (int m = 1; m < kScoreLanes; m <<= 1)
      exact_merge(acc, Exact3{__shfl_xor(acc.a0, m, kWave), __shfl_xor(acc.a1, m, kWave), __shfl_xor(acc.a2, m, kWave)});
    if (part == 0 && j < a.NB) {
      if (has_b) exact_add(acc, (double)h2f(sb));
      uint16_t sc = exact_to_f16(acc);
      if (!a.legacy_abs && (sc & 0x8000u)) sc = 0;  // clamp_min(0) (RT:4331)
      if (has_n) sc = f2h(h2f(sc) * h2f(sn));  // fp16 x fp16 is exact in fp32
      const long long o = (long long)(row0 + tt) * a.NB + j;
      a.scores[o] = sc;
      if (a.scores_out != nullptr) a.scores_out[o] = sc;
    }
  }
}

// From kLatSplitRows tokens on (16-byte score_w rows), the scores on the
// matrix cores, as the latent's first pass: with a basis_top_k mask (or a
// latent_out to write) k_scores_prep first writes the latent as scored;
// k_scores_mf sums each 16-token x 16-block tile in fp64
// (v_mfma_f64_16x16x4_f64, every term exact) with the terms' magnitudes in
// fp32 beside it, and where the error interval of sum + bias rounds to one
// fp16 value (the bound of k_latent_mfin, over R terms) that value is the
// score; the others (one in 425984 at the 405B shape and 256 tokens) go to a
// list that k_scores_fix sums exactly (Exact3), one output per wave.  Either
// way the score equals k_scores' bit for bit.  The latent kernels clear the
// list's count.
constexpr int kSmThreads = 256;  // 4 waves, one tile each
constexpr int kSfThreads = 256, kSfGroups = 16;

__device__ __forceinline__ void score_store(const RouteArgs& a, long long o, int j, uint16_t sc) {
  if (!a.legacy_abs && (sc & 0x8000u)) sc = 0;               // clamp_min(0) (RT:4331)
  if (a.dbn != nullptr) sc = f2h(h2f(sc) * h2f(a.dbn[j]));  // fp16 x fp16 is exact in fp32
  a.scores[o] = sc;
  if (a.scores_out != nullptr) a.scores_out[o] = sc;
}

// One wave per token: the basis_top_k mask over |latent| (ties keep the lower
// index, as k_scores), latent_out, and the latent as scored.
__global__ void __launch_bounds__(kWave) k_scores_prep(RouteArgs a) {
  const int row = (int)blockIdx.x, lane = threadIdx.x;
  const uint16_t* lt = a.lat16 + (long long)row * a.R;
  const int btk = a.basis_top_k < 1 ? 1 : (a.basis_top_k > a.R ? a.R : a.basis_top_k);
  for (int r = lane; r < a.R; r += kWave) {
    uint16_t v = lt[r];
    if (btk < a.R) {
      const uint32_t kr = f16_order_key((uint16_t)(v & 0x7FFFu));
      int rank = 0;
      for (int q = 0; q < a.R; ++q) {
        const uint32_t kq = f16_order_key((uint16_t)(lt[q] & 0x7FFFu));
        rank += (kq > kr) || (kq == kr && q < r);
      }
      if (rank >= btk) v = (uint16_t)(v & 0x8000u);
    }
    if (a.latent_out != nullptr) a.latent_out[(long long)row * a.R + r] = v;
    a.lat_m[(long long)row * a.R + r] = v;
  }
}

// Wave w of workgroup g takes tile 4 g + w (16 tokens x 16 blocks), reading
// the latent as scored from a.lat_m (the prepared copy, or the latent itself
// when nothing is masked; |latent| is taken here for legacy_abs).  Lane l
// (i = l % 16, g4 = l / 16) holds, per 64 basis terms, terms 16 g4 .. + 15 of
// token t0 + i's scored latent and of block b0 + i's score_w row (two
// 16-byte loads each; R % 8 == 0, so a load's 8 terms are all inside R or all
// past it); K slot g4 of MFMA step s is term 16 g4 + s.
__global__ void __launch_bounds__(kSmThreads) k_scores_mf(RouteArgs a) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int BT = (a.NB + 15) / 16, TT = (a.rows + 15) / 16;
  const int tile = 4 * (int)blockIdx.x + wave;
  if (tile >= BT * TT) return;  // whole waves; no barrier below
  const int t0 = (tile / BT) * 16, b0 = (tile % BT) * 16;
  const int i = lane & 15, g4 = lane >> 4;
  const int nt = min(16, a.rows - t0), nb = min(16, a.NB - b0);
  const rsrc_t rx = make_rsrc(a.lat_m + (long long)t0 * a.R, nt * a.R * 2);
  const rsrc_t rw = make_rsrc(a.score_w + (long long)b0 * a.R, nb * a.R * 2);
  const uint32_t xo = i < nt ? (uint32_t)(i * a.R) * 2u : kOffNone;
  const uint32_t wo = i < nb ? (uint32_t)(i * a.R) * 2u : kOffNone;
  typedef double d4 __attribute__((ext_vector_type(4)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  d4 acc = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
  f4 mag = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < a.R; c0 += 64) {
    uint4 xv[2], wv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = c0 + 16 * g4 + 8 * h;
      const bool in = c < a.R;
      xv[h] = buf_ld16c(rx, in ? xo : kOffNone, (uint32_t)c * 2u);
      wv[h] = buf_ld16c(rw, in ? wo : kOffNone, (uint32_t)c * 2u);
      if (a.legacy_abs) xv[h] = make_uint4(xv[h].x & 0x7FFF7FFFu, xv[h].y & 0x7FFF7FFFu, xv[h].z & 0x7FFF7FFFu,
                                           xv[h].w & 0x7FFF7FFFu);
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const uint32_t xw = s < 8 ? (&xv[0].x)[s >> 1] : (&xv[1].x)[(s - 8) >> 1];
      const uint32_t ww = s < 8 ? (&wv[0].x)[s >> 1] : (&wv[1].x)[(s - 8) >> 1];
      const float xf = h2f((uint16_t)(xw >> (16 * (s & 1))));
      const float wf = h2f((uint16_t)(ww >> (16 * (s & 1))));
      if (s & 1)
        acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64((double)xf, (double)wf, acc1, 0, 0, 0);
      else
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)xf, (double)wf, acc, 0, 0, 0);
      mag = __builtin_amdgcn_mfma_f32_16x16x4f32(fabsf(xf), fabsf(wf), mag, 0, 0, 0);
    }
  }
  mfma_drain();
  acc += acc1;
  // C layouts (measured): f64 lane L element q = (token 4 q + L / 16, block
  // L % 16); f32 lane L element q = (token 4 (L / 16) + q, block L % 16): the
  // magnitudes go through LDS into the f64 layout
  __shared__ float mg[4][256];
#pragma unroll
  for (int q = 0; q < 4; ++q) mg[wave][(4 * g4 + q) * 16 + i] = mag[q];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  const bool has_b = !a.legacy_abs && a.score_b != nullptr;
  const int j = b0 + i;
  const double bias = has_b && i < nb ? (double)h2f(a.score_b[j]) : 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int tt = 4 * q + g4;
    if (tt < nt && i < nb) {
      const float b = mg[wave][tt * 16 + i];
      const double sb = acc[q] + bias;
      // (R + 64) 2^-53 (2 b): the sums' roundings (at most one per term, the
      // two chains' addition; 2 b > sum|t|); 2^-49 (|sb| + |bias|): the bias
      // add and the interval ends' own rounding
      const double B = (double)(a.R + 64) * 1.1102230246251565e-16 * (2.0 * (double)b) +
                       1.7763568394002505e-15 * (fabs(sb) + fabs(bias));
      const uint16_t lo = exact_to_f16(Exact3{sb - B, 0.0, 0.0});
      const uint16_t hi = exact_to_f16(Exact3{sb + B, 0.0, 0.0});
      const long long o = (long long)(t0 + tt) * a.NB + j;
      if (b < 3.0e38f && fabs(sb) < 1.0e300 && lo == hi) {  // false for inf and nan
        score_store(a, o, j, lo);
      } else {
        const int slot = atomicAdd(a.sc_und_n, 1);
        a.sc_und[slot] = (int)o;
      }
    }
  }
}

// The undecided scores, exactly: wave g of the grid takes list entries g,
// g + G, ...; lane l sums terms l, l + 64, ... of its entry (Exact3 parts add
// exactly across lanes).
__global__ void __launch_bounds__(kSfThreads) k_scores_fix(RouteArgs a) {
  const int cnt = *a.sc_und_n;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = (int)(blockIdx.x * (kSfThreads / kWave) + threadIdx.x / kWave), nw = (int)gridDim.x * (kSfThreads / kWave);
  const bool has_b = !a.legacy_abs && a.score_b != nullptr;
  const uint16_t amask = a.legacy_abs ? 0x7FFFu : 0xFFFFu;
  for (int e = wv; e < cnt; e += nw) {
    const int o = a.sc_und[e];
    const int t = o / a.NB, j = o % a.NB;
    const uint16_t* lt = a.lat_m + (long long)t * a.R;
    const uint16_t* w = a.score_w + (long long)j * a.R;
    Exact3 acc = exact_zero();
    for (int r = lane; r < a.R; r += kWave) exact_add(acc, (double)(h2f((uint16_t)(lt[r] & amask)) * h2f(w[r])));
    acc = wave_sum_exact(acc);
    if (lane == 0) {
      if (has_b) exact_add(acc, (double)h2f(a.score_b[j]));
      score_store(a, o, j, exact_to_f16(acc));
    }
  }
}

void launch_scores(const RouteArgs& a, hipStream_t s) {
  if (a.sc_und != nullptr && a.svec) {
    RouteArgs b = a;
    if (a.basis_top_k < a.R || a.latent_out != nullptr)
      hipLaunchKernelGGL(k_scores_prep, dim3(a.rows), dim3(kWave), 0, s, a);
    else
      b.lat_m = a.lat16;  // nothing masked: the scores read the latent itself
    const long long tiles = (long long)((a.NB + 15) / 16) * ((a.rows + 15) / 16);
    hipLaunchKernelGGL(k_scores_mf, dim3((unsigned)((tiles + 3) / 4)), dim3(kSmThreads), 0, s, b);
    hipLaunchKernelGGL(k_scores_fix, dim3(kSfGroups), dim3(kSfThreads), 0, s, b);
    return;
  }
  const int tpw = scores_tokens_per_wg(a.rows, a.R);
  const dim3 g((a.NB + kScoresPerWg - 1) / kScoresPerWg, (a.rows + tpw - 1) / tpw);
  const size_t lds = (size_t)a.R * tpw * sizeof(uint16_t);
  if (a.svec)
    hipLaunchKernelGGL(k_scores<true>, g, dim3(kScoreThreads), lds, s, a);
  else
    hipLaunchKernelGGL(k_scores<false>, g, dim3(kScoreThreads), lds, s, a);
}

// Top-k of one token's scores (keys: fp16 order key, ties to the lower block
// index).  Each thread holds KPT consecutive keys in registers.  Two 8-bit
// histogram passes find the threshold score T and how many entries equal to
// T are taken (`need`); an ordered compaction then takes every score above T
// and the first `need` scores equal to T in block order.  Output: ascending
// block ids, or (sorted) score descending with ties by ascending id.
template <int KPT>
__global__ void __launch_bounds__(kSelThreads) k_select(RouteArgs a) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* sc = a.scores + (long long)row * a.NB;
  const int NB = a.NB;
  const int k = a.k;
  __shared__ TopkLds L;
  const int i0 = tid * KPT;
  uint32_t key[KPT];
#pragma unroll
  for (int m = 0; m < KPT; ++m) key[m] = i0 + m < NB ? f16_order_key(sc[i0 + m]) : 0u;
  topk_clear<kSelThreads>(L);
  lds_barrier();
  uint32_t T;
  unsigned need, gt, eq;
  topk_threshold<kSelThreads, KPT>(key, i0, NB, k, L, T, need, gt, eq);
  int32_t* out = a.sel + (long long)row * k;
  extern __shared__ uint32_t selkeys[];  // [k] (sorted output)
#pragma unroll
  for (int m = 0; m < KPT; ++m) {
    const int i = i0 + m;
    if (i >= NB) continue;
    const int pos = topk_position(key[m], T, need, gt, eq);
    gt += key[m] > T;
    eq += key[m] == T;
    if (pos < 0 || pos >= k) continue;
    if (!a.sorted)
      out[pos] = i;
    else
      selkeys[pos] = (key[m] << 16) | (0xFFFFu - (uint32_t)i);
  }
  if (!a.sorted) return;
  __syncthreads();
  for (int t = tid; t < k; t += kSelThreads) {
    const uint32_t kt = selkeys[t];
    int rank = 0;
    for (int q = 0; q < k; ++q) rank += selkeys[q] > kt;
    if (rank < k) out[rank] = (int32_t)(0xFFFFu - (kt & 0xFFFFu));
  }
}

}  // namespace

void launch_route_scores(const RouteArgs& a, hipStream_t s) {
  launch_latent(a, s);
  launch_scores(a, s);
}

void launch_route(const RouteArgs& a, hipStream_t s) {
  launch_latent(a, s);
  launch_scores(a, s);
  const size_t lds = a.sorted ? (size_t)a.k * sizeof(uint32_t) : 0;
  const int kpt = (a.NB + kSelThreads - 1) / kSelThreads;  // NB <= 65535: kpt <= 64
  const dim3 g3(a.rows), b3(kSelThreads);
  if (kpt <= 2)
    hipLaunchKernelGGL(k_select<2>, g3, b3, lds, s, a);
  else if (kpt <= 8)
    hipLaunchKernelGGL(k_select<8>, g3, b3, lds, s, a);
  else
    hipLaunchKernelGGL(k_select<64>, g3, b3, lds, s, a);
}

}  // namespace nsmlp
