// Hot-block cache maintenance on the device: the reference keeps its VRAM
// hot-block banks up to date on the host every token (promotion of the
// blocks that missed, RT:2809-3018, with the fixed-capacity slot plan of
// RT:2576-2617, and calibration hit counts, RT:2205-2243), with a .cpu()
// round trip per layer.  Here the same decisions are taken by kernels on the
// table's own stream:
//
//   k_cache_plan    one workgroup: the novel blocks of a selection (valid,
//                   not resident, first occurrence, in selection order), the
//                   slot of each (free slots first, then evictions) and the
//                   updated lookup / slot blocks / scores / active count;
//   k_cache_copy    the promoted blocks' gate/up rows and down columns (and
//                   their absmax) from the pinned host copies into their
//                   slots, 16 bytes per lane;
//   k_cache_record  calibration counts: counts[b] += w[r] for every entry b
//                   of row r, one thread per block adding in row order.
//
// The reference plans one novel block at a time: a free slot while there is
// one, else the argmin of the current scores, and the promoted block then
// scores base + (i + 1) 1e-3 with base = max(active scores) + 1.  Every
// promoted score is above every score in the bank before the plan, so the
// argmin never returns a slot promoted by the same plan, and the evicted
// slots are the old slots in ascending (score, slot) order (argmin returns
// the first of equal minima).  k_cache_plan computes that order with a
// bitonic sort of (score, slot) keys.
#include <mutex>

#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kPlanThreads = 1024;
constexpr int kPlanStage = 4096;  // entries staged in LDS for the duplicate checks

// fp32 score -> unsigned key with the same order (+0 and -0 equal, as the
// reference's argmin compares them)
__device__ __forceinline__ uint32_t score_order_key(float v) {
  const uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// k_cache_plan's dynamic LDS: the (score key << 32 | slot) sort keys of the
// old active slots, padded to a power of two (<= kMaxCacheSlots entries).
__global__ void __launch_bounds__(kPlanThreads) k_cache_plan(CacheArgs c) {
  extern __shared__ __attribute__((aligned(16))) unsigned long long key_s[];
  __shared__ int wsum[kPlanThreads / kWave];
  __shared__ float wmax[kPlanThreads / kWave];
  __shared__ __attribute__((aligned(16))) int32_t blk_s[kPlanStage];  // the first entries (duplicate checks)
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int cap = c.capacity;
  int active = *c.active;
  active = active < 0 ? 0 : (active > cap ? cap : active);
  for (int i = tid; i < min(c.n, kPlanStage); i += kPlanThreads) blk_s[i] = c.blocks[i];
  // base score: max over the active slots (fp32 max, exact), plus 1 in fp64
  float mx = -INFINITY;
  for (int s = tid; s < active; s += kPlanThreads) mx = fmaxf(mx, c.slot_score[s]);
  mx = wave_max(mx);
  if (lane == 0) wmax[wave] = mx;
  __syncthreads();
  // novel positions, compacted in selection order (chunks of 1024 entries)
  int carry = 0;
  for (int base = 0; base < c.n; base += kPlanThreads) {
    const int i = base + tid;
    int b = -1;
    bool novel = false;
    if (i < c.n) {
      b = c.blocks[i];
      novel = b >= 0 && b < c.NB && c.lookup[b] < 0;
      if (novel) {  // first occurrence: no earlier equal entry (independent reads, no early exit)
        const int js = min(i, kPlanStage), j4 = js & ~3;
        const int4* b4 = reinterpret_cast<const int4*>(blk_s);
        bool dup = false;
#pragma unroll 8
        for (int j = 0; j < j4; j += 4) {
          const int4 v = b4[j >> 2];
          dup |= (v.x == b) | (v.y == b) | (v.z == b) | (v.w == b);
        }
        for (int j = j4; j < js; ++j) dup |= blk_s[j] == b;
        for (int j = js; j < i; ++j) dup |= c.blocks[j] == b;
        novel = !dup;
      }
    }
    const unsigned long long m = __ballot(novel);
    const int before = __popcll(m & ((1ull << lane) - 1ull));
    if (lane == 0) wsum[wave] = __popcll(m);
    __syncthreads();
    int off = carry;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    int total = 0;
    for (int w = 0; w < kPlanThreads / kWave; ++w) total += wsum[w];
    if (novel) c.novel[off + before] = b;
    if (c.plan_out != nullptr && i < c.n) c.plan_out[i] = novel ? off + before : -1;  // novel index, slot below
    carry += total;
    __syncthreads();
  }
  const int n_novel = carry;
  const int n_free = cap - active;
  const int n_take = c.grow_only ? min(n_novel, n_free) : min(n_novel, cap);
  const int n_evict = max(0, n_take - n_free);
  // eviction order: the old active slots sorted by (score, slot), a bitonic
  // sort of 64-bit keys in LDS over the next power of two (padding sorts last)
  if (n_evict > 0) {
    int np2 = 1;
    while (np2 < active) np2 <<= 1;
    for (int i = tid; i < np2; i += kPlanThreads)
      key_s[i] = i < active ? ((unsigned long long)score_order_key(c.slot_score[i]) << 32) | (unsigned)i : ~0ull;
    __syncthreads();
    for (int kk = 2; kk <= np2; kk <<= 1) {
      for (int jj = kk >> 1; jj > 0; jj >>= 1) {
        for (int i = tid; i < np2; i += kPlanThreads) {
          const int l = i ^ jj;
          if (l > i) {
            const unsigned long long x = key_s[i], y = key_s[l];
            const bool up = (i & kk) == 0;
            if (up ? (x > y) : (x < y)) {
              key_s[i] = y;
              key_s[l] = x;
            }
          }
        }
        __syncthreads();
      }
    }
  }
  double base = 1.0;
  if (active > 0) {
    float m2 = -INFINITY;
    for (int w = 0; w < kPlanThreads / kWave; ++w) m2 = fmaxf(m2, wmax[w]);
    base = (double)m2 + 1.0;
  }
  // apply: slots are distinct, the evicted blocks are resident and the new
  // ones are not, so every write below has one writer
  for (int q = tid; q < n_take; q += kPlanThreads) {
    const int b = c.novel[q];
    const int s = q < n_free ? active + q : (int)(key_s[q - n_free] & 0xFFFFFFFFull);
    const int old = c.slot_block[s];
    if (old >= 0 && old < c.NB && c.lookup[old] == s) c.lookup[old] = -1;
    c.lookup[b] = s;
    c.slot_block[s] = b;
    c.slot_score[s] = (float)(base + (double)(q + 1) * 1e-3);
    c.copy_block[q] = b;
    c.copy_slot[q] = s;
  }
  if (c.plan_out != nullptr) {
    for (int i = tid; i < c.n; i += kPlanThreads) {
      const int q = c.plan_out[i];
      if (q >= 0)
        c.plan_out[i] = q < n_take ? (q < n_free ? active + q : (int)(key_s[q - n_free] & 0xFFFFFFFFull)) : -1;
    }
  }
  if (tid == 0) {
    *c.active = active + min(n_take, n_free);
    *c.n_copy = n_take;
  }
}

// Copy item q's block: part p of the block's bytes (kCopyPart per workgroup)
// over the six arrays of a block, laid out one after the other.
constexpr int kCopyThreads = 256;
constexpr long long kCopyPart = 64 * 1024;

__device__ __forceinline__ void copy16(uint8_t* dst, const uint8_t* src, long long off, long long len, int tid) {
  // len and both bases are multiples of 16
  for (long long i = off + (long long)tid * 16; i < len; i += (long long)kCopyThreads * 16)
    *reinterpret_cast<uint4*>(dst + i) = *reinterpret_cast<const uint4*>(src + i);
}

__global__ void __launch_bounds__(kCopyThreads) k_cache_copy(CacheArgs c) {
  const int q = blockIdx.y;
  if (q >= *c.n_copy) return;
  const int b = c.copy_block[q], s = c.copy_slot[q];
  const long long lo = (long long)blockIdx.x * kCopyPart, hi = lo + kCopyPart;
  long long at = 0;
  for (int a = 0; a < 6; ++a) {
    const long long n = c.bytes[a];
    const long long s0 = lo > at ? lo - at : 0, s1 = hi - at < n ? hi - at : n;
    if (s1 > s0) copy16(c.dst[a] + (long long)s * n, c.src[a] + (long long)b * n, s0, s1, threadIdx.x);
    at += n;
  }
}

// counts[b] += w[r] for each entry b of row r (rows in order, entries in
// order), as a row-by-row index_add_ adds them; w = 1 when absent.
constexpr int kRecThreads = 256;
constexpr int kRecTile = 2048;

__global__ void __launch_bounds__(kRecThreads) k_cache_record(float* counts, int NB, const int32_t* blocks, int rows,
                                                               int k, const float* w) {
  __shared__ int32_t tile[kRecTile];
  const int b = (int)blockIdx.x * kRecThreads + (int)threadIdx.x;
  float acc = b < NB ? counts[b] : 0.0f;
  const long long n = (long long)rows * k;
  for (long long t0 = 0; t0 < n; t0 += kRecTile) {
    const int len = (int)min((long long)kRecTile, n - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < len; i += kRecThreads) tile[i] = blocks[t0 + i];
    __syncthreads();
    if (b < NB) {
      for (int i = 0; i < len; ++i) {
        if (tile[i] == b) {
          const long long e = t0 + i;
          acc += w != nullptr ? w[e / k] : 1.0f;
        }
      }
    }
  }
  if (b < NB) counts[b] = acc;
}

}  // namespace

void launch_cache_promote(const CacheArgs& c, hipStream_t s) {
  static std::once_flag once;
  std::call_once(once, [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_cache_plan),
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)(kMaxCacheSlots * sizeof(unsigned long long)));
  });
  size_t np2 = 1;
  while (np2 < (size_t)c.capacity) np2 <<= 1;
  k_cache_plan<<<dim3(1), dim3(kPlanThreads), np2 * sizeof(unsigned long long), s>>>(c);
  long long total = 0;
  for (int a = 0; a < 6; ++a) total += c.bytes[a];
  const unsigned parts = (unsigned)((total + kCopyPart - 1) / kCopyPart);
  const unsigned items = (unsigned)min(c.n, c.capacity);
  if (items > 0 && parts > 0) k_cache_copy<<<dim3(parts, items), dim3(kCopyThreads), 0, s>>>(c);
}

void launch_cache_record(float* counts, int NB, const int32_t* blocks, int rows, int k, const float* w,
                         hipStream_t s) {
  k_cache_record<<<dim3((unsigned)((NB + kRecThreads - 1) / kRecThreads)), dim3(kRecThreads), 0, s>>>(
      counts, NB, blocks, rows, k, w);
}

}  // namespace nsmlp
