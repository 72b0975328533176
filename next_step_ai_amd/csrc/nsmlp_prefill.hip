// Chunked prefill of the sparse MLP: M tokens, each with its own top-k block
// set, over the union of the selected blocks (RT:4868-4901, RT:5453: every
// token's gate/up are masked to its own blocks, so a block contributes to a
// token only if the token selected it).  Grouped per block on MFMA
// (v_mfma_f32_16x16x32_f16, fp32 accumulation):
//
//   k_pf_mark / k_pf_scan / k_pf_list  token lists per block (CSR, ascending
//               token ids), from a [NB][M/32] membership bitmap and counts;
//   k_pf_gu     one workgroup per block: gate and up of the block's tokens
//               as a staged GEMM, the token rows gathered as the MFMA A
//               operand and the NF4 rows decoded to fp16(code * absmax) as the
//               B operand (the reference fallback's rounding of the weights,
//               RT:5439-5447); act = fp16(silu(gate) * up) per (block, token);
//   k_pf_down   one workgroup per 64 output rows and 128-token group: for
//               every block, act [tokens x 32] times the block's down columns
//               [32 x 64 rows] as fp16 codes, the absmax applied to the MFMA
//               result in fp32; each tile is added into the group's [128][64]
//               LDS accumulator at its tokens' rows as int64 fixed point
//               (2^-31), so the sum does not depend on the order the waves
//               add in; the result is rounded once to fp16.
//
// MFMA lane layout (16x16x32 f16, measured): A[i][k] and B[k][j] in lane l
// hold i (or j) = l % 16, k = 8 (l / 16) + 0..7; C[i][j] in lane l holds
// j = l % 16, i = 4 (l / 16) + r, r = 0..3.  The K order inside a 128-column
// chunk is permuted (lane group g takes columns 32 g .. 32 g + 31 over the
// chunk's four MFMA steps) so that each lane reads contiguous bytes; A and B
// use the same permutation, which leaves the dot products unchanged.
#include <cstring>
#include <mutex>
#include <type_traits>

#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kPfThreads = 512;
constexpr int kPfWaves = kPfThreads / kWave;
constexpr int kTokGroup = 128;   // tokens per down workgroup
constexpr double kFixInv = 1.0 / 2147483648.0;  // down accumulator: int64 units of 2^-31

// Code-pair table: entry e (a packed NF4 byte) holds fp16 code[e >> 4] in
// the low half (the even element) and fp16 code[e & 15] in the high half.
__device__ __forceinline__ void cpair_fill(uint32_t* cpair, const float* code, int tid, int nthr) {
  for (int e = tid; e < 256; e += nthr)
    cpair[e] = (uint32_t)f2h(code[e >> 4]) | ((uint32_t)f2h(code[e & 15]) << 16);
}

// 16 consecutive NF4 elements of two rows (words w0, w1: 4 bytes each, even
// element in the high nibble) as fp16(code * absmax), the reference
// fallback's rounding of the weights.  All eight pair lookups go out before
// any is used.
template <int kCopies>
__device__ __forceinline__ void deq8x2(uint32_t w0, float am0, uint32_t w1, float am1, const float2* cp,
                                       half8_t& h0, half8_t& h1) {
  float2 p[8];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    p[m] = cp[((w0 >> (8 * m)) & 0xFFu) * kCopies];
    p[4 + m] = cp[((w1 >> (8 * m)) & 0xFFu) * kCopies];
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    h0[2 * m] = (_Float16)(p[m].x * am0);
    h0[2 * m + 1] = (_Float16)(p[m].y * am0);
    h1[2 * m] = (_Float16)(p[4 + m].x * am1);
    h1[2 * m + 1] = (_Float16)(p[4 + m].y * am1);
  }
}

// 8 consecutive NF4 elements (4 bytes, even element in the high nibble) as
// their fp16 code values; the absmax (constant over the 32 columns of an
// MFMA step for a given weight row) scales the MFMA result instead.
__device__ __forceinline__ half8_t codes8(uint32_t word, const uint32_t* cpair) {
  const uint4 v = make_uint4(cpair[word & 0xFFu], cpair[(word >> 8) & 0xFFu], cpair[(word >> 16) & 0xFFu],
                             cpair[word >> 24]);
  return __builtin_bit_cast(half8_t, v);
}


// v * 2^31 truncated toward zero (|v| < 2^23), in fp32/int32 steps: hi =
// trunc(v * 2^8) carries the bits above 2^-8, the remainder v - hi * 2^-8 is
// exact and |rem| < 2^-8, so trunc(rem * 2^31) fits 23 bits.
__device__ __forceinline__ long long to_fix31(float v) {
  const int hi = (int)(v * 256.0f);
  const float rem = __builtin_fmaf((float)hi, -0.00390625f, v);
  const int lo = (int)(rem * 2147483648.0f);
  return ((long long)hi << 23) + (long long)lo;
}


}  // namespace


namespace {

// Membership bitmap and per-block token counts (offsets[b + 1]; a repeated
// (token, block) pair is counted once).
__global__ void k_pf_mark(PrefillArgs p) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)p.M * p.k) return;
  const int t = (int)(i / p.k);
  const int b = p.sel[i];
  if (b < 0 || b >= p.d.NB) {
    atomicOr(p.d.status, 1);
    return;
  }
  const uint32_t bit = 1u << (t & 31);
  if ((atomicOr(&p.bitmap[(long long)b * p.words + (t >> 5)], bit) & bit) == 0) atomicAdd(&p.offsets[b + 1], 1);
}

// Exclusive scan of the block counts, in place (one workgroup).
__global__ void __launch_bounds__(1024) k_pf_scan(PrefillArgs p) {
  __shared__ int wsum[16];
  __shared__ int carry_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NB = p.d.NB;
  if (tid == 0) carry_s = 0;
  __syncthreads();
  for (int base = 0; base < NB; base += 1024) {
    const int b = base + tid;
    int v = b < NB ? p.offsets[b + 1] : 0;
    int incl = v;
#pragma unroll
    for (int dd = 1; dd < kWave; dd <<= 1) {
      const int o = __shfl_up(incl, dd, kWave);
      if (lane >= dd) incl += o;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int before = carry_s;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    if (b < NB) p.offsets[b + 1] = before + incl;
    __syncthreads();
    if (tid == 1023) carry_s = before + incl;
    __syncthreads();
  }
}

// Token list of block b (ascending token ids) and its token-group starts, one
// thread per block; the bitmap words go out 8 at a time.
__global__ void __launch_bounds__(256) k_pf_list(PrefillArgs p) {
  const int b = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (b >= p.d.NB) return;
  int pos = p.offsets[b];
  int32_t* g = p.grp + (long long)b * (p.TG + 1);
  const uint32_t* bm = p.bitmap + (long long)b * p.words;
  for (int w0 = 0; w0 < p.words; w0 += 8) {
    uint32_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = w0 + u < p.words ? bm[w0 + u] : 0u;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int w = w0 + u;
      if (w >= p.words) break;
      if ((w & 3) == 0) g[w >> 2] = pos;
      uint32_t bits = v[u];
      while (bits) {
        p.tokens[pos++] = w * 32 + __builtin_ctz(bits);
        bits &= bits - 1;
      }
    }
  }
  for (int tg = (p.words + 3) >> 2; tg <= p.TG; ++tg) g[tg] = pos;
}

// Gate/up of one block for all its tokens, as a staged GEMM.  A pass takes
// up to kGuTok tokens (tiles of 16); K goes in 128-column chunks through a
// ring of kGuNS stages in LDS, filled by buffer loads straight into LDS
// (no registers), kGuNS - 1 chunks ahead: per chunk each thread issues the
// same loads (two 16-byte pieces of token rows, two dwords of the block's
// 64 NF4 rows, its absmax entry), so one s_waitcnt per chunk (the loads of
// the next kGuNS - 2 chunks may stay in flight) and one barrier hand a chunk
// to the waves.  Such a load puts lane l's bytes at a fixed LDS slot (16 l or
// 4 l from the wave's base); each lane picks the piece of global memory for
// its slot, so the rows are stored XOR-swizzled and the fragment reads below
// hit distinct banks.  Wave w takes MFMA step s = w % 4 of every chunk
// (columns 32 s .. 32 s + 31) for projection w / 4 (gate or up, 2 N-tiles of
// 16 rows): it decodes its B fragments to fp16(code * absmax) and multiplies
// them with every token tile's A fragment.  The four step partials are
// summed in LDS in step order at the end of the pass; act = fp16(silu(gate)
// * up).
constexpr int kGuChunk = 128;              // columns per chunk
constexpr int kGuTok = 64;                 // tokens per pass
constexpr int kGuTiles = kGuTok / 16;      // MFMA token tiles per pass
constexpr int kGuNS = 3;                   // LDS stages (chunks): 76 KB, two workgroups per CU
constexpr int kGuXBytes = kGuTok * kGuChunk * 2;   // token rows of a stage: [64][16 pieces of 16 B]
constexpr int kGuWBytes = 64 * kGuChunk / 2;       // NF4 rows of a stage: [64][16 dwords]
constexpr int kGuAux = 64 * 4;                     // absmax entries of a stage: [64 rows][4 pieces of 32 columns]
constexpr int kGuCopies = 4;                       // code-pair table copies (lane % 4)
struct GuLds {
  uint8_t x[kGuNS][kGuXBytes];
  uint8_t w[kGuNS][kGuWBytes];
  uint32_t qa[kGuNS][kGuAux];  // double-quantised: u8 code (low byte); fp32: the absmax bits
  float a2[kGuNS][kGuAux];     // double-quantised: the entry's absmax2 (fp32: a second copy of qa)
  float2 cpair[256 * kGuCopies];  // entry e, copy c at e * kGuCopies + c
  float c2[2][256];
};
static_assert(kGuTok * 64 * 4 <= kGuNS * kGuXBytes, "gate/up sums must fit the token stages");
static_assert(kGuTok * 16 == 2 * kPfThreads && 64 * 16 == 2 * kPfThreads && 2 * kGuAux == kPfThreads,
              "loads per chunk: two token pieces, two weight dwords, one absmax load per thread");

template <bool DQ>
__global__ void __launch_bounds__(kPfThreads, 4) k_pf_gu(PrefillArgs p) {  // 4 waves per SIMD: two workgroups per CU
  extern __shared__ __attribute__((aligned(16))) uint8_t pf_lds[];
  GuLds& L = *reinterpret_cast<GuLds*>(pf_lds);
  const DecodeArgs& d = p.d;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int beg = p.offsets[b], cnt = p.offsets[b + 1] - beg;
  if (cnt == 0) return;
  for (int i = tid; i < 256 * kGuCopies; i += kPfThreads) {
    const int e = i / kGuCopies;
    L.cpair[i] = make_float2(d.code[e >> 4], d.code[e & 15]);
  }
  if constexpr (DQ) L.c2[tid >> 8][tid & 255] = (tid < 256 ? d.gate.code2 : d.up.code2)[tid & 255];
  const BlockRef br = resolve_id(d, b);
  if (!br.ok && tid == 0) atomicOr(d.status, 1);
  const int H = d.H;
  const uint32_t rs = (uint32_t)d.gate.row_stride;
  const uint32_t A = (uint32_t)d.gate.abs_row_stride;
  const int nb = br.ok ? (int)(32 * rs) : 0;
  const rsrc_t rg = make_rsrc((br.dev ? d.gate.packed : d.host_gate.packed) + br.q * d.gate.blk_stride, nb);
  const rsrc_t ru = make_rsrc((br.dev ? d.up.packed : d.host_up.packed) + br.q * d.up.blk_stride, nb);
  rsrc_t rga = rg, rua = ru, rgq = rg, ruq = ru, rg2 = rg, ru2 = rg;
  if constexpr (DQ) {
    const int na = br.ok ? (int)(32 * A) : 0;
    rgq = make_rsrc((br.dev ? d.gate.qabsmax : d.host_gate.qabsmax) + br.q * d.gate.abs_blk_stride, na);
    ruq = make_rsrc((br.dev ? d.up.qabsmax : d.host_up.qabsmax) + br.q * d.up.abs_blk_stride, na);
    const int n2 = br.ok ? (int)((((long long)d.NB * 32 * A + (1 << d.dq_shift) - 1) >> d.dq_shift) * 4) : 0;
    rg2 = make_rsrc(d.gate.absmax2, n2);
    ru2 = make_rsrc(d.up.absmax2, n2);
  } else {
    const int na = br.ok ? (int)(32 * A * 4) : 0;
    rga = make_rsrc((br.dev ? d.gate.absmax : d.host_gate.absmax) + br.q * d.gate.abs_blk_stride, na);
    rua = make_rsrc((br.dev ? d.up.absmax : d.host_up.absmax) + br.q * d.up.abs_blk_stride, na);
  }
  const rsrc_t rx = make_rsrc(p.x, (int)((long long)p.M * H * 2));
  const rsrc_t rtok = make_rsrc(p.tokens + beg, cnt * 4);
  const int nchunks = H / kGuChunk;
  // loads of this thread per chunk (instruction i = 2 wave + h of 16 per
  // chunk, lane l): token row 4 i + l / 16, LDS slot l % 16 <- global piece
  // (l % 16) ^ (row % 16); weight row 4 i + l / 16 (gate rows 0-31 from waves
  // 0-3), LDS dword l % 16 <- global dword (l % 16) ^ 4 ((row / 4) % 4);
  // absmax entry e = tid % 256 = (row e / 4, 32-column piece e % 4): its u8
  // code from waves 0-3 and its absmax2 from waves 4-7 (fp32 absmax: the
  // value from both, into qa and a2)
  const int xslot = lane & 15;
  const bool wup = wave >= 4;
  const uint32_t wdw[2] = {(uint32_t)((lane & 15) ^ (((((8 * wave + 4 * 0 + (lane >> 4)) & 31) >> 2) & 3) << 2)),
                           (uint32_t)((lane & 15) ^ (((((8 * wave + 4 * 1 + (lane >> 4)) & 31) >> 2) & 3) << 2))};
  const uint32_t wrow_b[2] = {(uint32_t)((8 * wave + (lane >> 4)) & 31), (uint32_t)((8 * wave + 4 + (lane >> 4)) & 31)};
  const int ae = tid & (kGuAux - 1), ar = ae >> 2, apart = ae & 3;
  const uint32_t arow = (uint32_t)(ar & 31);
  const bool aup = (wave & 3) >= 2;  // ar >= 32, from the (uniform) wave index
  // this wave's MFMA step and projection; lane (j, g)
  const int s = wave & 3, proj = wave >> 2;
  const int j = lane & 15, g = lane >> 4;
  // per-lane load offsets, the same for every chunk (the chunk's column
  // offset goes in the scalar offset): weight dwords, absmax entries
  const rsrc_t rW = wup ? ru : rg;
  const rsrc_t rQ = DQ ? (aup ? ruq : rgq) : (aup ? rua : rga);
  const rsrc_t rA2 = aup ? ru2 : rg2;
  const rsrc_t rnone = make_rsrc(p.x, 0);
  const uint32_t wv0 = wrow_b[0] * rs + wdw[0] * 4u, wv1 = wrow_b[1] * rs + wdw[1] * 4u;
  const uint32_t ape = (32u * (uint32_t)apart) >> d.qbs_shift;  // the entry's group past the chunk's first
  const uint32_t qv = DQ ? ((arow >> 1) * A + ape) * 2u + (arow & 1u) : (arow * A + ape) * 4u;
  const uint32_t fb = (32u * (uint32_t)b + arow) * A + ape;  // absmax index of the entry in chunk 0
  __syncthreads();

  for (int t0 = 0; t0 < cnt; t0 += kGuTok) {
    const int T = min(kGuTok, cnt - t0);
    const int ntiles = (T + 15) >> 4;
    // token rows of this pass (rows past T load zeros)
    uint32_t xv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int tr = 8 * wave + 4 * h + (lane >> 4);
      const uint32_t pc = (uint32_t)(xslot ^ (tr & 15));
      const int tok = tr < T ? buf_ldic(rtok, (uint32_t)(t0 + tr) * 4u, 0) : -1;
      xv[h] = tok >= 0 ? ((uint32_t)tok * (uint32_t)H + pc * 8u) * 2u : kOffNone;
    }
    // chunk c into stage c % kGuNS (a chunk past the end: descriptors of
    // extent zero, so its loads write zeros without reading memory)
    auto issue = [&](int c, auto stc) {
      constexpr int st = decltype(stc)::value;
      const bool live = c < nchunks;
      const uint32_t col0 = (uint32_t)(live ? c : 0) * kGuChunk;
      const uint32_t cq = col0 >> d.qbs_shift;
      const rsrc_t rxc = live ? rx : rnone, rWc = live ? rW : rnone, rQc = live ? rQ : rnone;
      ld_lds16s(rxc, &L.x[st][(2 * wave) * 1024], xv[0], col0 * 2u);
      ld_lds16s(rxc, &L.x[st][(2 * wave + 1) * 1024], xv[1], col0 * 2u);
      ld_lds4s(rWc, &L.w[st][(2 * wave) * 256], wv0, col0 >> 1);
      ld_lds4s(rWc, &L.w[st][(2 * wave + 1) * 256], wv1, col0 >> 1);
      if constexpr (DQ) {
        if (!wup)
          ld_lds1s(rQc, &L.qa[st][wave * 64], qv, cq * 2u);
        else
          ld_lds4(live ? rA2 : rnone, &L.a2[st][(wave - 4) * 64], ((fb + cq) >> d.dq_shift) * 4u);
      } else {
        ld_lds4s(rQc, wup ? (const void*)&L.a2[st][(wave - 4) * 64] : (const void*)&L.qa[st][wave * 64], qv, cq * 4u);
      }
    };
    float4_t acc[kGuTiles][2];
#pragma unroll
    for (int tt = 0; tt < kGuTiles; ++tt) acc[tt][0] = acc[tt][1] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    issue(0, std::integral_constant<int, 0>());
    issue(1, std::integral_constant<int, 1>());
    // chunk c from stage ST = c % kGuNS (a compile-time constant: the loop
    // below is unrolled by kGuNS, so the stage offsets are immediates)
    auto chunk = [&](int c, auto stc) {
      constexpr int st = decltype(stc)::value;
      // this thread's loads of chunk c have landed (those of the next
      // kGuNS - 2 chunks may not), then every thread's
      asm volatile("s_waitcnt vmcnt(5)" ::: "memory");  // (kGuNS - 2) chunks x 5 loads
      lds_barrier();  // also: every wave is done with chunk c - 1, whose stage the next issue refills
      // every LDS read of the chunk that depends on no other goes out first
      // (the token tiles' A fragments, the two weight words, the absmax
      // entries), the next chunk's loads behind them; then the code-book
      // reads that need them.  Two LDS round trips per chunk before the
      // MFMAs (the A fragments read tile by tile after the decode made six).
      const int r0 = proj * 32 + j, r1 = r0 + 16;
      const int a0 = r0 * 4 + s, a1 = r1 * 4 + s;  // piece s: the step's 32 columns
      half8_t af[kGuTiles];
#pragma unroll
      for (int tt = 0; tt < kGuTiles; ++tt) {
        if (tt < ntiles) {
          const int row = tt * 16 + j;
          af[tt] = as_h8(*reinterpret_cast<const uint4*>(
              &L.x[st][row * 256 + ((uint32_t)(4 * s + g) ^ (uint32_t)(row & 15)) * 16]));
        }
      }
      const uint32_t w0 = *reinterpret_cast<const uint32_t*>(
          &L.w[st][r0 * 64 + ((uint32_t)(4 * s + g) ^ ((((uint32_t)(r0 & 31) >> 2) & 3u) << 2)) * 4]);
      const uint32_t w1 = *reinterpret_cast<const uint32_t*>(
          &L.w[st][r1 * 64 + ((uint32_t)(4 * s + g) ^ ((((uint32_t)(r1 & 31) >> 2) & 3u) << 2)) * 4]);
      const uint32_t q0 = L.qa[st][a0], q1 = L.qa[st][a1];
      const float x0 = DQ ? L.a2[st][a0] : 0.0f, x1 = DQ ? L.a2[st][a1] : 0.0f;
      __builtin_amdgcn_sched_barrier(0);
      issue(c + kGuNS - 1, std::integral_constant<int, (st + kGuNS - 1) % kGuNS>());
      half8_t bf[2];
      {
        float am0, am1;
        if constexpr (DQ) {
          const float* c2 = L.c2[proj];
          const float off = proj ? d.up.offset : d.gate.offset;
          am0 = dq_absmax(c2[q0 & 0xFFu], x0, off);
          am1 = dq_absmax(c2[q1 & 0xFFu], x1, off);
        } else {
          am0 = __uint_as_float(q0);
          am1 = __uint_as_float(q1);
        }
        deq8x2<kGuCopies>(w0, am0, w1, am1, L.cpair + (lane & (kGuCopies - 1)), bf[0], bf[1]);
      }
#pragma unroll
      for (int tt = 0; tt < kGuTiles; ++tt) {
        if (tt < ntiles) {
          acc[tt][0] = mfma16(af[tt], bf[0], acc[tt][0]);
          acc[tt][1] = mfma16(af[tt], bf[1], acc[tt][1]);
        }
      }
    };
    static_assert(kGuNS == 3, "the chunk loop is unrolled by 3");
    int c = 0;
    for (; c + 3 <= nchunks; c += 3) {
      chunk(c, std::integral_constant<int, 0>());
      chunk(c + 1, std::integral_constant<int, 1>());
      chunk(c + 2, std::integral_constant<int, 2>());
    }
    if (c < nchunks) chunk(c, std::integral_constant<int, 0>());
    if (c + 1 < nchunks) chunk(c + 1, std::integral_constant<int, 1>());
    // the stages are free once every load (the zeros past the end too) has
    // landed; step partials summed in step order into [kGuTok tok][64 rows]
    // fp32 (rows: gate 0-31, up 32-63), reusing the token stages
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    mfma_drain();
    float* cs = reinterpret_cast<float*>(&L.x[0][0]);
    for (int ss = 0; ss < 4; ++ss) {
      if (s == ss) {
#pragma unroll
        for (int tt = 0; tt < kGuTiles; ++tt) {
          if (tt < ntiles) {
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                float* dst = &cs[(tt * 16 + 4 * g + r) * 64 + proj * 32 + q * 16 + j];
                *dst = ss == 0 ? acc[tt][q][r] : *dst + acc[tt][q][r];
              }
          }
        }
      }
      __syncthreads();
    }
    for (int o = tid; o < T * 32; o += kPfThreads) {
      const int ti = o >> 5, row = o & 31;
      const float gs = cs[ti * 64 + row], us = cs[ti * 64 + 32 + row];
      const uint16_t a = br.ok ? f2h(silu_mul(gs, us)) : (uint16_t)0;
      if (p.act_dense != nullptr)  // token row, column 32 b + row of the zeroed dense act
        p.act_dense[(long long)p.tokens[beg + t0 + ti] * (d.NB * 32) + 32 * b + row] = a;
      else
        p.act[(long long)(beg + t0 + ti) * 32 + row] = a;
    }
    __syncthreads();
  }
}

// Down for 64 output rows and one 128-token group.  Wave w takes blocks w,
// w + 8, ...; their CSR ranges for the group and their slots sit in lane
// registers (256 blocks per segment), so each block's loads (down columns,
// absmax, the first 16 act rows and their token ids) are issued one block
// ahead, all unconditional.
struct DnPf {
  uint32_t w[4];    // 4 bytes of each N-tile row: nibbles 8 g .. 8 g + 7
  float am[4];      // fp32 absmax, or the absmax2 (double-quantised)
  uint32_t qa[4];   // u8 absmax code (double-quantised)
  uint4 act;        // act row s0 + j, columns 8 g .. 8 g + 7
  int tok[4];       // token ids of the C rows 4 g + r (entries s0 + 4 g + r), -1: none
  int s0, s1;
  int b;
};

constexpr int kPfA2Max = 1024;  // absmax2 entries of a 64-row chunk staged in LDS
constexpr int kDnDepth = 2;     // blocks in flight per wave

template <bool DQ>
__global__ void __launch_bounds__(kPfThreads, 2) k_pf_down(PrefillArgs p) {
  __shared__ unsigned long long acc_s[kTokGroup][64];
  __shared__ uint32_t cpair[256];
  __shared__ float c2_s[256];
  __shared__ float a2_s[DQ ? kPfA2Max : 1];
  const DecodeArgs& d = p.d;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int chunks = d.H / 64;
  // XCD-aware: the TG token groups of a row chunk go to one XCD (one L2 for
  // the chunk's down columns) when the chunk count allows it
  int rc, tg;
  if (chunks % 8 == 0) {
    const int xcd = blockIdx.x & 7, s = blockIdx.x >> 3;
    rc = xcd + 8 * (s / p.TG);
    tg = s % p.TG;
  } else {
    rc = blockIdx.x / p.TG;
    tg = blockIdx.x % p.TG;
  }
  const int o0 = rc * 64, t0 = tg * kTokGroup;
  for (int i = tid; i < kTokGroup * 64; i += kPfThreads) (&acc_s[0][0])[i] = 0ull;
  cpair_fill(cpair, d.code, tid, kPfThreads);
  const uint32_t Ad = (uint32_t)(d.NB * 32) >> d.qbs_shift;
  // double-quantised: the absmax2 entries of rows o0 .. o0 + 63 (from g_lo on)
  // in LDS when they fit, else read per block
  const uint32_t g_lo = DQ ? ((uint32_t)o0 * Ad) >> d.dq_shift : 0u;
  const bool a2_lds = DQ && (((64u * Ad - 1u) >> d.dq_shift) + 2u) <= (uint32_t)kPfA2Max;
  if constexpr (DQ) {
    if (tid < 256) c2_s[tid] = d.down.code2[tid];
    if (a2_lds) {
      const uint32_t last = (uint32_t)((((long long)d.H * Ad) - 1) >> d.dq_shift);
      for (int i = tid; i < kPfA2Max; i += kPfThreads) a2_s[i] = d.down.absmax2[min(g_lo + (uint32_t)i, last)];
    }
  }
  __syncthreads();
  const int j = lane & 15, g = lane >> 4;
  const int NB = d.NB;
  const int nbw = NB > wave ? (NB - wave + kPfWaves - 1) / kPfWaves : 0;  // this wave's blocks
  const long long nk = (long long)p.M * p.k;
  const rsrc_t r_act = make_rsrc(p.act, (int)(nk * 64));
  const rsrc_t r_tok = make_rsrc(p.tokens, (int)(nk * 4));
  const int n2 = DQ ? (int)((((long long)d.H * Ad + (1 << d.dq_shift) - 1) >> d.dq_shift) * 4) : 0;
  const rsrc_t r_a2 = make_rsrc(d.down.absmax2, n2);
  const bool have_host = d.host_down.packed != nullptr;
  bool out_of_range = false;  // a partial outside the fixed-point range (reported in the status word)

  for (int seg = 0; seg * 256 < nbw; ++seg) {
    const int nseg = min(256, nbw - seg * 256);
    // lane i: block m = seg 256 + 64 q + i: CSR range for the group, slot
    int s0v[4], s1v[4], slv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = seg * 256 + q * 64 + lane;
      const int b = wave + kPfWaves * m;
      const bool v = m < nbw;
      s0v[q] = v ? p.grp[(long long)b * (p.TG + 1) + tg] : 0;
      s1v[q] = v ? p.grp[(long long)b * (p.TG + 1) + tg + 1] : 0;
      slv[q] = v ? (d.lookup ? d.lookup[b] : b) : -1;
    }
    auto pick = [&](const int (&v)[4], int mm) {
      const int qi = (mm >> 6) & 3, li = mm & 63;
      const int x = qi == 0 ? v[0] : qi == 1 ? v[1] : qi == 2 ? v[2] : v[3];
      return __builtin_amdgcn_readlane(x, li);
    };
    auto issue = [&](DnPf& st, int mm) {
      const bool in = mm < nseg;
      const int b = wave + kPfWaves * (seg * 256 + mm);
      st.b = b;
      st.s0 = in ? pick(s0v, mm) : 0;
      st.s1 = in ? pick(s1v, mm) : 0;
      const int slot = in ? pick(slv, mm) : -1;
      const bool dev = slot >= 0;
      const bool ok = in && st.s0 < st.s1 && (dev ? slot < d.n_slots : have_host);
      if (!ok) st.s1 = st.s0;  // no contribution (the gate/up kernel flags invalid blocks)
      const long long q = ok ? (dev ? slot : b) : 0;
      const rsrc_t rw = make_rsrc((dev ? d.down.packed : d.host_down.packed) + q * d.down.blk_stride,
                                  ok ? d.H * 16 : 0);
      rsrc_t ra;
      if constexpr (DQ)
        ra = make_rsrc((dev ? d.down.qabsmax : d.host_down.qabsmax) + q * d.down.abs_blk_stride, ok ? d.H : 0);
      else
        ra = make_rsrc((dev ? d.down.absmax : d.host_down.absmax) + q * d.down.abs_blk_stride, ok ? d.H * 4 : 0);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const uint32_t o = (uint32_t)(o0 + nt * 16 + j);
        // cached: the other token groups of this row chunk read the same columns
        st.w[nt] = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)(o * 16u + 4u * g), 0, 0);
        if constexpr (DQ) {
          st.qa[nt] = buf_ldu8(ra, o, 0);
          const uint32_t f = o * Ad + ((32u * (uint32_t)b) >> d.qbs_shift);
          st.am[nt] = buf_ldfc(r_a2, (ok && !a2_lds) ? (f >> d.dq_shift) * 4u : kOffNone, 0);
        } else {
          st.qa[nt] = 0;
          st.am[nt] = buf_ldf(ra, o * 4u, 0);
        }
      }
      const int e = st.s0 + j;
      st.act = buf_ld16c(r_act, e < st.s1 ? (uint32_t)e * 64u + 16u * g : kOffNone, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int er = st.s0 + 4 * g + r;
        const int tv = buf_ldic(r_tok, er < st.s1 ? (uint32_t)er * 4u : kOffNone, 0);
        st.tok[r] = er < st.s1 ? tv : -1;
      }
    };
    DnPf st[kDnDepth];
#pragma unroll
    for (int i = 0; i < kDnDepth; ++i) issue(st[i], i);
    for (int m0 = 0; m0 < nseg; m0 += kDnDepth) {
#pragma unroll
      for (int ss = 0; ss < kDnDepth; ++ss) {
        DnPf& cur = st[ss];
        if (cur.s0 < cur.s1) {
          half8_t bf[4];
          float am[4];  // absmax of output row j of N-tile nt for this block
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            float a = cur.am[nt];
            if constexpr (DQ) {
              float a2 = cur.am[nt];
              if (a2_lds) {
                const uint32_t o = (uint32_t)(o0 + nt * 16 + j);
                a2 = a2_s[((o * Ad + ((32u * (uint32_t)cur.b) >> d.qbs_shift)) >> d.dq_shift) - g_lo];
              }
              a = dq_absmax(c2_s[cur.qa[nt]], a2, d.down.offset);
            }
            bf[nt] = codes8(cur.w[nt], cpair);
            am[nt] = a;
          }
          for (int e0 = cur.s0; e0 < cur.s1; e0 += 16) {
            uint4 av = cur.act;
            int tk[4] = {cur.tok[0], cur.tok[1], cur.tok[2], cur.tok[3]};
            if (e0 != cur.s0) {  // tiles after the first (more than 16 tokens of this group)
              const int e = e0 + j;
              av = buf_ld16c(r_act, e < cur.s1 ? (uint32_t)e * 64u + 16u * g : kOffNone, 0);
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int er = e0 + 4 * g + r;
                const int tv = buf_ldic(r_tok, er < cur.s1 ? (uint32_t)er * 4u : kOffNone, 0);
                tk[r] = er < cur.s1 ? tv : -1;
              }
            }
            const half8_t af = as_h8(av);
            float4_t c[4];
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) c[nt] = mfma16(af, bf[nt], float4_t{0.0f, 0.0f, 0.0f, 0.0f});
            mfma_drain();
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (tk[r] >= 0) {
                const int tl = tk[r] - t0;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                  const float v = c[nt][r] * am[nt];
                  out_of_range |= !(fabsf(v) < 8388608.0f);  // 2^23; also inf and nan
                  atomicAdd(&acc_s[tl][nt * 16 + j], (unsigned long long)to_fix31(v));
                }
              }
            }
          }
        }
        issue(cur, m0 + ss + kDnDepth);
      }
    }
  }
  if (out_of_range) atomicOr(d.status, NSMLP_STATUS_FIXED_RANGE);
  __syncthreads();
  for (int i = tid; i < kTokGroup * 64; i += kPfThreads) {
    const int tl = i >> 6, row = i & 63;
    const int t = t0 + tl;
    if (t >= p.M) continue;
    float y = (float)((double)(long long)acc_s[tl][row] * kFixInv);
    if (d.down_bias != nullptr) y += h2f(d.down_bias[o0 + row]);
    p.out[(long long)t * d.H + o0 + row] = f2h(y);
  }
}

}  // namespace

void launch_prefill(const PrefillArgs& p, hipStream_t s) {
  // the bitmap and the block counts (offsets, right after it) start at zero
  launch_zero_u32(p.bitmap, (long long)(reinterpret_cast<const uint32_t*>(p.offsets + p.d.NB + 1) - p.bitmap), s);
  const long long n = (long long)p.M * p.k;
  k_pf_mark<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(p);
  k_pf_scan<<<dim3(1), dim3(1024), 0, s>>>(p);
  k_pf_list<<<dim3((unsigned)((p.d.NB + 255) / 256)), dim3(256), 0, s>>>(p);
  if (p.act_dense != nullptr) launch_zero_u32(reinterpret_cast<uint32_t*>(p.act_dense), (long long)p.M * p.d.NB * 16, s);
  static std::once_flag gu_once;
  std::call_once(gu_once, [] {
    for (const void* f : {reinterpret_cast<const void*>(k_pf_gu<true>), reinterpret_cast<const void*>(k_pf_gu<false>)})
      (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(GuLds));
  });
  if (p.d.dq)
    k_pf_gu<true><<<dim3(p.d.NB), dim3(kPfThreads), sizeof(GuLds), s>>>(p);
  else
    k_pf_gu<false><<<dim3(p.d.NB), dim3(kPfThreads), sizeof(GuLds), s>>>(p);
  if (p.act_dense != nullptr) {
    // every token's act is zero outside its own blocks, so the dense down GEMM
    // over the scattered act is the per-token sum over the selected blocks
    DenseGuardArgs g;
    memset(&g, 0, sizeof(g));
    g.d = p.d;
    g.x = p.x;
    g.M = p.M;
    g.act = p.act_dense;
    g.part = p.part;
    g.S = p.S;
    g.out = p.out;
    g.offsets = p.offsets;  // blocks no token selected are skipped (their act is zero)
    launch_dense_down(g, s);
    return;
  }
  const dim3 gd((unsigned)((p.d.H / 64) * p.TG));
  if (p.d.dq)
    k_pf_down<true><<<gd, dim3(kPfThreads), 0, s>>>(p);
  else
    k_pf_down<false><<<gd, dim3(kPfThreads), 0, s>>>(p);
}

}  // namespace nsmlp
