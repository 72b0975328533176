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

// fp32 code pairs per packed byte: entry e = (code[e >> 4], code[e & 15]),
// the (even, odd) elements of byte e.
__device__ __forceinline__ void fpair_fill(float2* cp, const float* code, int tid, int nthr) {
  for (int e = tid; e < 256; e += nthr) cp[e] = make_float2(code[e >> 4], code[e & 15]);
}

// 16 consecutive NF4 elements of two rows (words w0, w1: 4 bytes each, even
// element in the high nibble) as fp16(code * absmax), the reference
// fallback's rounding of the weights.  All eight pair lookups go out before
// any is used.
__device__ __forceinline__ void deq8x2(uint32_t w0, float am0, uint32_t w1, float am1, const float2* cp,
                                       half8_t& h0, half8_t& h1) {
  float2 p[8];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    p[m] = cp[(w0 >> (8 * m)) & 0xFFu];
    p[4 + m] = cp[(w1 >> (8 * m)) & 0xFFu];
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
// up to kGuTok tokens (tiles of 16); K goes in 128-column chunks.  Per chunk
// the 512 threads load the pass's token rows (16 B pieces, 256 B per row),
// the block's 64 NF4 rows (8 B pieces, 64 B per row) and their absmax with
// coalesced loads two chunks ahead, and stage them in LDS (the absmax
// resolved to fp32 per row and 64 columns).  Wave w takes MFMA step
// s = w % 4 of every chunk (columns 32 s .. 32 s + 31) for projection
// w / 4 (gate or up, 2 N-tiles of 16 rows): it decodes its B fragments once
// per chunk to fp16(code * absmax) and multiplies them with every token
// tile's A fragment.  The four step partials are summed in LDS in step
// order at the end of the pass; act = fp16(silu(gate) * up).
constexpr int kGuChunk = 128;             // columns per chunk
constexpr int kGuTok = 64;                // tokens per pass
constexpr int kGuTiles = kGuTok / 16;      // MFMA token tiles per pass
constexpr int kXPieces = kGuTok * 16 / kPfThreads;  // 16-byte token-row pieces per thread and chunk
static_assert(kXPieces >= 1 && kGuTok * 16 == kXPieces * kPfThreads, "token pieces must cover the pass");
static_assert(kGuTok * 64 * 4 <= kGuTok * (kGuChunk * 2 + 16), "gate/up sums must fit the token buffer");
constexpr int kXRow = kGuChunk * 2 + 16;  // bytes per staged token row (padded)
constexpr int kWRow = kGuChunk / 2 + 16;  // bytes per staged NF4 row (padded)

struct GuRegs {
  uint4 x[kXPieces];  // 16-byte pieces of token rows
  uint2 w;        // 16 nibbles of one weight row
  float am;       // fp32 absmax, or the absmax2 (double-quantised)
  uint32_t qa;    // u8 absmax code (double-quantised)
};

template <bool DQ>
__global__ void __launch_bounds__(kPfThreads, 4) k_pf_gu(PrefillArgs p) {  // 4 waves per SIMD: two workgroups per CU
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kGuTok * kXRow];  // token rows, fp16
  __shared__ __attribute__((aligned(16))) uint8_t wsr[2][64 * kWRow];     // NF4 rows (gate 0-31, up 32-63)
  __shared__ float ams[2][64][8];                                          // absmax per row and 16 columns
  __shared__ float2 cpair_s[256];
  __shared__ float c2_s[2][256];
  const DecodeArgs& d = p.d;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int beg = p.offsets[b], cnt = p.offsets[b + 1] - beg;
  if (cnt == 0) return;
  fpair_fill(cpair_s, d.code, tid, kPfThreads);
  if constexpr (DQ) c2_s[tid >> 8][tid & 255] = (tid < 256 ? d.gate.code2 : d.up.code2)[tid & 255];
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
  // this thread's staged weight row (0..31 gate, 32..63 up) and 16-column piece
  const int wr = tid >> 3, wpart = tid & 7;
  const bool wup = wr >= 32;
  const uint32_t wrow = (uint32_t)(wr & 31);
  // this wave's MFMA step and projection; lane (j, g)
  const int s = wave & 3, proj = wave >> 2;
  const int j = lane & 15, g = lane >> 4;
  __syncthreads();

  for (int t0 = 0; t0 < cnt; t0 += kGuTok) {
    const int T = min(kGuTok, cnt - t0);
    const int ntiles = (T + 15) >> 4;
    int xtok[kXPieces];
#pragma unroll
    for (int h = 0; h < kXPieces; ++h) {
      const int tt = (tid + h * kPfThreads) >> 4;
      xtok[h] = tt < T ? buf_ldic(rtok, (uint32_t)(t0 + tt) * 4u, 0) : -1;
    }
    auto load = [&](GuRegs& R, int c) {
      const bool live = c < nchunks;
      const uint32_t col0 = (uint32_t)(live ? c : 0) * kGuChunk;
#pragma unroll
      for (int h = 0; h < kXPieces; ++h) {
        const uint32_t part = (uint32_t)((tid + h * kPfThreads) & 15);
        const uint32_t xo = (live && xtok[h] >= 0) ? ((uint32_t)xtok[h] * (uint32_t)H + col0 + part * 8u) * 2u
                                                   : kOffNone;
        R.x[h] = buf_ld16c(rx, xo, 0);
      }
      const uint32_t col = col0 + 16u * (uint32_t)wpart;
      const uint32_t ce = col >> d.qbs_shift;
      const u32x2_t wv = __builtin_amdgcn_raw_buffer_load_b64(wup ? ru : rg, (int)(live ? wrow * rs + (col >> 1)
                                                                                         : kOffNone), 0, 0);
      R.w = make_uint2(wv.x, wv.y);
      if constexpr (DQ) {
        R.qa = buf_ldu8(wup ? ruq : rgq, live ? ((wrow >> 1) * A + ce) * 2u + (wrow & 1u) : kOffNone, 0);
        const uint32_t f = (32u * (uint32_t)b + wrow) * A + ce;
        R.am = buf_ldfc(wup ? ru2 : rg2, live ? (f >> d.dq_shift) * 4u : kOffNone, 0);
      } else {
        R.qa = 0;
        R.am = buf_ldf(wup ? rua : rga, live ? (wrow * A + ce) * 4u : kOffNone, 0);
      }
    };
    auto store = [&](int bi, const GuRegs& R) {
#pragma unroll
      for (int h = 0; h < kXPieces; ++h) {
        const int piece = tid + h * kPfThreads;
        *reinterpret_cast<uint4*>(&xs[bi][(piece >> 4) * kXRow + (piece & 15) * 16]) = R.x[h];
      }
      *reinterpret_cast<uint2*>(&wsr[bi][wr * kWRow + wpart * 8]) = R.w;
      float am = R.am;
      if constexpr (DQ) am = dq_absmax(c2_s[wup ? 1 : 0][R.qa], R.am, wup ? d.up.offset : d.gate.offset);
      ams[bi][wr][wpart] = am;  // the absmax of this thread's 16 columns
    };
    float4_t acc[kGuTiles][2];
#pragma unroll
    for (int tt = 0; tt < kGuTiles; ++tt) acc[tt][0] = acc[tt][1] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    GuRegs R[2];
    load(R[0], 0);
    load(R[1], 1);
    store(0, R[0]);
    load(R[0], 2);
    __syncthreads();
    // chunk c computes from buffer c & 1 while the next chunk goes into the
    // other buffer; unrolled by two so the register stages are named
    auto step = [&](int c, int bi, GuRegs& Rn) {
      half8_t bf[2];
      {
        const int r0 = proj * 32 + j, r1 = r0 + 16;
        const uint32_t w0 = *reinterpret_cast<const uint32_t*>(&wsr[bi][r0 * kWRow + 16 * s + 4 * g]);
        const uint32_t w1 = *reinterpret_cast<const uint32_t*>(&wsr[bi][r1 * kWRow + 16 * s + 4 * g]);
        deq8x2(w0, ams[bi][r0][2 * s + (g >> 1)], w1, ams[bi][r1][2 * s + (g >> 1)], cpair_s, bf[0], bf[1]);
      }
#pragma unroll
      for (int tt = 0; tt < kGuTiles; ++tt) {
        if (tt < ntiles) {
          const half8_t af = as_h8(*reinterpret_cast<const uint4*>(&xs[bi][(tt * 16 + j) * kXRow + (32 * s + 8 * g) * 2]));
          acc[tt][0] = mfma16(af, bf[0], acc[tt][0]);
          acc[tt][1] = mfma16(af, bf[1], acc[tt][1]);
        }
      }
      if (c + 1 < nchunks) {
        store(bi ^ 1, Rn);
        load(Rn, c + 3);
      }
      __syncthreads();
    };
    for (int c = 0; c < nchunks; c += 2) {
      step(c, 0, R[1]);
      if (c + 1 < nchunks) step(c + 1, 1, R[0]);
    }
    // step partials summed in step order into [kGuTok tok][64 rows] fp32
    // (rows: gate 0-31, up 32-63), reusing the token staging buffer
    mfma_drain();
    float* cs = reinterpret_cast<float*>(&xs[0][0]);
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
  if (p.d.dq)
    k_pf_gu<true><<<dim3(p.d.NB), dim3(kPfThreads), 0, s>>>(p);
  else
    k_pf_gu<false><<<dim3(p.d.NB), dim3(kPfThreads), 0, s>>>(p);
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
