// Chunked prefill of the sparse MLP: M tokens, each with its own top-k block
// set, over the union of the selected blocks (RT:4868-4901, RT:5453: every
// token's gate/up are masked to its own blocks, so a block contributes to a
// token only if the token selected it).  Grouped per block on MFMA
// (v_mfma_f32_16x16x32_f16, fp32 accumulation):
//
//   k_pf_mark / k_pf_csr  token lists per block (CSR, ascending token ids),
//                         from a [NB][M/32] membership bitmap;
//   k_pf_gu     one workgroup per block: gate and up of the block's tokens,
//               the token rows gathered as the MFMA A operand and the NF4
//               rows dequantised in registers to fp16(code * absmax) as the
//               B operand (the reference fallback's rounding of the weights,
//               RT:5439-5447); the 8 waves split K, their sums meet in LDS in
//               wave order; act = fp16(silu(gate) * up) per (block, token);
//   k_pf_down   one workgroup per 64 output rows and 128-token group: for
//               every block, act [tokens x 32] times the block's down columns
//               [32 x 64 rows]; each tile is added into the group's [128][64]
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
#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kPfThreads = 512;
constexpr int kPfWaves = kPfThreads / kWave;
constexpr int kChunk = 128;      // gate/up columns per wave step
constexpr int kTokGroup = 128;   // tokens per down workgroup
constexpr double kFixInv = 1.0 / 2147483648.0;  // down accumulator: int64 units of 2^-31

__device__ __forceinline__ half8_t mfma_zero_h8() {
  half8_t h;
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = (_Float16)0.0f;
  return h;
}

// 8 consecutive NF4 elements (4 bytes, even element in the high nibble) as
// fp16(code * absmax).
__device__ __forceinline__ half8_t deq8(uint32_t word, float am, const float* code) {
  half8_t h;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t byte = (word >> (8 * m)) & 0xFFu;
    h[2 * m] = (_Float16)(code[byte >> 4] * am);
    h[2 * m + 1] = (_Float16)(code[byte & 15u] * am);
  }
  return h;
}

__device__ __forceinline__ half8_t as_h8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

// v * 2^31 truncated toward zero (|v| < 2^23), in fp32/int32 steps: hi =
// trunc(v * 2^8) carries the bits above 2^-8, the remainder v - hi * 2^-8 is
// exact and |rem| < 2^-8, so trunc(rem * 2^31) fits 23 bits.
__device__ __forceinline__ long long to_fix31(float v) {
  const int hi = (int)(v * 256.0f);
  const float rem = __builtin_fmaf((float)hi, -0.00390625f, v);
  const int lo = (int)(rem * 2147483648.0f);
  return ((long long)hi << 23) + (long long)lo;
}

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

}  // namespace


namespace {

__global__ void k_pf_mark(PrefillArgs p) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)p.M * p.k) return;
  const int t = (int)(i / p.k);
  const int b = p.sel[i];
  if (b < 0 || b >= p.d.NB) {
    atomicOr(p.d.status, 1);
    return;
  }
  atomicOr(&p.bitmap[(long long)b * p.words + (t >> 5)], 1u << (t & 31));
}

// One workgroup: counts, exclusive scan, token lists and group starts.
__global__ void __launch_bounds__(1024) k_pf_csr(PrefillArgs p) {
  __shared__ int wsum[16];
  __shared__ int carry_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NB = p.d.NB;
  for (int b = tid; b < NB; b += 1024) {
    int c = 0;
    for (int w = 0; w < p.words; ++w) c += __popc(p.bitmap[(long long)b * p.words + w]);
    p.offsets[b + 1] = c;
  }
  if (tid == 0) {
    p.offsets[0] = 0;
    carry_s = 0;
  }
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
  for (int b = tid; b < NB; b += 1024) {
    int pos = p.offsets[b];
    int32_t* g = p.grp + (long long)b * (p.TG + 1);
    for (int w = 0; w < p.words; ++w) {
      if ((w & 3) == 0) g[w >> 2] = pos;
      uint32_t bits = p.bitmap[(long long)b * p.words + w];
      while (bits) {
        p.tokens[pos++] = w * 32 + __builtin_ctz(bits);
        bits &= bits - 1;
      }
    }
    for (int tg = (p.words + 3) >> 2; tg <= p.TG; ++tg) g[tg] = pos;
  }
}

// Gate/up of one block for all its tokens.  A pass takes up to 8 tiles of
// 16 tokens; with nte (a power of two >= the tiles) tile groups the 8 waves
// split K 8 / nte ways: wave w computes tile w % nte over the 128-column
// chunks ks, ks + KS, ... (ks = w / nte), so every token of the block is done
// in one pass over its weights; the K-split sums meet in LDS in ks order.
template <bool DQ>
__global__ void __launch_bounds__(kPfThreads, 2) k_pf_gu(PrefillArgs p) {
  __shared__ float red[kPfWaves][4][256];  // per wave: N-tile (gate 0-15, 16-31, up 0-15, 16-31), C
  __shared__ float code_s[16];
  __shared__ float c2_s[2][256];
  const DecodeArgs& d = p.d;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int beg = p.offsets[b], cnt = p.offsets[b + 1] - beg;
  if (cnt == 0) return;
  if (tid < 16) code_s[tid] = d.code[tid];
  if constexpr (DQ) c2_s[tid >> 8][tid & 255] = (tid < 256 ? d.gate.code2 : d.up.code2)[tid & 255];
  const BlockRef br = resolve_id(d, b);
  if (!br.ok && tid == 0) atomicOr(d.status, 1);
  __syncthreads();
  const int H = d.H;
  const int j = lane & 15, g = lane >> 4;
  const long long rs = d.gate.row_stride;
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
  const int nchunks = H / kChunk;
  const int ntiles = (cnt + 15) / 16;

  for (int pass0 = 0; pass0 < ntiles; pass0 += kPfWaves) {
    const int ntp = min(kPfWaves, ntiles - pass0);
    const int nte = ntp <= 1 ? 1 : ntp <= 2 ? 2 : ntp <= 4 ? 4 : 8;
    const int KS = kPfWaves / nte;
    const int tile = wave % nte, ks = wave / nte;
    const int e_row = (pass0 + tile) * 16 + j;  // this lane's A row (token entry)
    const bool tv = br.ok && tile < ntp && e_row < cnt;
    const int tok = tv ? p.tokens[beg + e_row] : 0;
    const bool wlive = br.ok && tile < ntp;
    float4_t acc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[nt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // two-stage pipeline over this wave's chunks ks, ks + KS, ...; every load
    // is unconditional (a chunk past the end, an idle tile or an invalid block
    // reads zeros through an out-of-extent offset)
    uint4 w[2][4], xv[2][4];
    float am[2][4];
    uint32_t qa[2][4];
    auto issue = [&](int st, int c) {
      const bool live = c < nchunks && wlive;
      const uint32_t col = (uint32_t)(live ? c : 0) * kChunk + 32u * g;
      const uint32_t ce = col >> d.qbs_shift;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const uint32_t r = (uint32_t)((nt & 1) * 16 + j);
        // cached: the other tile waves of this K split read the same rows
        w[st][nt] = buf_ld16c(nt < 2 ? rg : ru, live ? r * (uint32_t)rs + (col >> 1) : kOffNone, 0);
        if constexpr (DQ) {
          qa[st][nt] = buf_ldu8(nt < 2 ? rgq : ruq, live ? ((r >> 1) * A + ce) * 2u + (r & 1u) : kOffNone, 0);
          const uint32_t f = (32u * (uint32_t)b + r) * A + ce;
          am[st][nt] = buf_ldfc(nt < 2 ? rg2 : ru2, live ? (f >> d.dq_shift) * 4u : kOffNone, 0);
        } else {
          qa[st][nt] = 0;
          am[st][nt] = buf_ldf(nt < 2 ? rga : rua, live ? (r * A + ce) * 4u : kOffNone, 0);
        }
      }
      const uint32_t xo = (live && tv) ? ((uint32_t)tok * (uint32_t)H + col) * 2u : kOffNone;
#pragma unroll
      for (int v = 0; v < 4; ++v) xv[st][v] = buf_ld16c(rx, xo, 16u * v);
    };
    issue(0, ks);
    issue(1, ks + KS);
    for (int c0 = ks; c0 < nchunks; c0 += 2 * KS) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int c = c0 + st * KS;
        if (c < nchunks && wlive) {
          float amv[4];
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            if constexpr (DQ)
              amv[nt] = dq_absmax(c2_s[nt < 2 ? 0 : 1][qa[st][nt]], am[st][nt], nt < 2 ? d.gate.offset : d.up.offset);
            else
              amv[nt] = am[st][nt];
          }
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const half8_t af = as_h8(xv[st][s]);
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
              const uint32_t word = s == 0 ? w[st][nt].x : s == 1 ? w[st][nt].y : s == 2 ? w[st][nt].z : w[st][nt].w;
              acc[nt] = mfma16(af, deq8(word, amv[nt], code_s), acc[nt]);
            }
          }
        }
        issue(st, c + 2 * KS);
      }
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][nt][(4 * g + r) * 16 + j] = acc[nt][r];
    __syncthreads();
    for (int o = tid; o < ntp * 16 * 32; o += kPfThreads) {
      const int t = o >> 9, i = (o >> 5) & 15, row = o & 31;
      const int e = (pass0 + t) * 16 + i;
      if (e >= cnt) continue;
      const int ng = row >> 4, jj = row & 15;
      float gs = 0.0f, us = 0.0f;
      for (int q = 0; q < KS; ++q) {
        gs += red[t + nte * q][ng][i * 16 + jj];
        us += red[t + nte * q][2 + ng][i * 16 + jj];
      }
      p.act[(long long)(beg + e) * 32 + row] = br.ok ? f2h(silu_mul(gs, us)) : (uint16_t)0;
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

template <bool DQ>
__global__ void __launch_bounds__(kPfThreads, 2) k_pf_down(PrefillArgs p) {
  __shared__ unsigned long long acc_s[kTokGroup][64];
  __shared__ float code_s[16];
  __shared__ float c2_s[256];
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
  if (tid < 16) code_s[tid] = d.code[tid];
  if constexpr (DQ) {
    if (tid < 256) c2_s[tid] = d.down.code2[tid];
  }
  __syncthreads();
  const int j = lane & 15, g = lane >> 4;
  const uint32_t Ad = (uint32_t)(d.NB * 32) >> d.qbs_shift;
  const int NB = d.NB;
  const int nbw = NB > wave ? (NB - wave + kPfWaves - 1) / kPfWaves : 0;  // this wave's blocks
  const long long nk = (long long)p.M * p.k;
  const rsrc_t r_act = make_rsrc(p.act, (int)(nk * 64));
  const rsrc_t r_tok = make_rsrc(p.tokens, (int)(nk * 4));
  const int n2 = DQ ? (int)((((long long)d.H * Ad + (1 << d.dq_shift) - 1) >> d.dq_shift) * 4) : 0;
  const rsrc_t r_a2 = make_rsrc(d.down.absmax2, n2);
  const bool have_host = d.host_down.packed != nullptr;

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
          st.am[nt] = buf_ldfc(r_a2, ok ? (f >> d.dq_shift) * 4u : kOffNone, 0);
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
    DnPf st[2];
    issue(st[0], 0);
    issue(st[1], 1);
    for (int m0 = 0; m0 < nseg; m0 += 2) {
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        DnPf& cur = st[ss];
        if (cur.s0 < cur.s1) {
          half8_t bf[4];
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            const float a = DQ ? dq_absmax(c2_s[cur.qa[nt]], cur.am[nt], d.down.offset) : cur.am[nt];
            bf[nt] = deq8(cur.w[nt], a, code_s);
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
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (tk[r] >= 0) {
                const int tl = tk[r] - t0;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                  atomicAdd(&acc_s[tl][nt * 16 + j], (unsigned long long)to_fix31(c[nt][r]));
                }
              }
            }
          }
        }
        issue(cur, m0 + ss + 2);
      }
    }
  }
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
  launch_zero_u32(p.bitmap, (long long)p.d.NB * p.words, s);
  const long long n = (long long)p.M * p.k;
  k_pf_mark<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(p);
  k_pf_csr<<<dim3(1), dim3(1024), 0, s>>>(p);
  if (p.d.dq)
    k_pf_gu<true><<<dim3(p.d.NB), dim3(kPfThreads), 0, s>>>(p);
  else
    k_pf_gu<false><<<dim3(p.d.NB), dim3(kPfThreads), 0, s>>>(p);
  const dim3 gd((unsigned)((p.d.H / 64) * p.TG));
  if (p.d.dq)
    k_pf_down<true><<<gd, dim3(kPfThreads), 0, s>>>(p);
  else
    k_pf_down<false><<<gd, dim3(kPfThreads), 0, s>>>(p);
}

}  // namespace nsmlp
