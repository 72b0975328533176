// Dense-guard prefill MLP (RT:5775-5831, _dense_guard_mlp_forward_exact_chunked_4bit):
// every intermediate block for every token, read from the slot table, as
// full-width GEMMs on v_mfma_f32_16x16x32_f16 with fp32 accumulation.  The
// reference dequantises each NF4 projection to an fp16 weight and runs
// F.linear three times; the rounding points kept here are its own:
//
//   W  = fp16(code * absmax)                   (bitsandbytes dequant to fp16)
//   g  = fp16(x W_gate^T),  s = fp16(silu(g))  (gate = F.silu(F.linear(x, Wg)))
//   u  = fp16(x W_up^T),    act = fp16(s * u)  (act = gate * up)
//   y  = fp16(act W_down^T + bias)             (F.linear(act, Wd, bias))
//
//   k_dg_gu    one workgroup per 128 intermediate rows and 256 tokens: the
//              tokens' rows and the 128 gate + 128 up weight rows go through
//              double-buffered LDS in 64-column chunks (the weights decoded
//              to fp16(code * absmax) as they are staged); wave w computes
//              64 tokens (w % 4) x 64 rows (w / 4) of both projections, so
//              the act epilogue pairs g and u in registers;
//   k_dg_down  one workgroup per 256 output rows, 256 tokens and one of S
//              ranges of the intermediate blocks: the same staged GEMM over
//              act and the down columns (two blocks per chunk); fp32
//              partial sums per range;
//   k_dg_fin   y = fp16(sum of the S partials in range order + bias).
//
// The tokens past the last whole 256-token tile (all of a prompt of fewer than
// 256) go in a second launch with the smallest tile of 64, 128 or 192 tokens
// that holds them (wave w then computes 16, 32 or 48 tokens x 64 rows; the
// per-element K order is the same, so every token's result equals the
// 256-token tiles' bit for bit).
//
// Every sum is taken in a fixed order, so the result does not change from run
// to run.
#include <mutex>

#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kDgThreads = 512;
constexpr int kDgTok = 256;                 // tokens per tile (64, 128 or 192 for shorter prompts)
constexpr int kDgK = 64;                    // columns per chunk
constexpr int kDgRow = 72;                  // halfs per staged row (64 + 8: conflict-free fragment reads)
constexpr int kDgStage = 256 * kDgRow;      // halfs per staged operand (256 rows)
constexpr int kDgPairCopies = 4;  // code-pair table copies (the gate/up kernel keeps 2 of each of its 2 tables)
constexpr size_t kDgLds =
    (size_t)4 * kDgStage * 2 + kDgPairCopies * 256 * sizeof(float2) + 2 * 256 * sizeof(float);

// fp32 code pairs per packed byte: (code[e >> 4], code[e & 15]) = (even, odd
// element), `copies` interleaved copies of each entry (entry e, copy c at
// e * copies + c): lanes reading their own copy spread random lookups over
// more banks.
__device__ __forceinline__ void dg_pairs(float2* cp, const float* code, int i, int copies) {
  const int e = i / copies;
  cp[i] = make_float2(code[e >> 4], code[e & 15]);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// 32 NF4 codes (16 bytes, even element in the high nibble) -> 32 fp16(code * am)
// (fp32 products rounded to nearest, two per v_cvt_pk_f16_f32) written as 64
// bytes to dst (16-byte aligned).
template <int COPIES>
__device__ __forceinline__ void dg_decode32(_Float16* dst, uint4 w, float am, const float2* cp) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t o[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float2 pr = cp[((words[q] >> (8 * b)) & 0xFFu) * COPIES];
      const float2_t v = {pr.x * am, pr.y * am};
      o[b] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2_t));
    }
    *reinterpret_cast<uint4*>(dst + 8 * q) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// One staged weight unit: 32 NF4 codes of one row and its absmax.
struct DgW {
  uint4 w;
  float am;     // fp32 absmax, or the absmax2 (double-quantised)
  uint32_t qa;  // u8 absmax code (double-quantised)
};

// The wave's 16 MT x 128 tile for one staged chunk (MT = 4: 256-token tiles,
// MT = 1: 64-token tiles): A rows (tokens) 16 MT mq + 16 mi + lane % 16, B
// rows brow(ni) + lane % 16, K halves 32 ks + 8 (lane / 16).
template <int MT, typename BRow>
__device__ __forceinline__ void dg_mma(float4_t (&acc)[MT][8], const _Float16* As, const _Float16* Bs, int mq,
                                       int lane, BRow brow) {
  const int j = lane & 15, g = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    half8_t a[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
      a[mi] = as_h8(*reinterpret_cast<const uint4*>(As + (16 * MT * mq + 16 * mi + j) * kDgRow + 32 * ks + 8 * g));
#pragma unroll
    for (int ni = 0; ni < 8; ++ni) {
      const half8_t b = as_h8(*reinterpret_cast<const uint4*>(Bs + (brow(ni) + j) * kDgRow + 32 * ks + 8 * g));
#pragma unroll
      for (int mi = 0; mi < MT; ++mi) acc[mi][ni] = mfma16(a[mi], b, acc[mi][ni]);
    }
    // keep the next step's fragment reads after this step's MFMAs (register pressure)
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Token rows of one chunk (64 MT tokens): piece p = tid + 512 h (h < MT) is
// token p / 8, columns 8 (p % 8) .. + 7 of the chunk.
template <int MT>
__device__ __forceinline__ void dg_load_rows(uint4 (&x)[MT], rsrc_t r, int tid, int t0, int M, uint32_t row_len,
                                             uint32_t k0, bool live) {
#pragma unroll
  for (int h = 0; h < MT; ++h) {
    const int p = tid + h * kDgThreads, t = t0 + (p >> 3);
    x[h] = buf_ld16c(r, (live && t < M) ? ((uint32_t)t * row_len + k0 + (uint32_t)(p & 7) * 8u) * 2u : kOffNone, 0);
  }
}

template <int MT>
__device__ __forceinline__ void dg_store_rows(_Float16* As, const uint4 (&x)[MT], int tid) {
#pragma unroll
  for (int h = 0; h < MT; ++h) {
    const int p = tid + h * kDgThreads;
    *reinterpret_cast<uint4*>(As + (p >> 3) * kDgRow + (p & 7) * 8) = x[h];
  }
}

// Staging schedule shared by both GEMMs (chunks c_lo .. c_hi - 1, buffer c & 1):
// chunk c computes from LDS while chunk c + 1 is written to the other buffer
// from registers and chunk c + 2 is loaded into registers, so each global
// load has a whole chunk of MFMAs to arrive; unrolled by two so the register
// stages are named.
template <int MT, typename LoadX, typename LoadW, typename StoreX, typename StoreW, typename Mma>
__device__ __forceinline__ void dg_pipeline(int c_lo, int c_hi, LoadX load_x, LoadW load_w, StoreX store_x,
                                            StoreW store_w, Mma mma) {
  uint4 X0[MT], X1[MT];
  DgW W0, W1;
  load_x(X0, c_lo);
  load_w(W0, c_lo);
  load_x(X1, c_lo + 1);
  load_w(W1, c_lo + 1);
  __syncthreads();  // code tables
  store_x(0, X0);
  store_w(0, W0);
  load_x(X0, c_lo + 2);
  load_w(W0, c_lo + 2);
  __syncthreads();
  for (int c = c_lo; c < c_hi; c += 2) {
    mma(0);
    store_x(1, X1);
    store_w(1, W1);
    load_x(X1, c + 3);
    load_w(W1, c + 3);
    __syncthreads();
    if (c + 1 < c_hi) mma(1);  // uniform
    store_x(0, X0);
    store_w(0, W0);
    load_x(X0, c + 4);
    load_w(W0, c + 4);
    __syncthreads();
  }
}

// Weight staging of the gate/up kernel in pairs of chunks: a row's 128
// columns of a pair are 64 contiguous bytes of packed NF4, read by 4
// consecutive lanes (a load that reads 32 bytes of each row per chunk runs at
// a lower rate).  Load j of lane l takes staged row 16 w + 128 j + l / 4 and
// 16-byte segment (l % 4) ^ 2 j of that row's 64 bytes, i.e. chunk
// ((l % 4) / 2) ^ j of the pair, columns 32 (l % 2) .. + 31: every lane
// decodes one piece per chunk.
struct DgPair {
  uint4 w[2];
  float am[2];     // fp32 absmax, or the absmax2 (double-quantised)
  uint32_t qa[2];  // u8 absmax codes (double-quantised)
};

template <bool DQ, int MT>
__global__ void __launch_bounds__(kDgThreads, 2) k_dg_gu(DenseGuardArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dg_lds[];
  _Float16* As = reinterpret_cast<_Float16*>(dg_lds);  // [2][256][72] token rows
  _Float16* Bs = As + 2 * kDgStage;                      // [2][256][72] gate rows 0-127, up rows 128-255
  float2* cp = reinterpret_cast<float2*>(Bs + 2 * kDgStage);  // [2][256 x 2] gate, up code pairs
  float* c2s = reinterpret_cast<float*>(cp + 1024);           // [2][256] second-level code books
  const DecodeArgs& d = g.d;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = blockIdx.x, t0 = g.t_base + (int)blockIdx.y * 64 * MT;
  const int H = d.H, I = d.NB * 32, M = g.M;
  dg_pairs(cp, d.code, tid, 2);
  dg_pairs(cp + 512, d.code_up, tid, 2);
  if constexpr (DQ) c2s[tid] = (tid < 256 ? d.gate.code2 : d.up.code2)[tid & 255];
  // load j of this wave: staged rows 16 wave + 128 j .. + 15, all in block
  // 4 nt + wave / 2 of the gate (j = 0) or up (j = 1) projection, so each
  // load's block and buffer descriptors are uniform over the wave
  const uint32_t rs = (uint32_t)d.gate.row_stride, A = (uint32_t)d.gate.abs_row_stride;
  const uint32_t wrow = (uint32_t)((16 * wave + (lane >> 2)) & 31);  // row inside the block
  const int u = (lane & 3) >> 1, half = lane & 1;
  const int blk = 4 * nt + (wave >> 1);
  const BlockRef br = resolve_id(d, blk);
  if (!br.ok && lane == 0) atomicOr(d.status, 1);
  rsrc_t rw[2], ra[2], r2[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const ProjView& pv = jj ? d.up : d.gate;
    const ProjView& hv = jj ? d.host_up : d.host_gate;
    rw[jj] = make_rsrc((br.dev ? pv.packed : hv.packed) + br.q * pv.blk_stride, br.ok ? (int)(32 * rs) : 0);
    if constexpr (DQ) {
      ra[jj] = make_rsrc((br.dev ? pv.qabsmax : hv.qabsmax) + br.q * pv.abs_blk_stride, br.ok ? (int)(32 * A) : 0);
      r2[jj] = make_rsrc(pv.absmax2,
                         br.ok ? (int)((((long long)I * A + (1 << d.dq_shift) - 1) >> d.dq_shift) * 4) : 0);
    } else {
      ra[jj] = make_rsrc((br.dev ? pv.absmax : hv.absmax) + br.q * pv.abs_blk_stride, br.ok ? (int)(32 * A * 4) : 0);
      r2[jj] = ra[jj];
    }
  }
  const rsrc_t rx = make_rsrc(g.x, (int)((long long)M * H * 2));
  const int nch = H / kDgK, np = (nch + 1) / 2;
  auto load_x = [&](uint4 (&X)[MT], int c) {
    const bool live = c < nch;
    dg_load_rows(X, rx, tid, t0, M, (uint32_t)H, (uint32_t)(live ? c : 0) * kDgK, live);
  };
  auto load_p = [&](DgPair& P, int pr) {
    const bool live = pr < np;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const uint32_t seg = (uint32_t)((lane & 3) ^ (2 * jj));  // chunk seg / 2, half seg % 2
      const uint32_t col = (uint32_t)pr * 128u + seg * 32u;
      const bool ok = live && (int)col < H;
      const uint32_t ce = col >> d.qbs_shift;
      P.w[jj] = buf_ld16(rw[jj], ok ? wrow * rs + (col >> 1) : kOffNone, 0);
      if constexpr (DQ) {
        P.qa[jj] = buf_ldu8(ra[jj], ok ? ((wrow >> 1) * A + ce) * 2u + (wrow & 1u) : kOffNone, 0);
        const uint32_t f = (32u * (uint32_t)blk + wrow) * A + ce;
        P.am[jj] = buf_ldfc(r2[jj], ok ? (f >> d.dq_shift) * 4u : kOffNone, 0);
      } else {
        P.qa[jj] = 0;
        P.am[jj] = buf_ldf(ra[jj], ok ? (wrow * A + ce) * 4u : kOffNone, 0);
      }
    }
  };
  // chunk k of a pair into buffer bi: this lane's piece jj = k ^ u (gate for
  // jj = 0, up for jj = 1)
  auto decode = [&](int bi, const DgPair& P, int k) {
    const bool up = (k ^ u) != 0;
    const uint4 w = up ? P.w[1] : P.w[0];
    float am = up ? P.am[1] : P.am[0];
    if constexpr (DQ) am = dq_absmax(c2s[(up ? 256 : 0) + (up ? P.qa[1] : P.qa[0])], am, up ? d.up.offset : d.gate.offset);
    const int row = 16 * wave + (up ? 128 : 0) + (lane >> 2);
    dg_decode32<2>(Bs + bi * kDgStage + row * kDgRow + 32 * half, w, am, cp + (up ? 512 : 0) + (lane & 1));
  };
  auto store_x = [&](int bi, const uint4 (&X)[MT]) { dg_store_rows<MT>(As + bi * kDgStage, X, tid); };
  const int mq = wave & 3, nh = wave >> 2;
  auto brow = [nh](int ni) { return (ni < 4 ? 0 : 128) + 64 * nh + 16 * (ni & 3); };
  float4_t acc[MT][8];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int ni = 0; ni < 8; ++ni) acc[mi][ni] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  uint4 X[2][MT];
  DgPair P[2];
  load_p(P[0], 0);
  load_p(P[1], 1);
  load_x(X[0], 0);
  load_x(X[1], 1);
  __syncthreads();  // code tables
  store_x(0, X[0]);
  decode(0, P[0], 0);
  load_x(X[0], 2);
  __syncthreads();
  // chunk c computes from buffer c & 1 while chunk c + 1 is staged into the
  // other buffer (token rows from registers, weights decoded from the pair
  // registers) and chunk c + 3's token rows are loaded; a pair's registers
  // are reloaded with the pair after next once its second chunk is decoded.
  // Unrolled by 4 chunks so every register index is static.
  for (int c = 0; c < nch; c += 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cc = c + i;
      if (cc < nch) dg_mma(acc, As + (i & 1) * kDgStage, Bs + (i & 1) * kDgStage, mq, lane, brow);  // uniform
      const int nb = (i + 1) & 1;
      store_x(nb, X[nb]);
      decode(nb, P[((i + 1) >> 1) & 1], (i + 1) & 1);
      load_x(X[nb], cc + 3);
      if (((i + 1) & 1) == 1) load_p(P[((i + 1) >> 1) & 1], ((cc + 1) >> 1) + 2);
      __syncthreads();
    }
  }
  mfma_drain();
  // act = fp16(fp16(silu(fp16(g))) * fp16(u)) for (token, row)
  const int j = lane & 15, gq = lane >> 4;
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int t = t0 + 16 * MT * mq + 16 * mi + 4 * gq + rr;
      if (t < M) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
          const float g16 = h2f(f2h(acc[mi][ni][rr]));
          const float s16 = h2f(f2h(g16 / (1.0f + expf(-g16))));
          const float u16 = h2f(f2h(acc[mi][4 + ni][rr]));
          g.act[(long long)t * I + 128 * nt + 64 * nh + 16 * ni + j] = f2h(s16 * u16);
        }
      }
    }
  }
}

template <bool DQ, int MT>
__global__ void __launch_bounds__(kDgThreads, 2) k_dg_down(DenseGuardArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dg_lds[];
  _Float16* As = reinterpret_cast<_Float16*>(dg_lds);  // [2][256][72] act rows
  _Float16* Bs = As + 2 * kDgStage;                      // [2][256][72] down rows
  float2* cp = reinterpret_cast<float2*>(Bs + 2 * kDgStage);  // [256 x 4] down code pairs
  float* c2s = reinterpret_cast<float*>(cp + 1024);
  const DecodeArgs& d = g.d;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = d.H, NB = d.NB, I = NB * 32, M = g.M, S = g.S;
  const int ntiles = H / 256;
  // XCD-aware: the workgroups of one block range (which read the same act
  // columns) share XCDs when the grid allows it
  int nt, s;
  if (S * ntiles == 256 && S <= 8 && 8 % S == 0) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per = 8 / S;
    s = xcd / per;
    nt = (xcd % per) * 32 + slot;
  } else {
    nt = blockIdx.x % ntiles;
    s = blockIdx.x / ntiles;
  }
  const int t0 = g.t_base + (int)blockIdx.y * 64 * MT, o0 = nt * 256;
  const int C = NB / 2;  // chunks of two blocks
  const int c_lo = (int)((long long)s * C / S), c_hi = (int)((long long)(s + 1) * C / S);
  dg_pairs(cp, d.code_down, tid, 4);
  dg_pairs(cp, d.code_down, tid + 512, 4);
  if constexpr (DQ) {
    if (tid < 256) c2s[tid] = d.down.code2[tid];
  }
  // staged down row o = o0 + tid % 256 of block 2 c + tid / 256 (uniform over the wave)
  const int orow = tid & 255, hb = wave >> 2;
  const uint32_t o = (uint32_t)(o0 + orow);
  const uint32_t Ad = (uint32_t)I >> d.qbs_shift;
  const bool have_host = d.host_down.packed != nullptr;
  const rsrc_t rx = make_rsrc(g.act, (int)((long long)M * I * 2));
  const rsrc_t r2 = DQ ? make_rsrc(d.down.absmax2, (int)((((long long)H * Ad + (1 << d.dq_shift) - 1) >> d.dq_shift) * 4))
                       : rx;
  auto load_x = [&](uint4 (&X)[MT], int c) {
    const bool live = c < c_hi;
    dg_load_rows(X, rx, tid, t0, M, (uint32_t)I, (uint32_t)(live ? c : c_lo) * kDgK, live);
  };
  auto load_w = [&](DgW& W, int c) {
    const bool live = c < c_hi;
    const int b = 2 * (live ? c : c_lo) + hb;
    const int slot = d.lookup ? d.lookup[b] : b;
    const bool dev = slot >= 0;
    const bool used = g.offsets == nullptr || g.offsets[b + 1] > g.offsets[b];
    const bool ok = live && used && (dev ? slot < d.n_slots : have_host);
    const long long q = ok ? (dev ? slot : b) : 0;
    const rsrc_t rw = make_rsrc((dev ? d.down.packed : d.host_down.packed) + q * d.down.blk_stride, ok ? H * 16 : 0);
    W.w = buf_ld16(rw, o * 16u, 0);
    if constexpr (DQ) {
      const rsrc_t ra = make_rsrc((dev ? d.down.qabsmax : d.host_down.qabsmax) + q * d.down.abs_blk_stride, ok ? H : 0);
      W.qa = buf_ldu8(ra, o, 0);
      const uint32_t f = o * Ad + ((32u * (uint32_t)b) >> d.qbs_shift);
      W.am = buf_ldfc(r2, ok ? (f >> d.dq_shift) * 4u : kOffNone, 0);
    } else {
      const rsrc_t ra = make_rsrc((dev ? d.down.absmax : d.host_down.absmax) + q * d.down.abs_blk_stride,
                                  ok ? H * 4 : 0);
      W.qa = 0;
      W.am = buf_ldf(ra, o * 4u, 0);
    }
  };
  auto store_x = [&](int bi, const uint4 (&X)[MT]) { dg_store_rows<MT>(As + bi * kDgStage, X, tid); };
  auto store_w = [&](int bi, const DgW& W) {
    float am = W.am;
    if constexpr (DQ) am = dq_absmax(c2s[W.qa], W.am, d.down.offset);
    dg_decode32<4>(Bs + bi * kDgStage + orow * kDgRow + 32 * hb, W.w, am, cp + (lane & 3));
  };
  const int mq = wave & 3, nh = wave >> 2;
  auto brow = [nh](int ni) { return 128 * nh + 16 * ni; };
  float4_t acc[MT][8];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int ni = 0; ni < 8; ++ni) acc[mi][ni] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  auto mma = [&](int bi) { dg_mma(acc, As + bi * kDgStage, Bs + bi * kDgStage, mq, lane, brow); };
  dg_pipeline<MT>(c_lo, c_hi, load_x, load_w, store_x, store_w, mma);
  mfma_drain();
  const int j = lane & 15, gq = lane >> 4;
  float* part = g.part + (long long)s * M * H;
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int t = t0 + 16 * MT * mq + 16 * mi + 4 * gq + rr;
      if (t < M) {
#pragma unroll
        for (int ni = 0; ni < 8; ++ni) part[(long long)t * H + o0 + 128 * nh + 16 * ni + j] = acc[mi][ni][rr];
      }
    }
  }
}

// y = fp16(sum_s part[s] + bias) (+ residual: fp16(residual + y))
__global__ void __launch_bounds__(256) k_dg_fin(DenseGuardArgs g) {
  const long long n = (long long)g.M * g.d.H;
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float y = 0.0f;
  for (int s = 0; s < g.S; ++s) y += g.part[(long long)s * n + i];
  const int o = (int)(i % g.d.H);
  if (g.d.down_bias != nullptr) y += h2f(g.d.down_bias[o]);
  uint16_t h = f2h(y);
  if (g.residual != nullptr) h = f2h(h2f(g.residual[i]) + h2f(h));
  g.out[i] = h;
}

using DgFn = void (*)(DenseGuardArgs);
// [dq][MT - 1 of the 64 MT-token tile]
const DgFn kDgGu[2][4] = {{k_dg_gu<false, 1>, k_dg_gu<false, 2>, k_dg_gu<false, 3>, k_dg_gu<false, 4>},
                          {k_dg_gu<true, 1>, k_dg_gu<true, 2>, k_dg_gu<true, 3>, k_dg_gu<true, 4>}};
const DgFn kDgDown[2][4] = {{k_dg_down<false, 1>, k_dg_down<false, 2>, k_dg_down<false, 3>, k_dg_down<false, 4>},
                            {k_dg_down<true, 1>, k_dg_down<true, 2>, k_dg_down<true, 3>, k_dg_down<true, 4>}};

// Token tiles: whole 256-token tiles, then the rest of the prompt in the
// smallest tile of 64, 128 or 192 tokens that holds it (a 256-token tile would
// spend its MFMAs and token-row staging on padding): one launch per tile size.
template <typename Launch>
void dg_token_tiles(const DenseGuardArgs& g, Launch launch) {
  const int full = g.M / kDgTok, rest = g.M - full * kDgTok;
  DenseGuardArgs a = g;
  if (full > 0) {
    a.t_base = 0;
    launch(a, 3, full);
  }
  if (rest > 0) {
    a.t_base = full * kDgTok;
    launch(a, (rest + 63) / 64 - 1, 1);
  }
}

void dg_set_lds() {
  static std::once_flag once;
  std::call_once(once, [] {
    for (int q = 0; q < 2; ++q)
      for (int m = 0; m < 4; ++m) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kDgGu[q][m]),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDgLds);
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kDgDown[q][m]),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDgLds);
      }
  });
}

}  // namespace

void launch_dense_down(const DenseGuardArgs& g, hipStream_t st) {
  dg_set_lds();
  dg_token_tiles(g, [&](const DenseGuardArgs& a, int mt_idx, int tiles) {
    kDgDown[a.d.dq ? 1 : 0][mt_idx]<<<dim3((unsigned)(a.d.H / 256 * a.S), (unsigned)tiles), dim3(kDgThreads), kDgLds,
                                      st>>>(a);
  });
  const long long n = (long long)g.M * g.d.H;
  k_dg_fin<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(g);
}

void launch_dense_guard(const DenseGuardArgs& g, hipStream_t st) {
  dg_set_lds();
  dg_token_tiles(g, [&](const DenseGuardArgs& a, int mt_idx, int tiles) {
    kDgGu[a.d.dq ? 1 : 0][mt_idx]<<<dim3((unsigned)(a.d.NB / 4), (unsigned)tiles), dim3(kDgThreads), kDgLds, st>>>(a);
  });
  launch_dense_down(g, st);
}

}  // namespace nsmlp
