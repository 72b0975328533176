// Streaming sparse-MLP decode for hidden sizes that are a multiple of 2048
// (one wave covers a 2048-column split: 64 lanes x 32 columns).
//
//   k_gu_rep    gate/up.  An 8-wave workgroup works in rounds; in a round every
//               wave decodes one item: gate rows 2p, 2p+1 and up rows 2p, 2p+1
//               of one selected block over the wave's split (4 x 1 KB of
//               packed NF4, 16 bytes per lane and row), the token's split held
//               in registers as fp16 pairs.  Items stream through a register
//               pipeline of kGuStages rounds.  Each wave reduces its 4 row sums
//               over its lanes into LDS slots of its own for that round, so
//               the waves never wait for each other during the stream; after
//               the last round one barrier joins them and silu(gate) * up of
//               every round's rows 2p, 2p+1 is written (fp32, splits added in
//               order).  Gate/up biases and the flat
//               mask are applied there, in a separate instantiation, so that
//               the plain path has no loads outside the weight stream.  The
//               kernel also publishes the resolved block references.
//   k_down_rep  down.  A workgroup owns 64 output rows (one per lane) and one
//               group of selected blocks, split over its 8 waves.  It turns
//               the group's activations into fp16 pairs scaled by a power of
//               two per block (max |act| in [0.5, 1)), then every wave streams
//               2-block items (16 packed bytes and one absmax per row and
//               block) through a register pipeline, accumulating in fp32 in
//               block order; the 8 wave sums meet in LDS (wave order).  When
//               the 64-row chunks alone give a workgroup per CU (one group),
//               the workgroup writes the fp16 output itself; otherwise it
//               writes a partial and k_fin_rep adds the groups in order.
//
// Weights are read with buffer loads through a per-block descriptor whose
// extent is zero for an invalid block or a round past the end: such a load
// returns zeros without touching memory, so every load in the stream is
// unconditional and the compiler's wait counts stay exact (a branch around a
// load would make it wait for the whole pipeline).  Both streaming kernels
// decode through the lane-replicated byte-pair table (64 KB of dynamic LDS at
// address 0; no static LDS in these kernels), filled with 16-byte LDS writes
// while the first weight loads are in flight.  Block references are resolved
// once, lane i holding item i, and read with v_readlane per item, so no
// dependent lookups sit in the stream.
#include <mutex>

#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

constexpr int kSplit = 2048;               // columns per split
constexpr int kWaves = 8;                  // waves per workgroup
constexpr int kThreads8 = kWaves * kWave;  // 512
constexpr int kGuStages = 2;
constexpr int kDnStages = 2;
constexpr int kMaxItems = 64;      // items per wave resolved up front (one per lane)
constexpr int kMaxDnBlocks = 512;  // blocks per down workgroup (activations in LDS)
constexpr int kLutWords = kRepLutBytes / 4;
// dynamic LDS: table, split sums of every round [kMaxItems][8][4] and the
// validity of every round's item [kMaxItems][8]; with double-quantised absmax
// the gate and up second-level code books [2][256]; with the in-kernel top-k
// also the selection state and the selected ids [k]
constexpr int kGuOkWord = kLutWords + kMaxItems * kWaves * 4;
constexpr int kGuCode2Word = kGuOkWord + kMaxItems * kWaves;
constexpr size_t kGuLds = (size_t)kGuCode2Word * 4;
constexpr size_t kGuDqLds = kGuLds + 2 * 256 * sizeof(float);
constexpr int kGuTopkWord = (int)(kGuDqLds / 4);
constexpr int kGuSelWord = kGuTopkWord + (int)((sizeof(TopkLds) + 15) / 16 * 4);
constexpr int kSelMaxNB = 4096;  // 8 scores per thread
constexpr int kSelMaxK = 2048;
constexpr size_t kGuSelLds = (size_t)kGuSelWord * 4 + kSelMaxK * sizeof(int32_t);
// dynamic LDS: table, activation pairs [512][16], scales [512], wave sums
// [8][64]; with double-quantised absmax also the down code book [256] and the
// absmax2 entries of the workgroup's 64 rows [kDnA2Max]
constexpr size_t kDnLds = kRepLutBytes + kMaxDnBlocks * 16 * 4 + kMaxDnBlocks * 4 + kWaves * kWave * 4;
constexpr int kDnA2Max = 1024;
constexpr size_t kDnDqLds = kDnLds + (256 + kDnA2Max) * sizeof(float);

// Encoded block reference: < 2^30 -> HBM slot; bit 30 -> host copy of the
// block id in the low bits; bit 31 -> invalid (zero contribution).
constexpr uint32_t kHostBit = 0x40000000u;
constexpr uint32_t kBad = 0x80000000u;

__device__ __forceinline__ uint32_t encode_ref(const BlockRef& br) {
  if (!br.ok) return kBad;
  return br.dev ? (uint32_t)br.q : (kHostBit | (uint32_t)br.q);
}

__device__ __forceinline__ uint32_t lane_value(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}

// Replicated pair table, filled by 512 threads in 8 passes of one 16-byte LDS
// write each: pass ps writes entry e = 32 ps + tid / 16, copies 4 (tid % 16)
// .. +3 (copies 0..31 decode code_a, 32..63 code_b).  The entry's low half is
// the code of its high nibble (e / 16 = 2 ps + tid / 256), the high half the
// code of its low nibble ((tid / 16) % 16).
struct LutCodes {
  float lo[8];
  float hi;
};

__device__ __forceinline__ void lut_codes_load(const float* code_a, const float* code_b, int tid, LutCodes& c) {
  const float* code = (tid & 15) >= 8 ? code_b : code_a;
#pragma unroll
  for (int ps = 0; ps < 8; ++ps) c.lo[ps] = code[2 * ps + (tid >> 8)];
  c.hi = code[(tid >> 4) & 15];
}

__device__ __forceinline__ void lut_store(uint32_t* lut, const LutCodes& c, int tid) {
  const uint32_t hi = (uint32_t)f2h(c.hi) << 16;
#pragma unroll
  for (int ps = 0; ps < 8; ++ps) {
    const uint32_t v = (uint32_t)f2h(c.lo[ps]) | hi;
    const int e = ps * 32 + (tid >> 4);
    *reinterpret_cast<uint4*>(lut + e * 64 + (tid & 15) * 4) = make_uint4(v, v, v, v);
  }
}

struct GuStage {
  uint4 w[4];      // gate 2p, gate 2p+1, up 2p, up 2p+1: this lane's 32 columns
  float am[4];     // fp32 absmax of the four rows
  uint32_t qa[2];  // double-quantised: u8 codes of gate rows 2p | 2p+1 << 8, same for up
};

// Issue the loads of one item (block reference enc, row pair p).  ca: this
// lane's absmax entry inside a row (its columns / qbs); cb: its byte offset
// inside a packed row.
template <bool DQ>
__device__ __forceinline__ void gu_issue(const DecodeArgs& a, uint32_t enc, int p, uint32_t cb, uint32_t ca,
                                         GuStage& st) {
  const bool bad = (enc & kBad) != 0;
  const bool dev = (enc & kHostBit) == 0;
  const long long q = bad ? 0 : (long long)(enc & (kHostBit - 1));
  const int nb = bad ? 0 : a.st_gu_bytes, na = bad ? 0 : a.st_gu_abytes;
  const rsrc_t rg = make_rsrc((dev ? a.gate.packed : a.host_gate.packed) + q * a.gate.blk_stride, nb);
  const rsrc_t ru = make_rsrc((dev ? a.up.packed : a.host_up.packed) + q * a.up.blk_stride, nb);
  const uint32_t rs = (uint32_t)a.gate.row_stride, ars = (uint32_t)a.gate.abs_row_stride;
  const uint32_t s0 = (uint32_t)(2 * p) * rs;
  st.w[0] = buf_ld16(rg, cb, s0);
  st.w[1] = buf_ld16(rg, cb, s0 + rs);
  st.w[2] = buf_ld16(ru, cb, s0);
  st.w[3] = buf_ld16(ru, cb, s0 + rs);
  if constexpr (DQ) {
    // codes of rows 2p and 2p+1 at entry ca: one 16-bit read per projection
    const rsrc_t rgq = make_rsrc((dev ? a.gate.qabsmax : a.host_gate.qabsmax) + q * a.gate.abs_blk_stride, na);
    const rsrc_t ruq = make_rsrc((dev ? a.up.qabsmax : a.host_up.qabsmax) + q * a.up.abs_blk_stride, na);
    const uint32_t qo = ((uint32_t)p * ars + ca) * 2u;
    st.qa[0] = buf_ldu16(rgq, qo, 0);
    st.qa[1] = buf_ldu16(ruq, qo, 0);
  } else {
    const rsrc_t rga = make_rsrc((dev ? a.gate.absmax : a.host_gate.absmax) + q * a.gate.abs_blk_stride, na);
    const rsrc_t rua = make_rsrc((dev ? a.up.absmax : a.host_up.absmax) + q * a.up.abs_blk_stride, na);
    const uint32_t ars4 = ars * 4u, as0 = (uint32_t)(2 * p) * ars4, ca4 = ca * 4u;
    st.am[0] = buf_ldf(rga, ca4, as0);
    st.am[1] = buf_ldf(rga, ca4, as0 + ars4);
    st.am[2] = buf_ldf(rua, ca4, as0);
    st.am[3] = buf_ldf(rua, ca4, as0 + ars4);
  }
}

// The absmax of row i of a gate/up stage; a2: the item's absmax2 of the row
// (double-quantised).
template <bool DQ>
__device__ __forceinline__ float gu_absmax(const DecodeArgs& a, const GuStage& st, const float* c2, int i, float a2) {
  if constexpr (DQ) {
    const uint32_t q = (st.qa[i >> 1] >> (8 * (i & 1))) & 0xFFu;
    return dq_absmax(c2[(i >= 2 ? 256 : 0) + q], a2, i >= 2 ? a.up.offset : a.gate.offset);
  } else {
    return st.am[i];
  }
}

// Reduce-scatter of 4 per-lane row sums over the 64 lanes: afterwards every
// lane holds the full sum of row (lane >> 4) & 3.
__device__ __forceinline__ float reduce4(const float (&v)[4], int lane) {
  const bool b5 = lane & 32, b4 = lane & 16;
  const float s0 = b5 ? v[0] : v[2], s1 = b5 ? v[1] : v[3];
  float k0 = b5 ? v[2] : v[0], k1 = b5 ? v[3] : v[1];
  k0 += __shfl_xor(s0, 32, kWave);
  k1 += __shfl_xor(s1, 32, kWave);
  const float s = b4 ? k0 : k1;
  float k = b4 ? k1 : k0;
  k += __shfl_xor(s, 16, kWave);
  k += __shfl_xor(k, 8, kWave);
  k += __shfl_xor(k, 4, kWave);
  k += __shfl_xor(k, 2, kWave);
  k += __shfl_xor(k, 1, kWave);
  return k;
}

// Kernel arguments are read from memory, and the compiler loads each field
// where it is first used: a field first used after a global load that it waits
// for costs a round trip of its own (the gate/up kernel had two before its
// first loads and three between the selection and its weight stream).  The
// kernels therefore pass their fields through empty asm statements ("+s":
// the field must be loaded before the statement, and its value afterwards is
// opaque, so it stays in SGPRs instead of being loaded again) in two batches:
// those the first global loads need, at the start, and the rest right after
// those loads are issued (behind a scheduling fence), so that their round
// trip overlaps the loads'.  Pointers go through as global pointers (through
// a generic pointer the loads would be flat loads, which also count as LDS
// operations in the wait counters).
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gptr(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

// Gate/up, first batch: the token, the selection or scores, the code books.
__device__ __forceinline__ void pin_gu_first(DecodeArgs& a, int& nwg) {
  nwg = (int)gridDim.x;
  auto x = gptr(a.x);
  auto sel = gptr(a.sel);
  auto sel_scores = gptr(a.sel_scores);
  auto code = gptr(a.code), code_up = gptr(a.code_up);
  auto gc2 = gptr(a.gate.code2), uc2 = gptr(a.up.code2);
  asm volatile(""
               : "+s"(nwg), "+s"(x), "+s"(sel), "+s"(sel_scores), "+s"(code), "+s"(code_up), "+s"(gc2), "+s"(uc2),
                 "+s"(a.splits), "+s"(a.NB), "+s"(a.k), "+s"(a.st_gu_rounds));
  a.x = (const uint16_t*)x;
  a.sel = (const int32_t*)sel;
  a.sel_scores = (const uint16_t*)sel_scores;
  a.code = (const float*)code;
  a.code_up = (const float*)code_up;
  a.gate.code2 = (const float*)gc2;
  a.up.code2 = (const float*)uc2;
}

// Gate/up, second batch: block references, weight views, workspace.
template <bool DQ>
__device__ __forceinline__ void pin_gu_rest(DecodeArgs& a) {
  auto sel_out = gptr(a.sel_out);
  auto lookup = gptr(a.lookup);
  auto status = gptr(a.status);
  auto st_enc = gptr(a.st_enc);
  auto st_bid = gptr(a.st_bid);
  auto st_act = gptr(a.st_act);
  auto gp = gptr(a.gate.packed), up = gptr(a.up.packed);
  auto hgp = gptr(a.host_gate.packed), hup = gptr(a.host_up.packed);
  auto ga = gptr(DQ ? a.gate.qabsmax : reinterpret_cast<const uint8_t*>(a.gate.absmax));
  auto ua = gptr(DQ ? a.up.qabsmax : reinterpret_cast<const uint8_t*>(a.up.absmax));
  auto hga = gptr(DQ ? a.host_gate.qabsmax : reinterpret_cast<const uint8_t*>(a.host_gate.absmax));
  auto hua = gptr(DQ ? a.host_up.qabsmax : reinterpret_cast<const uint8_t*>(a.host_up.absmax));
  auto g2 = gptr(a.gate.absmax2), u2 = gptr(a.up.absmax2);
  asm volatile(""
               : "+s"(sel_out), "+s"(lookup), "+s"(status), "+s"(st_enc), "+s"(st_bid), "+s"(st_act), "+s"(gp),
                 "+s"(up), "+s"(hgp), "+s"(hup), "+s"(ga), "+s"(ua), "+s"(hga), "+s"(hua), "+s"(g2), "+s"(u2),
                 "+s"(a.n_slots), "+s"(a.skip_negative), "+s"(a.st_gu_bytes), "+s"(a.st_gu_abytes),
                 "+s"(a.gate.blk_stride), "+s"(a.up.blk_stride), "+s"(a.gate.row_stride), "+s"(a.gate.abs_blk_stride),
                 "+s"(a.up.abs_blk_stride), "+s"(a.gate.abs_row_stride), "+s"(a.gate.offset), "+s"(a.up.offset),
                 "+s"(a.qbs_shift), "+s"(a.dq_shift));
  a.sel_out = (int32_t*)sel_out;
  a.lookup = (const int32_t*)lookup;
  a.status = (int*)status;
  a.st_enc = (uint32_t*)st_enc;
  a.st_bid = (int32_t*)st_bid;
  a.st_act = (float*)st_act;
  a.gate.packed = (const uint8_t*)gp;
  a.up.packed = (const uint8_t*)up;
  a.host_gate.packed = (const uint8_t*)hgp;
  a.host_up.packed = (const uint8_t*)hup;
  if constexpr (DQ) {
    a.gate.qabsmax = (const uint8_t*)ga;
    a.up.qabsmax = (const uint8_t*)ua;
    a.host_gate.qabsmax = (const uint8_t*)hga;
    a.host_up.qabsmax = (const uint8_t*)hua;
  } else {
    a.gate.absmax = (const float*)ga;
    a.up.absmax = (const float*)ua;
    a.host_gate.absmax = (const float*)hga;
    a.host_up.absmax = (const float*)hua;
  }
  a.gate.absmax2 = (const float*)g2;
  a.up.absmax2 = (const float*)u2;
  auto served = gptr(a.served);
  asm volatile("" : "+s"(served));
  a.served = (uint32_t*)served;
}

// SKPT > 0: the workgroup first selects the top k of a.sel_scores itself (SKPT
// scores per thread; ascending ids, ties to the lower id), so the selection
// needs no launch of its own; workgroup 0 also writes the ids to a.sel_out.
template <bool AFFINE, int SKPT, bool DQ>
__global__ void __launch_bounds__(kThreads8, 2) k_gu_rep(DecodeArgs args) {
  DecodeArgs a = args;
  int nwg;
  pin_gu_first(a, nwg);
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  float* comb = reinterpret_cast<float*>(lds + kLutWords);
  int* okl = reinterpret_cast<int*>(lds + kGuOkWord);
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
  const int S = a.splits;                                     // 1, 2, 4 or 8
  const int sh = __builtin_ctz((unsigned)S);  // S is a power of two
  const int NS = kWaves >> sh;
  const int s = wave & (S - 1), q = wave >> sh;
  const int R = a.st_gu_rounds;
  const int wg = (int)blockIdx.x;
  const int n_items = 16 * a.k;
  const uint32_t col = (uint32_t)(s * kSplit + lane * 32);
  const uint32_t cb = col >> 1, ca = col >> a.qbs_shift;
  const float* c2 = reinterpret_cast<const float*>(lds + kGuCode2Word);

  // Independent loads first: the block id of each lane's item (lane i:
  // round i), the code book and the token split.
  const int id0 = (lane * nwg + wg) * NS + q;
  const bool own = lane < R && id0 < n_items;
  const int jb = own ? id0 >> 4 : 0;
  int b_id = 0;
  constexpr int kKeys = SKPT > 0 ? SKPT : 1;
  uint32_t skey[kKeys];
  const int i0 = tid * kKeys;
  if constexpr (SKPT == 0) {
    b_id = a.sel ? a.sel[jb] : jb;
  } else {
#pragma unroll
    for (int m = 0; m < SKPT; ++m) {
      const int i = i0 + m < a.NB ? i0 + m : a.NB - 1;  // clamped: the load is unconditional
      skey[m] = f16_order_key(a.sel_scores[i]);
    }
  }
  LutCodes codes;
  lut_codes_load(a.code, a.code_up, tid, codes);
  float c2v = 0.0f;
  if constexpr (DQ) c2v = (tid < 256 ? a.gate.code2 : a.up.code2)[tid & 255];
  uint32_t xp[16];
  {
    const uint4* xv = reinterpret_cast<const uint4*>(a.x + col);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint4 t = xv[v];
      xp[4 * v] = t.x;
      xp[4 * v + 1] = t.y;
      xp[4 * v + 2] = t.z;
      xp[4 * v + 3] = t.w;
    }
  }
  sched_fence();
  pin_gu_rest<DQ>(a);
  int32_t* sel_l = reinterpret_cast<int32_t*>(lds + kGuSelWord);
  if constexpr (SKPT > 0) {
    TopkLds& tl = *reinterpret_cast<TopkLds*>(lds + kGuTopkWord);
    topk_clear<kThreads8>(tl);  // while the scores are loaded
    lds_barrier();
    uint32_t T;
    unsigned need, gt, eq;
    topk_threshold<kThreads8, SKPT>(skey, i0, a.NB, a.k, tl, T, need, gt, eq);
    // keys past NB are padding (the last thread's, after its real keys): the
    // counts they add come after every real key
#pragma unroll
    for (int m = 0; m < SKPT; ++m) {
      const int pos = topk_position(skey[m], T, need, gt, eq);
      gt += skey[m] > T;
      eq += skey[m] == T;
      if (i0 + m < a.NB && pos >= 0 && pos < a.k) sel_l[pos] = i0 + m;
    }
    lds_barrier();
    b_id = sel_l[jb];
    if (wg == 0 && a.sel_out != nullptr)
      for (int j = tid; j < a.k; j += kThreads8) a.sel_out[j] = sel_l[j];
  }
  // Block references (slot lookup).  Split 0 of row pair 0 reports an
  // invalid block and publishes the reference for the down kernel.
  // enc_v / bid_v: lane i holds item i's block reference and block id (0
  // for an invalid block, so that index arithmetic on it stays in range)
  uint32_t enc_v = kBad, bid_v = 0;
  if (own) {
    const BlockRef br = resolve_id(a, b_id);
    enc_v = encode_ref(br);
    bid_v = br.ok ? (uint32_t)b_id : 0u;
    if (s == 0 && (id0 & 15) == 0) {
      if (!br.ok && !br.silent) atomicOr(a.status, 1);
      a.st_enc[id0 >> 4] = enc_v;
      a.st_bid[id0 >> 4] = (int32_t)bid_v;
    }
  }
  // double-quantised: lane i also holds item i's absmax2 of its four rows at
  // this wave's split (a 2048-column split never straddles a second-level
  // block), read once here instead of in the weight stream
  float a2_v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (DQ) {
    const uint32_t ars = (uint32_t)a.gate.abs_row_stride;
    const uint32_t f0 = (32u * bid_v + 2u * (uint32_t)(id0 & 15)) * ars + (uint32_t)(s * kSplit >> a.qbs_shift);
    const uint32_t g0 = f0 >> a.dq_shift, g1 = (f0 + ars) >> a.dq_shift;
    a2_v[0] = a.gate.absmax2[g0];
    a2_v[1] = a.gate.absmax2[g1];
    a2_v[2] = a.up.absmax2[g0];
    a2_v[3] = a.up.absmax2[g1];
    sched_fence();  // before the weight stream: their wait then drains nothing of it
  }
  // The pipeline's stages go out first; the code table goes into LDS behind
  // them (its codes were loaded before them, so waiting for the codes drains
  // none of the stages) and one barrier publishes it.
  GuStage st[kGuStages];
#pragma unroll
  for (int i = 0; i < kGuStages; ++i)
    gu_issue<DQ>(a, i < R ? lane_value(enc_v, i) : kBad, ((i * nwg + wg) * NS + q) & 15, cb, ca, st[i]);
  sched_fence();
  // block-source counts (behind the stages: nothing waits for them early),
  // one per selected block: its row pair 0 at split 0
  if (a.served != nullptr && s == 0) {
    const bool first = own && (id0 & 15) == 0 && !(enc_v & kBad);
    const unsigned long long mh = __ballot(first && !(enc_v & kHostBit));
    const unsigned long long mc = __ballot(first && (enc_v & kHostBit));
    if (lane == 0) {
      if (mh) atomicAdd(a.served, (uint32_t)__popcll(mh));
      if (mc) atomicAdd(a.served + 1, (uint32_t)__popcll(mc));
    }
  }
  sched_fence();
  lut_store(lds, codes, tid);
  if constexpr (DQ) lds[kGuCode2Word + tid] = __float_as_uint(c2v);
  lds_barrier();

  uint32_t adg[4], adu[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    adg[i] = (uint32_t)(lane & 31) * 4u;
    adu[i] = 128u + (uint32_t)(lane & 31) * 4u;
  }

  for (int r0 = 0; r0 < R; r0 += kGuStages) {
#pragma unroll
    for (int i = 0; i < kGuStages; ++i) {
      const int r = r0 + i;
      const bool live = r < R;  // uniform over the workgroup
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (live) {
        float a2[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (DQ) {
#pragma unroll
          for (int m = 0; m < 4; ++m) a2[m] = __uint_as_float(lane_value(__float_as_uint(a2_v[m]), r));
        }
        acc[0] = rep_dot32(st[i].w[0], xp, adg) * gu_absmax<DQ>(a, st[i], c2, 0, a2[0]);
        acc[1] = rep_dot32(st[i].w[1], xp, adg) * gu_absmax<DQ>(a, st[i], c2, 1, a2[1]);
        acc[2] = rep_dot32(st[i].w[2], xp, adu) * gu_absmax<DQ>(a, st[i], c2, 2, a2[2]);
        acc[3] = rep_dot32(st[i].w[3], xp, adu) * gu_absmax<DQ>(a, st[i], c2, 3, a2[3]);
      }
      const int rn = r + kGuStages;
      const int rl = rn < R && rn < kMaxItems ? rn : 0;
      gu_issue<DQ>(a, rn < R ? lane_value(enc_v, rl) : kBad, ((rn * nwg + wg) * NS + q) & 15, cb, ca, st[i]);
      if (live) {
        const float v = reduce4(acc, lane);
        if ((lane & 15) == 0) comb[r * (kWaves * 4) + wave * 4 + (lane >> 4)] = v;
        if constexpr (AFFINE) {
          if (s == 0 && lane == 0) okl[r * kWaves + q] = !(lane_value(enc_v, r) & kBad);
        }
      }
    }
  }
  // The split sums of every round meet once, after the stream (each round
  // has its own LDS slots, so the waves never wait for each other before):
  // entry e = (round, item slot q, row of the pair); gate and up sums of row
  // 2p + (e & 1), splits added in order.
  lds_barrier();
  for (int e = tid; e < R * NS * 2; e += kThreads8) {
    const int ln = e & 1, qq = (e >> 1) % NS, r = (e >> 1) / NS;
    const int id = (r * nwg + wg) * NS + qq;
    if (id >= n_items) continue;
    const float* cs = comb + r * (kWaves * 4) + qq * S * 4;
    float g = 0.0f, u = 0.0f;
    for (int sp = 0; sp < S; ++sp) {
      g += cs[sp * 4 + ln];
      u += cs[sp * 4 + 2 + ln];
    }
    const int j = id >> 4;
    const int n = 2 * (id & 15) + ln;
    if constexpr (AFFINE) {
      if (okl[r * kWaves + qq]) {
        const int bj = SKPT > 0 ? sel_l[j] : (a.sel ? a.sel[j] : j);
        const long long bn = (long long)bj * 32 + n;
        if (a.gate_bias != nullptr) g += h2f(a.gate_bias[bn]);
        if (a.up_bias != nullptr) u += h2f(a.up_bias[bn]);
        if (a.mask != nullptr) {
          const float m = h2f(a.mask[bn]);
          g *= m;
          u *= m;
        }
      }
    }
    a.st_act[(long long)j * 32 + n] = silu_mul(g, u);
  }
}

struct DnStage {
  uint4 w[2];
  float am[2];     // absmax (fp32 absmax storage)
  uint32_t qa[2];  // u8 absmax code (double-quantised storage)
};

// aoff: this lane's absmax entry in a block (its row o).
template <bool DQ>
__device__ __forceinline__ void dn_issue(const DecodeArgs& a, uint32_t enc, uint32_t roff, uint32_t aoff, uint4& w,
                                         float& am, uint32_t& qa) {
  const bool bad = (enc & kBad) != 0;
  const bool dev = (enc & kHostBit) == 0;
  const long long q = bad ? 0 : (long long)(enc & (kHostBit - 1));
  const rsrc_t rp = make_rsrc((dev ? a.down.packed : a.host_down.packed) + q * a.down.blk_stride,
                              bad ? 0 : a.st_dn_bytes);
  w = buf_ld16(rp, roff, 0);
  if constexpr (DQ) {
    const rsrc_t ra = make_rsrc((dev ? a.down.qabsmax : a.host_down.qabsmax) + q * a.down.abs_blk_stride,
                                bad ? 0 : a.st_dn_abytes);
    qa = buf_ldu8(ra, aoff, 0);
  } else {
    const rsrc_t ra = make_rsrc((dev ? a.down.absmax : a.host_down.absmax) + q * a.down.abs_blk_stride,
                                bad ? 0 : a.st_dn_abytes);
    am = buf_ldf(ra, aoff * 4u, 0);
  }
}

// Down, first batch: what the first loads need (block references, code
// books, absmax2, activations) and the chunk geometry.
__device__ __forceinline__ void pin_dn_first(DecodeArgs& a) {
  auto st_enc = gptr(a.st_enc);
  auto st_bid = gptr(a.st_bid);
  auto st_act = gptr(a.st_act);
  auto code = gptr(a.code_down);
  auto c2 = gptr(a.down.code2), a2 = gptr(a.down.absmax2);
  asm volatile(""
               : "+s"(st_enc), "+s"(st_bid), "+s"(st_act), "+s"(code), "+s"(c2), "+s"(a2), "+s"(a.st_dn_gx),
                 "+s"(a.st_dn_per), "+s"(a.st_dn_a2n), "+s"(a.k), "+s"(a.H), "+s"(a.NB), "+s"(a.qbs_shift),
                 "+s"(a.dq_shift), "+s"(a.down.row_stride), "+s"(a.down.abs_row_stride));
  a.st_enc = (uint32_t*)st_enc;
  a.st_bid = (int32_t*)st_bid;
  a.st_act = (float*)st_act;
  a.code_down = (const float*)code;
  a.down.code2 = (const float*)c2;
  a.down.absmax2 = (const float*)a2;
}

// Down, second batch: weight views and outputs.
template <bool DQ>
__device__ __forceinline__ void pin_dn_rest(DecodeArgs& a) {
  auto dp = gptr(a.down.packed), hdp = gptr(a.host_down.packed);
  auto da = gptr(DQ ? a.down.qabsmax : reinterpret_cast<const uint8_t*>(a.down.absmax));
  auto hda = gptr(DQ ? a.host_down.qabsmax : reinterpret_cast<const uint8_t*>(a.host_down.absmax));
  auto out = gptr(a.out);
  auto out_f32 = gptr(a.out_f32);
  auto bias = gptr(a.down_bias);
  auto residual = gptr(a.residual);
  auto outpart = gptr(a.outpart);
  asm volatile(""
               : "+s"(dp), "+s"(hdp), "+s"(da), "+s"(hda), "+s"(out), "+s"(out_f32), "+s"(bias), "+s"(residual),
                 "+s"(outpart), "+s"(a.down.blk_stride), "+s"(a.down.abs_blk_stride), "+s"(a.down.offset),
                 "+s"(a.st_dn_bytes), "+s"(a.st_dn_abytes));
  a.down.packed = (const uint8_t*)dp;
  a.host_down.packed = (const uint8_t*)hdp;
  if constexpr (DQ) {
    a.down.qabsmax = (const uint8_t*)da;
    a.host_down.qabsmax = (const uint8_t*)hda;
  } else {
    a.down.absmax = (const float*)da;
    a.host_down.absmax = (const float*)hda;
  }
  a.out = (uint16_t*)out;
  a.out_f32 = (float*)out_f32;
  a.down_bias = (const uint16_t*)bias;
  a.residual = (const uint16_t*)residual;
  a.outpart = (float*)outpart;
}

template <bool DQ>
__global__ void __launch_bounds__(kThreads8, 2) k_down_rep(DecodeArgs args) {
  DecodeArgs a = args;
  pin_dn_first(a);
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  uint32_t* actp = lds + kLutWords;                                    // [512][16] fp16 pairs
  float* ascale = reinterpret_cast<float*>(actp + kMaxDnBlocks * 16);  // [512]
  float* wsum = ascale + kMaxDnBlocks;                                 // [8][64]
  float* c2 = wsum + kWaves * kWave;                                   // [256] (DQ)
  float* a2 = c2 + 256;                                                // [kDnA2Max] (DQ)
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int GX = a.st_dn_gx, per = a.st_dn_per;
  // XCD-aware mapping: workgroups go to the 8 XCDs round-robin (b % 8);
  // chunks 2m and 2m+1 share the 128-byte lines of the absmax codes, so
  // both are given to workgroups of one XCD (one L2).  The grid size
  // (H / 64) GX is a multiple of 16 (H a multiple of 2048).
  const uint32_t xcd = blockIdx.x & 7u, sidx = blockIdx.x >> 3;
  const uint32_t m = xcd + 8u * (sidx >> 1);
  const int gx = (int)(m % (uint32_t)GX), c = 2 * (int)(m / (uint32_t)GX) + (int)(sidx & 1u);
  const int nbw_all = (a.k + GX - 1) / GX;
  const int jb0 = gx * nbw_all;
  const int nbw = max(0, min(a.k - jb0, nbw_all));  // blocks of this workgroup
  const int jw0 = wave * per;                       // this wave's blocks (workgroup-local)
  const int nbv = max(0, min(nbw - jw0, per));
  const int T = (nbv + 1) >> 1;  // 2-block items (uniform per wave)
  const uint32_t o = (uint32_t)(c * kWave + lane);
  const uint32_t roff = o * (uint32_t)a.down.row_stride;
  const uint32_t aoff = o * (uint32_t)a.down.abs_row_stride;
  // double-quantised: absmax of (row o, block b) has flat index o * Ad +
  // 32 b / qbs; the workgroup stages the absmax2 entries of its 64 rows,
  // from g_lo on
  const uint32_t Ad = (uint32_t)(a.NB * 32) >> a.qbs_shift;
  const uint32_t g_lo = (uint32_t)(c * kWave) * Ad >> a.dq_shift;

  // Independent loads first: code book, block references, and (thread t <
  // nbw) the 32 activations of the workgroup's block t.  They are
  // unconditional loads from clamped, valid indices: a load under a branch
  // would be waited for on its own.
  const uint32_t* encs = a.st_enc + jb0;
  uint32_t enc_v = encs[lane < nbv ? jw0 + lane : 0];
  uint32_t bid_v = 0;
  if constexpr (DQ) bid_v = (uint32_t)a.st_bid[jb0 + (lane < nbv ? jw0 + lane : 0)];
  sched_fence();
  LutCodes codes;
  lut_codes_load(a.code_down, a.code_down, tid, codes);
  // Waves with nothing to stage skip the loads (wave-uniform tests): the
  // prologue's loads queue per CU, and the barrier after the staging waits
  // for the last wave's.
  float c2v = 0.0f, a2v[2] = {0.0f, 0.0f};
  if constexpr (DQ) {
    if (wave * kWave < 256) c2v = a.down.code2[tid & 255];
    // entries g_lo .. g_lo + st_dn_a2n - 1 (clamped: unconditional loads)
    const uint32_t last = min((uint32_t)((((long long)a.H * Ad) - 1) >> a.dq_shift), g_lo + a.st_dn_a2n - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (wave * kWave + h * kThreads8 < a.st_dn_a2n) {
        const uint32_t g = min(g_lo + (uint32_t)(tid + h * kThreads8), last);
        a2v[h] = a.down.absmax2[g];
      }
    }
  }
  const bool own = tid < nbw;
  uint32_t my_enc = kBad;
  float4 av[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) av[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (wave * kWave < nbw) {
    my_enc = encs[own ? tid : 0];
    if (!own) my_enc = kBad;
    const float4* ap = reinterpret_cast<const float4*>(a.st_act + (long long)(jb0 + (own ? tid : 0)) * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) av[i] = ap[i];
  }
  sched_fence();
  pin_dn_rest<DQ>(a);
  if (lane >= nbv) enc_v = kBad;
  DnStage st[kDnStages];
#pragma unroll
  for (int i = 0; i < kDnStages; ++i) {
    const bool in = i < T;
    dn_issue<DQ>(a, in ? lane_value(enc_v, 2 * i) : kBad, roff, aoff, st[i].w[0], st[i].am[0], st[i].qa[0]);
    dn_issue<DQ>(a, in ? lane_value(enc_v, 2 * i + 1) : kBad, roff, aoff, st[i].w[1], st[i].am[1], st[i].qa[1]);
  }
  sched_fence();

  lut_store(lds, codes, tid);
  if constexpr (DQ) {
    if (tid < 256) c2[tid] = c2v;
    a2[tid] = a2v[0];
    if (tid + kThreads8 < kDnA2Max) a2[tid + kThreads8] = a2v[1];
  }
  // block tid's activations as fp16 pairs scaled by a power of two (max |act|
  // in [0.5, 1)); invalid blocks and blocks past the group's end are zero
  {
    const bool live = !(my_enc & kBad);
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(av[i].x), fabsf(av[i].y)), fmaxf(fabsf(av[i].z), fabsf(av[i].w))));
    int ex = 0;
    if (live && mx > 0.0f) frexpf(mx, &ex);
    uint32_t hp[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float f[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
      uint32_t h[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) h[m] = live ? f2h(ldexpf(f[m], -ex)) : 0u;
      hp[2 * i] = h[0] | (h[1] << 16);
      hp[2 * i + 1] = h[2] | (h[3] << 16);
    }
    uint4* dst = reinterpret_cast<uint4*>(actp + tid * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(hp[4 * i], hp[4 * i + 1], hp[4 * i + 2], hp[4 * i + 3]);
    ascale[tid] = ldexpf(1.0f, ex);
  }
  lds_barrier();

  uint32_t ad[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ad[i] = (uint32_t)lane * 4u;
  const uint32_t* wact = actp + jw0 * 16;
  const float* wscale = ascale + jw0;
  float acc = 0.0f;
  for (int t0 = 0; t0 < T; t0 += kDnStages) {
#pragma unroll
    for (int i = 0; i < kDnStages; ++i) {
      const int t = t0 + i;
      if (t < T) {
        const int jj = 2 * t;
        float am0 = st[i].am[0], am1 = st[i].am[1];
        if constexpr (DQ) {
          // an invalid block or a pad entry reads code 0: its absmax must be
          // zero, as the zero-extent fp32 load gives it
          const uint32_t b0 = lane_value(bid_v, jj), b1 = lane_value(bid_v, jj + 1);
          const uint32_t f0 = o * Ad + ((32u * b0) >> a.qbs_shift), f1 = o * Ad + ((32u * b1) >> a.qbs_shift);
          am0 = dq_absmax(c2[st[i].qa[0]], a2[(f0 >> a.dq_shift) - g_lo], a.down.offset);
          am1 = dq_absmax(c2[st[i].qa[1]], a2[(f1 >> a.dq_shift) - g_lo], a.down.offset);
          if (lane_value(enc_v, jj) & kBad) am0 = 0.0f;
          if (lane_value(enc_v, jj + 1) & kBad) am1 = 0.0f;
        }
        acc += rep_dot32(st[i].w[0], wact + jj * 16, ad) * (am0 * wscale[jj]);
        acc += rep_dot32(st[i].w[1], wact + jj * 16 + 16, ad) * (am1 * wscale[jj + 1]);
      }
      const int tn = t + kDnStages;
      const bool in = tn < T;
      dn_issue<DQ>(a, in ? lane_value(enc_v, in ? 2 * tn : 0) : kBad, roff, aoff, st[i].w[0], st[i].am[0],
                   st[i].qa[0]);
      dn_issue<DQ>(a, in ? lane_value(enc_v, in ? 2 * tn + 1 : 0) : kBad, roff, aoff, st[i].w[1], st[i].am[1],
                   st[i].qa[1]);
    }
  }
  // wave sums added in wave (block) order
  wsum[wave * kWave + lane] = acc;
  lds_barrier();
  if (wave == 0) {
    float y = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) y += wsum[w * kWave + lane];
    if (GX == 1) {
      a.out[o] = decode_out(a, o, y);
    } else {
      a.outpart[(long long)gx * a.H + o] = y;
    }
  }
}

__global__ void __launch_bounds__(256) k_fin_rep(DecodeArgs a) {
  const int o = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (o >= a.H) return;
  const int G = a.st_dn_gx;
  const float* p = a.outpart + o;
  float y = 0.0f;
  int g = 0;
  for (; g + 8 <= G; g += 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = p[(long long)(g + i) * a.H];
#pragma unroll
    for (int i = 0; i < 8; ++i) y += v[i];
  }
  for (; g < G; ++g) y += p[(long long)g * a.H];
  a.out[o] = decode_out(a, o, y);
}

// Dense NF4 rows (the LM head: all rows of a row-major [out][in] NF4
// matrix times NT token vectors).  The structure of k_gu_rep without the
// block selection: an item is 4 consecutive rows; in a round every wave
// decodes one item over its 2048-column split (16 packed bytes per lane and
// row) through the replicated byte-pair table, dots it with each token's
// split (fp16 pairs in registers), scales each row sum by its absmax, and
// the split sums meet in LDS behind one LDS-only barrier per round.  S =
// ceil(in / 2048) splits, 8 / S items per workgroup round; lanes past the
// last column load zeros, waves past the last item group stay idle.
struct RwStage {
  uint4 w[4];
  float am[4];     // fp32 absmax, or the absmax2 (double-quantised)
  uint32_t qa[4];  // u8 absmax code (double-quantised)
};

// item < 0: zeros (idle wave or past the last round); colok: the lane's 32
// columns lie inside the row.
template <bool DQ>
__device__ __forceinline__ void rw_issue(const RowsArgs& a, int item, bool colok, uint32_t cb, uint32_t ca,
                                         RwStage& st) {
  const rsrc_t rp = make_rsrc(a.packed, a.p_bytes);
  const bool lane_ok = colok && item >= 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * item + i;  // uniform over the wave: its offset goes in soffset
    const bool live = lane_ok && row < a.out;
    st.w[i] = buf_ld16(rp, live ? cb : kOffNone, live ? (uint32_t)row * (uint32_t)a.rs : 0u);
    const uint32_t ai = (uint32_t)row * (uint32_t)a.ars + ca;  // flat absmax index
    if constexpr (DQ) {
      st.qa[i] = buf_ldu8(make_rsrc(a.qabsmax, a.a_bytes), live ? ai : kOffNone, 0);
      st.am[i] = buf_ldfc(make_rsrc(a.absmax2, a.a2_bytes), live ? (ai >> a.dq_shift) * 4u : kOffNone, 0);
    } else {
      st.qa[i] = 0;
      st.am[i] = buf_ldf(make_rsrc(a.absmax, a.a_bytes), live ? ca * 4u : kOffNone,
                         live ? (uint32_t)row * (uint32_t)a.ars * 4u : 0u);
    }
  }
}

constexpr int kRwStages = 2;

// One token fits 128 VGPRs (two workgroups per CU); two tokens take one.
template <int NT>
constexpr int rows_wgs_per_cu() {
  return NT == 1 ? 2 : 1;
}

template <bool DQ, int NT>
__global__ void __launch_bounds__(kThreads8, 2 * rows_wgs_per_cu<NT>()) k_rows_rep(RowsArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  float* comb = reinterpret_cast<float*>(lds + kLutWords);     // [2][8][4 NT]
  float* c2 = comb + 2 * kWaves * 4 * NT;                      // [256] (DQ)
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int S = a.splits, NS = kWaves / S;
  const int s = wave % S, q = wave / S;
  const bool idle = q >= NS;
  const int nwg = (int)gridDim.x, wg = (int)blockIdx.x;
  const uint32_t col = (uint32_t)(s * kSplit + lane * 32);
  const bool colok = (int)col < a.in;
  const uint32_t cb = col >> 1, ca = col >> a.qbs_shift;
  LutCodes codes;
  lut_codes_load(a.code, a.code, tid, codes);
  float c2v = 0.0f;
  if constexpr (DQ) c2v = a.code2[tid & 255];
  uint32_t xp[NT][16];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint4* xv = reinterpret_cast<const uint4*>(a.x + (long long)t * a.in + (colok ? col : 0u));
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint4 u = colok ? xv[v] : make_uint4(0u, 0u, 0u, 0u);
      xp[t][4 * v] = u.x;
      xp[t][4 * v + 1] = u.y;
      xp[t][4 * v + 2] = u.z;
      xp[t][4 * v + 3] = u.w;
    }
  }
  RwStage st[kRwStages];
#pragma unroll
  for (int i = 0; i < kRwStages; ++i)
    rw_issue<DQ>(a, !idle && i < a.rounds ? (i * nwg + wg) * NS + q : -1, colok, cb, ca, st[i]);
  sched_fence();
  lut_store(lds, codes, tid);
  if constexpr (DQ) {
    if (tid < 256) c2[tid] = c2v;
  }
  lds_barrier();
  uint32_t ad[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ad[i] = (uint32_t)lane * 4u;
  for (int r0 = 0; r0 < a.rounds; r0 += kRwStages) {
#pragma unroll
    for (int i = 0; i < kRwStages; ++i) {
      const int r = r0 + i;
      const bool live = r < a.rounds;  // uniform over the workgroup
      const int item = (r * nwg + wg) * NS + q;
      float acc[NT][4];
      if (live) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          float am = st[i].am[m];
          if constexpr (DQ) am = dq_absmax(c2[st[i].qa[m]], st[i].am[m], a.offset);
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[t][m] = rep_dot32(st[i].w[m], xp[t], ad) * am;
        }
      }
      const int rn = r + kRwStages;
      rw_issue<DQ>(a, !idle && rn < a.rounds ? (rn * nwg + wg) * NS + q : -1, colok, cb, ca, st[i]);
      if (live) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const float v = reduce4(acc[t], lane);
          if ((lane & 15) == 0) comb[((r & 1) * kWaves + wave) * 4 * NT + 4 * t + (lane >> 4)] = v;
        }
        lds_barrier();
        if (!idle && s == 0 && lane < 4 * NT) {
          // row 4 item + lane % 4 of token lane / 4: splits added in order
          const int t = lane >> 2, m = lane & 3, row = 4 * item + m;
          float y = 0.0f;
          for (int sp = 0; sp < S; ++sp) y += comb[((r & 1) * kWaves + q * S + sp) * 4 * NT + 4 * t + m];
          if (row < a.out) {
            if (a.out_f32 != nullptr) a.out_f32[(long long)t * a.out + row] = y;
            a.y[(long long)t * a.out + row] = f2h(y);
          }
        }
      }
    }
  }
}

int env_or(const char* name, int dflt) {
  const char* v = getenv(name);
  return (v != nullptr && *v != 0) ? atoi(v) : dflt;
}

std::once_flag g_attr_once;

template <typename K>
void set_lds_limit(K kernel, size_t bytes) {
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)bytes);
}

}  // namespace

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] == 0) {
    hipDeviceProp_t prop;
    cached[dev] = hipGetDeviceProperties(&prop, dev) == hipSuccess ? prop.multiProcessorCount : 256;
  }
  return cached[dev];
}

bool plan_streaming(DecodeArgs& a, int cus) {
  a.st_gu_wgs = 0;
  if (a.H % kSplit != 0 || a.H / kSplit > kWaves || cus <= 0) return false;
  if (a.n_slots >= (1 << 30)) return false;
  // one set of strides for HBM slots and host copies; 32-bit extents
  if (a.gate.row_stride != a.up.row_stride || a.gate.abs_row_stride != a.up.abs_row_stride) return false;
  if (a.host_gate.packed != nullptr &&
      (a.host_gate.row_stride != a.gate.row_stride || a.host_up.row_stride != a.gate.row_stride ||
       a.host_gate.abs_row_stride != a.gate.abs_row_stride || a.host_up.abs_row_stride != a.gate.abs_row_stride ||
       a.host_down.row_stride != a.down.row_stride || a.host_down.abs_row_stride != a.down.abs_row_stride))
    return false;
  const int ab = a.dq ? 1 : 4;  // bytes per stored absmax
  const long long gu_bytes = 31 * a.gate.row_stride + a.H / 2;
  const long long gu_abytes = (31 * a.gate.abs_row_stride + a.H / a.qbs) * ab;
  const long long dn_bytes = (long long)(a.H - 1) * a.down.row_stride + 16;
  const long long dn_abytes = ((long long)(a.H - 1) * a.down.abs_row_stride + 1) * ab;
  const long long lim = 1LL << 31;
  if (gu_bytes >= lim || gu_abytes >= lim || dn_bytes >= lim || dn_abytes >= lim) return false;
  if (a.dq) {
    // flat absmax indices in 32 bits; the down workgroup's absmax2 entries fit
    // its LDS stage
    const long long Ad = (long long)a.NB * 32 / a.qbs;
    const long long n_abs = (long long)a.H * Ad;
    if (n_abs >= lim) return false;
    const long long n2 = (n_abs + (1LL << a.dq_shift) - 1) >> a.dq_shift;
    const long long a2n = ((64 * Ad - 1) >> a.dq_shift) + 2;
    if (a2n > kDnA2Max) return false;
    a.st_gu_a2bytes = (int)(n2 * 4);
    a.st_dn_a2n = (int)a2n;
  }
  const int S = a.H / kSplit;
  const int NS = kWaves / S;
  // gate/up: rounds of NS items per workgroup, balanced over the workgroups
  const long long items = 16LL * a.k;
  static const int gu_per_cu = env_or("NSMLP_GU_WGS_PER_CU", 1) > 1 ? 2 : 1;  // measurement switch, read once
  const long long per_round = (long long)cus * gu_per_cu * NS;
  const long long R = (items + per_round - 1) / per_round;
  if (R > kMaxItems) return false;
  const long long nwg = (items + R * NS - 1) / (R * NS);
  // down: 64-row chunks x GX block groups, at least one workgroup per CU
  const long long chunks = a.H / kWave;
  long long GX = (cus + chunks - 1) / chunks;
  static const long long forced = env_or("NSMLP_DOWN_GX", 0);  // measurement switch, read once
  if (forced > 0) GX = forced;
  if (GX > a.k) GX = a.k;
  if (GX > 64) GX = 64;
  const long long nbw = (a.k + GX - 1) / GX;
  if (nbw > kMaxDnBlocks) return false;
  GX = (a.k + nbw - 1) / nbw;
  const long long per = (nbw + kWaves - 1) / kWaves;
  a.cs = kSplit;
  a.splits = S;
  a.st_gu_rounds = (int)R;
  a.st_gu_wgs = (int)nwg;
  a.st_dn_gx = (int)GX;
  a.st_dn_per = (int)per;
  a.st_gu_bytes = (int)gu_bytes;
  a.st_gu_abytes = (int)gu_abytes;
  a.st_dn_bytes = (int)dn_bytes;
  a.st_dn_abytes = (int)dn_abytes;
  return true;
}

bool streaming_can_select(int NB, int k) { return NB >= 1 && NB <= kSelMaxNB && k >= 1 && k <= NB && k <= kSelMaxK; }

void launch_decode_streaming(const DecodeArgs& a, hipStream_t s) {
  using GuFn = void (*)(DecodeArgs);
  // [dq][affine][0: given ids, 1: top-k of 4 scores per thread, 2: of 8]
  static const GuFn gu_fns[2][2][3] = {
      {{k_gu_rep<false, 0, false>, k_gu_rep<false, 4, false>, k_gu_rep<false, 8, false>},
       {k_gu_rep<true, 0, false>, k_gu_rep<true, 4, false>, k_gu_rep<true, 8, false>}},
      {{k_gu_rep<false, 0, true>, k_gu_rep<false, 4, true>, k_gu_rep<false, 8, true>},
       {k_gu_rep<true, 0, true>, k_gu_rep<true, 4, true>, k_gu_rep<true, 8, true>}}};
  std::call_once(g_attr_once, [] {
    for (int d = 0; d < 2; ++d)
      for (int f = 0; f < 2; ++f)
        for (int m = 0; m < 3; ++m) set_lds_limit(gu_fns[d][f][m], m ? kGuSelLds : (d ? kGuDqLds : kGuLds));
    set_lds_limit(k_down_rep<false>, kDnLds);
    set_lds_limit(k_down_rep<true>, kDnDqLds);
  });
  const bool affine = a.gate_bias != nullptr || a.up_bias != nullptr || a.mask != nullptr;
  const int mode = a.sel_scores == nullptr ? 0 : (a.NB <= 4 * kThreads8 ? 1 : 2);
  const GuFn gu = gu_fns[a.dq ? 1 : 0][affine ? 1 : 0][mode];
  const size_t gu_lds = mode ? (size_t)kGuSelWord * 4 + (size_t)a.k * sizeof(int32_t) : (a.dq ? kGuDqLds : kGuLds);
  gu<<<dim3(a.st_gu_wgs), dim3(kThreads8), gu_lds, s>>>(a);
  const dim3 gd((a.H / kWave) * a.st_dn_gx), bd(kThreads8);
  if (a.dq)
    k_down_rep<true><<<gd, bd, kDnDqLds, s>>>(a);
  else
    k_down_rep<false><<<gd, bd, kDnLds, s>>>(a);
  if (a.st_dn_gx > 1) hipLaunchKernelGGL(k_fin_rep, dim3(a.H / 256), dim3(256), 0, s, a);
}

bool plan_rows(RowsArgs& a, int nt, int cus) {
  if (a.in <= 0 || a.in % 32 != 0 || a.in > kWaves * kSplit || a.out <= 0 || cus <= 0 || nt < 1 || nt > 2)
    return false;
  const int S = (a.in + kSplit - 1) / kSplit, NS = kWaves / S;
  const long long items = (a.out + 3) / 4;
  const long long per_round = (long long)(nt == 1 ? rows_wgs_per_cu<1>() : rows_wgs_per_cu<2>()) * cus * NS;
  const long long R = (items + per_round - 1) / per_round;
  a.splits = S;
  a.rounds = (int)R;
  a.wgs = (int)((items + R * NS - 1) / (R * NS));
  return true;
}

void launch_rows(const RowsArgs& a, int nt, hipStream_t s) {
  using Fn = void (*)(RowsArgs);
  static const Fn fns[2][2] = {{k_rows_rep<false, 1>, k_rows_rep<false, 2>}, {k_rows_rep<true, 1>, k_rows_rep<true, 2>}};
  const size_t lds = (size_t)kRepLutBytes + 2 * kWaves * 4 * 2 * sizeof(float) + 256 * sizeof(float);
  static std::once_flag once;
  std::call_once(once, [] {
    for (int d = 0; d < 2; ++d)
      for (int t = 0; t < 2; ++t) set_lds_limit(fns[d][t], lds);
  });
  fns[a.dq ? 1 : 0][nt == 2 ? 1 : 0]<<<dim3(a.wgs), dim3(kThreads8), lds, s>>>(a);
}

}  // namespace nsmlp
