// Dense-guard prefill MLP (RT:5775-5831, _dense_guard_mlp_forward_exact_chunked_4bit):
// every intermediate block for every token, read from the slot table, as
// full-width GEMMs on v_mfma_f32_32x32x16_f16 with fp32 accumulation.  The
// reference dequantises each NF4 projection to an fp16 weight and runs
// F.linear three times; the rounding points kept here are its own:
//
//   W  = fp16(code * absmax)                   (bitsandbytes dequant to fp16)
//   g  = fp16(x W_gate^T),  s = fp16(silu(g))  (gate = F.silu(F.linear(x, Wg)))
//   u  = fp16(x W_up^T),    act = fp16(s * u)  (act = gate * up)
//   y  = fp16(act W_down^T + bias)             (F.linear(act, Wd, bias))
//
//   k_dg_gu2   one workgroup of 4 waves per 4 blocks and 256 tokens: wave w
//              owns block 4 bq + w, its 32 gate and 32 up rows x all the
//              tile's tokens in 256 fp32 accumulators; the weights are
//              decoded to fp16(code * absmax) in registers (each fed to 16
//              MFMAs), the token rows staged in LDS for the 4 waves; g and u
//              of a (token, row) meet in one lane, so act is formed there.
//              The blocks past the last whole round of the CUs are split in
//              K over all CUs (fp32 partial sums);
//   k_dg_gu_fix  adds a split block group's partial sums in K order, act;
//   k_dg_down  one workgroup per 256 output rows, 256 tokens and one of S
//              ranges of the intermediate blocks: the same register-decode
//              GEMM over act and the down columns (two blocks per step);
//              fp32 partial sums per range;
//   k_dg_fin   y = fp16(sum of the S partials in range order + bias).
//
// The tokens past the last whole 256-token tile (all of a prompt of fewer than
// 256) go in a second launch with the smallest tile of 64, 128 or 192 tokens
// that holds them (a wave then computes 64, 128 or 192 tokens; the
// per-element K order is the same, so every token's result equals the
// 256-token tiles' bit for bit).
//
// Every sum is taken in a fixed order, so the result does not change from run
// to run.
#include <mutex>

#include "nsmlp_regdecode.h"

namespace nsmlp {

namespace {

// ------------------------------------------------------------- down GEMM --
// part[s][t][o] = sum over the blocks of range s of act[t][i] * Wd[o][i],
// Wd = fp16(code * absmax).  A workgroup of 4 waves takes 256 output rows,
// 256 tokens and one block range; wave w owns rows 64 w .. + 63 as two
// 32-row tiles and keeps all 256 tokens x 64 rows in 256 fp32 accumulators
// (AGPRs: 8 token tiles x 2 row tiles of v_mfma_f32_32x32x16_f16), so each
// decoded weight feeds the MFMAs of all 256 tokens and every weight is read
// from HBM once.  A step covers 2 blocks (64 columns), 4 MFMA steps of 16:
//   - lane (j = l % 32, kh = l / 32) loads, for each row tile, the 16 packed
//     bytes of its row j of block 2 c + kh (the block's 32 columns); dword s
//     is its B fragment of MFMA step s: K slots 8 kh .. + 7 are columns
//     8 s .. + 7 of block 2 c + kh, i.e. columns 32 kh + 8 s .. + 7 of the
//     step.  The weights are decoded in registers (each row by one wave, no
//     LDS staging) through a lane-replicated fp32 code-pair table: two fp32
//     products rounded to fp16 by one v_cvt_pk_f16_f32;
//   - the 256 token rows of the 64 columns (128 bytes each) go into an LDS
//     stage by loads straight into LDS; row r's 16-byte piece p lands in
//     slot p ^ ((r / 2) % 8); the A fragment of token tile mi and MFMA step s
//     is piece 4 kh + s of row 32 mi + j, and the 16 rows a group of 16 lanes
//     reads at one piece hit 16 different 16-byte bank groups;
//   - every wave runs 4 MFMA steps x 2 row tiles x 8 token tiles.
// One wave per SIMD: 256 accumulators leave no room for a second.  The
// 32-cycle 32x32x16 MFMA leaves issue room for the decode between MFMAs
// (measured on this GPU at one wave per SIMD with independent MFMAs: 94% of
// the MFMA cycles busy with two VALU ops per MFMA and 91% with four, against
// 43-81% for the 16-cycle 16x16x32 shape with one or two; here about three
// VALU ops per MFMA, address arithmetic included), and every LDS read is
// issued a unit of MFMAs before its use (see the step schedule below).
constexpr int kDnThreads = 256;
constexpr int kDnTok = 256;                            // tokens per tile
constexpr int kDnRows = 256;                           // output rows per workgroup (64 per wave)
constexpr int kDnCopies = kRdCopies;                   // code-pair table copies (lane % 32)
constexpr uint32_t kDnTab = kRdTab;                    // 64 KB at LDS address 0
constexpr uint32_t kDnStage = kDnTok * 128u;           // 256 rows x 64 fp16
constexpr uint32_t kDnC2 = kDnTab + 2u * kDnStage;     // second-level code book [256]
constexpr uint32_t kDnRefs = kDnC2 + 256u * 4u;        // block references of the range
constexpr int kDnRefHost = 1 << 30;                    // reference bit: host copy
constexpr uint32_t kDnLdsMax = 160u * 1024u;

// Bytes spanned by the packed rows (abs = false, 16 bytes per row and block)
// or the absmax entries (elem bytes each) of `blocks` slots of a down view.
__host__ __device__ inline long long dn_extent(const ProjView& v, int blocks, int H, bool abs, int elem) {
  if (blocks <= 0) return 0;
  const long long bs = abs ? v.abs_blk_stride : v.blk_stride, rs = abs ? v.abs_row_stride : v.row_stride;
  return abs ? ((blocks - 1) * bs + (long long)(H - 1) * rs + 1) * elem : (blocks - 1) * bs + (long long)(H - 1) * rs + elem;
}

// The step schedule both GEMMs share: 4 units (MFMA step s = 0..3) of 16
// MFMAs (8 token tiles x 2 row tiles); unit s runs MFMA step s while it reads
// the A fragments of step s + 1, finishes the B fragments of step s + 1
// (looked up in unit s - 1) and looks up those of step s + 2.  Before the
// last unit the wave waits for step c + 1's loads and meets the others at the
// barrier (every wave has read its last A fragments of stage c & 1), sends
// step c + 2's token rows into that stage and reads step c + 1's first A
// fragments.  Three weight register sets (decoded, arrived, in flight) whose
// roles rotate from step to step; step c + 2's weights go out in unit 0, as
// soon as their set is free.
// NW: the vector memory instructions of one issue_w.
template <int NT, int NW, typename IssueW, typename IssueX, typename AmOf>
__device__ __forceinline__ void dn_gemm(float16_t (&acc)[NT][2], int nst, uint32_t abase, IssueW&& issue_w,
                                        IssueX&& issue_x, AmOf&& am_of) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t ad[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ad[i] = (uint32_t)(lane & (kDnCopies - 1)) * 8u;
  // A fragment (token tile mi, MFMA step s) of step c: abase holds the
  // lane's row and swizzled piece 4 kh; step s is piece 4 kh + s, whose slot
  // is the lane's slot with s XORed in
  auto read_a = [&](half8_t (&a)[NT], int c, int s) {
    const uint32_t base = (abase ^ ((uint32_t)s << 4)) + (uint32_t)(c & 1) * kDnStage;
#pragma unroll
    for (int mi = 0; mi < NT; ++mi) a[mi] = lds_ld_h8(base + (uint32_t)mi * 4096u);
  };
  auto lookup2 = [&](RdPairs (&pr)[2], const RdW& W, auto s) {
#pragma unroll
    for (int u = 0; u < 2; ++u) pr[u] = rd_lookup4(rd_word<decltype(s)::value>(W.w[u]), ad);
  };
  auto finish2 = [&](half8_t (&b)[2], const RdPairs (&pr)[2], const float (&am)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) b[u] = rd_finish8(pr[u], am[u]);
  };
  // 2 NT MFMAs, each followed by an LDS read and two VALU ops of the work
  // ahead
  auto mfma_unit = [&](const half8_t (&a)[NT], const half8_t (&b)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int mi = 0; mi < NT; ++mi) acc[mi][u] = mfma32(a[mi], b[u], acc[mi][u]);
#pragma unroll
    for (int i = 0; i < 2 * NT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // this wave's token rows of the next step have landed (loads complete in
  // issue order: only the NW weight loads of step c + 2, issued since, may
  // still be in flight) and its LDS reads are done; then every wave's.  The
  // last two steps wait for everything: their weight loads feed no later
  // step, so the compiler drops them and fewer than NW follow the rows.
  static_assert(NW >= 1 && NW <= 15, "vmcnt field");
  auto step_sync = [](bool tail) {
    if (tail)
      __builtin_amdgcn_s_waitcnt(0);
    else
      __builtin_amdgcn_s_waitcnt(NW | (7 << 4));  // vmcnt(NW) expcnt(7: none) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;

  RdW W0, W1, W2;
  half8_t a0[NT], a1[NT], b0[2], b1[2];
  RdPairs p0[2], p1[2];
  float am_c[2], am_n[2];
  issue_w(W0, 0);
  issue_x(0);
  issue_w(W1, 1);
  issue_x(1);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();  // step 0's token rows are in LDS (and step 1's)
  asm volatile("" ::: "memory");
  am_of(W0, am_c);
  read_a(a0, 0, 0);
  lookup2(p0, W0, S0{});
  finish2(b0, p0, am_c);
  lookup2(p1, W0, S1{});
  __builtin_amdgcn_sched_barrier(0);

  auto step = [&](int c, const RdW& Wc, const RdW& Wn, RdW& Wf, bool tail) {
    // unit 0: B of MFMA step 1 finished, step 2's looked up
    issue_w(Wf, c + 2);
    read_a(a1, c, 1);
    finish2(b1, p1, am_c);
    lookup2(p0, Wc, S2{});
    mfma_unit(a0, b0);
    // unit 1
    read_a(a0, c, 2);
    finish2(b0, p0, am_c);
    lookup2(p1, Wc, S3{});
    mfma_unit(a1, b1);
    // unit 2: the next step's absmax and its MFMA step 0 looked up
    read_a(a1, c, 3);
    finish2(b1, p1, am_c);
    am_of(Wn, am_n);
    lookup2(p0, Wn, S0{});
    mfma_unit(a0, b0);
    // unit 3
    step_sync(tail);
    issue_x(c + 2);
    read_a(a0, c + 1, 0);
    finish2(b0, p0, am_n);
    lookup2(p1, Wn, S1{});
    mfma_unit(a1, b1);
#pragma unroll
    for (int u = 0; u < 2; ++u) am_c[u] = am_n[u];
#pragma unroll
    for (int mi = 0; mi < NT; ++mi)
#pragma unroll
      for (int u = 0; u < 2; ++u) asm volatile("" : "+a"(acc[mi][u]));
  };
  // unrolled by the three register sets, whose roles rotate: no set is
  // copied, so step c + 2's weights only have to land by step c + 1's third
  // unit (a copy at the end of the step waited for them there)
  int c = 0;
  for (; c + 3 <= nst; c += 3) {
    step(c, W0, W1, W2, false);
    step(c + 1, W1, W2, W0, false);
    step(c + 2, W2, W0, W1, false);
  }
  if (c < nst) step(c, W0, W1, W2, true);
  if (c + 1 < nst) step(c + 1, W1, W2, W0, true);
  __builtin_amdgcn_s_waitcnt(0);
  mfma_drain();
}

// MT token groups of 16 per tile (16: 256 tokens; 4, 8 or 12 for the tokens
// past the last whole 256-token tile), i.e. MT / 2 tiles of 32.
template <bool DQ, bool HOST, int MT>
__global__ void __launch_bounds__(kDnThreads, 1) k_dg_down(DenseGuardArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dn_lds[];  // no static LDS: dn_lds is LDS address 0
  constexpr int NT = MT / 2;
  const DecodeArgs& d = g.d;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = d.H, NB = d.NB, I = NB * 32, M = g.M, S = g.S;
  // XCD-aware order: workgroups go to the 8 XCDs round-robin; when the grid
  // divides by 8, XCD x runs the consecutive tiles x N/8 .. (x+1) N/8 - 1:
  // row tiles of one (range, token tile), which read the same act columns
  // through the XCD's L2
  const int RT = (H + kDnRows - 1) / kDnRows, N = (int)gridDim.x;
  int idx = (int)blockIdx.x;
  if ((N & 7) == 0) idx = (idx & 7) * (N >> 3) + (idx >> 3);
  const int rt = idx % RT, combo = idx / RT, s = combo % S, tt = combo / S;
  const int t0 = g.t_base + tt * 16 * MT;
  const int G = NB / 2;  // 2-block steps
  const int g_lo = (int)((long long)s * G / S), g_hi = (int)((long long)(s + 1) * G / S);
  const int nst = g_hi - g_lo, b_lo = 2 * g_lo;
  float* c2s = reinterpret_cast<float*>(dn_lds + kDnC2);
  int32_t* refs = reinterpret_cast<int32_t*>(dn_lds + kDnRefs);

  rd_table_fill(dn_lds, d.code_down, tid);
  if constexpr (DQ) c2s[tid] = d.down.code2[tid];
  // block references: slot, or the block id with kDnRefHost for a host copy,
  // or -1 (out of the table, or no tokens when the block lists are given)
  const bool have_host = d.host_down.packed != nullptr;
  for (int i = tid; i < 2 * nst; i += kDnThreads) {
    const int b = b_lo + i;
    const int slot = d.lookup ? d.lookup[b] : b;
    const bool used = g.offsets == nullptr || g.offsets[b + 1] > g.offsets[b];
    const bool dev = slot >= 0;
    const bool ok = used && (dev ? slot < d.n_slots : have_host);
    refs[i] = !ok ? -1 : (dev ? slot : (kDnRefHost | b));
  }
  __syncthreads();

  const int j = lane & 31, kh = lane >> 5;
  const uint32_t o0 = (uint32_t)(rt * kDnRows + wave * 64 + j);  // row of tile 0; tile u: o0 + 32 u
  const uint32_t rs = (uint32_t)d.down.row_stride, bs = (uint32_t)d.down.blk_stride;
  const uint32_t ars = (uint32_t)d.down.abs_row_stride, abs_ = (uint32_t)d.down.abs_blk_stride;
  const uint32_t Ad = (uint32_t)I >> d.qbs_shift;
  const rsrc_t rw = make_rsrc(d.down.packed, (int)dn_extent(d.down, d.n_slots, H, false, 16));
  const rsrc_t rwh = HOST ? make_rsrc(d.host_down.packed, (int)dn_extent(d.down, NB, H, false, 16)) : rw;
  const rsrc_t ra = DQ ? make_rsrc(d.down.qabsmax, (int)dn_extent(d.down, d.n_slots, H, true, 1))
                       : make_rsrc(d.down.absmax, (int)dn_extent(d.down, d.n_slots, H, true, 4));
  const rsrc_t rah = !HOST ? ra
                     : DQ  ? make_rsrc(d.host_down.qabsmax, (int)dn_extent(d.down, NB, H, true, 1))
                           : make_rsrc(d.host_down.absmax, (int)dn_extent(d.down, NB, H, true, 4));
  const rsrc_t r2 = DQ ? make_rsrc(d.down.absmax2, (int)((((long long)H * Ad + (1 << d.dq_shift) - 1) >> d.dq_shift) * 4))
                       : ra;
  const rsrc_t rx = make_rsrc(g.act, (int)((long long)M * I * 2));

  // Offsets: a lane's row in tile u is o0 + 32 u, so the tile's part of every
  // weight and absmax offset is a uniform constant that goes into the load's
  // scalar offset; the rows of a wave (64, H % 256 == 0) are all inside H or
  // all outside.  Every offset is computed, then selected: a select between
  // two registers (an arm with arithmetic becomes a branch, which splits the
  // step into blocks the scheduler and the register allocator see
  // separately).
  const bool wrows = (int)(rt * kDnRows + wave * 64) < H;
  auto issue_w = [&](RdW& W, int c) {
    const int cc = max(0, min(c, nst - 1));  // clamped: the reference read stays in the range
    const int enc = refs[2 * cc + kh];
    const bool ok = (c < nst) & (enc >= 0) & wrows;
    const bool host = HOST & ((enc & kDnRefHost) != 0);
    const uint32_t qq = (uint32_t)(enc & (kDnRefHost - 1));
    const uint32_t b = (uint32_t)(b_lo + 2 * cc + kh);
    const bool dv = ok & !host, hv = ok & host;
    const uint32_t wo_d = qq * bs + o0 * rs, ao_d = qq * abs_ + o0 * ars;
    const uint32_t wo_h = b * bs + o0 * rs, ao_h = b * abs_ + o0 * ars;
    const uint32_t ab = DQ ? 1u : 4u;
    const uint32_t wo = dv ? wo_d : kOffNone, ao = dv ? ao_d * ab : kOffNone;
    const uint32_t who = hv ? wo_h : kOffNone, aho = hv ? ao_h * ab : kOffNone;
    const uint32_t f0 = o0 * Ad + ((32u * b) >> d.qbs_shift);
    W.ok = ok;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t so_w = 32u * (uint32_t)u * rs, so_a = 32u * (uint32_t)u * ars * ab;
      W.w[u] = buf_ld16(rw, wo, so_w);
      if constexpr (HOST) {
        const uint4 h = buf_ld16(rwh, who, so_w);
        W.w[u] = make_uint4(W.w[u].x | h.x, W.w[u].y | h.y, W.w[u].z | h.z, W.w[u].w | h.w);
      }
      if constexpr (DQ) {
        W.qa[u] = buf_ldu8(ra, ao, so_a);
        if constexpr (HOST) W.qa[u] |= buf_ldu8(rah, aho, so_a);
        const uint32_t fo = ((f0 + 32u * (uint32_t)u * Ad) >> d.dq_shift) * 4u;
        W.a[u] = buf_ldfc(r2, ok ? fo : kOffNone, 0);
      } else {
        W.a[u] = buf_ldf(ra, ao, so_a);
        if constexpr (HOST) W.a[u] = __uint_as_float(__float_as_uint(W.a[u]) | __float_as_uint(buf_ldf(rah, aho, so_a)));
      }
    }
  };
  // token rows of step c into stage c & 1: load i of wave w fills rows
  // 32 i + 8 w .. + 7 (lane l: row + l / 8, slot l % 8); row i's offset is
  // load 0's plus 32 i rows (a scalar offset)
  const int arow = 8 * wave + (lane >> 3);  // row of load 0 ((row / 2) % 8 is the same for every load)
  const uint32_t apiece = (uint32_t)((lane & 7) ^ ((arow >> 1) & 7));
  const uint32_t xrow = ((uint32_t)(t0 + arow) * (uint32_t)I + 8u * apiece) * 2u;
  auto issue_x = [&](int c) {
    const int tlim = c < nst ? M - t0 - arow : 0;  // rows 32 i with 32 i < tlim are tokens of this call
    const uint32_t xo = xrow + (uint32_t)(64 * (b_lo + 2 * c));
    const uint32_t sb = kDnTab + (uint32_t)(c & 1) * kDnStage;
#pragma unroll
    for (int i = 0; i < MT / 2; ++i) {  // 16 MT rows of 128 bytes: MT / 2 loads per wave
      const uint32_t xi = 32 * i < tlim ? xo : kOffNone;
      ld_lds16s(rx, dn_lds + sb + (32 * i + 8 * wave) * 128, xi, 64u * (uint32_t)i * (uint32_t)I);
    }
  };
  auto am_of = [&](const RdW& W, float (&am)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float v = W.a[u];
      if constexpr (DQ) v = dq_absmax(c2s[W.qa[u]], W.a[u], d.down.offset);
      am[u] = W.ok ? v : 0.0f;
    }
  };

  // 256 accumulators, kept in AGPRs: pinned there at the start and after
  // every step (otherwise part of them crosses the loop in VGPRs, which the
  // loads in flight and the decode need)
  float16_t acc[NT][2];
#pragma unroll
  for (int mi = 0; mi < NT; ++mi)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][u][r] = 0.0f;
      asm volatile("" : "+a"(acc[mi][u]));
    }
  // the lane's A fragment address of MFMA step 0 in stage 0: row j, piece 4 kh
  const uint32_t abase = kDnTab + (uint32_t)j * 128u + ((4u * (uint32_t)kh ^ (uint32_t)((j >> 1) & 7)) << 4);
  dn_gemm<NT, (DQ ? 3 : 2) * (HOST ? 2 : 1) * 2 - (DQ && HOST ? 2 : 0)>(acc, nst, abase, issue_w, issue_x, am_of);
  // C element r of lane (j, kh), tile (mi, u): token 32 mi + 8 (r / 4) +
  // 4 kh + r % 4, row o0 + 32 u
  float* part = g.part + (long long)s * M * H;
  if (wrows) {
#pragma unroll
    for (int mi = 0; mi < NT; ++mi) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = t0 + 32 * mi + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (t < M) {
#pragma unroll
          for (int u = 0; u < 2; ++u) part[(long long)t * H + o0 + 32u * (uint32_t)u] = acc[mi][u][r];
        }
      }
    }
  }
}

// ---------------------------------------------------------- gate/up GEMM --
// g[t][i], u[t][i] = sum over k of x[t][k] * W[i][k] for the gate and up rows,
// W = fp16(code * absmax), then act[t][i] = fp16(fp16(silu(fp16(g))) *
// fp16(u)).  The down kernel's scheme with the roles of the operands kept: a
// workgroup of 4 waves takes 4 consecutive blocks and 16 MT tokens, wave w
// owns block 4 bq + w, i.e. its 32 gate rows (row tile 0) and its 32 up rows
// (row tile 1) x all the tile's tokens in 8 MT fp32 accumulators per tile
// (AGPRs); each decoded weight feeds the MFMAs of all the tile's tokens and
// every weight is read from HBM once.  The 4 waves share the tile's token
// rows.  A step covers 64 columns:
//   - lane (j = l % 32, kh = l / 32) loads, for each row tile, 16 packed
//     bytes of its row j: bytes 16 kh .. + 15 of the step's 32, the step's
//     columns 32 kh .. + 31.  Dword s is its B fragment for MFMA step s, so K
//     slots 8 kh .. 8 kh + 7 of step s are columns 32 kh + 8 s .. + 7 of the
//     step (the A fragments use the same order); their absmax is the entry
//     (64 c + 32 kh) / qbs (qbs >= 32);
//   - the tokens' rows of the 64 columns (128 bytes each) go into an LDS
//     stage by loads straight into LDS (row r's 16-byte piece p in slot
//     p ^ ((r / 2) % 8)); the A fragment of token tile mi and MFMA step s is
//     piece 4 kh + s of token row 32 mi + j.
// Gate and up accumulators of the same (token, row) sit in the same lane, so
// act is formed in registers.  The code-pair table, the step schedule and the
// register pinning are the down kernel's.
constexpr uint32_t kGuC2 = kDnTab + 2u * kDnStage;  // second-level code books [2][256]
constexpr uint32_t kGuLds = kGuC2 + 2u * 256u * 4u;

// A launch covers one token tile (from t_base); its work is items, item q
// the 4 consecutive blocks 4 q .. 4 q + 3 (nq = NB / 4 items).  One workgroup
// per CU: the first gu_full items (whole rounds of the CUs) run one per
// workgroup over all of K; the rest (gu_tail < CUs items) would leave most CUs
// idle for a whole K loop, so their K steps are laid end to end and cut into
// ranges of gu_per steps, one per workgroup (tail workgroup i: steps
// i gu_per .. + gu_per - 1).  gu_per <= nst, so a range holds at most two
// segments, each within one item.  A segment that is a whole item forms act;
// any other writes its fp32 accumulators to slot 2 i + (second segment) of
// gu_part, and k_dg_gu_fix adds an item's segments in K order and forms act.
// The split depends on the layer shape and the CU count only, so a token's
// sums do not depend on how many tokens share the call.
__device__ __forceinline__ float dg_act(float gsum, float usum) {
  const float g16 = h2f(f2h(gsum));
  const float s16 = h2f(f2h(g16 / (1.0f + expf(-g16))));
  const float u16 = h2f(f2h(usum));
  return s16 * u16;
}

template <bool DQ, int MT>
__global__ void __launch_bounds__(kDnThreads, 1) k_dg_gu2(DenseGuardArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t gu_lds[];  // no static LDS: gu_lds is LDS address 0
  constexpr int NT = MT / 2;
  const DecodeArgs& d = g.d;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = d.H, I = d.NB * 32, M = g.M;
  const int nst = H / 64;
  float* c2s = reinterpret_cast<float*>(gu_lds + kGuC2);

  rd_table_fill(gu_lds, d.code, tid);
  if constexpr (DQ) {
    c2s[tid] = d.gate.code2[tid];
    c2s[256 + tid] = d.up.code2[tid];
  }
  // this workgroup's first segment: item, virtual steps v0 .. v1 - 1, its
  // partial slot (-1: a whole item); with nseg = 2 also steps 0 .. v1b - 1 of
  // the next item (slot + 1)
  const int wg = (int)blockIdx.x;
  int item = wg, v0 = 0, v1 = nst, slot = -1, nseg = 1, v1b = 0;
  if (wg >= g.gu_full) {
    const int i = wg - g.gu_full, per = g.gu_per;
    const long long s0 = (long long)i * per, s1 = min(s0 + per, (long long)g.gu_tail * nst);
    const int a = (int)(s0 / nst);
    item = g.gu_full + a;
    v0 = (int)(s0 - (long long)a * nst);
    v1 = (int)min((long long)nst, s1 - (long long)a * nst);
    slot = 2 * i;
    if (s1 > (long long)(a + 1) * nst) {  // the range runs into the next item
      nseg = 2;
      v1b = (int)(s1 - (long long)(a + 1) * nst);
    }
  }
  __syncthreads();

  const int j = lane & 31, kh = lane >> 5;
  const uint32_t rs = (uint32_t)d.gate.row_stride, A = (uint32_t)d.gate.abs_row_stride;
  const rsrc_t rx = make_rsrc(g.x, (int)((long long)M * H * 2));
  const int t0 = g.t_base;
  auto run = [&](const int quad, const int v0, const int v1, const int slot) {
    const int blk = 4 * quad + wave;
    const int len = v1 - v0;
    // the K loop of an item starts at a step that depends on its quad's index
    // within its XCD (4 starting points), so that the many rows that share a
    // cache set are not read at the same columns at the same time; the
    // workgroups of one starting point share their token columns in L2 (8,
    // 16 and 32 points were slower: more token columns fetched per XCD; 1 and
    // 2 too).  A segment's virtual step c is the item's step (v0 + c + rot)
    // mod nst.
    const int rot = (int)(((long long)((quad >> 3) & 3) * nst) >> 2);
    const int pbase = (v0 + rot) % nst;
    const BlockRef br = resolve_id(d, blk);
    if (!br.ok && lane == 0) atomicOr(d.status, 1);

    rsrc_t rw[2], ra[2], r2[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const ProjView& pv = u ? d.up : d.gate;
      const ProjView& hv = u ? d.host_up : d.host_gate;
      // the block is the wave's (blk is uniform): scalar descriptors
      rw[u] = make_rsrc_uniform((br.dev ? pv.packed : hv.packed) + br.q * pv.blk_stride, br.ok ? (int)(32 * rs) : 0);
      if constexpr (DQ) {
        ra[u] = make_rsrc_uniform((br.dev ? pv.qabsmax : hv.qabsmax) + br.q * pv.abs_blk_stride,
                                  br.ok ? (int)(32 * A) : 0);
        r2[u] = make_rsrc_uniform(pv.absmax2,
                                  br.ok ? (int)((((long long)I * A + (1 << d.dq_shift) - 1) >> d.dq_shift) * 4) : 0);
      } else {
        ra[u] = make_rsrc_uniform((br.dev ? pv.absmax : hv.absmax) + br.q * pv.abs_blk_stride,
                                  br.ok ? (int)(32 * A * 4) : 0);
        r2[u] = ra[u];
      }
    }
    // per-lane parts of the weight and absmax offsets (row j); double-quantised
    // u8 absmax codes are stored in row pairs ([row / 2][entry][row % 2])
    const uint32_t wv = (uint32_t)j * rs + 16u * (uint32_t)kh;
    const uint32_t qv = DQ ? ((uint32_t)(j >> 1) * A) * 2u + (uint32_t)(j & 1) : (uint32_t)j * A * 4u;
    const uint32_t fv = (32u * (uint32_t)blk + (uint32_t)j) * A;  // absmax index of row j, entry 0
    auto issue_w = [&](RdW& W, int c) {
      const bool live = c < len;
      c = pbase + c < nst ? pbase + c : pbase + c - nst;
      const uint32_t ce = ((uint32_t)(64 * c) + 32u * (uint32_t)kh) >> d.qbs_shift;  // the lane's absmax entry
      const uint32_t wo = live ? wv : kOffNone, qo = live ? qv + (DQ ? 2u : 4u) * ce : kOffNone;
      W.ok = br.ok;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        // temporal loads: a row's 128-byte line serves 4 steps (an
        // nontemporal load fetched it again for each)
        W.w[u] = buf_ld16c(rw[u], wo, 32u * (uint32_t)c);
        if constexpr (DQ) {
          W.qa[u] = buf_ldu8c(ra[u], qo, 0);
          const uint32_t fo = ((fv + ce) >> d.dq_shift) * 4u;
          W.a[u] = buf_ldfc(r2[u], live ? fo : kOffNone, 0);
        } else {
          W.a[u] = buf_ldfc(ra[u], qo, 0);
        }
      }
    };
    // token rows of step c into stage c & 1: load i of wave w fills rows
    // 32 i + 8 w .. + 7 (lane l: row + l / 8, slot l % 8); row i's offset is
    // load 0's plus 32 i rows (a scalar offset)
    const int arow = 8 * wave + (lane >> 3);
    const uint32_t apiece = (uint32_t)((lane & 7) ^ ((arow >> 1) & 7));
    const uint32_t xrow = ((uint32_t)(t0 + arow) * (uint32_t)H + 8u * apiece) * 2u;
    auto issue_x = [&](int c) {
      const int tlim = c < len ? M - t0 - arow : 0;  // rows 32 i with 32 i < tlim are tokens of this call
      const int cp = pbase + c < nst ? pbase + c : pbase + c - nst;
      const uint32_t xo = xrow + 128u * (uint32_t)cp;
      const uint32_t sb = kDnTab + (uint32_t)(c & 1) * kDnStage;
#pragma unroll
      for (int i = 0; i < MT / 2; ++i) {
        const uint32_t xi = 32 * i < tlim ? xo : kOffNone;
        ld_lds16s(rx, gu_lds + sb + (32 * i + 8 * wave) * 128, xi, 64u * (uint32_t)i * (uint32_t)H);
      }
    };
    auto am_of = [&](const RdW& W, float (&am)[2]) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float v = W.a[u];
        if constexpr (DQ) v = dq_absmax(c2s[u * 256 + W.qa[u]], W.a[u], u ? d.up.offset : d.gate.offset);
        am[u] = W.ok ? v : 0.0f;
      }
    };

    float16_t acc[NT][2];
#pragma unroll
    for (int mi = 0; mi < NT; ++mi)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mi][u][r] = 0.0f;
        asm volatile("" : "+a"(acc[mi][u]));
      }
    const uint32_t abase = kDnTab + (uint32_t)j * 128u + ((4u * (uint32_t)kh ^ (uint32_t)((j >> 1) & 7)) << 4);
    dn_gemm<NT, DQ ? 6 : 4>(acc, len, abase, issue_w, issue_x, am_of);
    if (slot < 0 || len == nst) {
      // act = fp16(fp16(silu(fp16(g))) * fp16(u)) for (token, row): C element
      // r of lane (j, kh) is row j of its tile for token 32 mi + 8 (r / 4) +
      // 4 kh + r % 4
#pragma unroll
      for (int mi = 0; mi < NT; ++mi) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = t0 + 32 * mi + 8 * (r >> 2) + 4 * kh + (r & 3);
          if (t < M) g.act[(long long)t * I + 32 * blk + j] = f2h(dg_act(acc[mi][0][r], acc[mi][1][r]));
        }
      }
    } else {
      // the segment's sums in fragment order: [slot][wave][mi][u][r][lane]
      float* pp = g.gu_part + ((size_t)slot * 4 + (size_t)wave) * (size_t)(NT * 2 * 16 * 64) + lane;
#pragma unroll
      for (int mi = 0; mi < NT; ++mi)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int r = 0; r < 16; ++r) pp[((mi * 2 + u) * 16 + r) * 64] = acc[mi][u][r];
    }
  };
  run(item, v0, v1, slot);
  if (nseg > 1) {
    __syncthreads();  // every wave is done with the token stages before the next loads refill them
    run(item + 1, 0, v1b, slot + 1);
  }
}

// act of the split tail items: workgroup (tail item a, wave w, 4 token tiles
// from 4 mg); a thread adds its (tile, lane) sums over the item's segments in
// K order (tail workgroups i_lo .. i_hi, the segment of workgroup i being its
// first or its second) and forms act as k_dg_gu2.
template <int MT>
__global__ void __launch_bounds__(256) k_dg_gu_fix(DenseGuardArgs g) {
  constexpr int NT = MT / 2, MG = (NT + 3) / 4;
  const int nst = g.d.H / 64, I = g.d.NB * 32;
  const int b = (int)blockIdx.x;
  const int a = b / (4 * MG), wave = (b / MG) & 3, mi = (b % MG) * 4 + (int)(threadIdx.x >> 6);
  const int lane = (int)threadIdx.x & 63;
  if (mi >= NT) return;
  const long long per = g.gu_per, s0 = (long long)a * nst;
  const int i_lo = (int)(s0 / per), i_hi = (int)((s0 + nst - 1) / per);
  float gs[16], us[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) gs[r] = us[r] = 0.0f;
  for (int i = i_lo; i <= i_hi; ++i) {
    const int slot = 2 * i + ((long long)i * per / nst == a ? 0 : 1);
    const float* pp = g.gu_part + (((size_t)slot * 4 + (size_t)wave) * NT + (size_t)mi) * (size_t)(2 * 16 * 64) + lane;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      gs[r] += pp[r * 64];
      us[r] += pp[(16 + r) * 64];
    }
  }
  const int quad = g.gu_full + a;
  const int t0 = g.t_base, blk = 4 * quad + wave;
  const int j = lane & 31, kh = lane >> 5;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int t = t0 + 32 * mi + 8 * (r >> 2) + 4 * kh + (r & 3);
    if (t < g.M) g.act[(long long)t * I + 32 * blk + j] = f2h(dg_act(gs[r], us[r]));
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
// [dq][MT / 4 - 1 of the 16 MT-token tile]
const DgFn kDgGu2[2][4] = {{k_dg_gu2<false, 4>, k_dg_gu2<false, 8>, k_dg_gu2<false, 12>, k_dg_gu2<false, 16>},
                           {k_dg_gu2<true, 4>, k_dg_gu2<true, 8>, k_dg_gu2<true, 12>, k_dg_gu2<true, 16>}};
const DgFn kDgGuFix[4] = {k_dg_gu_fix<4>, k_dg_gu_fix<8>, k_dg_gu_fix<12>, k_dg_gu_fix<16>};
constexpr int kGuTailWgs = 256;  // CUs counted at most (the partial slots, 2 per tail workgroup, are sized for it)

// CUs of the current device (one gate/up workgroup each), at most kGuTailWgs
int dg_tail_wgs() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kGuTailWgs;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = kGuTailWgs;
    cus[dev] = n < kGuTailWgs ? n : kGuTailWgs;
  }
  return cus[dev];
}

// gate/up of one MT-token tile (from g.t_base): whole rounds of the CUs
// first, then the rest's K steps in equal ranges over the CUs (see k_dg_gu2);
// the fix-up runs before the next launch reuses the partial slots
void launch_gu2(const DenseGuardArgs& g, int MT, hipStream_t st) {
  const int items = g.d.NB / 4;
  const int W = dg_tail_wgs(), nst = g.d.H / 64;
  DenseGuardArgs a = g;
  a.gu_full = items / W * W;
  a.gu_tail = items - a.gu_full;
  a.gu_per = a.gu_tail > 0 ? (int)(((long long)a.gu_tail * nst + W - 1) / W) : nst;  // <= nst: gu_tail < W
  const int wt = a.gu_tail > 0 ? (int)(((long long)a.gu_tail * nst + a.gu_per - 1) / a.gu_per) : 0;
  kDgGu2[g.d.dq ? 1 : 0][MT / 4 - 1]<<<dim3((unsigned)(a.gu_full + wt)), dim3(kDnThreads), kGuLds, st>>>(a);
  if (a.gu_tail > 0 && a.gu_per < nst) {  // every tail item is split
    const int mg = (MT / 2 + 3) / 4;
    kDgGuFix[MT / 4 - 1]<<<dim3((unsigned)(a.gu_tail * 4 * mg)), dim3(256), 0, st>>>(a);
  }
}
// [dq][MT - 1 of the 64 MT-token tile]
// [dq][host copies][MT / 4 - 1 of the 16 MT-token tile]
const DgFn kDgDown[2][2][4] = {
    {{k_dg_down<false, false, 4>, k_dg_down<false, false, 8>, k_dg_down<false, false, 12>, k_dg_down<false, false, 16>},
     {k_dg_down<false, true, 4>, k_dg_down<false, true, 8>, k_dg_down<false, true, 12>, k_dg_down<false, true, 16>}},
    {{k_dg_down<true, false, 4>, k_dg_down<true, false, 8>, k_dg_down<true, false, 12>, k_dg_down<true, false, 16>},
     {k_dg_down<true, true, 4>, k_dg_down<true, true, 8>, k_dg_down<true, true, 12>, k_dg_down<true, true, 16>}}};

void dg_set_lds() {
  static std::once_flag once;
  std::call_once(once, [] {
    for (int q = 0; q < 2; ++q)
      for (int h = 0; h < 2; ++h)
        for (int m = 0; m < 4; ++m)
          (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kDgDown[q][h][m]),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDnLdsMax);
    for (int q = 0; q < 2; ++q)
      for (int m = 0; m < 4; ++m)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kDgGu2[q][m]),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGuLds);
  });
}

}  // namespace

size_t dense_gu_tail_bytes(int M) {
  const int mc = M < kDnTok ? M : kDnTok;
  const int nt = 2 * ((mc + 63) / 64);  // accumulator tiles of the widest token tile of the call
  return (size_t)2 * kGuTailWgs * 4 * nt * 2 * 16 * 64 * 4;
}

// k_dg_down and k_dg_gu2 read their code-pair table and token stages at
// fixed LDS addresses (immediate offsets from 0): that holds only while the
// kernels have no static LDS, so that their dynamic LDS starts at address 0.
// Checked once per process on the compiled kernels, before the first launch.
int dense_down_check() {
  static std::once_flag once;
  static size_t static_lds = 0;
  static int rc_attr = 0;
  std::call_once(once, [] {
    for (int q = 0; q < 2; ++q)
      for (int h = 0; h < 2; ++h)
        for (int m = 0; m < 4; ++m) {
          hipFuncAttributes attr;
          if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kDgDown[q][h][m])) != hipSuccess) {
            rc_attr = 1;
            continue;
          }
          if (attr.sharedSizeBytes > static_lds) static_lds = attr.sharedSizeBytes;
        }
    for (int q = 0; q < 2; ++q)
      for (int m = 0; m < 4; ++m) {
        hipFuncAttributes attr;
        if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kDgGu2[q][m])) != hipSuccess) {
          rc_attr = 1;
          continue;
        }
        if (attr.sharedSizeBytes > static_lds) static_lds = attr.sharedSizeBytes;
      }
  });
  if (rc_attr) {
    (void)hipGetLastError();
    return set_error(NSMLP_EHIP, "dense down GEMM: kernel attributes unavailable");
  }
  if (static_lds != 0)
    return set_error(NSMLP_EHIP, "dense down GEMM has %zu bytes of static LDS; its LDS reads assume its dynamic LDS "
                                 "starts at address 0", static_lds);
  return NSMLP_OK;
}

int dense_down_refs(int NB, int S) { return 2 * ((NB / 2 + S - 1) / S); }

bool dense_down_fits(const DecodeArgs& d, int S) {
  const long long lim = (1LL << 31) - 1;
  const int ab = d.dq ? 1 : 4;
  if (d.NB % 4 != 0 || S < 1) return false;
  if (kDnRefs + 4LL * dense_down_refs(d.NB, S) > (long long)kDnLdsMax) return false;
  if (dn_extent(d.down, d.n_slots, d.H, false, 16) > lim || dn_extent(d.down, d.n_slots, d.H, true, ab) > lim)
    return false;
  return d.host_down.packed == nullptr ||
         (dn_extent(d.down, d.NB, d.H, false, 16) <= lim && dn_extent(d.down, d.NB, d.H, true, ab) <= lim);
}

void launch_dense_down(const DenseGuardArgs& g, hipStream_t st) {
  dg_set_lds();
  const int RT = (g.d.H + kDnRows - 1) / kDnRows;
  const size_t lds = kDnRefs + 4u * (size_t)dense_down_refs(g.d.NB, g.S);
  const bool host = g.d.host_down.packed != nullptr;
  // whole 256-token tiles, then the rest in the smallest 64-, 128- or
  // 192-token tile that holds it (per token the same sums, bit for bit)
  const int full = g.M / kDnTok, rest = g.M - full * kDnTok;
  DenseGuardArgs a = g;
  if (full > 0) {
    a.t_base = 0;
    kDgDown[g.d.dq ? 1 : 0][host ? 1 : 0][3]<<<dim3((unsigned)(RT * full * g.S)), dim3(kDnThreads), lds, st>>>(a);
  }
  if (rest > 0) {
    a.t_base = full * kDnTok;
    kDgDown[g.d.dq ? 1 : 0][host ? 1 : 0][(rest + 63) / 64 - 1]<<<dim3((unsigned)(RT * g.S)), dim3(kDnThreads), lds, st>>>(a);
  }
  const long long n = (long long)g.M * g.d.H;
  k_dg_fin<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(g);
}

void launch_dense_guard(const DenseGuardArgs& g, hipStream_t st) {
  dg_set_lds();
  // whole 256-token tiles, then the rest in the smallest 64-, 128- or
  // 192-token tile that holds it (per token the same sums, bit for bit)
  const int full = g.M / kDnTok, rest = g.M - full * kDnTok;
  DenseGuardArgs a = g;
  a.gu_part = g.part;  // free until the down GEMM writes its partials there
  for (int ty = 0; ty < full; ++ty) {
    a.t_base = ty * kDnTok;
    launch_gu2(a, 16, st);
  }
  if (rest > 0) {
    a.t_base = full * kDnTok;
    launch_gu2(a, 4 * ((rest + 63) / 64), st);
  }
  launch_dense_down(g, st);
}

}  // namespace nsmlp
