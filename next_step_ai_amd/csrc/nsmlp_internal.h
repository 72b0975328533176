// Internal device/host helpers shared by the nsmlp HIP translation units.
// CDNA4 (gfx950) only: wave64, fp16 via _Float16, fp64 vector ALU.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/nsmlp.h"

namespace nsmlp {

constexpr int kBlock = 32;         // intermediate rows per sparse block
constexpr int kWave = 64;          // CDNA wavefront width
constexpr int kMaxSelect = 65535;  // selection keys pack the index in 16 bits

// ---------------------------------------------------------------- errors --
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// ------------------------------------------------------------------ fp16 --
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Monotone 16-bit key of an fp16 value (larger value -> larger key); -0 == +0.
__device__ __forceinline__ uint32_t f16_order_key(uint16_t h) {
  if (h == 0x8000u) h = 0;
  return (h & 0x8000u) ? (uint32_t)(~h & 0xFFFFu) : (uint32_t)(h | 0x8000u);
}

// ------------------------------------------------- exact fp16 dot product --
// A product of two finite fp16 values is exact in fp32 (22-bit significand,
// magnitude in [2^-48, 2^32]) and is a multiple of 2^-48.  Each product d is
// split without error into three parts aligned to 2^12, 2^-11 and 2^-48
// (round-to-nearest "add and subtract 1.5*2^(52+B)").  Summing each part in
// its own fp64 accumulator is exact for up to 2^16 terms, in any order:
//   a2: multiples of 2^12,  |sum| <= 2^16 * (2^32 + 2^11) < 2^65
//   a1: multiples of 2^-11, |sum| <= 2^16 * 2^12          < 2^42
//   a0: multiples of 2^-48, |sum| <= 2^16 * 2^-12         < 2^5
// so partial accumulators of different threads/workgroups can be added with
// plain fp64 adds and the total stays exact (order independent).
struct Exact3 {
  double a0, a1, a2;
};

__device__ __forceinline__ Exact3 exact_zero() { return Exact3{0.0, 0.0, 0.0}; }

__device__ __forceinline__ void exact_add(Exact3& e, double d) {
  const double C2 = 27670116110564327424.0;  // 1.5 * 2^64  -> rounds to multiples of 2^12
  const double C1 = 3298534883328.0;         // 1.5 * 2^41  -> rounds to multiples of 2^-11
  double t2 = d + C2;  // no fast-math: (d + C) - C is not folded
  double c2 = t2 - C2;
  double r = d - c2;
  double t1 = r + C1;
  double c1 = t1 - C1;
  double c0 = r - c1;
  e.a2 += c2;
  e.a1 += c1;
  e.a0 += c0;
}

__device__ __forceinline__ void exact_merge(Exact3& e, const Exact3& o) {
  e.a0 += o.a0;
  e.a1 += o.a1;
  e.a2 += o.a2;
}

// Exact conversion of a double that is a multiple of 2^-48 (|v| < 2^78) to
// fixed point with LSB 2^-48.
__device__ __forceinline__ __int128 dbl_to_fix48(double v) {
  uint64_t bits = (uint64_t)__double_as_longlong(v);
  uint64_t ex = (bits >> 52) & 0x7FFull;
  if (ex == 0) return 0;
  __int128 m = (__int128)((bits & 0xFFFFFFFFFFFFFull) | (1ull << 52));
  int s = (int)ex - 1075 + 48;
  __int128 r = s >= 0 ? (m << s) : (m >> (-s));
  return (bits >> 63) ? -r : r;
}

// Round v * 2^-48 to the nearest fp16 (ties to even); overflow -> inf.
__device__ __forceinline__ uint16_t fix48_to_f16(__int128 v) {
  uint16_t sign = v < 0 ? 0x8000u : 0u;
  unsigned __int128 M = v < 0 ? (unsigned __int128)(-v) : (unsigned __int128)v;
  if (M == 0) return sign;
  uint64_t hi = (uint64_t)(M >> 64), lo = (uint64_t)M;
  int msb = hi ? 127 - __clzll((long long)hi) : 63 - __clzll((long long)lo);
  int X = msb - 48;
  if (X > 15) return sign | 0x7C00u;
  int q = X >= -14 ? X - 10 : -24;
  int shift = q + 48;  // in [24, 53]
  unsigned __int128 R = M >> shift;
  unsigned __int128 rem = M - (R << shift);
  unsigned __int128 half = (unsigned __int128)1 << (shift - 1);
  if (rem > half || (rem == half && (R & 1))) R += 1;
  if (q == -24) return sign | (uint16_t)R;
  if (R == 2048) {
    R = 1024;
    q += 1;
  }
  int ef = q + 25;
  if (ef >= 31) return sign | 0x7C00u;
  return sign | (uint16_t)(ef << 10) | (uint16_t)(R - 1024);
}

__device__ __forceinline__ uint16_t exact_to_f16(const Exact3& e) {
  __int128 v = dbl_to_fix48(e.a0) + dbl_to_fix48(e.a1) + dbl_to_fix48(e.a2);
  return fix48_to_f16(v);
}

// --------------------------------------------------------- wave helpers --
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ Exact3 wave_sum_exact(Exact3 e) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) {
    Exact3 o{__shfl_xor(e.a0, m, kWave), __shfl_xor(e.a1, m, kWave), __shfl_xor(e.a2, m, kWave)};
    exact_merge(e, o);
  }
  return e;
}

// ------------------------------------------------------------ NF4 decode --
// 32 NF4 nibbles packed in 16 bytes (element 2i in the high nibble of byte i)
// dotted with 32 fp32 activations; the code book sits in LDS.
__device__ __forceinline__ float nf4_dot32(const uint4 w, const float* __restrict__ xf, const float* lut) {
  float acc = 0.0f;
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t v = words[q];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      uint32_t byte = (v >> (8 * b)) & 0xFFu;
      acc = __builtin_fmaf(lut[byte >> 4], xf[8 * q + 2 * b], acc);
      acc = __builtin_fmaf(lut[byte & 0xFu], xf[8 * q + 2 * b + 1], acc);
    }
  }
  return acc;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// ------------------------------------------------------------- launches --
// Descriptor of one NF4 projection's block storage.  A block (slot) holds 32
// rows of a gate/up weight, or a 32-column block of the down weight.
struct ProjView {
  const uint8_t* packed;
  const float* absmax;
  long long blk_stride;      // bytes between consecutive slots
  long long row_stride;      // bytes between consecutive rows inside a slot
  long long abs_blk_stride;  // absmax entries between consecutive slots
  long long abs_row_stride;  // absmax entries between consecutive rows
};

struct DecodeArgs {
  const uint16_t* x;    // [H] fp16
  int H;
  int qbs;
  int k;                 // selected blocks
  int cs;                // columns per gate/up split
  int splits;            // H / cs
  int groups;            // down block groups
  int rows_per_chunk;    // down rows per workgroup (256)
  const int32_t* sel;    // [k] block ids, or nullptr (identity)
  const int32_t* lookup; // [NB] slot of a block, -1 = host; nullptr = identity
  int NB;
  int n_slots;
  ProjView gate, up, down;            // device slot storage
  ProjView host_gate, host_up, host_down;  // miss source indexed by block id (may be empty)
  const float* code;     // [16] gate code book
  const float* code_up;  // [16] up code book
  const float* code_down;  // [16] down code book
  const uint16_t* down_bias;  // [H] fp16 or nullptr
  const uint16_t* gate_bias;  // [NB*32] fp16 or nullptr (indexed by block id)
  const uint16_t* up_bias;    // [NB*32] fp16 or nullptr
  const uint16_t* mask;       // [NB*32] fp16 flat mask or nullptr
  int skip_negative;          // sel[j] < 0 means "no block" (not an error)
  uint16_t* out;         // [H] fp16
  float* out_f32;        // [H] fp32 result before rounding, or nullptr
  // workspace
  float* part;           // [k][splits][64]
  float* act;            // [k][32]
  int* blk_count;        // [k]
  float* outpart;        // [groups][H]
  int* row_count;        // [H / rows_per_chunk]
  int* status;           // [1] device error flag
};

// Resolve selected position j to (storage view index, validity):
// slot >= 0 -> HBM slot, slot < 0 -> host copy indexed by block id.  An id or
// slot out of range, or a missing host copy, marks the block invalid (its
// contribution is zero and status bit 1 is set).
struct BlockRef {
  long long q;
  int b;
  bool dev;
  bool ok;
  bool silent;  // invalid but expected (skipped entry)
};

__device__ __forceinline__ BlockRef resolve_block(const DecodeArgs& a, int j) {
  BlockRef r;
  const int b = a.sel ? a.sel[j] : j;
  r.b = b;
  r.ok = b >= 0 && b < a.NB;
  r.silent = a.skip_negative && b < 0;
  const int slot = r.ok ? (a.lookup ? a.lookup[b] : b) : -1;
  r.dev = slot >= 0;
  if (slot >= a.n_slots) r.ok = false;
  if (!r.dev && a.host_gate.packed == nullptr) r.ok = false;
  r.q = r.dev ? slot : b;
  return r;
}

void launch_decode_gate_up(const DecodeArgs& a, hipStream_t s);
void launch_decode_down(const DecodeArgs& a, hipStream_t s);

struct RouteArgs {
  const uint16_t* x;       // [rows][H]
  int rows, H;
  const uint16_t* enc_w;   // [R][H]
  const uint16_t* enc_b;   // [R] or nullptr
  int R, basis_top_k;
  const uint16_t* score_w; // [NB][R]
  const uint16_t* score_b; // [NB] or nullptr
  const uint16_t* dbn;     // [NB] fp16 or nullptr
  int NB, legacy_abs, sorted, k;
  int lat_splits;          // H / lat_cols
  int lat_cols;            // columns per latent workgroup
  int vec;                 // 16-byte loads allowed for x / enc_w
  int32_t* sel;            // [rows][k]
  uint16_t* latent_out;    // [rows][R] or nullptr
  uint16_t* scores_out;    // [rows][NB] or nullptr
  // workspace
  double* lat_part;        // [rows][R][lat_splits][3]
  uint16_t* scores;        // [rows][NB]
  int* status;
};

void launch_route(const RouteArgs& a, hipStream_t s);

struct LinearArgs {
  const uint16_t* x;          // [rows][in_dim]
  int rows, in_dim, out_dim;  // out_dim: input linear only
  const int32_t* active_idx;  // [rows][kk]
  int kk, A;                  // A: gathered slots (output linear)
  const uint8_t* packed;
  const float* absmax;
  const float* code;
  int qbs;
  const uint16_t* mask;       // [rows][A*32] or nullptr
  const uint16_t* bias;       // or nullptr
  uint16_t* out;
  int cs, splits;             // output linear column split
  float* part;                // [rows*kk][splits][32]
};

void launch_output_linear(const LinearArgs& a, hipStream_t s);
void launch_input_linear(const LinearArgs& a, hipStream_t s);
void launch_zero_u32(uint32_t* p, long long n, hipStream_t s);
void launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, long long n, hipStream_t s);
void launch_gather_rows(const uint8_t* src, const float* src_abs, const int32_t* blocks, int src_blocks, int n,
                        long long bpb, long long apb, uint8_t* dst, float* dst_abs, hipStream_t s);
void launch_gather_down(const uint8_t* src, const float* src_abs, const int32_t* blocks, int n, int out_f, int in_f,
                        int qbs, int layout, uint8_t* dst, float* dst_abs, hipStream_t s);
void set_nf4_midpoints(const float* mid15);
void launch_nf4_quant(const float* w, uint64_t seed, float std, long long n, int qbs, bool synth, uint8_t* packed,
                      float* absmax, hipStream_t s);
void launch_synth_normal_f16(uint64_t seed, long long n, float std, uint16_t* out, hipStream_t s);
void launch_synth_normal_f32(uint64_t seed, long long n, float std, float* out, hipStream_t s);

}  // namespace nsmlp
