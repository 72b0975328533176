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

// Round the exact sum a2 + a1 + a0 of an Exact3 to the nearest fp16 (ties to
// even; overflow -> inf; zero -> +0).  Valid for sums of up to 2^16 + 1
// products of two fp16 values: then |a1| < 2^27.1 (each part at most 2^11)
// and |a0| < 17 (each part at most 2^-12), so
//   * |a2| >= 2^30 means |sum| > 65520: inf with the sign of a2;
//   * otherwise hi = a2 + a1 is exact (a multiple of 2^-11 below 2^30.2);
//   * s + err = hi + a0 exactly (TwoSum), |err| <= half an ulp of s.
// s is then rounded to fp16 by scaling its fp16 ulp to 1 (exact): the
// fraction of the scaled s decides, and only an exact half is settled by
// the sign of err (any other fraction is at least one ulp of s from a half,
// more than |err|).  A sum just below a power of two whose s rounded up to
// it rounds to that power, as s does.
__host__ __device__ inline uint16_t exact_to_f16(const Exact3& e) {
  const double a2 = e.a2, a1 = e.a1, a0 = e.a0;
  if (fabs(a2) >= 1073741824.0) return a2 < 0.0 ? (uint16_t)0xFC00u : (uint16_t)0x7C00u;
  const double hi = a2 + a1;
  const double s = hi + a0;
  const double bb = s - hi;
  const double err = (hi - (s - bb)) + (a0 - bb);
  if (s == 0.0) return 0;
  const uint16_t sign = s < 0.0 ? (uint16_t)0x8000u : (uint16_t)0u;
  const double as = fabs(s), ae = s < 0.0 ? -err : err;
  int ex = 0;
  (void)frexp(as, &ex);  // as in [2^(ex-1), 2^ex)
  int q = ex - 1 >= -14 ? ex - 11 : -24;  // fp16 ulp exponent of as
  const double R = ldexp(as, -q);
  const double Ri = floor(R), frac = R - Ri;
  uint32_t Rn = (uint32_t)Ri;
  if (frac > 0.5 || (frac == 0.5 && (ae > 0.0 || (ae == 0.0 && (Rn & 1u))))) Rn += 1;
  if (q == -24) return sign | (uint16_t)Rn;  // subnormal (1024: the smallest normal)
  if (Rn == 2048u) {
    Rn = 1024u;
    q += 1;
  }
  const int ef = q + 25;
  if (ef >= 31) return sign | 0x7C00u;
  return sign | (uint16_t)(ef << 10) | (uint16_t)(Rn - 1024u);
}

// --------------------------------------------------------- wave helpers --
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
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
// A byte holds two NF4 codes: element 2i in the high nibble, 2i+1 in the low
// nibble.  The code books live in LDS as fp16 values at a 16-byte stride
// (entry n at byte 16n: the 16 entries sit in 16 distinct banks), so the LDS
// address of a nibble is the nibble times 16, which one SDWA instruction
// produces straight from the packed byte:
//   high nibble: byte & 0xF0                    -> v_and_b32_sdwa  (src1_sel:BYTE_b)
//   low nibble : (byte << 4) & 0xFF             -> v_lshlrev_b32_sdwa (dst_sel:BYTE_0)
// The two fp16 codes of a byte form a half2 that v_dot2_f32_f16 multiplies
// with the matching fp16 activation pair, accumulating in fp32.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

#define NSMLP_NIB_HELPERS(B)                                                                          \
  __device__ __forceinline__ uint32_t nib_hi16_##B(uint32_t w) {                                      \
    uint32_t r;                                                                                       \
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_" #B \
        : "=v"(r) : "v"(0xF0u), "v"(w));                                                              \
    return r;                                                                                         \
  }                                                                                                   \
  __device__ __forceinline__ uint32_t nib_lo16_##B(uint32_t w) {                                      \
    uint32_t r;                                                                                       \
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_" #B \
        : "=v"(r) : "v"(4u), "v"(w));                                                                 \
    return r;                                                                                         \
  }
NSMLP_NIB_HELPERS(0)
NSMLP_NIB_HELPERS(1)
NSMLP_NIB_HELPERS(2)
NSMLP_NIB_HELPERS(3)
#undef NSMLP_NIB_HELPERS

__device__ __forceinline__ half2_t as_half2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }

__device__ __forceinline__ _Float16 lut_at(const char* lut, uint32_t off) {
  return *reinterpret_cast<const _Float16*>(lut + off);
}

// Codes of the 8 nibbles of one packed dword, dotted with 4 activation pairs.
__device__ __forceinline__ float nf4_dot8(uint32_t v, const uint32_t* xp, const char* lut, float acc) {
  half2_t c0 = {lut_at(lut, nib_hi16_0(v)), lut_at(lut, nib_lo16_0(v))};
  half2_t c1 = {lut_at(lut, nib_hi16_1(v)), lut_at(lut, nib_lo16_1(v))};
  half2_t c2 = {lut_at(lut, nib_hi16_2(v)), lut_at(lut, nib_lo16_2(v))};
  half2_t c3 = {lut_at(lut, nib_hi16_3(v)), lut_at(lut, nib_lo16_3(v))};
  acc = __builtin_amdgcn_fdot2(c0, as_half2(xp[0]), acc, false);
  acc = __builtin_amdgcn_fdot2(c1, as_half2(xp[1]), acc, false);
  acc = __builtin_amdgcn_fdot2(c2, as_half2(xp[2]), acc, false);
  acc = __builtin_amdgcn_fdot2(c3, as_half2(xp[3]), acc, false);
  return acc;
}

// 32 NF4 codes (16 bytes) dotted with 16 activation pairs.
__device__ __forceinline__ float nf4_dot32(const uint4 w, const uint32_t* xp, const char* lut) {
  float acc = nf4_dot8(w.x, xp, lut, 0.0f);
  acc = nf4_dot8(w.y, xp + 4, lut, acc);
  acc = nf4_dot8(w.z, xp + 8, lut, acc);
  return nf4_dot8(w.w, xp + 12, lut, acc);
}

// Byte-indexed code-pair table: entry b (4 bytes at offset 4b) holds the fp16
// codes of the byte's high nibble (low half) and low nibble (high half), so
// one LDS read yields the half2 for v_dot2.  The offset 4b comes from one
// SDWA shift.
#define NSMLP_BYTE4_HELPER(B)                                                                         \
  __device__ __forceinline__ uint32_t byte_x4_##B(uint32_t w) {                                       \
    uint32_t r;                                                                                       \
    asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_" #B \
        : "=v"(r) : "v"(2u), "v"(w));                                                                 \
    return r;                                                                                         \
  }
NSMLP_BYTE4_HELPER(0)
NSMLP_BYTE4_HELPER(1)
NSMLP_BYTE4_HELPER(2)
NSMLP_BYTE4_HELPER(3)
#undef NSMLP_BYTE4_HELPER

__device__ __forceinline__ uint32_t pair_at(const char* lut, uint32_t off) {
  return *reinterpret_cast<const uint32_t*>(lut + off);
}

__device__ __forceinline__ float nf4_dot8_pairs(uint32_t v, const uint32_t* xp, const char* lut, float acc) {
  const uint32_t p0 = pair_at(lut, byte_x4_0(v)), p1 = pair_at(lut, byte_x4_1(v));
  const uint32_t p2 = pair_at(lut, byte_x4_2(v)), p3 = pair_at(lut, byte_x4_3(v));
  acc = __builtin_amdgcn_fdot2(as_half2(p0), as_half2(xp[0]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_half2(p1), as_half2(xp[1]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_half2(p2), as_half2(xp[2]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_half2(p3), as_half2(xp[3]), acc, false);
  return acc;
}

// 32 NF4 codes dotted with 16 activation pairs through the byte-pair table.
__device__ __forceinline__ float nf4_dot32_pairs(const uint4 w, const uint32_t* xp, const char* lut) {
  float acc = nf4_dot8_pairs(w.x, xp, lut, 0.0f);
  acc = nf4_dot8_pairs(w.y, xp + 4, lut, acc);
  acc = nf4_dot8_pairs(w.z, xp + 8, lut, acc);
  return nf4_dot8_pairs(w.w, xp + 12, lut, acc);
}

// Fill the 256-entry byte-pair table (1 KB of LDS); needs >= 256 threads.
__device__ __forceinline__ void pair_lut_fill(char* lut, const float* code, int tid) {
  if (tid < 256) {
    const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)code[tid >> 4]);
    const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)code[tid & 15]);
    reinterpret_cast<uint32_t*>(lut)[tid] = hi | (lo << 16);
  }
}

// Lane-replicated byte-pair table (64 KB of LDS, which must start at LDS
// address 0): entry e of copy c sits at byte e * 256 + c * 4, so a lane that
// always reads copy c always hits bank c and the 64 lookups of a wave never
// conflict, whatever bytes they decode.  The lane keeps c * 4 in the low byte
// of an address register; one SDWA move writes the packed byte into bits
// 8..15 and preserves the rest, so a lookup costs one VALU op and one
// ds_read_b32.
constexpr int kRepLutBytes = 65536;

#define NSMLP_SET_BYTE1(ad, w, sel) \
  asm("v_mov_b32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:" sel : "+v"(ad) : "v"(w))

typedef const __attribute__((address_space(3))) uint32_t* lds_u32_ptr;
__device__ __forceinline__ uint32_t lds_ld_u32(uint32_t byte_addr) {
  return *reinterpret_cast<lds_u32_ptr>(static_cast<uintptr_t>(byte_addr));
}

__device__ __forceinline__ float rep_dot8(uint32_t v, const uint32_t* xp, uint32_t (&ad)[4], float acc) {
  NSMLP_SET_BYTE1(ad[0], v, "BYTE_0");
  NSMLP_SET_BYTE1(ad[1], v, "BYTE_1");
  NSMLP_SET_BYTE1(ad[2], v, "BYTE_2");
  NSMLP_SET_BYTE1(ad[3], v, "BYTE_3");
  const uint32_t p0 = lds_ld_u32(ad[0]), p1 = lds_ld_u32(ad[1]);
  const uint32_t p2 = lds_ld_u32(ad[2]), p3 = lds_ld_u32(ad[3]);
  acc = __builtin_amdgcn_fdot2(as_half2(p0), as_half2(xp[0]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_half2(p1), as_half2(xp[1]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_half2(p2), as_half2(xp[2]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_half2(p3), as_half2(xp[3]), acc, false);
  return acc;
}

// 32 NF4 codes (16 packed bytes) dotted with 16 fp16 pairs, fp32 accumulation
// in element order (the same sequence of v_dot2 as nf4_dot32_pairs).
__device__ __forceinline__ float rep_dot32(const uint4 w, const uint32_t* xp, uint32_t (&ad)[4]) {
  float acc = rep_dot8(w.x, xp, ad, 0.0f);
  acc = rep_dot8(w.y, xp + 4, ad, acc);
  acc = rep_dot8(w.z, xp + 8, ad, acc);
  return rep_dot8(w.w, xp + 12, ad, acc);
}

// Nontemporal (streaming) loads for weight data read exactly once.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_stream16(const uint8_t* p) {
  const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ float ld_stream_f32(const float* p) { return __builtin_nontemporal_load(p); }

// fp32 variant for the multi-row linears: code book as 16 fp32 values in LDS.
__device__ __forceinline__ float nf4_dot32_f32(const uint4 w, const float* __restrict__ xf, const float* lut) {
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

// Fill a 16-entry fp16 code book at a 16-byte stride (256 bytes of LDS).
__device__ __forceinline__ void lut_fill(char* lut, const float* code, int tid) {
  if (tid < 16) *reinterpret_cast<_Float16*>(lut + 16 * tid) = (_Float16)code[tid];
}

// Coherent (L2 write-through / bypass) accesses for data handed between
// workgroups inside one launch; ordering: stores, then s_waitcnt vmcnt(0),
// then the counter atomic.
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ int ld_coherent_i32(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coherent_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent_i32(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// ------------------------------------------------------------------ MFMA --
// v_mfma_f32_16x16x32_f16 lane layout (measured): A[i][k] and B[k][j] in lane
// l hold i (or j) = l % 16, k = 8 (l / 16) + 0..7; C[i][j] in lane l holds
// j = l % 16, i = 4 (l / 16) + r, r = 0..3.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half8_t as_h8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_f16 lane layout (measured with one-hot operands):
// A[i][k] and B[k][j] in lane l hold i (or j) = l % 32, k = 8 (l / 32) +
// 0..7; C[i][j] in lane l holds j = l % 32, element r = 0..15 holding
// i = 8 (r / 4) + 4 (l / 32) + r % 4.
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float16_t mfma32(half8_t a, half8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Wait states between MFMAs and VALU reads of their results, beyond what the
// compiler inserts: reads of a 16x16x32 result that follow its MFMA closely
// have returned values that changed from run to run in the last elements
// (written last), so MFMA results are read only after this drain (long
// enough for the 32x32x16 shape's 16 passes too).
__device__ __forceinline__ void mfma_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------- buffer loads --
// Weight streams use raw buffer loads through per-block descriptors: a
// descriptor whose extent is zero (or an offset past the extent) makes the
// load return zeros without touching memory, so loads stay unconditional and
// the compiler's wait counts stay exact (a branch around a load makes it wait
// for every load in flight).
// Keeps the compiler from moving instructions across this point (load issue
// order decides which waits drain the weight stream).
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Kernel arguments are read from memory (the kernarg segment), and the
// compiler places each field's load where the field is first used, so a field
// first used after a global load costs a round trip of its own.  Reading every
// 64-byte line of the arguments at the start of a kernel (one batch of scalar
// loads, data discarded) puts them in the scalar cache; the compiler's own
// loads of the fields then hit it wherever they are placed.
template <int kBytes>
__device__ __forceinline__ void kernarg_warm() {
  static_assert(kBytes >= 64 && kBytes <= 4096 && kBytes % 4 == 0, "argument block size");
  // whole 64-byte pieces, then one piece ending at the block's end (it
  // overlaps the previous one): no load reads past the argument block
  constexpr int kFull = kBytes / 64;
  constexpr int kTail = kBytes % 64 != 0 ? kBytes - 64 : -1;
  const auto kp = __builtin_amdgcn_kernarg_segment_ptr();
  typedef int v16i __attribute__((ext_vector_type(16)));
  v16i d;
  asm volatile(
      ".set .Lnsmlp_kw, 0\n\t"
      ".rept %2\n\t"
      "s_load_dwordx16 %0, %1, .Lnsmlp_kw\n\t"
      ".set .Lnsmlp_kw, .Lnsmlp_kw + 64\n\t"
      ".endr\n\t"
      ".if %3 >= 0\n\t"
      "s_load_dwordx16 %0, %1, %3\n\t"
      ".endif\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(d)
      : "s"(kp), "i"(kFull), "i"(kTail)
      : "memory");
}

// Raw buffer descriptors (gfx9 family dword format) and nontemporal loads.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kNontemporal = 2;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRsrcWord3);
}
// Descriptor of a range that is the same in every lane of the wave, built in
// scalar registers: the compiler cannot always tell that a value derived
// from a global load is uniform, and a descriptor in vector registers turns
// every load through it into a loop over the lanes' values.
__device__ __forceinline__ rsrc_t make_rsrc_uniform(const void* base, int bytes) {
  const unsigned long long v = reinterpret_cast<unsigned long long>(base);
  const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)v);
  const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(v >> 32));
  return make_rsrc(reinterpret_cast<const void*>(((unsigned long long)hi << 32) | lo),
                   __builtin_amdgcn_readfirstlane(bytes));
}
__device__ __forceinline__ uint4 buf_ld16(rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kNontemporal);
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint2 buf_ld8(rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x2_t t = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, kNontemporal);
  return make_uint2(t.x, t.y);
}
__device__ __forceinline__ float buf_ldf(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, kNontemporal));
}
__device__ __forceinline__ uint32_t buf_ldu8(rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)voff, (int)soff, kNontemporal);
}
// Cached (temporal) variants, for data that other workgroups read again.
__device__ __forceinline__ uint4 buf_ld16c(rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint2 buf_ld8c(rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x2_t t = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
  return make_uint2(t.x, t.y);
}
__device__ __forceinline__ uint32_t buf_ldu8c(rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ int buf_ldic(rsrc_t r, uint32_t voff, uint32_t soff) {
  return (int)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}
__device__ __forceinline__ float buf_ldfc(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
constexpr uint32_t kOffNone = 0x80000000u;  // an offset past every extent: the load returns zeros
__device__ __forceinline__ uint32_t buf_ldu16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, kNontemporal);
}

// Buffer loads into LDS (lane l's bytes at LDS address base + 16 l, or 4 l
// for the dword and byte forms; the byte form zero-extends to a dword).
// Written as asm: the compiler then neither counts them in its own wait
// counts (which only makes those waits longer than needed, never shorter)
// nor waits for them before every later LDS read; the kernel waits for
// them itself.  `base` is the wave's LDS byte address (uniform).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)p);
}
__device__ __forceinline__ void ld_lds16(rsrc_t r, const void* lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(voff), "s"(lds_addr(lds)), "s"(r)
               : "memory", "m0");
}
// Same, with a uniform byte offset added to every lane's (an SGPR operand).
__device__ __forceinline__ void ld_lds16s(rsrc_t r, const void* lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, %3 offen lds" ::"v"(voff), "s"(lds_addr(lds)), "s"(r),
               "s"(soff)
               : "memory", "m0");
}
__device__ __forceinline__ void ld_lds4(rsrc_t r, const void* lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dword %0, %2, 0 offen lds" ::"v"(voff), "s"(lds_addr(lds)), "s"(r)
               : "memory", "m0");
}
__device__ __forceinline__ void ld_lds4s(rsrc_t r, const void* lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dword %0, %2, %3 offen lds" ::"v"(voff), "s"(lds_addr(lds)), "s"(r),
               "s"(soff)
               : "memory", "m0");
}
__device__ __forceinline__ void ld_lds1s(rsrc_t r, const void* lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_ubyte %0, %2, %3 offen lds" ::"v"(voff), "s"(lds_addr(lds)), "s"(r),
               "s"(soff)
               : "memory", "m0");
}
__device__ __forceinline__ void ld_lds1(rsrc_t r, const void* lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_ubyte %0, %2, 0 offen lds" ::"v"(voff), "s"(lds_addr(lds)), "s"(r)
               : "memory", "m0");
}
// Workgroup barrier after this wave's LDS accesses: waits for the LDS
// counter only (no memory fence, no wait for vector loads in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ------------------------------------------------------------------ top-k --
// Workgroup top-k of NB fp16 scores.  Keys are fp16 order keys; among equal
// scores the lower block index ranks higher (the order of the unique key
// order16 << 16 | ~index).  Each of NTHR threads holds KPT consecutive keys
// (thread t: indices t*KPT ..).  Two 8-bit histogram passes find the k-th
// largest score T and how many entries equal to T are taken (`need`); the
// scan gives each thread the counts above T (gt) and equal to T (eq) before
// its range, so an ordered compaction can place every selected index.
struct TopkLds {
  unsigned hist[2][256];  // one histogram per pass, both cleared up front
  unsigned wsum[16];
};

// Inclusive prefix sum over the 64 lanes (all active) with DPP moves: a
// Hillis-Steele scan inside each row of 16 lanes (row_shr 1, 2, 4, 8; lanes
// shifted in from before the row read 0), then the row totals carried over
// (row_bcast:15 adds lane 15 to row 1 and lane 47 to row 3; row_bcast:31
// adds lane 31 to rows 2 and 3).  No LDS round trip per step.
__device__ __forceinline__ unsigned wave_incl_scan(unsigned v, int lane) {
  (void)lane;
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// Run by every wave on its own (no barrier after it): the digit (from the
// top) holding the remaining-th largest entry of hist, and the count of
// entries in higher digits, in every lane.
__device__ __forceinline__ void topk_find_digit(const unsigned* hist, unsigned remaining, int lane, unsigned& digit,
                                                unsigned& above) {
  // lane l holds digits 255 - 4l .. 252 - 4l (plain registers: no array, so
  // nothing is placed in scratch memory)
  const unsigned c0 = hist[255 - 4 * lane], c1 = hist[254 - 4 * lane];
  const unsigned c2 = hist[253 - 4 * lane], c3 = hist[252 - 4 * lane];
  const unsigned local = c0 + c1 + c2 + c3;
  const unsigned incl = wave_incl_scan(local, lane);
  const unsigned excl = incl - local;
  const bool mine = excl < remaining && remaining <= incl;
  unsigned b = 3, cum = excl + c0 + c1 + c2;
  if (excl + c0 >= remaining) {
    b = 0;
    cum = excl;
  } else if (excl + c0 + c1 >= remaining) {
    b = 1;
    cum = excl + c0;
  } else if (excl + c0 + c1 + c2 >= remaining) {
    b = 2;
    cum = excl + c0 + c1;
  }
  const unsigned long long m = __ballot(mine);
  const int src = m ? __ffsll((long long)m) - 1 : 0;
  digit = (unsigned)__shfl((int)(255u - 4u * lane - b), src, kWave);
  above = (unsigned)__shfl((int)cum, src, kWave);
}

// Clears both histograms; the caller puts a barrier between this and
// topk_threshold (best while the keys are still being loaded).
template <int NTHR>
__device__ __forceinline__ void topk_clear(TopkLds& L) {
  for (int i = threadIdx.x; i < 2 * 256; i += NTHR) (&L.hist[0][0])[i] = 0;
}

template <int NTHR, int KPT>
__device__ __forceinline__ void topk_threshold(const uint32_t (&key)[KPT], int i0, int NB, int k, TopkLds& L,
                                               uint32_t& T, unsigned& need, unsigned& gt, unsigned& eq) {
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  T = 0;
  unsigned remaining = (unsigned)k;
  for (int pass = 0; pass < 2; ++pass) {
    // Scores clamped at zero are common (about half at the 405B shape) and
    // share one bin: they are counted per wave and added once, instead of
    // contending on one LDS counter.
    constexpr uint32_t kZeroKey = 0x8000u;  // order key of +0.0
    unsigned nzero = 0;  // this wave's zero keys of the pass (ballot counts: uniform over the wave)
#pragma unroll
    for (int m = 0; m < KPT; ++m) {
      const bool in = i0 + m < NB;
      const bool isz = in && key[m] == kZeroKey;
      nzero += (unsigned)__popcll(__ballot(isz && (pass == 0 || (T >> 8) == (kZeroKey >> 8))));
      if (!in || isz) continue;
      if (pass == 0) {
        atomicAdd(&L.hist[0][key[m] >> 8], 1u);
      } else if ((key[m] >> 8) == (T >> 8)) {
        atomicAdd(&L.hist[1][key[m] & 0xFFu], 1u);
      }
    }
    if (lane == 0 && nzero != 0)
      atomicAdd(&L.hist[pass][pass == 0 ? (kZeroKey >> 8) : (kZeroKey & 0xFFu)], nzero);
    __syncthreads();
    unsigned digit, above;
    topk_find_digit(L.hist[pass], remaining, lane, digit, above);
    T |= digit << (pass == 0 ? 8 : 0);
    remaining -= above;
  }
  need = remaining;
  // counts of keys above T (high half) and equal to T (low half) before this
  // thread's keys; both stay below 2^16 since NB <= 65535
  unsigned cnt = 0;
#pragma unroll
  for (int m = 0; m < KPT; ++m)
    if (i0 + m < NB) cnt += key[m] > T ? (1u << 16) : (key[m] == T ? 1u : 0u);
  const unsigned incl = wave_incl_scan(cnt, lane);
  if (lane == kWave - 1) L.wsum[wave] = incl;
  __syncthreads();
  // the earlier waves' totals: every wave reads all of them at once (a loop
  // of dependent reads up to the wave index made the last wave the slowest)
  unsigned before = incl - cnt;
#pragma unroll
  for (int w = 0; w < NTHR / kWave; ++w) before += w < wave ? L.wsum[w] : 0u;
  gt = before >> 16;
  eq = before & 0xFFFFu;
}

// Position of a key in ascending block order among the selected, or -1; gt /
// eq count the keys above / equal to T before it.  The caller advances them
// (gt += key > T, eq += key == T): plain values, so nothing goes to scratch.
__device__ __forceinline__ int topk_position(uint32_t key, uint32_t T, unsigned need, unsigned gt, unsigned eq) {
  // selects, not branches: every key of every thread goes through it
  const int p = (int)(gt + (eq < need ? eq : need));  // above T, or equal and among the first `need`
  const bool take = key > T || (key == T && eq < need);
  return take ? p : -1;
}

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
  // double-quantised absmax (DecodeArgs::dq): u8 codes at the absmax
  // positions, second-level scales of the full weight, code book, offset
  const uint8_t* qabsmax;
  const float* absmax2;
  const float* code2;
  float offset;
};

// Double-quantised absmax value: fp32(fp32(code2[q] * absmax2) + offset),
// both roundings kept (no fused multiply-add), as the reference resolves it
// (dequantize_blockwise, then + offset; RT:4621-4625).
__device__ __forceinline__ float dq_absmax(float code2_q, float absmax2, float offset) {
#pragma clang fp contract(off)
  return code2_q * absmax2 + offset;
}

struct DecodeArgs {
  const uint16_t* x;    // [H] fp16
  int H;
  int qbs;
  int qbs_shift;         // log2(qbs)
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
  const uint16_t* residual;  // [H] fp16 added to the rounded output, or nullptr
  // workspace
  float* part;           // [k][splits][64]
  uint32_t* act;         // [k][16] fp16 pairs of silu(gate)*up, scaled by 2^act_exp
  float* act_scale;      // [k] 2^-act_exp (undoes the scaling)
  int* blk_count;        // [k]
  float* outpart;        // [groups][H]
  int* row_count;        // [H / rows_per_chunk]
  int* status;           // [1] device error flag
  int chunks;            // down row chunks
  // streaming path (hidden size a multiple of 2048)
  float* st_act;         // [k][32] silu(gate) * up of the selected blocks
  uint32_t* st_enc;      // [k] resolved block references
  int st_gu_wgs;         // gate/up workgroups (0: streaming path not used)
  int st_gu_rounds;      // gate/up rounds per workgroup
  int st_dn_gx;          // down workgroups per 64-row chunk (block groups)
  int st_dn_per;         // blocks per down wave (<= 64)
  int st_gu_bytes;       // extent of one gate/up slot: packed bytes, absmax bytes
  int st_gu_abytes;
  int st_dn_bytes;       // extent of one down block: packed bytes, absmax bytes
  int st_dn_abytes;
  // with sel_scores != nullptr the gate/up kernel selects the top k of these
  // fp16 scores itself (ascending ids, ties to the lower id) and writes them
  // to sel_out; sel is then unused
  const uint16_t* sel_scores;  // [NB]
  int32_t* sel_out;            // [k]
  // double-quantised absmax: absmax of flat index f (in the full weight:
  // gate/up (32 b + r) * (H / qbs) + c / qbs, down o * (I / qbs) + 32 b / qbs)
  // uses absmax2[f >> dq_shift]
  int dq;
  int dq_shift;
  int32_t* st_bid;       // [k] block ids of the selected positions (streaming)
  int st_gu_a2bytes;     // extent of gate/up absmax2 (bytes)
  int st_dn_a2n;         // down absmax2 entries staged per 64-row chunk
  // [2] selected blocks read from HBM slots, from host copies (added per
  // call, kept until taken); nullptr: not counted
  uint32_t* served;
};

// Output row o of a decode: the MLP sum y (+ bias) rounded once to fp16;
// with a residual, fp16(residual[o] + that value), the decode loop's fp16 add
// (hidden = residual + mlp_out).  out_f32 keeps the sum before the bias.
__device__ __forceinline__ uint16_t decode_out(const DecodeArgs& a, int o, float y) {
  if (a.out_f32 != nullptr) a.out_f32[o] = y;
  if (a.down_bias != nullptr) y += h2f(a.down_bias[o]);
  uint16_t h = f2h(y);
  if (a.residual != nullptr) h = f2h(h2f(a.residual[o]) + h2f(h));
  return h;
}

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

// Same, from the block id b = sel[j] already loaded.
__device__ __forceinline__ BlockRef resolve_id(const DecodeArgs& a, int b) {
  BlockRef r;
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

__device__ __forceinline__ BlockRef resolve_block(const DecodeArgs& a, int j) {
  return resolve_id(a, a.sel ? a.sel[j] : j);
}

// Chunked prefill (M tokens, per-token block sets) over a slot table.
struct PrefillArgs {
  DecodeArgs d;           // slot table views, H, qbs, NB, code, dq state, status
  const uint16_t* x;      // [M][H] fp16
  int M;
  const int32_t* sel;     // [M][k] block ids
  int k;
  uint16_t* out;          // [M][H] fp16
  uint32_t* bitmap;       // [NB][words]
  int words;              // ceil(M / 32)
  int32_t* offsets;       // [NB + 1] CSR offsets
  int32_t* grp;           // [NB][TG + 1] CSR index of the first token of each 128-token group
  int TG;                 // token groups
  int32_t* tokens;        // [M k] token ids per block, ascending
  uint16_t* act;          // [M k][32] fp16 silu(gate) * up per (block, token) entry (grouped down)
  // dense down (when the union covers most blocks): act scattered into a
  // zeroed [M][NB 32] matrix, then the dense-guard down GEMM over it
  uint16_t* act_dense;    // or nullptr
  float* part;            // [S][M][H] fp32 partial sums
  int S;
};
void launch_prefill(const PrefillArgs& p, hipStream_t s);
int prefill_gu_check();  // NSMLP_OK, or the error (static LDS in the gate/up kernel)

// Dense-guard prefill MLP: every block for every token (M tokens) over a slot
// table, as staged GEMMs on MFMA.  H % 256 == 0, NB % 4 == 0.
struct DenseGuardArgs {
  DecodeArgs d;              // slot table views, H, NB, qbs, code books, dq state, status, down_bias
  const uint16_t* x;         // [M][H] fp16
  int M;
  uint16_t* act;             // [M][NB*32] fp16 (workspace)
  float* part;               // [S][M][H] fp32 partial sums over S block ranges (workspace)
  int S;
  uint16_t* out;             // [M][H] fp16
  const uint16_t* residual;  // [M][H] fp16 added to the rounded output, or nullptr
  int t_base;                // first token of the launch's tiles (set by the launchers)
  // the prefill's dense down: CSR offsets [NB + 1] of the blocks' token lists;
  // a block with no tokens has an all-zero act column and its down weights
  // are not read (nullptr: every block is read)
  const int32_t* offsets;
  // gate/up work split (set by the launcher): gu_full whole items first,
  // then the K steps of gu_tail items in ranges of gu_per steps; the split
  // items' fp32 sums in gu_part (the down partials' space, free until the
  // down GEMM)
  int gu_full, gu_tail, gu_per;
  float* gu_part;
};
void launch_dense_guard(const DenseGuardArgs& g, hipStream_t s);
// Bytes of the gate/up tail's partial sums for a dense call of M tokens per
// chunk (g.part must hold at least this many).
size_t dense_gu_tail_bytes(int M);
// The down GEMM and the final sum alone, over g.act (the prefill's dense path).
void launch_dense_down(const DenseGuardArgs& g, hipStream_t s);
// Whether the down GEMM takes this table with S block ranges: every slot and
// host copy addressable by 31-bit offsets, the range's block references in LDS.
bool dense_down_fits(const DecodeArgs& d, int S);
int dense_down_refs(int NB, int S);
// NSMLP_OK when the down GEMM's compiled kernels have no static LDS (its LDS
// addressing assumes so); otherwise an error status with the message set.
int dense_down_check();

// Dense NF4 rows (the LM head): y[t][o] = sum_i W[o][i] x[t][i] over a
// row-major [out][in] NF4 matrix, in % 32 == 0, in <= 16384.
struct RowsArgs {
  const uint16_t* x;  // [nt][in] fp16
  int in, out;
  int qbs_shift;
  const uint8_t* packed;  // [out][in/2]
  int rs;                 // bytes per row (in / 2)
  int p_bytes;            // out * rs (buffer extent)
  int ars;                // absmax per row (in / qbs)
  const float* absmax;    // [out][in/qbs] f32 (dq = 0)
  const uint8_t* qabsmax; // [out][in/qbs] u8 codes (dq = 1)
  int a_bytes;            // extent of the absmax array
  const float* absmax2;   // per dq block of the flat absmax index
  int a2_bytes;
  const float* code2;     // [256]
  float offset;
  int dq, dq_shift;
  const float* code;      // [16]
  uint16_t* y;            // [nt][out] fp16
  float* out_f32;         // [nt][out] or NULL
  int splits, rounds, wgs;
};
bool plan_rows(RowsArgs& a, int nt, int cus);  // nt tokens per pass (1 or 2)
void launch_rows(const RowsArgs& a, int nt, hipStream_t s);

// Hot-block cache maintenance (fixed-capacity promotion and calibration
// counts) over a slot table with pinned host copies.
constexpr int kMaxCacheSlots = 8192;  // capacity limit (eviction order staged in LDS)
struct CacheArgs {
  int NB;
  int capacity;
  int n;          // entries of blocks
  int grow_only;  // 1: free slots only, no eviction
  int32_t* lookup;      // [NB] block -> slot or -1
  int32_t* slot_block;  // [capacity] slot -> block or -1
  float* slot_score;    // [capacity]
  int32_t* active;      // [1]
  const int32_t* blocks;  // [n] candidate blocks (a token's selection)
  int32_t* plan_out;      // [n] slot given to each entry or -1; nullable
  int32_t* novel;         // workspace [n]
  int32_t* copy_block;    // workspace [min(n, capacity)]
  int32_t* copy_slot;     // workspace [min(n, capacity)]
  int32_t* n_copy;        // workspace [1]
  const uint8_t* src[6];  // host copies by block id: gate packed, gate absmax, up packed, up absmax,
  uint8_t* dst[6];        //   down packed, down absmax; slots by slot index
  long long bytes[6];     // bytes per block of each array (multiples of 16)
};
void launch_cache_promote(const CacheArgs& c, hipStream_t s);
void launch_cache_record(float* counts, int NB, const int32_t* blocks, int rows, int k, const float* w,
                         hipStream_t s);

void launch_decode_gate_up(const DecodeArgs& a, hipStream_t s);
void launch_decode_down(const DecodeArgs& a, hipStream_t s);
// Streaming decode (hidden size a multiple of 2048): gate/up, down, final sum.
// Sets the st_* tiling fields for a device with `cus` compute units; false
// (and st_gu_wgs = 0) when the streaming kernels do not apply.
bool plan_streaming(DecodeArgs& a, int cus);
// Whether the streaming kernels can select the top k themselves (NB, k limits).
bool streaming_can_select(int NB, int k);
void launch_decode_streaming(const DecodeArgs& a, hipStream_t s);
int device_cus();

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
  int vec;                 // 16-byte loads allowed for x / enc_w
  int svec;                // 16-byte loads allowed for score_w rows (R % 8 == 0, aligned)
  int32_t* sel;            // [rows][k]
  uint16_t* latent_out;    // [rows][R] or nullptr
  uint16_t* scores_out;    // [rows][NB] or nullptr
  // workspace
  uint16_t* lat16;         // [rows][R] fp16 latent
  uint16_t* scores;        // [rows][NB]
  int* status;
  // fewer than kLatSplitRows rows: the latent's exact sums in kLatParts
  // column ranges [rows][R][kLatParts] x (a0, a1, a2), merged and rounded by
  // the scores kernel; nullptr otherwise
  double* lat_part;
  // [kClearWords] words zeroed by the first latent kernel before anything of
  // the call is written (the per-call status and block counts of a shared
  // scratch); nullptr: none
  int* clear_words;
  // kLatSplitRows rows or more (16-byte loads): the matrix-core first pass's
  // fp64 sums in lat_nparts column ranges [nparts][rows][R], their magnitude
  // sums (fp32, same layout), the outputs left undecided [rows R] and their
  // count; nullptr otherwise
  double* lat_p64;
  float* lat_p32;
  int* lat_und;
  int* lat_und_n;
  int lat_nparts;
  // kLatSplitRows rows or more: the scores on the matrix cores (16-byte
  // score_w rows): the latent with the basis_top_k mask ([rows][R] fp16),
  // the undecided scores [rows NB] and their count; nullptr otherwise
  uint16_t* lat_m;
  int* sc_und;
  int* sc_und_n;
};
constexpr int kClearWords = 8;
constexpr int kLatSplitRows = 8;
constexpr int kLatParts = 4;
// Column ranges of the matrix-core latent: two 4-wave workgroups per CU over
// the 16 x 16 (token, latent row) tiles, at most 32 ranges, each wave at
// least 32 columns.
__host__ __device__ inline int latent_mf_parts(int rows, int R, int H) {
  const int tiles = ((rows + 15) / 16) * ((R + 15) / 16);
  int P = (512 + tiles - 1) / tiles;
  if (P > 32) P = 32;
  while (P > 1 && 4 * P * 32 > H) P >>= 1;
  return P < 1 ? 1 : P;
}

void launch_route(const RouteArgs& a, hipStream_t s);
// The latent and score kernels only (the top-k runs inside the decode).
void launch_route_scores(const RouteArgs& a, hipStream_t s);

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
  int bm;                     // input linear: 32-column slots per active block
};

void launch_output_linear(const LinearArgs& a, hipStream_t s);
void launch_input_linear(const LinearArgs& a, hipStream_t s);
void launch_zero_u32(uint32_t* p, long long n, hipStream_t s);
void launch_take_status(int* status, int* dst, hipStream_t s);
void launch_take_counts(uint32_t* counts, long long* dst, hipStream_t s);
void launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, long long n, hipStream_t s);
template <typename AbsT>  // float or uint8_t (double-quantised codes)
void launch_gather_rows(const uint8_t* src, const AbsT* src_abs, const int32_t* blocks, int src_blocks, int n,
                        long long bpb, long long apb, uint8_t* dst, AbsT* dst_abs, hipStream_t s);
template <typename AbsT>
void launch_gather_down(const uint8_t* src, const AbsT* src_abs, const int32_t* blocks, int n, int out_f, int in_f,
                        int qbs, int layout, uint8_t* dst, AbsT* dst_abs, hipStream_t s);
// u8 absmax codes into the interleaved slot layout (and, when src_packed is
// non-NULL, the packed bytes as launch_gather_rows does).
void launch_gather_rows_q8(const uint8_t* src_packed, const uint8_t* src_q, const int32_t* blocks, int src_blocks,
                           int n, long long bpb, int A, uint8_t* dst_packed, uint8_t* dst_q, hipStream_t s);
void launch_absmax_dq(const float* absmax, long long n, int dq_block, const float* code2, float offset, uint8_t* q,
                      float* absmax2, hipStream_t s);
void launch_absmax_undq(const uint8_t* q, long long n, int dq_shift, const float* code2, const float* absmax2,
                        float offset, float* out, hipStream_t s);
void set_nf4_midpoints(const float* mid15);
void launch_nf4_quant(const float* w, uint64_t seed, float std, long long n, int qbs, bool synth, uint8_t* packed,
                      float* absmax, hipStream_t s);
void launch_synth_normal_f16(uint64_t seed, long long n, float std, uint16_t* out, hipStream_t s);
void launch_synth_normal_f32(uint64_t seed, long long n, float std, float* out, hipStream_t s);

}  // namespace nsmlp
