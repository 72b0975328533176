// NF4 decode in registers for the MFMA GEMMs (dense-guard gate/up and down,
// prefill gate/up): packed NF4 bytes -> fp16(code * absmax), the reference
// fallback's rounding of the weights (bitsandbytes dequantisation to fp16,
// RT:5439-5447), through a lane-replicated fp32 code-pair table in LDS.
//
// The table sits at LDS address 0 (the kernels that use it have no static
// LDS): entry e (a packed byte) holds (code[e >> 4], code[e & 15]) as two
// fp32, in kRdCopies copies of 8 bytes; lane l reads copy l % kRdCopies, so
// the 16 lanes an LDS cycle serves read 16 different bank pairs whatever
// their bytes are.  A lookup address is the lane's copy offset (low byte)
// with the packed byte in bits 8..15, set by one SDWA move.
#pragma once

#include "nsmlp_internal.h"

namespace nsmlp {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float rd_f2_t __attribute__((ext_vector_type(2)));

constexpr int kRdCopies = 32;                          // code-pair table copies (lane % 32)
constexpr uint32_t kRdTab = 256u * kRdCopies * 8u;     // 64 KB at LDS address 0

typedef const __attribute__((address_space(3))) rd_f2_t* lds_f2_ptr;
typedef const __attribute__((address_space(3))) half8_t* lds_h8_ptr;
__device__ __forceinline__ rd_f2_t lds_ld_f2(uint32_t byte_addr) {
  return *reinterpret_cast<lds_f2_ptr>(static_cast<uintptr_t>(byte_addr));
}
__device__ __forceinline__ half8_t lds_ld_h8(uint32_t byte_addr) {
  return *reinterpret_cast<lds_h8_ptr>(static_cast<uintptr_t>(byte_addr));
}

// The table, filled by 256 threads: thread e writes the 32 copies of entry e,
// 256 contiguous bytes.
__device__ __forceinline__ void rd_table_fill(uint8_t* lds0, const float* code, int tid) {
  const float hi = code[tid >> 4], lo = code[tid & 15];
  uint4* dst = reinterpret_cast<uint4*>(lds0 + tid * 256);
  const uint4 v = make_uint4(__float_as_uint(hi), __float_as_uint(lo), __float_as_uint(hi), __float_as_uint(lo));
#pragma unroll
  for (int i = 0; i < 16; ++i) dst[i] = v;
}

// 8 NF4 codes (one packed dword, even element in the high nibble) ->
// 8 fp16(code * am) in element order, in two halves so that the table
// lookups can go out a unit ahead of their use: rd_lookup4 reads the four
// code pairs, rd_finish8 scales them and rounds to fp16 (two fp32 products
// per v_cvt_pk_f16_f32).  ad[i] holds this lane's copy offset (copy * 8) in
// its low byte; the packed byte goes into bits 8..15.
struct RdPairs {
  rd_f2_t p[4];
};
__device__ __forceinline__ RdPairs rd_lookup4(uint32_t v, uint32_t (&ad)[4]) {
  NSMLP_SET_BYTE1(ad[0], v, "BYTE_0");
  NSMLP_SET_BYTE1(ad[1], v, "BYTE_1");
  NSMLP_SET_BYTE1(ad[2], v, "BYTE_2");
  NSMLP_SET_BYTE1(ad[3], v, "BYTE_3");
  return RdPairs{{lds_ld_f2(ad[0]), lds_ld_f2(ad[1]), lds_ld_f2(ad[2]), lds_ld_f2(ad[3])}};
}
__device__ __forceinline__ half8_t rd_finish8(const RdPairs& pr, float am) {
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float2_t w = {pr.p[i].x * am, pr.p[i].y * am};
    o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(w, half2_t));
  }
  return as_h8(make_uint4(o[0], o[1], o[2], o[3]));
}
// dword s (a constant) of a 16-byte weight load
template <int s>
__device__ __forceinline__ uint32_t rd_word(const uint4& w) {
  return s == 0 ? w.x : s == 1 ? w.y : s == 2 ? w.z : w.w;
}

// One 64-column step's weight loads of a lane for two 32-row tiles: 16 packed
// bytes per tile (its 32 columns) and their absmax (u8 code + second-level
// scale, or fp32).
struct RdW {
  uint4 w[2];
  uint32_t qa[2];
  float a[2];
  int ok;  // the lane's block is valid (its absmax is forced to zero otherwise)
};

}  // namespace nsmlp
