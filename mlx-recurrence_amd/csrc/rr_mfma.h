// rr_mfma.h — gfx950 bf16 MFMA helpers shared by the chunked kernels.
//
// Operand fragments (verified on gfx950 by an in-bounds lane-layout check):
//   v_mfma_f32_32x32x16_bf16: A[row = lane%32][k = 8*(lane/32) + e], e < 8;
//       B[k = 8*(lane/32) + e][col = lane%32];
//       D element r: row = 8*(r/4) + 4*(lane/32) + r%4, col = lane%32.
//   v_mfma_f32_16x16x32_bf16: A[row = lane%16][k = 8*(lane/16) + e];
//       B[k = 8*(lane/16) + e][col = lane%16];
//       D element r: row = 4*(lane/16) + r, col = lane%16.
//   v_mfma_f32_16x16x16_bf16: A[row = lane%16][k = 4*(lane/16) + e], e < 4;
//       B[k = 4*(lane/16) + e][col = lane%16]; D as for 16x16x32.  A 16x16
//       accumulator block X is therefore, element for element, the B operand
//       of X (contracting over X's rows) without any data movement.
// Every operand is kept in LDS "K-contiguous" (row-major [M][K] for A, [N][K]
// for B) so a fragment is one 16-byte LDS read.  fp32 quantities used as an
// operand are split into bf16 hi + lo (x = hi + lo + O(2^-17 |x|)) and fed as
// two MFMAs; bf16 inputs are exact and need one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rr {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(unsigned short)))) unsigned short u16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned short)))) unsigned short u16x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

// fp32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint16_t bf_bits(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float bf_val(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ void bf_split(float x, uint16_t& hi, uint16_t& lo) {
  hi = bf_bits(x);
  lo = bf_bits(x - bf_val(hi));
}

__device__ __forceinline__ f32x4_t mfma16(const u16x8_t& a, const u16x8_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32(const u16x8_t& a, const u16x8_t& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t mfma16k16(const u16x4_t& a, const u16x4_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, a),
                                                   __builtin_bit_cast(i16x4_t, b), c, 0, 0, 0);
}

// Split four fp32 values into bf16 hi and lo operand fragments.
__device__ __forceinline__ void bf_split4(const f32x4_t& x, u16x4_t& hi, u16x4_t& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint16_t h, l;
    bf_split(x[e], h, l);
    hi[e] = h;
    lo[e] = l;
  }
}

// Store an fp32 value as bf16 (round to nearest even).
__device__ __forceinline__ void st_bf16(uint16_t* p, int64_t i, float v) { p[i] = bf_bits(v); }

// 16-byte fragment read from LDS (address must be 16-byte aligned).
__device__ __forceinline__ u16x8_t frag(const uint16_t* p) {
  return *reinterpret_cast<const u16x8_t*>(p);
}

// 8-byte fragment read from LDS (address must be 8-byte aligned).
__device__ __forceinline__ u16x4_t frag4(const uint16_t* p) {
  return *reinterpret_cast<const u16x4_t*>(p);
}

// Make one wave's LDS writes visible to its own later LDS reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Raw 16-bit load of an input element (bf16 inputs stay bits; used by the
// chunked kernels, which take bf16 operands).
__device__ __forceinline__ uint16_t ld_bits(const uint16_t* p, int64_t i) { return p[i]; }

}  // namespace rr
