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

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t bf_bits(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
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

// Two fp32 values -> packed bf16 pair (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t bf_pack2(float a, float b) {
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  const bf16x2_v v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
// Split four fp32 values into bf16 hi and lo operand fragments.
__device__ __forceinline__ void bf_split4(const f32x4_t& x, u16x4_t& hi, u16x4_t& lo) {
  const uint32_t h01 = bf_pack2(x[0], x[1]), h23 = bf_pack2(x[2], x[3]);
  const uint32_t l01 = bf_pack2(x[0] - __uint_as_float(h01 << 16), x[1] - __uint_as_float(h01 & 0xffff0000u));
  const uint32_t l23 = bf_pack2(x[2] - __uint_as_float(h23 << 16), x[3] - __uint_as_float(h23 & 0xffff0000u));
  hi = __builtin_bit_cast(u16x4_t, make_uint2(h01, h23));
  lo = __builtin_bit_cast(u16x4_t, make_uint2(l01, l23));
}

// Split eight fp32 values into bf16 hi and lo operand fragments.
__device__ __forceinline__ void bf_split8(const float (&x)[8], u16x8_t& hi, u16x8_t& lo) {
  u16x4_t h0, l0, h1, l1;
  bf_split4(f32x4_t{x[0], x[1], x[2], x[3]}, h0, l0);
  bf_split4(f32x4_t{x[4], x[5], x[6], x[7]}, h1, l1);
  hi = u16x8_t{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
  lo = u16x8_t{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
}

// Store an fp32 value as bf16 (round to nearest even).
__device__ __forceinline__ void st_bf16(uint16_t* p, int64_t i, float v) { p[i] = bf_bits(v); }
// Accesses at a uniform base plus a 32-bit per-lane offset: the byte offset
// is formed in 32 bits (element i of a chunk, i * sizeof(E) < 2^32), so the
// address is the SGPR base plus a VGPR offset with no 64-bit math per element.
// ld32<T>: a T (e.g. a 16-byte vector) starting at element i.
template <typename T, typename E>
__device__ __forceinline__ T ld32(const E* base, uint32_t i) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + i * (uint32_t)sizeof(E));
}
template <typename T, typename E>
__device__ __forceinline__ T ld32(const __attribute__((address_space(1))) E* base, uint32_t i) {
  typedef const __attribute__((address_space(1))) char gchar;
  typedef const __attribute__((address_space(1))) T gT;
  return *(gT*)((gchar*)base + i * (uint32_t)sizeof(E));
}
__device__ __forceinline__ void st_bf16_u32(uint16_t* base, uint32_t i, float v) {
  *reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(base) + i * 2u) = bf_bits(v);
}

// 16-byte fragment read from LDS (address must be 16-byte aligned).
__device__ __forceinline__ u16x8_t frag(const uint16_t* p) {
  return *reinterpret_cast<const u16x8_t*>(p);
}

// 8-byte fragment read from LDS (address must be 8-byte aligned).
__device__ __forceinline__ u16x4_t frag4(const uint16_t* p) {
  return *reinterpret_cast<const u16x4_t*>(p);
}

// Cross-lane sums without LDS traffic.  Every lane of the group receives the
// same value (each butterfly step adds two equal-valued pairs, so the
// rounding is identical across the group).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over the 16 lanes of a row (lanes 16k .. 16k + 15).
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x141>(v);   // row_half_mirror: quad q <-> quad q ^ 1
  v += dpp_mov<0x140>(v);   // row_mirror: half h <-> half h ^ 1
  return v;
}
// Sum over the four rows: lanes l, l ^ 16, l ^ 32, l ^ 48 (LDS-unit
// permutes; used a few times per chunk).
__device__ __forceinline__ float rows4_sum(float v) {
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}
__device__ __forceinline__ float wave_sum(float v) { return rows4_sum(row16_sum(v)); }
// Sum of lanes l and l ^ 32.
__device__ __forceinline__ float halves_sum(float v) { return v + __shfl_xor(v, 32); }
// Inclusive prefix sum over lanes 0..31 and, separately, 32..63: shifts
// within each 16-lane row, then row 0 (2) hands its total to row 1 (3).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_in(float v) {   // 0 where the source lane is outside the row
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, true));
}
__device__ __forceinline__ float prefix32_sum(float v) {
  v += dpp_in<0x111, 0xF>(v);   // row_shr:1
  v += dpp_in<0x112, 0xF>(v);   // row_shr:2
  v += dpp_in<0x114, 0xF>(v);   // row_shr:4
  v += dpp_in<0x118, 0xF>(v);   // row_shr:8
  v += dpp_in<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
  return v;
}

// Operand fragments of a matrix stored k-major in LDS (X[k][col] at
// base[k * pitch + col], col contiguous) with gfx950's transposing read
// ds_read_b64_tr_b16: within each 16-lane group the lanes supply 16 4-element
// row pieces and lane j receives element j % 4 of the pieces of lanes
// 4 e + j / 4, e = 0..3 (checked on gfx950 by an in-bounds lane-layout probe).
// Supplying &X[k0 + i / 4][4 (i % 4)] from lane i of group g gives lane j the
// k-run X[k0 .. k0 + 3][j]: a fragment with k = 4 (lane / 16) + e (16x16x16)
// or, two reads, k = 8 (lane / 16) + e (16x16x32), for columns col0 .. col0 + 15.
// base must address X[0][col0]; pitch and col0 are multiples of 4.
__device__ __forceinline__ u16x4_t tr_read4(const uint16_t* p) {
  typedef short i16x4v __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(
      u16x4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4v*)(p)));
}
__device__ __forceinline__ u16x4_t frag4_tr(const uint16_t* base, int pitch, int lane) {
  const int g = lane >> 4, i = lane & 15;
  return tr_read4(base + (4 * g + (i >> 2)) * pitch + 4 * (i & 3));
}
__device__ __forceinline__ u16x8_t frag_tr(const uint16_t* base, int pitch, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const uint16_t* a = base + (8 * g + (i >> 2)) * pitch + 4 * (i & 3);
  const u16x4_t lo = tr_read4(a), hi = tr_read4(a + 4 * pitch);
  return u16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Pins a loaded value in a VGPR at this point, in every lane.  A value that
// only some lanes use (a select on the lane index) lets the compiler move its
// load into a divergent branch, where it then waits for every load in flight;
// pinning it after the other loads are issued makes the wait cover only the
// loads issued before it.
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }

// A bf16 matrix X[step][col] (W columns) staged in LDS for transposing reads.
// Rows are padded to 32 or 96 bytes past a multiple of 128, so the four rows
// that 16 lanes of a transposing read take hit four distinct 32-byte bank
// groups (16-column rows, 32 bytes, tile the banks unpadded).  With PACK, rows
// of a multiple of 64 columns are stored unpadded instead, their 16-column
// pieces permuted by row (piece p of row t at p ^ (t % 4)): 20 % less LDS, for
// a few more address registers (the piece offsets differ per lane).
template <int W, bool PACK = false>
struct Staged {
  static constexpr bool SWZ = PACK && W % 64 == 0;
  static constexpr int P = SWZ ? W : W == 16 ? 16 : W + 16;   // row pitch (elements)
  static constexpr int SIZE = 32 * P;                          // elements of 32 rows
  // element offset of X[t][col]; an 8-aligned run of 8 columns stays contiguous
  static __device__ __forceinline__ int off(int t, int col) { return t * P + (SWZ ? col ^ (16 * (t & 3)) : col); }
};
// frag_tr for a Staged matrix: columns col0 .. col0 + 15 (col0 % 16 == 0),
// k-runs from row 0.
template <typename S>
__device__ __forceinline__ u16x8_t frag_tr_st(const uint16_t* x, int col0, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const uint16_t* a = x + S::off(8 * g + (i >> 2), col0) + 4 * (i & 3);   // rows r and r + 4 share r % 4
  const u16x4_t lo = tr_read4(a), hi = tr_read4(a + 4 * S::P);
  return u16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// A pointer into global memory as such: loads through it are global (not
// flat) loads, which count only against vmcnt, so waits for LDS traffic
// (lgkmcnt, e.g. at a barrier) do not also wait for them.  For pointers the
// compiler cannot trace to a kernel argument (selected between several).
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* as_global(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
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
