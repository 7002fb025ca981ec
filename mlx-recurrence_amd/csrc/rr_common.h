// rr_common.h — shared device helpers and host-side error plumbing for the
// gfx950 recurrence kernels.
//
// Element access: inputs arrive as fp32, bf16 or fp16 and are widened to fp32
// on load; state and accumulation are always fp32.  bf16 is carried as raw
// uint16_t bits (widening is a 16-bit shift; narrowing is the hardware
// conversion, round to nearest even) so the kernels do not depend on a vendor
// bf16 class.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/recurrence.h"

namespace rr {

struct bf16 { uint16_t bits; };
using f16 = _Float16;

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
// fp32 -> bf16 with gfx950's v_cvt_pk_bf16_f32 (round to nearest even, NaN
// stays NaN).
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  return bf16{__builtin_bit_cast(uint16_t, static_cast<__bf16>(v))};
}
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }
template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = from_f32<T>(v); }

// ---------------------------------------------------------------- host side
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// Device address of the library's status word on the current device (a
// 32-bit __device__ variable; kernels OR error bits into it, rr_async_status
// reads and clears it), or nullptr with the error set.  Looked up once per
// device.
uint32_t* status_word();

// Checkpoint interval: the largest power of two <= 32 that divides seg.
inline int64_t chunk_len(int64_t L, int64_t seg) {
  if (seg <= 0 || L <= 0 || L % seg != 0) return 0;
  int64_t t = 1;
  while (t < 32 && (seg % (t * 2)) == 0) t *= 2;
  return t;
}

// The reference's shape rules (_chassis.py:104-115), same conditions and text.
int check_segment_shape(int64_t L, int64_t seg, int64_t lane_dim, const char* lane_name);

inline bool valid_dtype(int dtype) { return dtype == RR_F32 || dtype == RR_BF16 || dtype == RR_F16; }

}  // namespace rr

// Dispatch on the input element type: instantiates BODY with `using InT = ...`.
#define RR_DISPATCH_DTYPE(dtype, ...)                 \
  switch (dtype) {                                    \
    case RR_F32: { using InT = float; __VA_ARGS__; } break;    \
    case RR_BF16: { using InT = rr::bf16; __VA_ARGS__; } break; \
    case RR_F16: { using InT = rr::f16; __VA_ARGS__; } break;   \
    default: return rr::fail(RR_EINVAL, "unsupported dtype");  \
  }
