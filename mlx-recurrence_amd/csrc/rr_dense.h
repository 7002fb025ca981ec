// rr_dense.h — shared pieces of the per-chunk fp32-MFMA kernels (ssd_dense.hip,
// gla_dense.hip): the 16 x 16 fp32 MFMA block product, register-staged LDS
// slabs, and the walk over the chunk maps.
#pragma once

#include "rr_common.h"
#include "rr_mfma.h"

namespace rr {
namespace dense {

using rr::f32x4_t;

constexpr int Q = 32;   // chunk length (steps)

// acc += A . B over K (a multiple of 4) for the 16 x 16 output block whose
// lane holds column lane % 16 of rows 4 (lane / 16) + r, on the fp32 MFMA
// v_mfma_f32_16x16x4_f32 (A[row = lane % 16][k = lane / 16],
// B[k = lane / 16][col = lane % 16]): products and sums in fp32, no operand
// splitting.  fa(row, k) and fb(k, col) read the operands (rows and columns
// relative to the block).
// mm16r sums k over [K0, K1) only.
template <int K0, int K1, class FA, class FB>
__device__ __forceinline__ f32x4_t mm16r(FA fa, FB fb, int lane, f32x4_t acc) {
  const int r = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int k0 = K0; k0 < K1; k0 += 4)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa(r, k0 + kq), fb(k0 + kq, r), acc, 0, 0, 0);
  return acc;
}
template <int K, class FA, class FB>
__device__ __forceinline__ f32x4_t mm16(FA fa, FB fb, int lane, f32x4_t acc) {
  return mm16r<0, K>(fa, fb, lane, acc);
}

// exp(x) where keep, else 0 (formed in every lane, then selected: no branch,
// and an overflowing exponential of a masked element is dropped, not multiplied).
__device__ __forceinline__ float kept_exp(bool keep, float x) {
  const float e = __expf(x);
  return keep ? e : 0.f;
}

// A [ROWS][W] fp32 slab staged through registers by NT threads: load() issues
// one global load per element (row r at src + r * stride, element w at + w;
// every thread takes elements tid, tid + NT, ...), store() writes them to LDS.
// A kernel calls every load() before the first store(), so all of its loads
// are in flight at once.
template <int ROWS, int W, int NT = 256>
struct Slab {
  static constexpr int N = (ROWS * W + NT - 1) / NT;   // elements per thread
  static constexpr bool kExact = ROWS * W % NT == 0;   // else the last pass is partial
  float v[N];
  template <typename T>
  __device__ __forceinline__ void load(const T* src, int64_t stride, int tid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int i = min(tid + NT * j, ROWS * W - 1);   // (partial pass: a duplicate, in bounds, not stored)
      v[j] = rr::ld(src, (int64_t)(i / W) * stride + i % W);
    }
  }
  // the transpose of a [W][ROWS] block: element (r, w) from src[w * stride + r]
  template <typename T>
  __device__ __forceinline__ void load_t(const T* src, int64_t stride, int tid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int i = min(tid + NT * j, ROWS * W - 1);
      v[j] = rr::ld(src, (int64_t)(i % W) * stride + i / W);
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = 0.f;
  }
  template <int P>
  __device__ __forceinline__ void store(float (&dst)[ROWS][P], int tid) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int i = tid + NT * j;
      if (kExact || i < ROWS * W) dst[i / W][i % W] = v[j];
    }
  }
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}


// Chunk (b, h, c) of workgroup blockIdx.x = (b * H + h) * nC + c.
struct ChunkPos {
  int b, h, c;
  int64_t bh, row0;   // b * H + h; first (b, t) row of the chunk
};
__device__ __forceinline__ ChunkPos chunk_pos(int H, int L, int nC) {
  const int id = blockIdx.x, c = id % nC, bh = id / nC;
  return ChunkPos{bh / H, bh % H, c, (int64_t)bh, (int64_t)(bh / H) * L + (int64_t)c * Q};
}

// ------------------------------------------------------------------ the walk over chunks
// One thread per state element (b, h, d, n): x_c = P_c x_{c-1} + E_c over the
// chunks (forward from h0, in order, writing the state after each chunk;
// backward from dfinal, in reverse, writing the adjoint flowing into each
// chunk before its own map, and dh0 at the end).  The maps of kWalkBatch
// chunks are loaded at once.  Maps and out are [d][n] per chunk; x0 and xlast
// are [d][n] (SSD) or [n][d] (GLA: the reference's [i, j]).
constexpr int kWalkBatch = 16;
template <bool BWD, bool GLA>
__global__ __launch_bounds__(256) void dense_compose_kernel(const float* __restrict__ mapE,
                                                            const float* __restrict__ mapP,
                                                            const float* __restrict__ x0, float* __restrict__ out,
                                                            float* __restrict__ xlast, int64_t total, int DL, int NS,
                                                            int nC) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int DN = DL * NS;
  if (i >= total) return;
  const int64_t bh = i / DN;
  const int e = (int)(i % DN), n = e % NS;
  const int64_t xi = GLA ? bh * DN + (int64_t)n * DL + e / NS : i;   // this element in x0 / xlast
  float x = x0 != nullptr ? x0[xi] : 0.f;
  for (int i0 = 0; i0 < nC; i0 += kWalkBatch) {
    float ev[kWalkBatch], pv[kWalkBatch];
#pragma unroll
    for (int q = 0; q < kWalkBatch; ++q) {
      const int k = min(i0 + q, nC - 1), c = BWD ? nC - 1 - k : k;
      ev[q] = mapE[(bh * nC + c) * DN + e];
      pv[q] = mapP[(bh * nC + c) * NS + n];
    }
#pragma unroll
    for (int q = 0; q < kWalkBatch; ++q) {
      const int k = i0 + q, c = BWD ? nC - 1 - k : k;
      if (k < nC) {
        if (BWD) out[(bh * nC + c) * DN + e] = x;
        x = pv[q] * x + ev[q];
        if (!BWD) out[(bh * nC + c) * DN + e] = x;
      }
    }
  }
  if (xlast != nullptr) xlast[xi] = x;
}


}  // namespace dense
}  // namespace rr
