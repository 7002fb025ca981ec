// step.hip — single-token decode steps of the four recurrences on gfx950: the
// O(1)-per-token recurrent update of a cached state, one launch per token.
//
// The reference names this as its next inference step (docs/validation/
// BOTTLENECK_ANALYSIS.md:105-119: fuse the per-layer recurrent update into one
// kernel per layer type, on the final-state cache layouts that
// ssd_scan_with_state / gla_scan_with_state / rglru_ / rotlru_scan_with_state
// return, ssd.py:365-375, gla.py:321-329, rglru.py:259-267, rotlru.py:323-331).
// Per token, with the state updated in place (fp32) and y written in fp32:
//   SSD     h[d,n] = exp(delta A[h,n]) h[d,n] + delta B[n] u[d];  y[d] = sum_n h[d,n] C[n]
//   GLA     S[i,j] = g S[i,j] + k[i] v[j];                          y[j] = sum_i q[i] S[i,j]
//   RG-LRU  h = a h + x;                                            y = h
//   rotLRU  (u,w) = a R(theta) (u,w) + (x0,x1);                     y = (u,w)
// (the reference's per-step recurrences, ssd.py:85-111, gla.py:78-100,
// rglru.py:88-99, rotlru.py:101-122, for one t).
//
// Each step reads and writes the whole state once: the kernels are HBM-bound
// (SSD B8 H80 Dh64 N128: 42 MB per token) or, at small batch, launch-bound.
// SSD / GLA: one workgroup per (batch, head); lanes run along the state's
// contiguous axis (4 consecutive elements per lane, one 16-byte access), the
// per-lane decay / input coefficients of those 4 columns are formed once, and
// rows are spread over lane groups and waves.  The row sums of SSD (over n)
// are butterfly reductions within a lane group; the column sums of GLA (over
// i) are reduced across the lane groups of a wave and then across the waves
// in a fixed order (deterministic).
#include "rr_common.h"

#include <algorithm>
#include <string>

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

// Sum over the G consecutive lanes of a group (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Loads the 4 consecutive fp32 values of a row at columns c .. c + 3 (row
// length n): every lane loads, at columns clamped into the row, and columns
// past n read as 0 (a select on the loaded registers; a load under a branch
// makes the branch's join wait for every load in flight).  VEC: rows a
// multiple of 4 long, one 16-byte access.
template <bool VEC>
__device__ __forceinline__ void ld4(const float* row, int c, int n, float (&v)[4]) {
  if constexpr (VEC) {
    const float4 q = *reinterpret_cast<const float4*>(row + min(c, n - 4));
    v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = row[min(c + e, n - 1)];
  }
}
__device__ __forceinline__ void mask4(int c, int n, float (&v)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    asm volatile("" : "+v"(v[e]));
    v[e] = c + e < n ? v[e] : 0.f;
  }
}
template <bool VEC>
__device__ __forceinline__ void st4(float* row, int c, int n, const float (&v)[4]) {
  if constexpr (VEC) {
    if (c < n) *reinterpret_cast<float4*>(row + c) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c + e < n) row[c + e] = v[e];
  }
}

// ------------------------------------------------------------------ SSD
// Lane l of a wave: column group col = l % G (states n = 4 col .. 4 col + 3),
// row slot l / G; the workgroup walks the Dh rows 4 * (64 / G) at a time, the
// next row's u and state loaded while the current one is updated.
template <typename InT, int G, bool VEC>
__global__ __launch_bounds__(kThreads) void ssd_step_kernel(const InT* __restrict__ u, const InT* __restrict__ delta,
                                                            const InT* __restrict__ Bm, const InT* __restrict__ Cm,
                                                            const float* __restrict__ A, int a_sn, int H, int Dh,
                                                            int N, float* __restrict__ state, float* __restrict__ y) {
  constexpr int kRowsPerWave = 64 / G, kStep = kWaves * kRowsPerWave;
  const int bh = blockIdx.x, h = bh % H;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane % G, c0 = 4 * col;
  float* S = state + (int64_t)bh * Dh * N;
  // every load of the token and of the first row first (clamped indices)
  const float dt = rr::ld(delta, bh);
  float Av[4], Bv[4], Cv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int nn = min(c0 + e, N - 1);
    Av[e] = A[(int64_t)h * (a_sn ? N : 1) + (int64_t)nn * a_sn];
    Bv[e] = rr::ld(Bm, (int64_t)bh * N + nn);
    Cv[e] = rr::ld(Cm, (int64_t)bh * N + nn);
  }
  int d = wave * kRowsPerWave + lane / G;
  float ud = rr::ld(u, (int64_t)bh * Dh + min(d, Dh - 1));
  float s[4];
  ld4<VEC>(S + (int64_t)min(d, Dh - 1) * N, c0, N, s);
  float dA[4], dB[4], Cn[4];
  mask4(c0, N, Av);
  mask4(c0, N, Bv);
  mask4(c0, N, Cv);
  mask4(c0, N, s);   // states past N read as 0 (they enter the row sum)
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    dA[e] = c0 + e < N ? __expf(dt * Av[e]) : 0.f;
    dB[e] = dt * Bv[e];
    Cn[e] = Cv[e];
  }
  for (; d < Dh; d += kStep) {
    // the next row's loads (clamped; dropped past the last row)
    const int dn = min(d + kStep, Dh - 1);
    const float un = rr::ld(u, (int64_t)bh * Dh + dn);
    float sn[4];
    ld4<VEC>(S + (int64_t)dn * N, c0, N, sn);
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[e] = dA[e] * s[e] + dB[e] * ud;   // ssd.py:97-98 for one step
      acc += s[e] * Cn[e];
    }
    st4<VEC>(S + (int64_t)d * N, c0, N, s);
    acc = group_sum<G>(acc);              // y[d] = sum_n h[d,n] C[n] (ssd.py:99-101)
    if (col == 0) y[(int64_t)bh * Dh + d] = acc;
    ud = un;
    mask4(c0, N, sn);
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] = sn[e];
  }
}

// ------------------------------------------------------------------ GLA
// State S[i][j], j contiguous.  Lane l: columns j = 4 col .. 4 col + 3
// (col = l % G), row slot l / G; the column sums over i go lane groups ->
// waves (LDS) in a fixed order.
template <typename InT, int G, bool VEC>
__global__ __launch_bounds__(kThreads) void gla_step_kernel(const InT* __restrict__ q, const InT* __restrict__ k,
                                                                  const InT* __restrict__ v, const InT* __restrict__ gates,
                                                                  int Dh, float* __restrict__ state,
                                                                  float* __restrict__ y) {
  constexpr int kRowsPerWave = 64 / G, kStep = kWaves * kRowsPerWave;
  __shared__ float part[kWaves][4 * G];
  const int bh = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane % G, c0 = 4 * col;
  float* S = state + (int64_t)bh * Dh * Dh;
  // every load of the token and of the first row first (clamped indices)
  const float g = rr::ld(gates, bh);
  float vj[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) vj[e] = rr::ld(v, (int64_t)bh * Dh + min(c0 + e, Dh - 1));
  int i = wave * kRowsPerWave + lane / G;
  float ki = rr::ld(k, (int64_t)bh * Dh + min(i, Dh - 1)), qi = rr::ld(q, (int64_t)bh * Dh + min(i, Dh - 1));
  float s[4];
  ld4<VEC>(S + (int64_t)min(i, Dh - 1) * Dh, c0, Dh, s);
  mask4(c0, Dh, vj);
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  for (; i < Dh; i += kStep) {
    // the next row's loads (clamped; dropped past the last row)
    const int in = min(i + kStep, Dh - 1);
    const float kn = rr::ld(k, (int64_t)bh * Dh + in), qn = rr::ld(q, (int64_t)bh * Dh + in);
    float sn[4];
    ld4<VEC>(S + (int64_t)in * Dh, c0, Dh, sn);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[e] = g * s[e] + ki * vj[e];       // gla.py:86-87 for one step
      o[e] += qi * s[e];
    }
    st4<VEC>(S + (int64_t)i * Dh, c0, Dh, s);
    ki = kn, qi = qn;
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] = sn[e];
  }
  // column sums: over the row slots of the wave (lanes col, col + G, ...) ...
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int off = G; off < 64; off <<= 1) o[e] += __shfl_xor(o[e], off, 64);
  }
  if (lane < G) {
#pragma unroll
    for (int e = 0; e < 4; ++e) part[wave][4 * lane + e] = o[e];
  }
  __syncthreads();
  // ... then over the waves, in order (gla.py:88-90: y[j] = sum_i q[i] S[i,j])
  for (int j = threadIdx.x; j < Dh && j < 4 * G; j += kThreads) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += part[w][j];
    y[(int64_t)bh * Dh + j] = t;
  }
}

// ------------------------------------------------------------- RG-LRU / rotLRU
template <typename InT>
__global__ __launch_bounds__(kThreads) void rglru_step_kernel(const InT* __restrict__ a, const InT* __restrict__ x,
                                                              int64_t n, float* __restrict__ state,
                                                              float* __restrict__ y) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float h = rr::ld(a, i) * state[i] + rr::ld(x, i);   // rglru.py:92
    state[i] = h;
    y[i] = h;
  }
}

template <typename InT>
__global__ __launch_bounds__(kThreads) void rotlru_step_kernel(const InT* __restrict__ a, const InT* __restrict__ cs,
                                                               const InT* __restrict__ sn, const InT* __restrict__ x,
                                                               int64_t npairs, float* __restrict__ state,
                                                               float* __restrict__ y) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < npairs; p += stride) {
    const float av = rr::ld(a, p), c = rr::ld(cs, p), s = rr::ld(sn, p);
    const float2 h = reinterpret_cast<const float2*>(state)[p];
    const float un = av * (c * h.x - s * h.y) + rr::ld(x, 2 * p);       // rotlru.py:110-111
    const float wn = av * (s * h.x + c * h.y) + rr::ld(x, 2 * p + 1);
    reinterpret_cast<float2*>(state)[p] = make_float2(un, wn);
    reinterpret_cast<float2*>(y)[p] = make_float2(un, wn);
  }
}

// Lanes per row: the power of two >= ceil(cols / 4), at most 64.
inline int lanes_for(int64_t cols) {
  int g = 1;
  while (g < 64 && 4 * g < cols) g *= 2;
  return g;
}

int elementwise_grid(int64_t n) {
  const int64_t blocks = (n + kThreads - 1) / kThreads;
  return (int)std::min<int64_t>(std::max<int64_t>(blocks, 1), 65536);
}

}  // namespace

// Dispatch over the lanes-per-row template parameter.
#define RR_STEP_G_DISPATCH(g, ...)                        \
  switch (g) {                                            \
    case 1: { constexpr int G = 1; __VA_ARGS__; } break;  \
    case 2: { constexpr int G = 2; __VA_ARGS__; } break;  \
    case 4: { constexpr int G = 4; __VA_ARGS__; } break;  \
    case 8: { constexpr int G = 8; __VA_ARGS__; } break;  \
    case 16: { constexpr int G = 16; __VA_ARGS__; } break; \
    case 32: { constexpr int G = 32; __VA_ARGS__; } break; \
    default: { constexpr int G = 64; __VA_ARGS__; } break; \
  }

extern "C" int rr_ssd_step(const void* u, const void* delta, const void* Bm, const void* Cm, const float* A_neg,
                           int64_t A_stride_n, int dtype, int64_t B, int64_t H, int64_t Dh, int64_t N,
                           float* state, float* y, void* stream) {
  if (B <= 0 || H <= 0 || Dh <= 0 || N <= 0) return rr::fail(RR_EINVAL, "ssd_step: all dimensions must be positive");
  if (!u || !delta || !Bm || !Cm || !A_neg || !state || !y) return rr::fail(RR_EINVAL, "ssd_step: null pointer argument");
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, "ssd_step: unsupported dtype");
  if (A_stride_n != 0 && A_stride_n != 1) return rr::fail(RR_EINVAL, "ssd_step: A_stride_n must be 0 or 1");
  if (N > 256) return rr::fail(RR_EUNSUPPORTED, "ssd_step: N > 256 is not supported");
  if (B * H >= ((int64_t)1 << 31) || B * H * Dh * N >= ((int64_t)1 << 40))
    return rr::fail(RR_EUNSUPPORTED, "ssd_step: state too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int g = lanes_for(N);
  const bool vec = N % 4 == 0;
  RR_DISPATCH_DTYPE(dtype, RR_STEP_G_DISPATCH(g, {
    if (vec)
      hipLaunchKernelGGL((ssd_step_kernel<InT, G, true>), dim3((unsigned)(B * H)), dim3(kThreads), 0, s,
                         static_cast<const InT*>(u), static_cast<const InT*>(delta), static_cast<const InT*>(Bm),
                         static_cast<const InT*>(Cm), A_neg, (int)A_stride_n, (int)H, (int)Dh, (int)N, state, y);
    else
      hipLaunchKernelGGL((ssd_step_kernel<InT, G, false>), dim3((unsigned)(B * H)), dim3(kThreads), 0, s,
                         static_cast<const InT*>(u), static_cast<const InT*>(delta), static_cast<const InT*>(Bm),
                         static_cast<const InT*>(Cm), A_neg, (int)A_stride_n, (int)H, (int)Dh, (int)N, state, y);
  }));
  return rr::check_launch("rr_ssd_step");
}

extern "C" int rr_gla_step(const void* q, const void* k, const void* v, const void* gates, int dtype, int64_t B,
                           int64_t H, int64_t Dh, float* state, float* y, void* stream) {
  if (B <= 0 || H <= 0 || Dh <= 0) return rr::fail(RR_EINVAL, "gla_step: all dimensions must be positive");
  if (!q || !k || !v || !gates || !state || !y) return rr::fail(RR_EINVAL, "gla_step: null pointer argument");
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, "gla_step: unsupported dtype");
  if (Dh > 256) return rr::fail(RR_EUNSUPPORTED, "gla_step: Dh > 256 is not supported");
  if (B * H >= ((int64_t)1 << 31)) return rr::fail(RR_EUNSUPPORTED, "gla_step: state too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int g = lanes_for(Dh);
  const bool vec = Dh % 4 == 0;
  RR_DISPATCH_DTYPE(dtype, RR_STEP_G_DISPATCH(g, {
    if (vec)
      hipLaunchKernelGGL((gla_step_kernel<InT, G, true>), dim3((unsigned)(B * H)), dim3(kThreads), 0, s,
                         static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(v),
                         static_cast<const InT*>(gates), (int)Dh, state, y);
    else
      hipLaunchKernelGGL((gla_step_kernel<InT, G, false>), dim3((unsigned)(B * H)), dim3(kThreads), 0, s,
                         static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(v),
                         static_cast<const InT*>(gates), (int)Dh, state, y);
  }));
  return rr::check_launch("rr_gla_step");
}

extern "C" int rr_rglru_step(const void* a, const void* x, int dtype, int64_t B, int64_t D, float* state, float* y,
                             void* stream) {
  if (B <= 0 || D <= 0) return rr::fail(RR_EINVAL, "rglru_step: B and D must be positive");
  if (!a || !x || !state || !y) return rr::fail(RR_EINVAL, "rglru_step: null pointer argument");
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, "rglru_step: unsupported dtype");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = B * D;
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rglru_step_kernel<InT>), dim3((unsigned)elementwise_grid(n)),
                                              dim3(kThreads), 0, s, static_cast<const InT*>(a),
                                              static_cast<const InT*>(x), n, state, y));
  return rr::check_launch("rr_rglru_step");
}

extern "C" int rr_rotlru_step(const void* a, const void* cs, const void* sn, const void* x, int dtype, int64_t B,
                              int64_t Dp, float* state, float* y, void* stream) {
  if (B <= 0 || Dp <= 0) return rr::fail(RR_EINVAL, "rotlru_step: B and Dp must be positive");
  if (!a || !cs || !sn || !x || !state || !y) return rr::fail(RR_EINVAL, "rotlru_step: null pointer argument");
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, "rotlru_step: unsupported dtype");
  if ((reinterpret_cast<uintptr_t>(state) | reinterpret_cast<uintptr_t>(y)) % 8 != 0)
    return rr::fail(RR_EINVAL, "rotlru_step: state and y must be 8-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t np = B * Dp;
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rotlru_step_kernel<InT>), dim3((unsigned)elementwise_grid(np)),
                                              dim3(kThreads), 0, s, static_cast<const InT*>(a),
                                              static_cast<const InT*>(cs), static_cast<const InT*>(sn),
                                              static_cast<const InT*>(x), np, state, y));
  return rr::check_launch("rr_rotlru_step");
}
