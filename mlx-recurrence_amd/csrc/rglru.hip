// rglru.hip — RG-LRU diagonal scan h_t = a_t * h_{t-1} + x_t on gfx950.
//
// Reference: mlx_recurrence/rglru.py (forward kernel :64-123, backward kernel
// :130-203, VJP formulas :36-39).  The reference gives every (batch, channel)
// one thread that walks all L steps; that exposes B*D threads of parallelism
// and one dependent FMA chain of length L.  Here a workgroup owns 64 channels
// of one batch row for the whole sequence and its NW waves work on NW
// consecutive chunks of T steps at once:
//   1. each wave loads its chunk's inputs into registers (read from HBM once)
//      and folds them into the chunk's affine map h -> P*h + E;
//   2. the maps are exchanged through LDS and each wave composes the maps of
//      the chunks before it with the carried state to get its entering state;
//   3. each wave replays its chunk from that state, writing y and the chunk's
//      end-of-chunk checkpoint.
// The backward pass runs the same three steps in reverse time on the adjoint
// recurrence, recomputing the chunk's states from the forward checkpoints.
#include "rr_common.h"

namespace {

constexpr int kMaxT = 32;

template <typename InT, int NW>
__global__ __launch_bounds__(64 * NW) void rglru_fwd_kernel(
    const InT* __restrict__ a, const InT* __restrict__ x, const float* __restrict__ h0,
    float* __restrict__ y, float* __restrict__ ckpt, int L, int D, int T, int nC) {
  __shared__ float sP[NW][64];
  __shared__ float sE[NW][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int d = blockIdx.x * 64 + lane;
  const int b = blockIdx.y;
  const bool dok = d < D;
  const int64_t base = (int64_t)b * L * D + d;
  float carry = (h0 != nullptr && dok) ? h0[(int64_t)b * D + d] : 0.f;

  for (int c0 = 0; c0 < nC; c0 += NW) {
    const int c = c0 + w;
    const bool act = dok && c < nC;
    float av[kMaxT], xv[kMaxT];
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      av[t] = 1.f;  // chunks past the end act as the identity map (P=1, E=0)
      xv[t] = 0.f;
      if (t < T && act) {
        const int64_t i = base + (int64_t)(c * T + t) * D;
        av[t] = rr::ld(a, i);
        xv[t] = rr::ld(x, i);
      }
    }
    float P = 1.f, E = 0.f;
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      if (t < T) {
        E = av[t] * E + xv[t];
        P *= av[t];
      }
    }
    sP[w][lane] = P;
    sE[w][lane] = E;
    __syncthreads();
    float hin = carry, nxt = carry;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const float pj = sP[j][lane], ej = sE[j][lane];
      if (j < w) hin = pj * hin + ej;
      nxt = pj * nxt + ej;
    }
    float h = hin;
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      if (t < T) {
        h = av[t] * h + xv[t];  // same update as rglru.py:92
        if (act) y[base + (int64_t)(c * T + t) * D] = h;
      }
    }
    if (act) ckpt[((int64_t)b * nC + c) * D + d] = h;
    __syncthreads();
    carry = nxt;
  }
}

// Adjoint (rglru.py:36-39, :173-178): lam += dy_t; dx_t = lam;
// da_t = lam * h_{t-1}; lam *= a_t.
template <typename InT, int NW>
__global__ __launch_bounds__(64 * NW) void rglru_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ dfinal, const InT* __restrict__ a,
    const InT* __restrict__ x, const float* __restrict__ h0, const float* __restrict__ ckpt,
    InT* __restrict__ da, InT* __restrict__ dx, float* __restrict__ dh0, int L, int D, int T,
    int nC) {
  __shared__ float sP[NW][64];
  __shared__ float sE[NW][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int d = blockIdx.x * 64 + lane;
  const int b = blockIdx.y;
  const bool dok = d < D;
  const int64_t base = (int64_t)b * L * D + d;
  float carry = (dfinal != nullptr && dok) ? dfinal[(int64_t)b * D + d] : 0.f;

  for (int r0 = 0; r0 < nC; r0 += NW) {
    const int c = nC - 1 - (r0 + w);  // wave 0 takes the latest chunk of the round
    const bool act = dok && c >= 0;
    float hst = 0.f;
    if (act) {
      if (c > 0) hst = ckpt[((int64_t)b * nC + (c - 1)) * D + d];
      else if (h0 != nullptr) hst = h0[(int64_t)b * D + d];
    }
    float av[kMaxT], gy[kMaxT], hs[kMaxT];
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      av[t] = 1.f;
      gy[t] = 0.f;
      hs[t] = 0.f;
      if (t < T && act) {
        const int64_t i = base + (int64_t)(c * T + t) * D;
        av[t] = rr::ld(a, i);
        gy[t] = dy[i];
        hs[t] = rr::ld(x, i);
      }
    }
    // Recompute the chunk's states from its checkpoint (hs[t] = h_t).
    float h = hst;
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      if (t < T) {
        h = av[t] * h + hs[t];
        hs[t] = h;
      }
    }
    // Chunk map of the adjoint: lam_out = P * lam_in + E.
    float lam = 0.f, P = 1.f;
#pragma unroll
    for (int t = kMaxT - 1; t >= 0; --t) {
      if (t < T) {
        lam += gy[t];
        lam *= av[t];
        P *= av[t];
      }
    }
    sP[w][lane] = P;
    sE[w][lane] = lam;
    __syncthreads();
    float lin = carry, nxt = carry;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const float pj = sP[j][lane], ej = sE[j][lane];
      if (j < w) lin = pj * lin + ej;
      nxt = pj * nxt + ej;
    }
    lam = lin;
#pragma unroll
    for (int t = kMaxT - 1; t >= 0; --t) {
      if (t < T) {
        lam += gy[t];
        const float hprev = (t > 0) ? hs[t - 1] : hst;
        if (act) {
          const int64_t i = base + (int64_t)(c * T + t) * D;
          rr::st(dx, i, lam);
          rr::st(da, i, lam * hprev);
        }
        lam *= av[t];
      }
    }
    __syncthreads();
    carry = nxt;
  }
  if (dh0 != nullptr && dok && w == 0) dh0[(int64_t)b * D + d] = carry;
}

int check_common(int64_t B, int64_t L, int64_t D, int64_t seg, int dtype) {
  if (B <= 0 || L <= 0 || D <= 0) {
    return rr::fail(RR_EINVAL, "rglru: B, L and D must be positive");
  }
  if (int rc = rr::check_segment_shape(L, seg, D, "D")) return rc;
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, "rglru: unsupported dtype");
  if (B > 65535) return rr::fail(RR_EUNSUPPORTED, "rglru: B > 65535 is not supported");
  if (L * D > (int64_t)1 << 40) return rr::fail(RR_EUNSUPPORTED, "rglru: tensor too large");
  return RR_OK;
}

constexpr int kFwdWaves = 16;
constexpr int kBwdWaves = 8;

}  // namespace

extern "C" int rr_rglru_fwd(const void* a, const void* x, int dtype, int64_t B, int64_t L,
                            int64_t D, int64_t seg, const float* h0, float* y, float* ckpt,
                            void* stream) {
  if (int rc = check_common(B, L, D, seg, dtype)) return rc;
  if (!a || !x || !y || !ckpt) return rr::fail(RR_EINVAL, "rglru_fwd: null pointer argument");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  const dim3 grid((unsigned)((D + 63) / 64), (unsigned)B);
  hipStream_t s = static_cast<hipStream_t>(stream);
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rglru_fwd_kernel<InT, kFwdWaves>), grid,
                                              dim3(64 * kFwdWaves), 0, s,
                                              static_cast<const InT*>(a),
                                              static_cast<const InT*>(x), h0, y, ckpt, (int)L,
                                              (int)D, T, nC));
  return rr::check_launch("rr_rglru_fwd");
}

extern "C" int rr_rglru_bwd(const float* dy, const float* dfinal, const void* a, const void* x,
                            int dtype, int64_t B, int64_t L, int64_t D, int64_t seg,
                            const float* h0, const float* ckpt, void* da, void* dx, float* dh0,
                            void* stream) {
  if (int rc = check_common(B, L, D, seg, dtype)) return rc;
  if (!dy || !a || !x || !ckpt || !da || !dx) {
    return rr::fail(RR_EINVAL, "rglru_bwd: null pointer argument");
  }
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  const dim3 grid((unsigned)((D + 63) / 64), (unsigned)B);
  hipStream_t s = static_cast<hipStream_t>(stream);
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rglru_bwd_kernel<InT, kBwdWaves>), grid,
                                              dim3(64 * kBwdWaves), 0, s, dy, dfinal,
                                              static_cast<const InT*>(a),
                                              static_cast<const InT*>(x), h0, ckpt,
                                              static_cast<InT*>(da), static_cast<InT*>(dx), dh0,
                                              (int)L, (int)D, T, nC));
  return rr::check_launch("rr_rglru_bwd");
}
