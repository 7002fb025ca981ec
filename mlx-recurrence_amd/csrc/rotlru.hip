// rotlru.hip — rotational LRU, a pair-diagonal (complex) scan on gfx950:
//   u_t = a_t (c_t u_{t-1} - s_t w_{t-1}) + x_t[2p]
//   w_t = a_t (s_t u_{t-1} + c_t w_{t-1}) + x_t[2p+1]
// i.e. h_t = z_t h_{t-1} + x_t with the complex gate z_t = a_t (c_t + i s_t).
//
// Reference: mlx_recurrence/rotlru.py (forward :80-146, backward :153-266, VJP
// :317-322).  Same chunk-parallel workgroup structure as rglru.hip: a workgroup
// owns 64 pairs of one batch row for all L steps; its waves take consecutive
// chunks, fold them into complex affine maps (P, E), exchange the maps through
// LDS, then replay their chunk from the composed entering state.  The adjoint
// multiplies by conj(z_t) (the transpose of a_t R(theta_t)), so the backward
// pass has the same map structure in reverse time.
#include "rr_common.h"

namespace {

constexpr int kMaxT = 32;

template <typename InT, int NW>
__global__ __launch_bounds__(64 * NW) void rotlru_fwd_kernel(
    const InT* __restrict__ a, const InT* __restrict__ cs, const InT* __restrict__ sn,
    const InT* __restrict__ x, const float* __restrict__ h0, float* __restrict__ y,
    float* __restrict__ ckpt, int L, int Dp, int T, int nC) {
  __shared__ float sPr[NW][64], sPi[NW][64], sEu[NW][64], sEw[NW][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int p = blockIdx.x * 64 + lane;
  const int b = blockIdx.y;
  const int D = 2 * Dp;
  const bool pok = p < Dp;
  const int64_t pbase = (int64_t)b * L * Dp + p;
  const int64_t xbase = (int64_t)b * L * D + 2 * p;
  float cu = 0.f, cw = 0.f;
  if (h0 != nullptr && pok) {
    cu = h0[(int64_t)b * D + 2 * p];
    cw = h0[(int64_t)b * D + 2 * p + 1];
  }

  for (int c0 = 0; c0 < nC; c0 += NW) {
    const int c = c0 + w;
    const bool act = pok && c < nC;
    float av[kMaxT], cv[kMaxT], sv[kMaxT], xu[kMaxT], xw[kMaxT];
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      av[t] = 1.f;  // identity step past the end
      cv[t] = 1.f;
      sv[t] = 0.f;
      xu[t] = 0.f;
      xw[t] = 0.f;
      if (t < T && act) {
        const int64_t ip = pbase + (int64_t)(c * T + t) * Dp;
        const int64_t ix = xbase + (int64_t)(c * T + t) * D;
        av[t] = rr::ld(a, ip);
        cv[t] = rr::ld(cs, ip);
        sv[t] = rr::ld(sn, ip);
        xu[t] = rr::ld(x, ix);
        xw[t] = rr::ld(x, ix + 1);
      }
    }
    float pr = 1.f, pi = 0.f, eu = 0.f, ew = 0.f;
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      if (t < T) {
        const float un = av[t] * (cv[t] * eu - sv[t] * ew) + xu[t];
        const float wn = av[t] * (sv[t] * eu + cv[t] * ew) + xw[t];
        eu = un;
        ew = wn;
        const float zr = av[t] * cv[t], zi = av[t] * sv[t];
        const float npr = zr * pr - zi * pi;
        const float npi = zr * pi + zi * pr;
        pr = npr;
        pi = npi;
      }
    }
    sPr[w][lane] = pr;
    sPi[w][lane] = pi;
    sEu[w][lane] = eu;
    sEw[w][lane] = ew;
    __syncthreads();
    float hu = cu, hw = cw, nu = cu, nw = cw;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const float qr = sPr[j][lane], qi = sPi[j][lane], qu = sEu[j][lane], qw = sEw[j][lane];
      if (j < w) {
        const float tu = qr * hu - qi * hw + qu;
        const float tw = qi * hu + qr * hw + qw;
        hu = tu;
        hw = tw;
      }
      const float tu = qr * nu - qi * nw + qu;
      const float tw = qi * nu + qr * nw + qw;
      nu = tu;
      nw = tw;
    }
    float u = hu, v = hw;
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      if (t < T) {
        // same update and operation order as rotlru.py:101-104
        const float un = av[t] * (cv[t] * u - sv[t] * v) + xu[t];
        const float wn = av[t] * (sv[t] * u + cv[t] * v) + xw[t];
        u = un;
        v = wn;
        if (act) {
          const int64_t ix = xbase + (int64_t)(c * T + t) * D;
          *reinterpret_cast<float2*>(y + ix) = make_float2(u, v);
        }
      }
    }
    if (act) {
      *reinterpret_cast<float2*>(ckpt + ((int64_t)b * nC + c) * D + 2 * p) = make_float2(u, v);
    }
    __syncthreads();
    cu = nu;
    cw = nw;
  }
}

// Adjoint (rotlru.py:317-322, :212-234):
//   lam += dy_t; dx_t = lam; da_t = lam . (R_t h_{t-1});
//   dcs_t = a_t (lamU u_{t-1} + lamW w_{t-1}); dsn_t = a_t (lamW u_{t-1} - lamU w_{t-1});
//   lam <- a_t R_t^T lam.
template <typename InT, int NW>
__global__ __launch_bounds__(64 * NW) void rotlru_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ dfinal, const InT* __restrict__ a,
    const InT* __restrict__ cs, const InT* __restrict__ sn, const InT* __restrict__ x,
    const float* __restrict__ h0, const float* __restrict__ ckpt, InT* __restrict__ da,
    InT* __restrict__ dcs, InT* __restrict__ dsn, InT* __restrict__ dx,
    float* __restrict__ dh0, int L, int Dp, int T, int nC) {
  __shared__ float sPr[NW][64], sPi[NW][64], sEu[NW][64], sEw[NW][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int p = blockIdx.x * 64 + lane;
  const int b = blockIdx.y;
  const int D = 2 * Dp;
  const bool pok = p < Dp;
  const int64_t pbase = (int64_t)b * L * Dp + p;
  const int64_t xbase = (int64_t)b * L * D + 2 * p;
  float cu = 0.f, cw = 0.f;
  if (dfinal != nullptr && pok) {
    cu = dfinal[(int64_t)b * D + 2 * p];
    cw = dfinal[(int64_t)b * D + 2 * p + 1];
  }

  for (int r0 = 0; r0 < nC; r0 += NW) {
    const int c = nC - 1 - (r0 + w);
    const bool act = pok && c >= 0;
    float su = 0.f, sw = 0.f;  // state entering the chunk
    if (act) {
      if (c > 0) {
        const float2 h = *reinterpret_cast<const float2*>(ckpt + ((int64_t)b * nC + (c - 1)) * D + 2 * p);
        su = h.x;
        sw = h.y;
      } else if (h0 != nullptr) {
        su = h0[(int64_t)b * D + 2 * p];
        sw = h0[(int64_t)b * D + 2 * p + 1];
      }
    }
    float av[kMaxT], cv[kMaxT], sv[kMaxT], hu[kMaxT], hw[kMaxT];
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      av[t] = 1.f;
      cv[t] = 1.f;
      sv[t] = 0.f;
      hu[t] = 0.f;
      hw[t] = 0.f;
      if (t < T && act) {
        const int64_t ip = pbase + (int64_t)(c * T + t) * Dp;
        const int64_t ix = xbase + (int64_t)(c * T + t) * D;
        av[t] = rr::ld(a, ip);
        cv[t] = rr::ld(cs, ip);
        sv[t] = rr::ld(sn, ip);
        hu[t] = rr::ld(x, ix);
        hw[t] = rr::ld(x, ix + 1);
      }
    }
    // Recompute the chunk's states (hu/hw[t] = state after step t).
    {
      float u = su, v = sw;
#pragma unroll
      for (int t = 0; t < kMaxT; ++t) {
        if (t < T) {
          const float un = av[t] * (cv[t] * u - sv[t] * v) + hu[t];
          const float wn = av[t] * (sv[t] * u + cv[t] * v) + hw[t];
          u = un;
          v = wn;
          hu[t] = u;
          hw[t] = v;
        }
      }
    }
    // Chunk map of the adjoint from a zero carry: (P, E).
    float pr = 1.f, pi = 0.f, eu = 0.f, ew = 0.f;
#pragma unroll
    for (int t = kMaxT - 1; t >= 0; --t) {
      if (t < T) {
        const float* g = dy + xbase + (int64_t)(c * T + t) * D;
        float gu = 0.f, gw = 0.f;
        if (act) {
          const float2 gg = *reinterpret_cast<const float2*>(g);
          gu = gg.x;
          gw = gg.y;
        }
        eu += gu;
        ew += gw;
        const float nU = av[t] * (cv[t] * eu + sv[t] * ew);
        const float nW = av[t] * (-sv[t] * eu + cv[t] * ew);
        eu = nU;
        ew = nW;
        const float zr = av[t] * cv[t], zi = -av[t] * sv[t];
        const float npr = zr * pr - zi * pi;
        const float npi = zr * pi + zi * pr;
        pr = npr;
        pi = npi;
      }
    }
    sPr[w][lane] = pr;
    sPi[w][lane] = pi;
    sEu[w][lane] = eu;
    sEw[w][lane] = ew;
    __syncthreads();
    float lu = cu, lw = cw, nu = cu, nw = cw;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const float qr = sPr[j][lane], qi = sPi[j][lane], qu = sEu[j][lane], qw = sEw[j][lane];
      if (j < w) {
        const float tu = qr * lu - qi * lw + qu;
        const float tw = qi * lu + qr * lw + qw;
        lu = tu;
        lw = tw;
      }
      const float tu = qr * nu - qi * nw + qu;
      const float tw = qi * nu + qr * nw + qw;
      nu = tu;
      nw = tw;
    }
#pragma unroll
    for (int t = kMaxT - 1; t >= 0; --t) {
      if (t < T) {
        const int64_t ip = pbase + (int64_t)(c * T + t) * Dp;
        const int64_t ix = xbase + (int64_t)(c * T + t) * D;
        float gu = 0.f, gw = 0.f;
        if (act) {
          const float2 gg = *reinterpret_cast<const float2*>(dy + ix);
          gu = gg.x;
          gw = gg.y;
        }
        lu += gu;
        lw += gw;
        const float up = (t > 0) ? hu[t - 1] : su;
        const float wp = (t > 0) ? hw[t - 1] : sw;
        const float ru = cv[t] * up - sv[t] * wp;
        const float rw = sv[t] * up + cv[t] * wp;
        if (act) {
          rr::st(dx, ix, lu);
          rr::st(dx, ix + 1, lw);
          rr::st(da, ip, lu * ru + lw * rw);
          rr::st(dcs, ip, av[t] * (lu * up + lw * wp));
          rr::st(dsn, ip, av[t] * (lw * up - lu * wp));
        }
        const float nU = av[t] * (cv[t] * lu + sv[t] * lw);
        const float nW = av[t] * (-sv[t] * lu + cv[t] * lw);
        lu = nU;
        lw = nW;
      }
    }
    __syncthreads();
    cu = nu;
    cw = nw;
  }
  if (dh0 != nullptr && pok && w == 0) {
    dh0[(int64_t)b * D + 2 * p] = cu;
    dh0[(int64_t)b * D + 2 * p + 1] = cw;
  }
}

int check_common(int64_t B, int64_t L, int64_t Dp, int64_t seg, int dtype) {
  if (B <= 0 || L <= 0 || Dp <= 0) {
    return rr::fail(RR_EINVAL, "rotlru: B, L and Dp must be positive");
  }
  if (int rc = rr::check_segment_shape(L, seg, 2 * Dp, "D")) return rc;
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, "rotlru: unsupported dtype");
  if (B > 65535) return rr::fail(RR_EUNSUPPORTED, "rotlru: B > 65535 is not supported");
  return RR_OK;
}

constexpr int kFwdWaves = 8;
constexpr int kBwdWaves = 4;

}  // namespace

extern "C" int rr_rotlru_fwd(const void* a, const void* cs, const void* sn, const void* x,
                             int dtype, int64_t B, int64_t L, int64_t Dp, int64_t seg,
                             const float* h0, float* y, float* ckpt, void* stream) {
  if (int rc = check_common(B, L, Dp, seg, dtype)) return rc;
  if (!a || !cs || !sn || !x || !y || !ckpt) {
    return rr::fail(RR_EINVAL, "rotlru_fwd: null pointer argument");
  }
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  const dim3 grid((unsigned)((Dp + 63) / 64), (unsigned)B);
  hipStream_t s = static_cast<hipStream_t>(stream);
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rotlru_fwd_kernel<InT, kFwdWaves>), grid,
                                              dim3(64 * kFwdWaves), 0, s,
                                              static_cast<const InT*>(a),
                                              static_cast<const InT*>(cs),
                                              static_cast<const InT*>(sn),
                                              static_cast<const InT*>(x), h0, y, ckpt, (int)L,
                                              (int)Dp, T, nC));
  return rr::check_launch("rr_rotlru_fwd");
}

extern "C" int rr_rotlru_bwd(const float* dy, const float* dfinal, const void* a,
                             const void* cs, const void* sn, const void* x, int dtype,
                             int64_t B, int64_t L, int64_t Dp, int64_t seg, const float* h0,
                             const float* ckpt, void* da, void* dcs, void* dsn, void* dx,
                             float* dh0, void* stream) {
  if (int rc = check_common(B, L, Dp, seg, dtype)) return rc;
  if (!dy || !a || !cs || !sn || !x || !ckpt || !da || !dcs || !dsn || !dx) {
    return rr::fail(RR_EINVAL, "rotlru_bwd: null pointer argument");
  }
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  const dim3 grid((unsigned)((Dp + 63) / 64), (unsigned)B);
  hipStream_t s = static_cast<hipStream_t>(stream);
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rotlru_bwd_kernel<InT, kBwdWaves>), grid,
                                              dim3(64 * kBwdWaves), 0, s, dy, dfinal,
                                              static_cast<const InT*>(a),
                                              static_cast<const InT*>(cs),
                                              static_cast<const InT*>(sn),
                                              static_cast<const InT*>(x), h0, ckpt,
                                              static_cast<InT*>(da), static_cast<InT*>(dcs),
                                              static_cast<InT*>(dsn), static_cast<InT*>(dx), dh0,
                                              (int)L, (int)Dp, T, nC));
  return rr::check_launch("rr_rotlru_bwd");
}
