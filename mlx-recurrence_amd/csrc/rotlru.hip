// rotlru.hip — rotational LRU, a pair-diagonal (complex) scan on gfx950:
//   u_t = a_t (c_t u_{t-1} - s_t w_{t-1}) + x_t[2p]
//   w_t = a_t (s_t u_{t-1} + c_t w_{t-1}) + x_t[2p+1]
// i.e. h_t = z_t h_{t-1} + x_t with the complex gate z_t = a_t (c_t + i s_t).
//
// Reference: mlx_recurrence/rotlru.py (forward :80-146, backward :153-266, VJP
// :35-40, :206-235).  Same tiled chained scan as rglru.hip (rr_tiles.h): a
// workgroup of NW waves owns a tile of 64 * CP pairs of one batch row and
// NW * U steps; lane l holds pairs CP*l .. CP*l + CP - 1 (a/cs/sn: one CP-wide
// access per step; x and y: one 2*CP-wide access).  The maps h -> P h + E are
// complex; the adjoint multiplies by conj(z_t) (the transpose of a_t R(theta_t)),
// so the backward pass has the same structure in reverse time.
#include "rr_tiles.h"

namespace {

using rr::tiles::Pack;
using rr::tiles::ld_pack;
using rr::tiles::pack_fill;

constexpr int kNW = 8;
constexpr int kCP = 2;   // pairs per lane
constexpr int kU = 8;    // steps per wave

struct TileGrid {
  int G;   // pair tiles per batch row
  int K;   // step tiles
  int64_t tiles() const { return (int64_t)G * K; }
};
inline TileGrid tile_grid(int64_t L, int64_t Dp) {
  const int64_t S = (int64_t)kU * kNW;
  return TileGrid{(int)((Dp + 64 * kCP - 1) / (64 * kCP)), (int)((L + S - 1) / S)};
}

struct cplx {
  float r, i;
};
__device__ __forceinline__ cplx cmul(cplx p, cplx q) { return {p.r * q.r - p.i * q.i, p.r * q.i + p.i * q.r}; }
__device__ __forceinline__ cplx cfma(cplx p, cplx q, cplx e) {   // p q + e
  return {p.r * q.r - p.i * q.i + e.r, p.r * q.i + p.i * q.r + e.i};
}
__device__ __forceinline__ cplx conj(cplx p) { return {p.r, -p.i}; }

// The inputs of one wave: U steps of CP pairs.
// TH: the rotation comes as the angle theta (one input instead of cos and
// sin; the reference forms cos / sin in MLX host code, rotlru.py:18-23), and
// the kernel takes sincosf of it in registers.
template <typename InT, int U, bool TH>
struct WaveIn {
  Pack<InT, kCP> a[U], c[U], s[TH ? 1 : U];   // TH: c holds theta
  float cf[TH ? U : 1][kCP], sf[TH ? U : 1][kCP];
  Pack<InT, 2 * kCP> x[U];
  __device__ float cosv(int u, int q) const {
    if constexpr (TH) return cf[u][q];
    else return c[u][q];
  }
  __device__ float sinv(int u, int q) const {
    if constexpr (TH) return sf[u][q];
    else return s[u][q];
  }
  __device__ cplx z(int u, int q) const { return {a[u][q] * cosv(u, q), a[u][q] * sinv(u, q)}; }
  __device__ cplx xin(int u, int q) const { return {x[u][2 * q], x[u][2 * q + 1]}; }
};

// Step u of pair p sits at element rb + u Dp + p of a / cs / sn and at twice
// that in x (rb: the wave's first step row, uniform).  issue_wave loads every
// step in every lane at a clamped step and pair (in bounds); finish_wave,
// called once all of the wave's loads are issued, gives the steps past L or
// Dp the identity (z = 1, x = 0, theta = 0) and forms cos / sin of theta.
__device__ __forceinline__ uint32_t step_off(int u, int t0, int L, int Dp, int pc) {
  return (uint32_t)((min(t0 + u, L - 1) - min(t0, L - 1)) * Dp + pc);   // the step clamped to L - 1
}
template <typename InT, int U, bool TH>
__device__ __forceinline__ void issue_wave(WaveIn<InT, U, TH>& in, const InT* a, const InT* cs, const InT* sn,
                                           const InT* x, int64_t rb, int t0, int L, int Dp, int pc) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t ip = step_off(u, t0, L, Dp, pc);
    in.a[u] = rr::tiles::ld_pack_at<InT, kCP>(a + rb, ip);
    in.c[u] = rr::tiles::ld_pack_at<InT, kCP>(cs + rb, ip);
    if constexpr (!TH) in.s[u] = rr::tiles::ld_pack_at<InT, kCP>(sn + rb, ip);
    in.x[u] = rr::tiles::ld_pack_at<InT, 2 * kCP>(x + 2 * rb, 2 * ip);
  }
}
template <typename InT, int U, bool TH>
__device__ __forceinline__ void finish_wave(WaveIn<InT, U, TH>& in, int t0, int L, bool pok) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool ok = pok && t0 + u < L;
    in.a[u] = rr::tiles::pick<InT, kCP>(ok, in.a[u], pack_fill<InT, kCP>(1.f));
    in.c[u] = rr::tiles::pick<InT, kCP>(ok, in.c[u], pack_fill<InT, kCP>(TH ? 0.f : 1.f));
    if constexpr (!TH) in.s[u] = rr::tiles::pick<InT, kCP>(ok, in.s[u], pack_fill<InT, kCP>(0.f));
    in.x[u] = rr::tiles::pick<InT, 2 * kCP>(ok, in.x[u], pack_fill<InT, 2 * kCP>(0.f));
  }
  if constexpr (TH) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int q = 0; q < kCP; ++q) sincosf(in.c[u][q], &in.sf[u][q], &in.cf[u][q]);
  }
}

template <typename InT, bool TH>
__global__ __launch_bounds__(64 * kNW, 4) void rotlru_fwd_kernel(
    const InT* __restrict__ a, const InT* __restrict__ cs, const InT* __restrict__ sn,
    const InT* __restrict__ x, const float* __restrict__ h0, float* __restrict__ y,
    float* __restrict__ ckpt, uint32_t* counter, uint64_t* slots, uint32_t* status, int B, int L, int Dp, int T,
    int nC, int G, int K) {
  constexpr int GP = 64 * kCP, S = kU * kNW;
  __shared__ cplx sP[kNW][GP], sE[kNW][GP];
  __shared__ cplx sIn[GP];
  __shared__ int sTicket;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nGrp = B * G;
  const int ticket = rr::tiles::take_ticket(counter, nGrp * K, &sTicket);
  if (ticket < 0) return;
  const rr::tiles::TileOfTicket tt = rr::tiles::tile_of_ticket(ticket, nGrp, K, false);
  const int k = tt.k, grp = tt.grp;
  const int b = grp / G, g = grp % G;
  const int p = g * GP + lane * kCP;
  const bool pok = p < Dp;
  const int D = 2 * Dp;
  const int t0 = k * S + w * kU;
  const int64_t row0 = (int64_t)b * L;
  const int64_t rb = (row0 + min(t0, L - 1)) * Dp;   // the wave's first step row (clamped)
  const int pc = min(p, Dp - kCP);                    // clamped pair: every lane loads

  WaveIn<InT, kU, TH> in;
  issue_wave<InT, kU, TH>(in, a, cs, sn, x, rb, t0, L, Dp, pc);
  finish_wave<InT, kU, TH>(in, t0, L, pok);
#pragma unroll
  for (int q = 0; q < kCP; ++q) {
    cplx P{1.f, 0.f}, E{0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const cplx z = in.z(u, q);
      E = cfma(z, E, in.xin(u, q));
      P = cmul(z, P);
    }
    sP[w][lane * kCP + q] = P;
    sE[w][lane * kCP + q] = E;
  }
  __syncthreads();
  if (w == 0) {
    // slot of (tile, lane, q, real / imaginary part j): tile * 2 GP +
    // 64 (2 q + j) + lane (a wave's hand-off stores and loads cover whole
    // 32-byte sectors)
    uint64_t* mine = slots + ((int64_t)grp * K + k) * (2 * GP) + lane;
#pragma unroll
    for (int q = 0; q < kCP; ++q) {
      cplx hin{0.f, 0.f};
      if (k > 0) {
        hin.r = rr::tiles::take_value(mine - 2 * GP + 128 * q, status);
        hin.i = rr::tiles::take_value(mine - 2 * GP + 128 * q + 64, status);
      } else if (h0 != nullptr && pok) {
        hin = {h0[(int64_t)b * D + 2 * (p + q)], h0[(int64_t)b * D + 2 * (p + q) + 1]};
      }
      sIn[lane * kCP + q] = hin;
      if (k + 1 < K) {
        cplx hout = hin;
#pragma unroll
        for (int j = 0; j < kNW; ++j) hout = cfma(sP[j][lane * kCP + q], hout, sE[j][lane * kCP + q]);
        rr::tiles::publish(mine + 128 * q, hout.r);
        rr::tiles::publish(mine + 128 * q + 64, hout.i);
      }
    }
  }
  __syncthreads();
  cplx h[kCP];
#pragma unroll
  for (int q = 0; q < kCP; ++q) {
    h[q] = sIn[lane * kCP + q];
    for (int j = 0; j < w; ++j) h[q] = cfma(sP[j][lane * kCP + q], h[q], sE[j][lane * kCP + q]);
  }
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int t = t0 + u;
    float out[2 * kCP];
#pragma unroll
    for (int q = 0; q < kCP; ++q) {
      h[q] = cfma(in.z(u, q), h[q], in.xin(u, q));   // rotlru.py:101-122
      out[2 * q] = h[q].r;
      out[2 * q + 1] = h[q].i;
    }
    if (pok && t < L) {
      rr::tiles::st_f32_at<2 * kCP>(y + 2 * rb, (uint32_t)(u * D + 2 * p), out);
      if ((t + 1) % T == 0) rr::tiles::st_f32<2 * kCP>(ckpt, ((int64_t)b * nC + (t + 1) / T - 1) * D + 2 * p, out);
    }
  }
}

// Adjoint (rotlru.py:35-40, :206-235), per step t going backwards with
// r = R(theta_t) h_{t-1}:
//   lam += dy_t; dx_t = lam; da_t = lam . r;
//   dcs_t = a_t (lamU u_{t-1} + lamW w_{t-1}); dsn_t = a_t (lamW u_{t-1} - lamU w_{t-1});
//   lam = conj(z_t) lam.
template <typename InT, bool TH>
__global__ __launch_bounds__(64 * kNW, 2) void rotlru_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ dfinal, const InT* __restrict__ a,
    const InT* __restrict__ cs, const InT* __restrict__ sn, const InT* __restrict__ x,
    const float* __restrict__ h0, const float* __restrict__ ckpt, InT* __restrict__ da,
    InT* __restrict__ dcs, InT* __restrict__ dsn, InT* __restrict__ dx, float* __restrict__ dh0,
    uint32_t* counter, uint64_t* slots, uint32_t* status, int B, int L, int Dp, int T, int nC, int G, int K) {
  constexpr int GP = 64 * kCP, S = kU * kNW;
  __shared__ cplx sP[kNW][GP], sEf[kNW][GP], sEb[kNW][GP];
  __shared__ cplx sIn[GP];
  __shared__ int sTicket;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nGrp = B * G;
  const int ticket = rr::tiles::take_ticket(counter, nGrp * K, &sTicket);
  if (ticket < 0) return;
  const rr::tiles::TileOfTicket tt = rr::tiles::tile_of_ticket(ticket, nGrp, K, true);
  const int k = tt.k, grp = tt.grp;
  const int b = grp / G, g = grp % G;
  const int p = g * GP + lane * kCP;
  const bool pok = p < Dp;
  const int D = 2 * Dp;
  const int t0 = k * S + w * kU;
  const int64_t row0 = (int64_t)b * L;
  const int64_t rb = (row0 + min(t0, L - 1)) * Dp;   // the wave's first step row (clamped)
  const int pc = min(p, Dp - kCP);                    // clamped pair: every lane loads

  // every load first: dy, the inputs, and the state entering the wave's
  // checkpoint interval (checkpoint row crow, or h0 at tb = 0, or zero: then
  // any valid row is read and dropped)
  Pack<float, 2 * kCP> g4[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) g4[u] = rr::tiles::ld_pack_at<float, 2 * kCP>(dy + 2 * rb, 2 * step_off(u, t0, L, Dp, pc));
  WaveIn<InT, kU, TH> in;
  issue_wave<InT, kU, TH>(in, a, cs, sn, x, rb, t0, L, Dp, pc);
  const int tb = t0 - t0 % T;   // start of the checkpoint interval (inside the tile: S % 32 == 0)
  const int crow = rr::tiles::bwd_ckpt_row(t0, T, L);
  const bool from_h0 = crow < 0 && tb == 0 && h0 != nullptr;
  const bool huse = crow >= 0 || from_h0;
  const float* const hsrc = crow >= 0 ? ckpt + ((int64_t)b * nC + crow) * D : (from_h0 ? h0 + (int64_t)b * D : ckpt);
  Pack<float, 2 * kCP> h4 = rr::tiles::ld_pack_at<float, 2 * kCP>(hsrc, (uint32_t)(2 * pc));
  finish_wave<InT, kU, TH>(in, t0, L, pok);
  cplx gy[kU][kCP];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    g4[u] = rr::tiles::pick<float, 2 * kCP>(pok && t0 + u < L, g4[u], pack_fill<float, 2 * kCP>(0.f));
#pragma unroll
    for (int q = 0; q < kCP; ++q) gy[u][q] = {g4[u][2 * q], g4[u][2 * q + 1]};
  }
  // forward map (from a zero state) and adjoint map (from a zero adjoint)
#pragma unroll
  for (int q = 0; q < kCP; ++q) {
    cplx P{1.f, 0.f}, Ef{0.f, 0.f}, Eb{0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const cplx z = in.z(u, q);
      Ef = cfma(z, Ef, in.xin(u, q));
      P = cmul(z, P);
    }
#pragma unroll
    for (int u = kU - 1; u >= 0; --u) {
      Eb = {Eb.r + gy[u][q].r, Eb.i + gy[u][q].i};
      Eb = cmul(conj(in.z(u, q)), Eb);
    }
    sP[w][lane * kCP + q] = P;
    sEf[w][lane * kCP + q] = Ef;
    sEb[w][lane * kCP + q] = Eb;
  }
  __syncthreads();
  if (w == 0) {
    uint64_t* mine = slots + ((int64_t)grp * K + k) * (2 * GP) + lane;   // slot layout as in the forward
#pragma unroll
    for (int q = 0; q < kCP; ++q) {
      cplx lin{0.f, 0.f};   // adjoint entering the tile from later steps
      if (k + 1 < K) {
        lin.r = rr::tiles::take_value(mine + 2 * GP + 128 * q, status);
        lin.i = rr::tiles::take_value(mine + 2 * GP + 128 * q + 64, status);
      } else if (dfinal != nullptr && pok) {
        lin = {dfinal[(int64_t)b * D + 2 * (p + q)], dfinal[(int64_t)b * D + 2 * (p + q) + 1]};
      }
      sIn[lane * kCP + q] = lin;
      cplx lout = lin;
#pragma unroll
      for (int j = kNW - 1; j >= 0; --j) lout = cfma(conj(sP[j][lane * kCP + q]), lout, sEb[j][lane * kCP + q]);
      if (k > 0) {
        rr::tiles::publish(mine + 128 * q, lout.r);
        rr::tiles::publish(mine + 128 * q + 64, lout.i);
      } else if (dh0 != nullptr && pok) {
        dh0[(int64_t)b * D + 2 * (p + q)] = lout.r;
        dh0[(int64_t)b * D + 2 * (p + q) + 1] = lout.i;
      }
    }
  }
  __syncthreads();
  cplx lam[kCP], hin[kCP];
  h4 = rr::tiles::pick<float, 2 * kCP>(huse && pok, h4, pack_fill<float, 2 * kCP>(0.f));
#pragma unroll
  for (int q = 0; q < kCP; ++q) {
    lam[q] = sIn[lane * kCP + q];
    for (int j = kNW - 1; j > w; --j) lam[q] = cfma(conj(sP[j][lane * kCP + q]), lam[q], sEb[j][lane * kCP + q]);
    hin[q] = {h4[2 * q], h4[2 * q + 1]};
    for (int j = w - (t0 - tb) / kU; j < w; ++j) hin[q] = cfma(sP[j][lane * kCP + q], hin[q], sEf[j][lane * kCP + q]);
  }
  cplx hs[kU][kCP];   // hs[u] = h_{t0+u}
#pragma unroll
  for (int q = 0; q < kCP; ++q) {
    cplx h = hin[q];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      h = cfma(in.z(u, q), h, in.xin(u, q));
      hs[u][q] = h;
    }
  }
#pragma unroll
  for (int u = kU - 1; u >= 0; --u) {
    const int t = t0 + u;
    float gx[2 * kCP], ga[kCP], gc[kCP], gs[kCP];
#pragma unroll
    for (int q = 0; q < kCP; ++q) {
      const cplx hp = u > 0 ? hs[u - 1][q] : hin[q];
      const float av = in.a[u][q], cv = in.cosv(u, q), sv = in.sinv(u, q);
      lam[q] = {lam[q].r + gy[u][q].r, lam[q].i + gy[u][q].i};
      gx[2 * q] = lam[q].r;
      gx[2 * q + 1] = lam[q].i;
      const float ru = cv * hp.r - sv * hp.i, rw = sv * hp.r + cv * hp.i;
      ga[q] = lam[q].r * ru + lam[q].i * rw;
      gc[q] = av * (lam[q].r * hp.r + lam[q].i * hp.i);
      gs[q] = av * (lam[q].i * hp.r - lam[q].r * hp.i);
      lam[q] = cmul(conj(in.z(u, q)), lam[q]);
    }
    if (pok && t < L) {
      const uint32_t ip = (uint32_t)(u * Dp + p);
      rr::tiles::st_pack_at<InT, kCP>(da + rb, ip, ga);
      if constexpr (TH) {   // d theta = -sin * dcos + cos * dsin
        float gt[kCP];
#pragma unroll
        for (int q = 0; q < kCP; ++q) gt[q] = in.cosv(u, q) * gs[q] - in.sinv(u, q) * gc[q];
        rr::tiles::st_pack_at<InT, kCP>(dcs + rb, ip, gt);
      } else {
        rr::tiles::st_pack_at<InT, kCP>(dcs + rb, ip, gc);
        rr::tiles::st_pack_at<InT, kCP>(dsn + rb, ip, gs);
      }
      rr::tiles::st_pack_at<InT, 2 * kCP>(dx + 2 * rb, 2 * ip, gx);
    }
  }
}

int check_common(int64_t B, int64_t L, int64_t Dp, int64_t seg, int dtype) {
  if (B <= 0 || L <= 0 || Dp <= 0) return rr::fail(RR_EINVAL, "rotlru: B, L and Dp must be positive");
  if (int rc = rr::check_segment_shape(L, seg, 2 * Dp, "D")) return rc;   // rotlru.py:283
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, "rotlru: unsupported dtype");
  if (B * L * 2 * Dp >= ((int64_t)1 << 40)) return rr::fail(RR_EUNSUPPORTED, "rotlru: tensor too large");
  return RR_OK;
}

size_t ws_bytes_for(int64_t B, int64_t L, int64_t Dp) {
  return rr::tiles::ws_bytes(B * tile_grid(L, Dp).tiles(), 2 * 64 * kCP);
}

}  // namespace

rr::tiles::Geometry rr::rotlru_geometry(int64_t L, int64_t Dp) {
  const TileGrid tg = tile_grid(L, Dp);
  return rr::tiles::Geometry{tg.G, tg.K, kU, kNW};
}

extern "C" size_t rr_rotlru_workspace_bytes(int64_t B, int64_t L, int64_t Dp, int64_t seg, int dtype,
                                            int pass) {
  (void)pass;
  if (B <= 0 || L <= 0 || Dp <= 0 || rr::chunk_len(L, seg) == 0 || !rr::valid_dtype(dtype)) return 0;
  return ws_bytes_for(B, L, Dp);
}

extern "C" int rr_rotlru_fwd(const void* a, const void* cs, const void* sn, const void* x, int dtype,
                             int64_t B, int64_t L, int64_t Dp, int64_t seg, const float* h0, float* y,
                             float* ckpt, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_common(B, L, Dp, seg, dtype)) return rc;
  if (!a || !cs || !sn || !x || !y || !ckpt) return rr::fail(RR_EINVAL, "rotlru_fwd: null pointer argument");
  const size_t need = ws_bytes_for(B, L, Dp);
  if (!workspace || workspace_bytes < need) return rr::fail(RR_EWORKSPACE, "rotlru_fwd: workspace too small");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  const TileGrid tg = tile_grid(L, Dp);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* status = rr::status_word();
  if (status == nullptr) return RR_EHIP;
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rotlru_fwd_kernel<InT, false>), dim3((unsigned)(B * tg.tiles())),
                                              dim3(64 * kNW), 0, s, static_cast<const InT*>(a),
                                              static_cast<const InT*>(cs), static_cast<const InT*>(sn),
                                              static_cast<const InT*>(x), h0, y, ckpt,
                                              rr::tiles::ws_counter(workspace), rr::tiles::ws_slots(workspace),
                                              status, (int)B, (int)L, (int)Dp, T, nC, tg.G, tg.K));
  return rr::check_launch("rr_rotlru_fwd");
}

extern "C" int rr_rotlru_bwd(const float* dy, const float* dfinal, const void* a, const void* cs,
                             const void* sn, const void* x, int dtype, int64_t B, int64_t L,
                             int64_t Dp, int64_t seg, const float* h0, const float* ckpt, void* da,
                             void* dcs, void* dsn, void* dx, float* dh0, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (int rc = check_common(B, L, Dp, seg, dtype)) return rc;
  if (!dy || !a || !cs || !sn || !x || !ckpt || !da || !dcs || !dsn || !dx)
    return rr::fail(RR_EINVAL, "rotlru_bwd: null pointer argument");
  const size_t need = ws_bytes_for(B, L, Dp);
  if (!workspace || workspace_bytes < need) return rr::fail(RR_EWORKSPACE, "rotlru_bwd: workspace too small");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  const TileGrid tg = tile_grid(L, Dp);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* status = rr::status_word();
  if (status == nullptr) return RR_EHIP;
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rotlru_bwd_kernel<InT, false>), dim3((unsigned)(B * tg.tiles())),
                                              dim3(64 * kNW), 0, s, dy, dfinal, static_cast<const InT*>(a),
                                              static_cast<const InT*>(cs), static_cast<const InT*>(sn),
                                              static_cast<const InT*>(x), h0, ckpt, static_cast<InT*>(da),
                                              static_cast<InT*>(dcs), static_cast<InT*>(dsn),
                                              static_cast<InT*>(dx), dh0, rr::tiles::ws_counter(workspace),
                                              rr::tiles::ws_slots(workspace), status, (int)B, (int)L, (int)Dp, T, nC,
                                              tg.G, tg.K));
  return rr::check_launch("rr_rotlru_bwd");
}

extern "C" int rr_rotlru_theta_fwd(const void* a, const void* theta, const void* x, int dtype, int64_t B,
                                   int64_t L, int64_t Dp, int64_t seg, const float* h0, float* y, float* ckpt,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_common(B, L, Dp, seg, dtype)) return rc;
  if (!a || !theta || !x || !y || !ckpt) return rr::fail(RR_EINVAL, "rotlru_theta_fwd: null pointer argument");
  const size_t need = ws_bytes_for(B, L, Dp);
  if (!workspace || workspace_bytes < need) return rr::fail(RR_EWORKSPACE, "rotlru_theta_fwd: workspace too small");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  const TileGrid tg = tile_grid(L, Dp);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* status = rr::status_word();
  if (status == nullptr) return RR_EHIP;
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rotlru_fwd_kernel<InT, true>), dim3((unsigned)(B * tg.tiles())),
                                              dim3(64 * kNW), 0, s, static_cast<const InT*>(a),
                                              static_cast<const InT*>(theta), nullptr, static_cast<const InT*>(x),
                                              h0, y, ckpt, rr::tiles::ws_counter(workspace),
                                              rr::tiles::ws_slots(workspace), status, (int)B, (int)L, (int)Dp, T, nC,
                                              tg.G, tg.K));
  return rr::check_launch("rr_rotlru_theta_fwd");
}

extern "C" int rr_rotlru_theta_bwd(const float* dy, const float* dfinal, const void* a, const void* theta,
                                   const void* x, int dtype, int64_t B, int64_t L, int64_t Dp, int64_t seg,
                                   const float* h0, const float* ckpt, void* da, void* dtheta, void* dx,
                                   float* dh0, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_common(B, L, Dp, seg, dtype)) return rc;
  if (!dy || !a || !theta || !x || !ckpt || !da || !dtheta || !dx)
    return rr::fail(RR_EINVAL, "rotlru_theta_bwd: null pointer argument");
  const size_t need = ws_bytes_for(B, L, Dp);
  if (!workspace || workspace_bytes < need) return rr::fail(RR_EWORKSPACE, "rotlru_theta_bwd: workspace too small");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  const TileGrid tg = tile_grid(L, Dp);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* status = rr::status_word();
  if (status == nullptr) return RR_EHIP;
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((rotlru_bwd_kernel<InT, true>), dim3((unsigned)(B * tg.tiles())),
                                              dim3(64 * kNW), 0, s, dy, dfinal, static_cast<const InT*>(a),
                                              static_cast<const InT*>(theta), nullptr, static_cast<const InT*>(x),
                                              h0, ckpt, static_cast<InT*>(da), static_cast<InT*>(dtheta), nullptr,
                                              static_cast<InT*>(dx), dh0, rr::tiles::ws_counter(workspace),
                                              rr::tiles::ws_slots(workspace), status, (int)B, (int)L, (int)Dp, T, nC,
                                              tg.G, tg.K));
  return rr::check_launch("rr_rotlru_theta_bwd");
}
