// rglru.hip — RG-LRU diagonal scan h_t = a_t * h_{t-1} + x_t on gfx950.
//
// Reference: mlx_recurrence/rglru.py (forward kernel :64-123, backward kernel
// :130-203, VJP formulas :36-39).  The reference gives every (batch, channel)
// one thread that walks all L steps.  Here a pass is one tiled chained scan
// (rr_tiles.h): a workgroup of NW waves owns a tile of 64 * CH channels of one
// batch row and NW * U steps; lane l holds channels CH*l .. CH*l + CH - 1 (one
// 8- or 16-byte access per step) and wave w steps w*U .. w*U + U - 1 of the
// tile.  Each wave folds its steps into the affine map h -> P h + E, the maps
// meet in LDS, wave 0 takes the state entering the tile from the previous tile
// of the same channels and hands on the state leaving it, and every wave
// replays its steps from registers (inputs are read from HBM once).
//
// The backward pass runs the same scheme in reverse time on the adjoint
// lam_{t-1} = a_t lam_t + dy_{t-1} (reference :36-39, :173-178:
// lam += dy_t; dx_t = lam; da_t = lam * h_{t-1}; lam *= a_t), recomputing the
// states of each wave's steps from the forward checkpoint at the start of the
// checkpoint interval that contains them.
#include "rr_tiles.h"

namespace {

using rr::tiles::Pack;
using rr::tiles::ld_pack;
using rr::tiles::pack_fill;

// Tile shapes (measured on MI355X at B8 L4096 D2560): CH = 2 channels per
// lane; U steps per wave: forward 16 for 16-bit inputs, otherwise 8 (the
// backward also holds dy and the recomputed states; the gated passes hold
// the gates in fp32, the gated backward 4 steps); NW = 8 waves, two
// workgroups per CU.  A tile's NW * U steps are a multiple of 32, so it holds
// whole checkpoint intervals.
template <typename InT, bool BWD, bool GATED> constexpr int steps_per_wave() {
  return BWD && GATED ? 4 : sizeof(InT) == 4 || BWD || GATED ? 8 : 16;
}
constexpr int kNW = 8;
constexpr int kFwdCh = 2, kBwdCh = 2;

struct TileGrid {
  int G;   // channel tiles per batch row
  int K;   // step tiles
  int64_t tiles() const { return (int64_t)G * K; }
};
inline int steps_per_wave(int dtype, int pass, bool gated) {
  return pass == 1 && gated ? 4 : dtype == RR_F32 || pass == 1 || gated ? 8 : 16;
}
inline TileGrid tile_grid(int64_t L, int64_t D, int ch, int dtype, int pass, bool gated = false) {
  const int64_t S = (int64_t)steps_per_wave(dtype, pass, gated) * kNW;
  return TileGrid{(int)((D + 64 * ch - 1) / (64 * ch)), (int)((L + S - 1) / S)};
}

// Gated RG-LRU (the Griffin gate math of reference rglru.py:13-14, which the
// reference computes in MLX before its scan kernel): with c' = c softplus(lam)
// per channel, a = exp(-c' sigmoid(r)) and x' = sqrt(1 - a^2) (i x).  The
// per-element math uses the hardware exp / reciprocal / square root (about
// 1 ulp each; the correctly rounded library forms made the passes VALU-bound),
// and 1 - a^2 = -expm1(2z), z = -c' sigmoid(r), takes its Taylor series
// through z^5 where 1 - a^2 would cancel (2z > -1/8; truncation < 1e-7
// relative), so s = sqrt(1 - a^2) keeps its relative accuracy as a -> 1.
__device__ __forceinline__ float softplus_f(float v) { return v > 20.f ? v : log1pf(expf(v)); }
__device__ __forceinline__ float sigmoid_f(float v) { return __builtin_amdgcn_rcpf(1.f + __expf(-v)); }
// (from sr = sigmoid(r))
__device__ __forceinline__ void gate_s(float sr, float csp, float& a, float& s) {
  const float z = -csp * sr;
  a = __expf(z);
  const float t = 2.f * z;
  float p = -t * (1.f + t * (0.5f + t * (1.f / 6 + t * (1.f / 24 + t * (1.f / 120)))));
  float q = 1.f - a * a;
  asm volatile("" : "+v"(p));   // both forms, then a select (no divergent branch per element)
  asm volatile("" : "+v"(q));
  s = __builtin_amdgcn_sqrtf(t > -0.125f ? p : q);
}

// c' = c softplus(lam) of a lane's CH channels, formed once per workgroup:
// the waves w < CH form channel 64 w + lane of the tile from lv (its lam,
// loaded by every wave before the step inputs) into sC; after a workgroup
// barrier each lane reads its own.  Channels past D read 0.
template <int CH, bool GATED>
__device__ __forceinline__ void tile_csp(float lv, float gc, int w, int lane, bool cok, float* sC, float (&csp)[CH]) {
  if constexpr (GATED) {
    if (w < CH) sC[64 * w + lane] = gc * softplus_f(lv);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CH; ++c) csp[c] = cok ? sC[lane * CH + c] : 0.f;
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c) csp[c] = 0.f;
  }
}

// A wave's U steps of the scan inputs.  Plain: pa = a, px = x.  Gated:
// pa = r, px = x, pi = i, and the fp32 gates av = a, sv = sqrt(1 - a^2),
// sr = sigmoid(r).  Steps past L or D are identity steps (a = 1, x' = 0).
// rb: element offset of the wave's first step row (uniform), so step u of
// channel ch is at rb + u D + ch.  issue_steps loads every step in every lane
// at a clamped step and channel (in bounds); finish_steps, called once all
// of the wave's loads are issued, gives masked positions the identity values
// and forms the gates.
__device__ __forceinline__ uint32_t step_off(int u, int t0, int L, int D, int chc) {
  return (uint32_t)((min(t0 + u, L - 1) - min(t0, L - 1)) * D + chc);   // the step clamped to L - 1
}
template <typename InT, int CH, int U, bool GATED>
__device__ __forceinline__ void issue_steps(const InT* a, const InT* x, const InT* gi, int t0, int L, int64_t rb,
                                            int D, int chc, Pack<InT, CH> (&pa)[U], Pack<InT, CH> (&px)[U],
                                            Pack<InT, CH> (&pi)[GATED ? U : 1]) {
  const InT* const aw = a + rb;
  const InT* const xw = x + rb;
  const InT* const iw = GATED ? gi + rb : nullptr;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = step_off(u, t0, L, D, chc);
    pa[u] = rr::tiles::ld_pack_at<InT, CH>(aw, i);
    px[u] = rr::tiles::ld_pack_at<InT, CH>(xw, i);
    if constexpr (GATED) pi[u] = rr::tiles::ld_pack_at<InT, CH>(iw, i);
  }
}
template <typename InT, int CH, int U, bool GATED>
__device__ __forceinline__ void finish_steps(const float (&csp)[CH], bool cok, int t0, int L,
                                             Pack<InT, CH> (&pa)[U], Pack<InT, CH> (&px)[U],
                                             Pack<InT, CH> (&pi)[GATED ? U : 1], float (&av)[GATED ? U : 1][CH],
                                             float (&sv)[GATED ? U : 1][CH], float (&sr)[GATED ? U : 1][CH]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {   // identity steps past L or D
    const bool ok = cok && t0 + u < L;
    pa[u] = rr::tiles::pick<InT, CH>(ok, pa[u], pack_fill<InT, CH>(1.f));
    px[u] = rr::tiles::pick<InT, CH>(ok, px[u], pack_fill<InT, CH>(0.f));
    if constexpr (GATED) pi[u] = rr::tiles::pick<InT, CH>(ok, pi[u], pack_fill<InT, CH>(0.f));
  }
  if constexpr (GATED) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = cok && t0 + u < L;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        sr[u][c] = sigmoid_f(pa[u][c]);
        gate_s(sr[u][c], csp[c], av[u][c], sv[u][c]);
        if (!ok) av[u][c] = 1.f, sv[u][c] = 0.f;
      }
    }
  }
}

template <typename InT, int CH, int U, bool GATED>
__global__ __launch_bounds__(64 * kNW, 4) void rglru_fwd_kernel(
    const InT* __restrict__ a, const InT* __restrict__ x, const InT* __restrict__ gi,
    const float* __restrict__ glam, float gc, const float* __restrict__ h0, float* __restrict__ y,
    float* __restrict__ ckpt, uint32_t* counter, uint64_t* slots, uint32_t* status, int B, int L, int D, int T,
    int nC, int G, int K) {
  constexpr int GCH = 64 * CH, S = U * kNW;
  __shared__ float sP[kNW][GCH], sE[kNW][GCH];
  __shared__ float sIn[GCH];
  __shared__ float sC[GATED ? GCH : 1];
  __shared__ int sTicket;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // tickets run over step tiles slowest, so the tile before (same channels,
  // previous steps) always holds a smaller ticket
  const int nGrp = B * G;
  const int ticket = rr::tiles::take_ticket(counter, nGrp * K, &sTicket);
  if (ticket < 0) return;
  const rr::tiles::TileOfTicket tt = rr::tiles::tile_of_ticket(ticket, nGrp, K, false);
  const int k = tt.k, grp = tt.grp;
  const int b = grp / G, g = grp % G;
  const int ch = g * GCH + lane * CH;
  const bool cok = ch < D;
  const int t0 = k * S + w * U;
  const int64_t row0 = (int64_t)b * L;
  // the wave's first step row (clamped: a wave wholly past L touches nothing)
  const int64_t rb = (row0 + min(t0, L - 1)) * D;

  // every load first (clamped channel: every lane loads), then masks and gates
  const int chc = min(ch, D - CH);
  const float lv = GATED ? glam[min(g * GCH + 64 * (w % CH) + lane, D - 1)] : 0.f;
  Pack<InT, CH> pa[U], px[U], pi[GATED ? U : 1];
  issue_steps<InT, CH, U, GATED>(a, x, gi, t0, L, rb, D, chc, pa, px, pi);
  float csp[CH];
  tile_csp<CH, GATED>(lv, gc, w, lane, cok, sC, csp);
  float av[GATED ? U : 1][CH], sv[GATED ? U : 1][CH], sr[GATED ? U : 1][CH];
  finish_steps<InT, CH, U, GATED>(csp, cok, t0, L, pa, px, pi, av, sv, sr);
  // the step's decay and input
  auto A = [&](int u, int c) -> float {
    if constexpr (GATED) return av[u][c];
    else return pa[u][c];
  };
  auto X = [&](int u, int c) -> float {
    if constexpr (GATED) return sv[u][c] * (pi[u][c] * px[u][c]);
    else return px[u][c];
  };
  float P[CH], E[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    P[c] = 1.f;
    E[c] = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      E[c] = A(u, c) * E[c] + X(u, c);
      P[c] *= A(u, c);
    }
    sP[w][lane * CH + c] = P[c];
    sE[w][lane * CH + c] = E[c];
  }
  __syncthreads();
  if (w == 0) {
    // slot of (tile, lane, c): tile * GCH + 64 c + lane (a wave's hand-off
    // stores and loads cover whole 32-byte sectors)
    uint64_t* mine = slots + ((int64_t)grp * K + k) * GCH + lane;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float hin = 0.f;
      if (k > 0) hin = rr::tiles::take_value(mine - GCH + 64 * c, status);   // exit state of tile k - 1
      else if (h0 != nullptr && cok) hin = h0[(int64_t)b * D + ch + c];
      sIn[lane * CH + c] = hin;
      if (k + 1 < K) {
        float hout = hin;
#pragma unroll
        for (int j = 0; j < kNW; ++j) hout = sP[j][lane * CH + c] * hout + sE[j][lane * CH + c];
        rr::tiles::publish(mine + 64 * c, hout);
      }
    }
  }
  __syncthreads();
  float h[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    h[c] = sIn[lane * CH + c];
    for (int j = 0; j < w; ++j) h[c] = sP[j][lane * CH + c] * h[c] + sE[j][lane * CH + c];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = t0 + u;
#pragma unroll
    for (int c = 0; c < CH; ++c) h[c] = A(u, c) * h[c] + X(u, c);   // rglru.py:92
    if (cok && t < L) {
      rr::tiles::st_f32_at<CH>(y + rb, (uint32_t)(u * D + ch), h);
      if ((t + 1) % T == 0) rr::tiles::st_f32_at<CH>(ckpt + ((int64_t)b * nC + (t + 1) / T - 1) * D, (uint32_t)ch, h);
    }
  }
}

// Backward.  Plain: da, dx.  Gated: da receives dr, dx dx, dgi di, and dpart
// the tile's sums over its steps of dz * sigmoid(r) per channel (z = log a),
// row b * K + k of a [B * K, D] array that rglru_dlam_kernel reduces.
template <typename InT, int CH, int U, bool GATED>
__global__ __launch_bounds__(64 * kNW, 4) void rglru_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ dfinal, const InT* __restrict__ a,
    const InT* __restrict__ x, const InT* __restrict__ gi, const float* __restrict__ glam, float gc,
    const float* __restrict__ h0, const float* __restrict__ ckpt, InT* __restrict__ da, InT* __restrict__ dx,
    InT* __restrict__ dgi, float* __restrict__ dpart, float* __restrict__ dh0, uint32_t* counter,
    uint64_t* slots, uint32_t* status, int B, int L, int D, int T, int nC, int G, int K) {
  constexpr int GCH = 64 * CH, S = U * kNW;
  __shared__ float sP[kNW][GCH], sEf[kNW][GCH], sEb[kNW][GCH];
  __shared__ float sD[GATED ? kNW : 1][GCH];
  __shared__ float sIn[GCH];
  __shared__ float sC[GATED ? GCH : 1];
  __shared__ int sTicket;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // step tiles are taken from the end: the tile after (same channels, later
  // steps) always holds a smaller ticket
  const int nGrp = B * G;
  const int ticket = rr::tiles::take_ticket(counter, nGrp * K, &sTicket);
  if (ticket < 0) return;
  const rr::tiles::TileOfTicket tt = rr::tiles::tile_of_ticket(ticket, nGrp, K, true);
  const int k = tt.k, grp = tt.grp;
  const int b = grp / G, g = grp % G;
  const int ch = g * GCH + lane * CH;
  const bool cok = ch < D;
  const int t0 = k * S + w * U;
  const int64_t row0 = (int64_t)b * L;
  // the wave's first step row (clamped: a wave wholly past L touches nothing)
  const int64_t rb = (row0 + min(t0, L - 1)) * D;

  // every load first (clamped channel: every lane loads), then masks and
  // gates: dy, the inputs, lam, and the state entering the wave's checkpoint
  // interval (checkpoint row crow, or h0 at tb = 0, or zero: then any valid
  // row is read and dropped)
  const int chc = min(ch, D - CH);
  const float lv = GATED ? glam[min(g * GCH + 64 * (w % CH) + lane, D - 1)] : 0.f;
  Pack<float, CH> g2[U];
#pragma unroll
  for (int u = 0; u < U; ++u) g2[u] = rr::tiles::ld_pack_at<float, CH>(dy + rb, step_off(u, t0, L, D, chc));
  Pack<InT, CH> pa[U], px[U], pi[GATED ? U : 1];
  issue_steps<InT, CH, U, GATED>(a, x, gi, t0, L, rb, D, chc, pa, px, pi);
  const int tb = t0 - t0 % T;
  const int crow = rr::tiles::bwd_ckpt_row(t0, T, L);
  const bool from_h0 = crow < 0 && tb == 0 && h0 != nullptr;
  const bool huse = crow >= 0 || from_h0;
  const float* const hsrc = crow >= 0 ? ckpt + ((int64_t)b * nC + crow) * D : (from_h0 ? h0 + (int64_t)b * D : ckpt);
  float hin[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) hin[c] = hsrc[chc + c];
  float gy[U][CH];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    g2[u] = rr::tiles::pick<float, CH>(cok && t0 + u < L, g2[u], pack_fill<float, CH>(0.f));
#pragma unroll
    for (int c = 0; c < CH; ++c) gy[u][c] = g2[u][c];
  }
  float csp[CH];
  tile_csp<CH, GATED>(lv, gc, w, lane, cok, sC, csp);
  float av[GATED ? U : 1][CH], sv[GATED ? U : 1][CH], sr[GATED ? U : 1][CH];
  finish_steps<InT, CH, U, GATED>(csp, cok, t0, L, pa, px, pi, av, sv, sr);
  auto A = [&](int u, int c) -> float {
    if constexpr (GATED) return av[u][c];
    else return pa[u][c];
  };
  auto X = [&](int u, int c) -> float {
    if constexpr (GATED) return sv[u][c] * (pi[u][c] * px[u][c]);
    else return px[u][c];
  };
  // forward map (from a zero state) and adjoint map (from a zero adjoint)
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float P = 1.f, Ef = 0.f, Eb = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      Ef = A(u, c) * Ef + X(u, c);
      P *= A(u, c);
    }
#pragma unroll
    for (int u = U - 1; u >= 0; --u) Eb = A(u, c) * (Eb + gy[u][c]);
    sP[w][lane * CH + c] = P;
    sEf[w][lane * CH + c] = Ef;
    sEb[w][lane * CH + c] = Eb;
  }
  __syncthreads();
  if (w == 0) {
    uint64_t* mine = slots + ((int64_t)grp * K + k) * GCH + lane;   // slot layout as in the forward
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float lin = 0.f;   // adjoint entering the tile from later steps
      if (k + 1 < K) lin = rr::tiles::take_value(mine + GCH + 64 * c, status);
      else if (dfinal != nullptr && cok) lin = dfinal[(int64_t)b * D + ch + c];
      sIn[lane * CH + c] = lin;
      float lout = lin;
#pragma unroll
      for (int j = kNW - 1; j >= 0; --j) lout = sP[j][lane * CH + c] * lout + sEb[j][lane * CH + c];
      if (k > 0) rr::tiles::publish(mine + 64 * c, lout);
      else if (dh0 != nullptr && cok) dh0[(int64_t)b * D + ch + c] = lout;
    }
  }
  __syncthreads();
  // adjoint entering this wave's steps from the later waves of the tile
  float lam[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    lam[c] = sIn[lane * CH + c];
    for (int j = kNW - 1; j > w; --j) lam[c] = sP[j][lane * CH + c] * lam[c] + sEb[j][lane * CH + c];
  }
  // state entering this wave's steps: checkpoint at the start of the
  // checkpoint interval, then the earlier waves of the interval (the tile
  // holds whole intervals: S is a multiple of 32 >= T)
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    asm volatile("" : "+v"(hin[c]));
    hin[c] = huse && cok ? hin[c] : 0.f;
    for (int j = w - (t0 - tb) / U; j < w; ++j) hin[c] = sP[j][lane * CH + c] * hin[c] + sEf[j][lane * CH + c];
  }
  // recompute the states (hs[u] = h_{t0+u}), then sweep the adjoint backwards
  float hs[U][CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float h = hin[c];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      h = A(u, c) * h + X(u, c);
      hs[u][c] = h;
    }
  }
  float dsum[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) dsum[c] = 0.f;
#pragma unroll
  for (int u = U - 1; u >= 0; --u) {
    const int t = t0 + u;
    float gx[CH], ga[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      lam[c] += gy[u][c];
      gx[c] = lam[c];
      ga[c] = lam[c] * (u > 0 ? hs[u - 1][c] : hin[c]);
      lam[c] *= A(u, c);
    }
    const bool ok = cok && t < L;
    if constexpr (GATED) {
      // x' = s (i x), s = sqrt(1 - a^2): ds/da = -a / s; a = exp(z),
      // z = -c' sigmoid(r).  (At a = 1, s = 0, where the s branch has no
      // finite derivative, its term is dropped.)
      float gr[CH], gi2[CH], gxx[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const float sg = sr[u][c], iv = pi[u][c], xv = px[u][c], av_ = av[u][c], s = sv[u][c];
        const float ds = gx[c] * (iv * xv);
        float q = ds * av_ * __builtin_amdgcn_rcpf(s);
        asm volatile("" : "+v"(q));
        const float dz = (ga[c] - (s > 0.f ? q : 0.f)) * av_;
        gr[c] = dz * -csp[c] * (sg * (1.f - sg));
        gi2[c] = gx[c] * s * xv;
        gxx[c] = gx[c] * s * iv;
        if (ok) dsum[c] += dz * sg;
      }
      if (ok) {
        const uint32_t i = (uint32_t)(u * D + ch);
        rr::tiles::st_pack_at<InT, CH>(da + rb, i, gr);
        rr::tiles::st_pack_at<InT, CH>(dgi + rb, i, gi2);
        rr::tiles::st_pack_at<InT, CH>(dx + rb, i, gxx);
      }
    } else if (ok) {
      const uint32_t i = (uint32_t)(u * D + ch);
      rr::tiles::st_pack_at<InT, CH>(dx + rb, i, gx);
      rr::tiles::st_pack_at<InT, CH>(da + rb, i, ga);
    }
  }
  if constexpr (GATED) {   // the tile's dz * sigmoid(r) sums, waves added in order
#pragma unroll
    for (int c = 0; c < CH; ++c) sD[w][lane * CH + c] = dsum[c];
    __syncthreads();
    if (w == 0 && cok) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < kNW; ++j) t += sD[j][lane * CH + c];
        dpart[((int64_t)b * K + k) * D + ch + c] = t;
      }
    }
  }
}

// dlam[d] = -c sigmoid(lam[d]) * sum over rows of dpart[row, d] (d softplus /
// d lam = sigmoid), rows in a fixed order: wave w of a workgroup of 16 sums
// rows w, w + 16, ... of 64 channels with 8 loads in flight, then the waves'
// sums are added in order.
constexpr int kDlamWaves = 16;
__global__ __launch_bounds__(64 * kDlamWaves) void rglru_dlam_kernel(const float* __restrict__ dpart,
                                                                     const float* __restrict__ glam, float gc,
                                                                     float* __restrict__ dlam, int rows, int D) {
  __shared__ float red[kDlamWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int d = blockIdx.x * 64 + lane;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (d < D) {
    for (int j0 = w; j0 < rows; j0 += 8 * kDlamWaves) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int j = j0 + q * kDlamWaves;
        if (j < rows) acc[q] += dpart[(int64_t)j * D + d];
      }
    }
  }
  red[w][lane] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (w == 0 && d < D) {
    float t = 0.f;
    for (int j = 0; j < kDlamWaves; ++j) t += red[j][lane];
    dlam[d] = -gc * t * sigmoid_f(glam[d]);
  }
}

int check_common(int64_t B, int64_t L, int64_t D, int64_t seg, int dtype) {
  if (B <= 0 || L <= 0 || D <= 0) {
    return rr::fail(RR_EINVAL, "rglru: B, L and D must be positive");
  }
  if (int rc = rr::check_segment_shape(L, seg, D, "D")) return rc;
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, "rglru: unsupported dtype");
  if (B * L * D >= ((int64_t)1 << 40)) return rr::fail(RR_EUNSUPPORTED, "rglru: tensor too large");
  return RR_OK;
}

size_t ws_bytes_for(int64_t B, int64_t L, int64_t D, int dtype, int pass, bool gated = false) {
  const int ch = pass == 0 ? kFwdCh : kBwdCh;
  return rr::tiles::ws_bytes(B * tile_grid(L, D, ch, dtype, pass, gated).tiles(), 64 * ch);
}
// Gated backward: the hand-off words, then the [B * K, D] fp32 tile sums.
size_t gated_part_offset(int64_t B, int64_t L, int64_t D, int dtype) {
  return (ws_bytes_for(B, L, D, dtype, 1, true) + 255) / 256 * 256;
}
size_t gated_ws_bytes(int64_t B, int64_t L, int64_t D, int dtype, int pass) {
  if (pass == 0) return ws_bytes_for(B, L, D, dtype, 0, true);
  const int K = tile_grid(L, D, kBwdCh, dtype, 1, true).K;
  return gated_part_offset(B, L, D, dtype) + (size_t)(B * K * D) * 4;
}

}  // namespace

rr::tiles::Geometry rr::rglru_geometry(int64_t L, int64_t D, int dtype, int pass, bool gated) {
  const TileGrid tg = tile_grid(L, D, pass == 0 ? kFwdCh : kBwdCh, dtype, pass, gated);
  return rr::tiles::Geometry{tg.G, tg.K, steps_per_wave(dtype, pass, gated), kNW};
}

extern "C" size_t rr_rglru_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t seg, int dtype,
                                           int pass) {
  if (B <= 0 || L <= 0 || D <= 0 || rr::chunk_len(L, seg) == 0 || !rr::valid_dtype(dtype)) return 0;
  return ws_bytes_for(B, L, D, dtype, pass);
}

extern "C" int rr_rglru_fwd(const void* a, const void* x, int dtype, int64_t B, int64_t L,
                            int64_t D, int64_t seg, const float* h0, float* y, float* ckpt,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_common(B, L, D, seg, dtype)) return rc;
  if (!a || !x || !y || !ckpt) return rr::fail(RR_EINVAL, "rglru_fwd: null pointer argument");
  const size_t need = ws_bytes_for(B, L, D, dtype, 0);
  if (!workspace || workspace_bytes < need) return rr::fail(RR_EWORKSPACE, "rglru_fwd: workspace too small");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* status = rr::status_word();
  if (status == nullptr) return RR_EHIP;
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, {
    constexpr int U = steps_per_wave<InT, false, false>();
    const TileGrid tg = tile_grid(L, D, kFwdCh, dtype, 0);
    hipLaunchKernelGGL((rglru_fwd_kernel<InT, kFwdCh, U, false>), dim3((unsigned)(B * tg.tiles())), dim3(64 * kNW),
                       0, s, static_cast<const InT*>(a), static_cast<const InT*>(x), nullptr, nullptr, 0.f, h0, y,
                       ckpt, rr::tiles::ws_counter(workspace), rr::tiles::ws_slots(workspace), status, (int)B,
                       (int)L, (int)D, T, nC, tg.G, tg.K);
  });
  return rr::check_launch("rr_rglru_fwd");
}

extern "C" int rr_rglru_bwd(const float* dy, const float* dfinal, const void* a, const void* x,
                            int dtype, int64_t B, int64_t L, int64_t D, int64_t seg,
                            const float* h0, const float* ckpt, void* da, void* dx, float* dh0,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_common(B, L, D, seg, dtype)) return rc;
  if (!dy || !a || !x || !ckpt || !da || !dx) {
    return rr::fail(RR_EINVAL, "rglru_bwd: null pointer argument");
  }
  const size_t need = ws_bytes_for(B, L, D, dtype, 1);
  if (!workspace || workspace_bytes < need) return rr::fail(RR_EWORKSPACE, "rglru_bwd: workspace too small");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* status = rr::status_word();
  if (status == nullptr) return RR_EHIP;
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, {
    constexpr int U = steps_per_wave<InT, true, false>();
    const TileGrid tg = tile_grid(L, D, kBwdCh, dtype, 1);
    hipLaunchKernelGGL((rglru_bwd_kernel<InT, kBwdCh, U, false>), dim3((unsigned)(B * tg.tiles())), dim3(64 * kNW),
                       0, s, dy, dfinal, static_cast<const InT*>(a), static_cast<const InT*>(x), nullptr, nullptr,
                       0.f, h0, ckpt, static_cast<InT*>(da), static_cast<InT*>(dx), nullptr, nullptr, dh0,
                       rr::tiles::ws_counter(workspace), rr::tiles::ws_slots(workspace), status, (int)B, (int)L, (int)D,
                       T, nC, tg.G, tg.K);
  });
  return rr::check_launch("rr_rglru_bwd");
}

extern "C" size_t rr_rglru_gated_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t seg, int dtype,
                                                 int pass) {
  if (B <= 0 || L <= 0 || D <= 0 || rr::chunk_len(L, seg) == 0 || !rr::valid_dtype(dtype)) return 0;
  return gated_ws_bytes(B, L, D, dtype, pass);
}

extern "C" int rr_rglru_gated_fwd(const void* r, const void* i, const void* x, const float* lam, float c,
                                  int dtype, int64_t B, int64_t L, int64_t D, int64_t seg, const float* h0,
                                  float* y, float* ckpt, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  if (int rc = check_common(B, L, D, seg, dtype)) return rc;
  if (!r || !i || !x || !lam || !y || !ckpt) return rr::fail(RR_EINVAL, "rglru_gated_fwd: null pointer argument");
  if (!(c > 0.f) || !(c < INFINITY)) return rr::fail(RR_EINVAL, "rglru_gated_fwd: c must be positive and finite");
  const size_t need = gated_ws_bytes(B, L, D, dtype, 0);
  if (!workspace || workspace_bytes < need) return rr::fail(RR_EWORKSPACE, "rglru_gated_fwd: workspace too small");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* status = rr::status_word();
  if (status == nullptr) return RR_EHIP;
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, {
    constexpr int U = steps_per_wave<InT, false, true>();
    const TileGrid tg = tile_grid(L, D, kFwdCh, dtype, 0, true);
    hipLaunchKernelGGL((rglru_fwd_kernel<InT, kFwdCh, U, true>), dim3((unsigned)(B * tg.tiles())), dim3(64 * kNW), 0,
                       s, static_cast<const InT*>(r), static_cast<const InT*>(x), static_cast<const InT*>(i), lam,
                       c, h0, y, ckpt, rr::tiles::ws_counter(workspace), rr::tiles::ws_slots(workspace), status,
                       (int)B, (int)L, (int)D, T, nC, tg.G, tg.K);
  });
  return rr::check_launch("rr_rglru_gated_fwd");
}

extern "C" int rr_rglru_gated_bwd(const float* dy, const float* dfinal, const void* r, const void* i,
                                  const void* x, const float* lam, float c, int dtype, int64_t B, int64_t L,
                                  int64_t D, int64_t seg, const float* h0, const float* ckpt, void* dr, void* di,
                                  void* dx, float* dlam, float* dh0, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  if (int rc = check_common(B, L, D, seg, dtype)) return rc;
  if (!dy || !r || !i || !x || !lam || !ckpt || !dr || !di || !dx || !dlam) {
    return rr::fail(RR_EINVAL, "rglru_gated_bwd: null pointer argument");
  }
  if (!(c > 0.f) || !(c < INFINITY)) return rr::fail(RR_EINVAL, "rglru_gated_bwd: c must be positive and finite");
  const size_t need = gated_ws_bytes(B, L, D, dtype, 1);
  if (!workspace || workspace_bytes < need) return rr::fail(RR_EWORKSPACE, "rglru_gated_bwd: workspace too small");
  const int T = (int)rr::chunk_len(L, seg);
  const int nC = (int)(L / T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* status = rr::status_word();
  if (status == nullptr) return RR_EHIP;
  // only the hand-off words need clearing; every tile writes its row of sums
  if (int rc = rr::tiles::launch_clear(workspace, ws_bytes_for(B, L, D, dtype, 1, true), s)) return rc;
  float* dpart = reinterpret_cast<float*>(static_cast<char*>(workspace) + gated_part_offset(B, L, D, dtype));
  const TileGrid tg = tile_grid(L, D, kBwdCh, dtype, 1, true);
  RR_DISPATCH_DTYPE(dtype, {
    constexpr int U = steps_per_wave<InT, true, true>();
    hipLaunchKernelGGL((rglru_bwd_kernel<InT, kBwdCh, U, true>), dim3((unsigned)(B * tg.tiles())), dim3(64 * kNW), 0,
                       s, dy, dfinal, static_cast<const InT*>(r), static_cast<const InT*>(x),
                       static_cast<const InT*>(i), lam, c, h0, ckpt, static_cast<InT*>(dr), static_cast<InT*>(dx),
                       static_cast<InT*>(di), dpart, dh0, rr::tiles::ws_counter(workspace),
                       rr::tiles::ws_slots(workspace), status, (int)B, (int)L, (int)D, T, nC, tg.G, tg.K);
  });
  if (int rc = rr::check_launch("rr_rglru_gated_bwd")) return rc;
  hipLaunchKernelGGL(rglru_dlam_kernel, dim3((unsigned)((D + 63) / 64)), dim3(64 * kDlamWaves), 0, s, dpart, lam, c,
                     dlam, (int)(B * tg.K), (int)D);
  return rr::check_launch("rr_rglru_gated_bwd dlam");
}
