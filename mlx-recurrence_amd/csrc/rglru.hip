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

// Tile shapes (measured on MI355X at BASELINE config 3): CH = 2 channels per
// lane; U steps per wave: forward 16 for 16-bit inputs, otherwise 8 (the
// backward also holds dy and the recomputed states); NW = 8 waves, two
// workgroups per CU.
template <typename InT, bool BWD> constexpr int steps_per_wave() { return sizeof(InT) == 4 || BWD ? 8 : 16; }
constexpr int kNW = 8;
constexpr int kFwdCh = 2, kBwdCh = 2;

struct TileGrid {
  int G;   // channel tiles per batch row
  int K;   // step tiles
  int64_t tiles() const { return (int64_t)G * K; }
};
inline int steps_per_wave(int dtype, int pass) { return dtype == RR_F32 || pass == 1 ? 8 : 16; }
inline TileGrid tile_grid(int64_t L, int64_t D, int ch, int dtype, int pass) {
  const int64_t S = (int64_t)steps_per_wave(dtype, pass) * kNW;
  return TileGrid{(int)((D + 64 * ch - 1) / (64 * ch)), (int)((L + S - 1) / S)};
}

template <typename InT, int CH, int U>
__global__ __launch_bounds__(64 * kNW, 4) void rglru_fwd_kernel(
    const InT* __restrict__ a, const InT* __restrict__ x, const float* __restrict__ h0,
    float* __restrict__ y, float* __restrict__ ckpt, uint32_t* counter, uint64_t* slots, int B, int L,
    int D, int T, int nC, int G, int K) {
  constexpr int GCH = 64 * CH, S = U * kNW;
  __shared__ float sP[kNW][GCH], sE[kNW][GCH];
  __shared__ float sIn[GCH];
  __shared__ int sTicket;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // tickets run over step tiles slowest, so the tile before (same channels,
  // previous steps) always holds a smaller ticket
  const int nGrp = B * G;
  const int ticket = rr::tiles::take_ticket(counter, nGrp * K, &sTicket);
  if (ticket < 0) return;
  const int k = ticket / nGrp, grp = ticket % nGrp;
  const int b = grp / G, g = grp % G;
  const int ch = g * GCH + lane * CH;
  const bool cok = ch < D;
  const int t0 = k * S + w * U;
  const int64_t row0 = (int64_t)b * L;

  Pack<InT, CH> pa[U], px[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = t0 + u;
    if (cok && t < L) {
      const int64_t i = (row0 + t) * D + ch;
      pa[u] = ld_pack<InT, CH>(a, i);
      px[u] = ld_pack<InT, CH>(x, i);
    } else {   // identity step
      pa[u] = pack_fill<InT, CH>(1.f);
      px[u] = pack_fill<InT, CH>(0.f);
    }
  }
  float P[CH], E[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    P[c] = 1.f;
    E[c] = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      E[c] = pa[u][c] * E[c] + px[u][c];
      P[c] *= pa[u][c];
    }
    sP[w][lane * CH + c] = P[c];
    sE[w][lane * CH + c] = E[c];
  }
  __syncthreads();
  if (w == 0) {
    uint64_t* mine = slots + ((int64_t)grp * K + k) * GCH + lane * CH;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float hin = 0.f;
      if (k > 0) hin = rr::tiles::take_value(mine - GCH + c);   // exit state of tile k - 1
      else if (h0 != nullptr && cok) hin = h0[(int64_t)b * D + ch + c];
      sIn[lane * CH + c] = hin;
      if (k + 1 < K) {
        float hout = hin;
#pragma unroll
        for (int j = 0; j < kNW; ++j) hout = sP[j][lane * CH + c] * hout + sE[j][lane * CH + c];
        rr::tiles::publish(mine + c, hout);
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
    for (int c = 0; c < CH; ++c) h[c] = pa[u][c] * h[c] + px[u][c];   // rglru.py:92
    if (cok && t < L) {
      rr::tiles::st_f32<CH>(y, (row0 + t) * D + ch, h);
      if ((t + 1) % T == 0) rr::tiles::st_f32<CH>(ckpt, ((int64_t)b * nC + (t + 1) / T - 1) * D + ch, h);
    }
  }
}

template <typename InT, int CH, int U>
__global__ __launch_bounds__(64 * kNW, 4) void rglru_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ dfinal, const InT* __restrict__ a,
    const InT* __restrict__ x, const float* __restrict__ h0, const float* __restrict__ ckpt,
    InT* __restrict__ da, InT* __restrict__ dx, float* __restrict__ dh0, uint32_t* counter,
    uint64_t* slots, int B, int L, int D, int T, int nC, int G, int K) {
  constexpr int GCH = 64 * CH, S = U * kNW;
  __shared__ float sP[kNW][GCH], sEf[kNW][GCH], sEb[kNW][GCH];
  __shared__ float sIn[GCH];
  __shared__ int sTicket;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // step tiles are taken from the end: the tile after (same channels, later
  // steps) always holds a smaller ticket
  const int nGrp = B * G;
  const int ticket = rr::tiles::take_ticket(counter, nGrp * K, &sTicket);
  if (ticket < 0) return;
  const int k = K - 1 - ticket / nGrp, grp = ticket % nGrp;
  const int b = grp / G, g = grp % G;
  const int ch = g * GCH + lane * CH;
  const bool cok = ch < D;
  const int t0 = k * S + w * U;
  const int64_t row0 = (int64_t)b * L;

  Pack<InT, CH> pa[U], px[U];
  float gy[U][CH];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = t0 + u;
    if (cok && t < L) {
      const int64_t i = (row0 + t) * D + ch;
      pa[u] = ld_pack<InT, CH>(a, i);
      px[u] = ld_pack<InT, CH>(x, i);
      const Pack<float, CH> g2 = ld_pack<float, CH>(dy, i);
#pragma unroll
      for (int c = 0; c < CH; ++c) gy[u][c] = g2[c];
    } else {
      pa[u] = pack_fill<InT, CH>(1.f);
      px[u] = pack_fill<InT, CH>(0.f);
#pragma unroll
      for (int c = 0; c < CH; ++c) gy[u][c] = 0.f;
    }
  }
  // forward map (from a zero state) and adjoint map (from a zero adjoint)
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float P = 1.f, Ef = 0.f, Eb = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      Ef = pa[u][c] * Ef + px[u][c];
      P *= pa[u][c];
    }
#pragma unroll
    for (int u = U - 1; u >= 0; --u) Eb = pa[u][c] * (Eb + gy[u][c]);
    sP[w][lane * CH + c] = P;
    sEf[w][lane * CH + c] = Ef;
    sEb[w][lane * CH + c] = Eb;
  }
  __syncthreads();
  if (w == 0) {
    uint64_t* mine = slots + ((int64_t)grp * K + k) * GCH + lane * CH;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float lin = 0.f;   // adjoint entering the tile from later steps
      if (k + 1 < K) lin = rr::tiles::take_value(mine + GCH + c);
      else if (dfinal != nullptr && cok) lin = dfinal[(int64_t)b * D + ch + c];
      sIn[lane * CH + c] = lin;
      float lout = lin;
#pragma unroll
      for (int j = kNW - 1; j >= 0; --j) lout = sP[j][lane * CH + c] * lout + sEb[j][lane * CH + c];
      if (k > 0) rr::tiles::publish(mine + c, lout);
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
  const int tb = t0 - t0 % T;
  float hin[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    hin[c] = 0.f;
    if (cok) {
      if (tb > 0) hin[c] = ckpt[((int64_t)b * nC + tb / T - 1) * D + ch + c];
      else if (h0 != nullptr) hin[c] = h0[(int64_t)b * D + ch + c];
    }
    for (int j = w - (t0 - tb) / U; j < w; ++j) hin[c] = sP[j][lane * CH + c] * hin[c] + sEf[j][lane * CH + c];
  }
  // recompute the states (hs[u] = h_{t0+u}), then sweep the adjoint backwards
  float hs[U][CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float h = hin[c];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      h = pa[u][c] * h + px[u][c];
      hs[u][c] = h;
    }
  }
#pragma unroll
  for (int u = U - 1; u >= 0; --u) {
    const int t = t0 + u;
    float gx[CH], ga[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      lam[c] += gy[u][c];
      gx[c] = lam[c];
      ga[c] = lam[c] * (u > 0 ? hs[u - 1][c] : hin[c]);
      lam[c] *= pa[u][c];
    }
    if (cok && t < L) {
      const int64_t i = (row0 + t) * D + ch;
      rr::tiles::st_pack<InT, CH>(dx, i, gx);
      rr::tiles::st_pack<InT, CH>(da, i, ga);
    }
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

size_t ws_bytes_for(int64_t B, int64_t L, int64_t D, int dtype, int pass) {
  const int ch = pass == 0 ? kFwdCh : kBwdCh;
  return rr::tiles::ws_bytes(B * tile_grid(L, D, ch, dtype, pass).tiles(), 64 * ch);
}

}  // namespace

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
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, {
    constexpr int U = steps_per_wave<InT, false>();
    const TileGrid tg = tile_grid(L, D, kFwdCh, dtype, 0);
    hipLaunchKernelGGL((rglru_fwd_kernel<InT, kFwdCh, U>), dim3((unsigned)(B * tg.tiles())), dim3(64 * kNW), 0, s,
                       static_cast<const InT*>(a), static_cast<const InT*>(x), h0, y, ckpt,
                       rr::tiles::ws_counter(workspace), rr::tiles::ws_slots(workspace), (int)B, (int)L, (int)D,
                       T, nC, tg.G, tg.K);
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
  if (int rc = rr::tiles::launch_clear(workspace, need, s)) return rc;
  RR_DISPATCH_DTYPE(dtype, {
    constexpr int U = steps_per_wave<InT, true>();
    const TileGrid tg = tile_grid(L, D, kBwdCh, dtype, 1);
    hipLaunchKernelGGL((rglru_bwd_kernel<InT, kBwdCh, U>), dim3((unsigned)(B * tg.tiles())), dim3(64 * kNW), 0, s,
                       dy, dfinal, static_cast<const InT*>(a), static_cast<const InT*>(x), h0, ckpt,
                       static_cast<InT*>(da), static_cast<InT*>(dx), dh0, rr::tiles::ws_counter(workspace),
                       rr::tiles::ws_slots(workspace), (int)B, (int)L, (int)D, T, nC, tg.G, tg.K);
  });
  return rr::check_launch("rr_rglru_bwd");
}
