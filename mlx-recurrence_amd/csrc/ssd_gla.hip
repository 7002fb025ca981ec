// ssd_gla.hip — SSD and GLA scans on gfx950 (chunk-parallel VALU engine).
//
// Both recurrences are instances of one "diagonal decay, rank-1 input, linear
// readout" scan over a state h[d, n] per (batch, head):
//
//     h_t[d, n] = dec_t[n] * h_{t-1}[d, n] + inB_t[n] * u_t[d]
//     y_t[d]    = sum_n outC_t[n] * h_t[d, n]
//
//   SSD (reference ssd.py:85-111):  d = channel (Dh), n = state (N),
//       dec = exp(delta_t A[n]), inB = delta_t B_t[n], outC = C_t[n], u = u_t.
//   GLA (reference gla.py:78-100):  d = j (value index), n = i (key index),
//       dec = g_t, inB = k_t[i], outC = q_t[i], u = v_t[j].
//
// Its adjoint (reference ssd.py:203-268, gla.py:184-236), with lam[d, n]:
//     lam += gy_t[d] outC_t[n]
//     gu_t[d]   = sum_n lam inB_t[n]           (SSD du, GLA dv)
//     Gin_t[n]  = sum_d lam u_t[d]             (SSD dB / delta, GLA dk)
//     Gout_t[n] = sum_d h_t gy_t[d]            (SSD dC, GLA dq)
//     Hp_t[n]   = sum_d lam h_{t-1}            (SSD d(delta), dA; GLA dgates)
//     lam *= dec_t[n]
//
// Work decomposition.  A workgroup owns a 16(d) x 16(n) tile of one head's
// state for the whole sequence; lane = 16*ng + dl holds d = 16*dt + dl and the
// four states n = 16*nt + 4*ng + k (a row of 16 lanes is one n-group, so sums
// over d stay within a row: DPP, no LDS traffic).  Its NW waves take NW consecutive chunks of
// T steps at once (chunk-parallel scan): each wave stages its chunk's per-step
// coefficients (dec, inB, outC; one exp per (t, n) instead of one per lane)
// in LDS, folds the chunk into the affine map h -> P*h + E, the maps are
// exchanged through LDS, and each wave replays its chunk from the composed
// entering state.  The backward pass recomputes each chunk from the forward
// checkpoint (history kept in registers) and runs the same scheme in reverse
// time for the adjoint.  Sums over n of a tile and over d of a tile are done
// with cross-lane shuffles; sums across tiles go through fp32 partial buffers
// in the caller's workspace and a finalize kernel that also applies the
// recurrence-specific epilogue (dB = delta*Gin, d(delta), dA, dgates).
#include "rr_common.h"
#include "rr_internal.h"
#include "rr_mfma.h"

#include <atomic>
#include <type_traits>
#include <string>

namespace {

constexpr int kMaxT = 32;
constexpr int kTile = 16;
constexpr int kChunkWaves = 4;    // chunks per workgroup of the chunk-parallel kernels
constexpr int kFinRows = 32;  // (b, t) rows per finalize workgroup

// Sum over the 4 rows (the 4 n-groups of one d: lanes l, l ^ 16, l ^ 32,
// l ^ 48) with gfx950's row-swapping permutes (VALU, no LDS traffic); every
// lane of the group gets the same value.
__device__ __forceinline__ float ngroup_sum(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto h = __builtin_amdgcn_permlane32_swap(u, u, false, false);   // lanes l % 32, l % 32 + 32
  v = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const uint32_t x = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);   // rows 2k, 2k + 1
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Sums over the 16 lanes of a row (the 16 d of a tile) of N values at once,
// butterfly level by level across the values (independent DPP adds back to
// back, none waiting on the one before); every lane of the row gets the sum.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int N>
__device__ __forceinline__ void dsum16(float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_add<0xB1>(v[i]);    // quad_perm [1, 0, 3, 2]
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_add<0x4E>(v[i]);    // quad_perm [2, 3, 0, 1]
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_add<0x141>(v[i]);   // row_half_mirror
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_add<0x140>(v[i]);   // row_mirror
}

template <typename InT>
struct Args {
  // SSD: lane_in=u, step=delta, in_coef=B, out_coef=C, A=A_neg.
  // GLA: lane_in=v, step=gates, in_coef=k, out_coef=q, A=null.
  const InT* lane_in;
  const InT* step;
  const InT* in_coef;
  const InT* out_coef;
  const float* A;
  int64_t a_sh, a_sn;   // A[h * a_sh + n * a_sn]
  const float* h0;      // initial state (nullable)
  const float* dy;      // bwd: upstream gradient of y
  const float* dfinal;  // bwd: cotangent of the final state (nullable)
  float* y;             // fwd output, or its per-n-tile partials
  float* ckpt;          // [B,H,nC,DL,NS]
  InT* gu;              // bwd: du / dv when NN == 1
  float* gu_part;       // bwd: per-n-tile partials of gu when NN > 1
  float* g3;            // bwd: [3][ND][B*L*H][NS] partial Gin, Gout, Hp
  float* dh0;           // bwd: gradient of the initial state (nullable)
  float* lamws;         // bwd: adjoint flowing into each chunk [B,H,nC,DL,NS] (workspace)
  float* mapE;          // chunk maps x -> P x + E (workspace): E [B,H,nC,DL,NS]
  float* mapP;          //   P [B,H,nC,NS]
  int L, H, DL, NS, T, nC, ND, NN;
  int Bsz;              // batch rows
  int64_t rows;         // B*L*H
};

// State layout of h0 / dfinal / dh0 within one (b, head): SSD [Dh, N] (d-major),
// GLA [i, j] = [n, d] (n-major).
template <bool GLA>
__device__ __forceinline__ int64_t state_idx(int d, int n, int DL, int NS) {
  return GLA ? (int64_t)n * DL + d : (int64_t)d * NS + n;
}

// Every staging load below is issued first, at a clamped in-bounds index, and
// masked afterwards: loads under a branch would each wait out a full memory
// latency in turn.
constexpr int kStageIt = kMaxT * kTile / 64;   // (step, column) pairs per lane

// The chunk's per-step coefficients of state columns nt*16 .. nt*16 + 15:
// lane holds column nn = lane % 16 of steps lane / 16 + 4 j.
template <typename InT, bool GLA>
__device__ __forceinline__ void stage_chunk(const Args<InT>& p, float4 (*coef)[kMaxT][4],
                                            int b, int h, int c, bool act, int nt, int lane) {
  const int nn = lane & 15, n = nt * kTile + nn;
  const bool nok = n < p.NS;
  const int nc = min(n, p.NS - 1), cc = act ? c : 0;
  const float an = GLA ? 0.f : p.A[(int64_t)h * p.a_sh + (int64_t)nc * p.a_sn];
  float sv[kStageIt], bv[kStageIt], cv[kStageIt];
#pragma unroll
  for (int j = 0; j < kStageIt; ++j) {
    const int t = (lane >> 4) + 4 * j, tc = min(t, p.T - 1);
    const int64_t row = ((int64_t)b * p.L + (int64_t)cc * p.T + tc) * p.H + h;
    sv[j] = rr::ld(p.step, row);
    bv[j] = rr::ld(p.in_coef, row * p.NS + nc);
    cv[j] = rr::ld(p.out_coef, row * p.NS + nc);
  }
#pragma unroll
  for (int j = 0; j < kStageIt; ++j) {
    const int t = (lane >> 4) + 4 * j;
    const bool ok = act && t < p.T && nok;
    const float dec = GLA ? sv[j] : expf(sv[j] * an);
    const float inb = GLA ? bv[j] : sv[j] * bv[j];
    reinterpret_cast<float*>(&coef[0][t][0])[nn] = ok ? dec : 1.f;
    reinterpret_cast<float*>(&coef[1][t][0])[nn] = ok ? inb : 0.f;
    reinterpret_cast<float*>(&coef[2][t][0])[nn] = ok ? cv[j] : 0.f;
  }
}

__device__ __forceinline__ void unpack(float4 v, float (&a)[4]) {
  a[0] = v.x;
  a[1] = v.y;
  a[2] = v.z;
  a[3] = v.w;
}

// FULL: the chunk is kMaxT steps (the checkpoint interval of the default
// seg = 32), so the per-step loops carry no run-time bound and the compiler
// can issue each step's LDS reads ahead of the steps before it.

// Workgroup of a chunk-parallel kernel (fold, replay): a 1-D grid over the
// units u = (b * H + h) * groups + g (chunk group g: NW chunks) times the
// ND * NN state tiles, decoded so that every tile of a unit runs on the same
// XCD (the GPU hands workgroups to its 8 XCDs round-robin by linear index):
// the tiles of a unit read the same step inputs, B and C rows, which one L2
// then holds once.
struct TileUnit {
  int tile, grp, h, b;
  bool valid;   // false for the padding workgroups of the last unit group
};
template <int NW, typename InT>
__device__ __forceinline__ TileUnit tile_unit(const Args<InT>& p) {
  const int id = blockIdx.x, x = id % 8, rest = id / 8, tiles = p.ND * p.NN;
  const int groups = (p.nC + NW - 1) / NW;
  const int u = (rest / tiles) * 8 + x, bh = u / groups;
  return TileUnit{rest % tiles, u % groups, bh % p.H, bh / p.H, (int64_t)bh < (int64_t)p.Bsz * p.H};
}
inline int64_t tile_grid(int64_t B, int64_t H, int64_t groups, int64_t tiles) {
  return (B * H * groups + 7) / 8 * 8 * tiles;
}

// Each pass runs in three kernels:
//   r1_fold_kernel (every chunk at once, NW chunks per workgroup): each wave
//     folds its chunk into the affine map x -> P x + E of the state (forward,
//     from the coefficients and u) or of the adjoint (backward, from the
//     coefficients and dy, walking the steps backwards), P per state column,
//     E per state element, into the workspace;
//   r1_compose_kernel (one wave per state tile of a (head, batch row)): walks
//     the maps in order, writing the state after each chunk to the checkpoints
//     (forward) or the adjoint flowing into each chunk from the later ones to
//     `lamws` (backward; the last one is dh0): the only serial part of the
//     scan, and a cheap one (a multiply-add per state element per chunk);
//   r1_out_kernel / r1_bwd_kernel (every chunk at once): each wave replays its
//     chunk from its entering state (checkpoint c - 1, h0 or zero) and writes
//     y, or recomputes its states and walks the adjoint back from lamws,
//     writing the per-step partial sums.
template <typename InT, bool GLA, int NW, bool BWD>
__global__ __launch_bounds__(64 * NW) void r1_fold_kernel(Args<InT> p) {
  constexpr bool FULL = false;   // (a run-time bound keeps the read-ahead, and the registers, in check)
  __shared__ float4 sCoef[NW][3][kMaxT][4];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ng = lane >> 4, dl = lane & 15;
  const TileUnit tu = tile_unit<NW>(p);
  if (!tu.valid) return;
  const int tile = tu.tile, grp = tu.grp, h = tu.h, b = tu.b;
  const int dt = tile / p.NN, nt = tile % p.NN;
  const int d = dt * kTile + dl;
  const bool dok = d < p.DL;
  const int nb = nt * kTile + ng * 4;
  const int64_t bh = (int64_t)b * p.H + h;
  const int c = grp * NW + w;
  const bool act = c < p.nC;
  stage_chunk<InT, GLA>(p, sCoef[w], b, h, c, act, nt, lane);
  float xv[kMaxT];   // forward: u_t[d]; backward: dy_t[d]
  {
    const int cc = act ? c : 0, dc = min(d, p.DL - 1);
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      const int64_t i = (((int64_t)b * p.L + (int64_t)cc * p.T + min(t, p.T - 1)) * p.H + h) * p.DL + dc;
      xv[t] = BWD ? p.dy[i] : rr::ld(p.lane_in, i);
    }
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) xv[t] = t < p.T && act && dok ? xv[t] : 0.f;
  }
  __syncthreads();
  float e[4] = {0.f, 0.f, 0.f, 0.f}, P[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (BWD) {
#pragma unroll
    for (int t = kMaxT - 1; t >= 0; --t) {
      if (FULL || t < p.T) {
        float dec[4], outc[4];
        unpack(sCoef[w][0][t][ng], dec);
        unpack(sCoef[w][2][t][ng], outc);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          e[k] = (e[k] + xv[t] * outc[k]) * dec[k];
          P[k] *= dec[k];
        }
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      if (FULL || t < p.T) {
        float dec[4], inb[4];
        unpack(sCoef[w][0][t][ng], dec);
        unpack(sCoef[w][1][t][ng], inb);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          e[k] = dec[k] * e[k] + inb[k] * xv[t];
          P[k] *= dec[k];
        }
      }
    }
  }
  if (act && dok) {
    float* em = p.mapE + ((bh * p.nC + c) * p.DL + d) * p.NS;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (nb + k < p.NS) em[nb + k] = e[k];
  }
  if (act && dl == 0) {
    float* pm = p.mapP + (bh * p.nC + c) * p.NS;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (nb + k < p.NS) pm[nb + k] = P[k];
  }
}

// One wave per (tile, head, batch row): x_c = P_c x_{c-1} + E_c over the chunks
// (forward from h0, in order; backward from dfinal, in reverse), maps loaded
// kCompPF chunks ahead.
constexpr int kCompPF = 8;
template <bool GLA, bool BWD>
__global__ __launch_bounds__(64) void r1_compose_kernel(const float* __restrict__ mapE, const float* __restrict__ mapP,
                                                        const float* __restrict__ x0, float* __restrict__ out,
                                                        float* __restrict__ xlast, int H, int DL, int NS, int nC,
                                                        int NN) {
  const int lane = threadIdx.x, ng = lane >> 4, dl = lane & 15;
  const int dt = blockIdx.x / NN, nt = blockIdx.x % NN;
  const int h = blockIdx.y, b = blockIdx.z;
  const int d = dt * kTile + dl, dc = min(d, DL - 1);
  const bool dok = d < DL;
  const int nb = nt * kTile + ng * 4;
  const int64_t bh = (int64_t)b * H + h;
  int ncl[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) ncl[k] = min(nb + k, NS - 1);
  float x[4] = {0.f, 0.f, 0.f, 0.f};
  if (x0 != nullptr) {
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = x0[bh * DL * NS + state_idx<GLA>(dc, ncl[k], DL, NS)];
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = dok && nb + k < NS ? x[k] : 0.f;
  }
  for (int i0 = 0; i0 < nC; i0 += kCompPF) {
    float ev[kCompPF][4], pv[kCompPF][4];
#pragma unroll
    for (int q = 0; q < kCompPF; ++q) {
      const int i = min(i0 + q, nC - 1), c = BWD ? nC - 1 - i : i;
      const float* em = mapE + ((bh * nC + c) * DL + dc) * NS;
      const float* pm = mapP + (bh * nC + c) * NS;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        ev[q][k] = em[ncl[k]];
        pv[q][k] = pm[ncl[k]];
      }
    }
#pragma unroll
    for (int q = 0; q < kCompPF; ++q) {
      const int i = i0 + q, c = BWD ? nC - 1 - i : i;
      if (i < nC) {
        // backward: the adjoint flowing into chunk c, before its own map
        if (BWD && dok) {
          float* o = out + ((bh * nC + c) * DL + d) * NS;
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (nb + k < NS) o[nb + k] = x[k];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = pv[q][k] * x[k] + ev[q][k];
        // forward: the state after chunk c
        if (!BWD && dok) {
          float* o = out + ((bh * nC + c) * DL + d) * NS;
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (nb + k < NS) o[nb + k] = x[k];
        }
      }
    }
  }
  if (xlast != nullptr && dok) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (nb + k < NS) xlast[bh * DL * NS + state_idx<GLA>(d, nb + k, DL, NS)] = x[k];
  }
}


// Short heads (nC <= kDirectMaxChunks): the replay kernels compose the chunk
// maps themselves instead of reading the compose kernel's output.  The
// workgroup loads the maps of chunks j0 .. j0 + cnt - 1 of its tile into LDS
// (wave w takes maps w, w + NW, ...; every load issued first, at a clamped
// chunk), and each wave then walks the ones it needs from LDS.
constexpr int kDirectMaxChunks = 16;
struct MapSmem {
  float4 E[kDirectMaxChunks][64];   // E of the tile, this lane's four states
  float4 P[kDirectMaxChunks][4];    // P of the tile's 16 columns, by n-group
};
template <bool DIRECT>
struct MaybeMaps {
  MapSmem m;
};
template <>
struct MaybeMaps<false> {};
template <int NW, typename InT>
__device__ __forceinline__ void load_maps(const Args<InT>& p, MapSmem& sm, int64_t bh, int d, int nb, int lane, int w,
                                          int j0, int cnt) {
  const int ng = lane >> 4, dl = lane & 15, dc = min(d, p.DL - 1);
  constexpr int PER = kDirectMaxChunks / NW;
  float ev[PER][4], pv[PER][4];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int j = min(j0 + w + NW * i, p.nC - 1);
    const float* em = p.mapE + ((bh * p.nC + j) * p.DL + dc) * p.NS;
    const float* pm = p.mapP + (bh * p.nC + j) * p.NS;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int ncl = min(nb + k, p.NS - 1);
      ev[i][k] = em[ncl];
      pv[i][k] = pm[ncl];
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int jj = w + NW * i;
    if (jj < cnt) {
      sm.E[jj][lane] = make_float4(ev[i][0], ev[i][1], ev[i][2], ev[i][3]);
      if (dl == 0) sm.P[jj][ng] = make_float4(pv[i][0], pv[i][1], pv[i][2], pv[i][3]);
    }
  }
}

template <typename InT, bool GLA, int NW, bool FULL, bool DIRECT>
__global__ __launch_bounds__(64 * NW) void r1_out_kernel(Args<InT> p) {
  __shared__ float4 sCoef[NW][3][kMaxT][4];
  __shared__ MaybeMaps<DIRECT> sMap;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ng = lane >> 4, dl = lane & 15;
  const TileUnit tu = tile_unit<NW>(p);
  if (!tu.valid) return;
  const int tile = tu.tile, grp = tu.grp, h = tu.h, b = tu.b;
  const int dt = tile / p.NN, nt = tile % p.NN;
  const int d = dt * kTile + dl;
  const bool dok = d < p.DL;
  const int nb = nt * kTile + ng * 4;
  const int64_t bh = (int64_t)b * p.H + h;
  const int c = grp * NW + w;
  const bool act = c < p.nC;
  stage_chunk<InT, GLA>(p, sCoef[w], b, h, c, act, nt, lane);
  float uv[kMaxT], hs[4];
  {
    const int cc = act ? c : 0, dc = min(d, p.DL - 1);
#pragma unroll
    for (int t = 0; t < kMaxT; ++t)
      uv[t] = rr::ld(p.lane_in, (((int64_t)b * p.L + (int64_t)cc * p.T + min(t, p.T - 1)) * p.H + h) * p.DL + dc);
    // the entering state: checkpoint slot c - 1, else h0, else zero (DIRECT:
    // h0 or zero here, the maps of chunks 0 .. c - 1 applied below)
    const bool from_ck = !DIRECT && cc > 0, has = from_ck || p.h0 != nullptr;
    const float* hsrc = from_ck ? p.ckpt : has ? p.h0 : p.ckpt;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int ncl = min(nb + k, p.NS - 1);
      const int64_t i = from_ck ? ((bh * p.nC + (cc - 1)) * p.DL + dc) * p.NS + ncl
                        : has   ? bh * p.DL * p.NS + state_idx<GLA>(dc, ncl, p.DL, p.NS)
                                : 0;
      hs[k] = hsrc[i];
    }
    if constexpr (DIRECT) load_maps<NW>(p, sMap.m, bh, d, nb, lane, w, 0, min(grp * NW + NW - 1, p.nC - 1));
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) uv[t] = t < p.T && act && dok ? uv[t] : 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) hs[k] = act && dok && has && nb + k < p.NS ? hs[k] : 0.f;
  }
  __syncthreads();
  if constexpr (DIRECT) {
    // x <- P_j x + E_j over the chunks before this one
    for (int j = 0; j < (act ? c : 0); ++j) {
      float pj[4], ej[4];
      unpack(sMap.m.P[j][ng], pj);
      unpack(sMap.m.E[j][lane], ej);
#pragma unroll
      for (int k = 0; k < 4; ++k) hs[k] = pj[k] * hs[k] + ej[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) hs[k] = act && dok && nb + k < p.NS ? hs[k] : 0.f;
  }
  float* yout = p.y + (p.NN > 1 ? (int64_t)nt * p.rows * p.DL : 0);
  // this lane's y of step 0 of the chunk; step t is t * H * DL further
  float* const ylane = yout + (((int64_t)b * p.L + (int64_t)(act ? c : 0) * p.T) * p.H + h) * p.DL + d;
  const int64_t ystep = (int64_t)p.H * p.DL;
#pragma unroll
  for (int t = 0; t < kMaxT; ++t) {
    if (FULL || t < p.T) {
      float dec[4], inb[4], outc[4];
      unpack(sCoef[w][0][t][ng], dec);
      unpack(sCoef[w][1][t][ng], inb);
      unpack(sCoef[w][2][t][ng], outc);
      float yp = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        hs[k] = dec[k] * hs[k] + inb[k] * uv[t];
        yp += outc[k] * hs[k];
      }
      yp = ngroup_sum(yp);
      if (act && dok && ng == (t & 3)) ylane[t * ystep] = yp;
    }
  }
  if (DIRECT && act && dok) {   // the state after the chunk: its checkpoint
    float* ck = p.ckpt + ((bh * p.nC + c) * p.DL + d) * p.NS;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (nb + k < p.NS) ck[nb + k] = hs[k];
  }
}

// g[i] for i < 12 (a select tree over the bits of i; i >= 12: any of them).
__device__ __forceinline__ float pick12(const float (&g)[12], int i) {
  const bool b0 = i & 1, b1 = i & 2, b2 = i & 4, b3 = i & 8;
  const float a0 = b0 ? g[1] : g[0], a1 = b0 ? g[3] : g[2], a2 = b0 ? g[5] : g[4];
  const float a3 = b0 ? g[7] : g[6], a4 = b0 ? g[9] : g[8], a5 = b0 ? g[11] : g[10];
  const float c0 = b1 ? a1 : a0, c1 = b1 ? a3 : a2, c2 = b1 ? a5 : a4;
  return b3 ? c2 : b2 ? c1 : c0;
}

// PART: the grid has several n-tiles (NN > 1) and du / dv goes to per-tile
// fp32 partials, else straight to gu.
// LDS of the backward replay: u_t[d] and dy_t[d] of each wave's chunk, and
// (DIRECT) the chunk maps, which are dead before u and dy are staged.
template <int NW, bool DIRECT>
struct BwdLds {
  struct UG {
    float U[NW][kMaxT][kTile];
    float G[NW][kMaxT][kTile];
  };
  union {
    UG x;
    MapSmem m;
  };
};
template <int NW>
struct BwdLds<NW, false> {
  struct UG {
    float U[NW][kMaxT][kTile];
    float G[NW][kMaxT][kTile];
  } x;
};

template <typename InT, bool GLA, int NW, bool PART, bool FULL, bool DIRECT>
__global__ __launch_bounds__(64 * NW) void r1_bwd_kernel(Args<InT> p) {
  __shared__ float4 sCoef[NW][3][kMaxT][4];
  __shared__ BwdLds<NW, DIRECT> sx;
  auto& sU = sx.x.U;
  auto& sG = sx.x.G;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ng = lane >> 4, dl = lane & 15;
  const TileUnit tu = tile_unit<NW>(p);
  if (!tu.valid) return;
  const int tile = tu.tile, grp = tu.grp, h = tu.h, b = tu.b;
  const int dt = tile / p.NN, nt = tile % p.NN;
  const int d = dt * kTile + dl;
  const bool dok = d < p.DL;
  const int nb = nt * kTile + ng * 4;
  const int64_t bh = (int64_t)b * p.H + h;
  const int64_t sbase = bh * p.DL * p.NS;
  float* gin_p = p.g3 + (int64_t)dt * p.rows * p.NS;   // then Gout, Hp, ND * rows * NS apart

  {
    const int c = grp * NW + w;
    const bool act = c < p.nC;
    stage_chunk<InT, GLA>(p, sCoef[w], b, h, c, act, nt, lane);
    float hst[4], lam[4];
    // u and dy of columns dt*16 + lane % 16, steps lane / 16 + 4 j
    const int dd = dt * kTile + (lane & 15);
    float uvv[kStageIt], gyv[kStageIt];
    auto stage_ug = [&]() {
#pragma unroll
      for (int j = 0; j < kStageIt; ++j) {
        const int t = (lane >> 4) + 4 * j;
        const bool ok = act && t < p.T && dd < p.DL;
        sU[w][t][lane & 15] = ok ? uvv[j] : 0.f;
        sG[w][t][lane & 15] = ok ? gyv[j] : 0.f;
      }
    };
    {
      const int cc = act ? c : 0, ddc = min(dd, p.DL - 1);
#pragma unroll
      for (int j = 0; j < kStageIt; ++j) {
        const int t = (lane >> 4) + 4 * j;
        const int64_t i = (((int64_t)b * p.L + (int64_t)cc * p.T + min(t, p.T - 1)) * p.H + h) * p.DL + ddc;
        uvv[j] = rr::ld(p.lane_in, i);
        gyv[j] = p.dy[i];
      }
      // the entering state: checkpoint slot c - 1, else h0, else zero (an
      // inactive wave, c >= nC, reads chunk 0's and drops it)
      const bool from_ck = cc > 0, has = from_ck || p.h0 != nullptr;
      const float* hsrc = from_ck ? p.ckpt : has ? p.h0 : p.ckpt;
      const int dc = min(d, p.DL - 1);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int ncl = min(nb + k, p.NS - 1);
        const int64_t i = from_ck ? ((bh * p.nC + (cc - 1)) * p.DL + dc) * p.NS + ncl
                          : has   ? sbase + state_idx<GLA>(dc, ncl, p.DL, p.NS)
                                  : 0;
        hst[k] = hsrc[i];
      }
      if constexpr (!DIRECT) stage_ug();
#pragma unroll
      for (int k = 0; k < 4; ++k) hst[k] = act && dok && has && nb + k < p.NS ? hst[k] : 0.f;
      // the adjoint flowing into the chunk from the later ones (r1_compose_kernel;
      // DIRECT: dfinal, the maps of chunks nC - 1 .. c + 1 applied below)
      if constexpr (DIRECT) {
        const float* fsrc = p.dfinal != nullptr ? p.dfinal : p.ckpt;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          lam[k] = fsrc[p.dfinal != nullptr ? sbase + state_idx<GLA>(dc, min(nb + k, p.NS - 1), p.DL, p.NS) : 0];
#pragma unroll
        for (int k = 0; k < 4; ++k) lam[k] = act && dok && p.dfinal != nullptr && nb + k < p.NS ? lam[k] : 0.f;
        // maps grp * NW + 1 .. nC - 1
        load_maps<NW>(p, sx.m, bh, d, nb, lane, w, grp * NW + 1, p.nC - 1 - grp * NW);
      } else {
        const float* lsrc = p.lamws + ((bh * p.nC + cc) * p.DL + dc) * p.NS;
#pragma unroll
        for (int k = 0; k < 4; ++k) lam[k] = lsrc[min(nb + k, p.NS - 1)];
#pragma unroll
        for (int k = 0; k < 4; ++k) lam[k] = act && dok && nb + k < p.NS ? lam[k] : 0.f;
      }
    }
    __syncthreads();
    if constexpr (DIRECT) {
      // lam <- P_j lam + E_j over the later chunks, last first
      for (int j = p.nC - 1; j > (act ? c : p.nC - 1); --j) {
        const int jj = j - (grp * NW + 1);
        float pj[4], ej[4];
        unpack(sx.m.P[jj][ng], pj);
        unpack(sx.m.E[jj][lane], ej);
#pragma unroll
        for (int k = 0; k < 4; ++k) lam[k] = pj[k] * lam[k] + ej[k];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) lam[k] = act && dok && nb + k < p.NS ? lam[k] : 0.f;
      __syncthreads();   // every wave has read the maps: u and dy take their place
      stage_ug();        // (a wave reads back only its own rows: no barrier after)
    }
    // The chunk's states are recomputed from its checkpoint in two halves of
    // 16 steps (16 x 4 registers at a time): here the state after step 15,
    // below each half again from its entering state as the adjoint walks it.
    constexpr int kHalf = kMaxT / 2;
    float hmid[4] = {hst[0], hst[1], hst[2], hst[3]};
#pragma unroll
    for (int t = 0; t < kHalf; ++t) {
      if (FULL || t < p.T) {
        float dec[4], inb[4];
        unpack(sCoef[w][0][t][ng], dec);
        unpack(sCoef[w][1][t][ng], inb);
        const float uvt = sU[w][t][dl];
#pragma unroll
        for (int k = 0; k < 4; ++k) hmid[k] = dec[k] * hmid[k] + inb[k] * uvt;
      }
    }
    // Steps t0 .. t0 + 15 of the adjoint, backwards, beside their states
    // recomputed from hbeg (the state entering step t0).  Per step, lane
    // dl < 12 of each row stores quantity dl / 4 (Gin, Gout, Hp) of state
    // nb + dl % 4, and the row ng == t % 4 stores du / dv of its 16 columns:
    // per-lane bases here, a uniform row offset per step.
    const int64_t crow = ((int64_t)b * p.L + (int64_t)(act ? c : 0) * p.T) * p.H + h;   // step 0's row
    float* const gq = gin_p + (int64_t)(dl >> 2) * p.ND * p.rows * p.NS + nb + (dl & 3);
    const bool gq_ok = act && dl < 12 && nb + (dl & 3) < p.NS;
    float* const gu_f = PART ? p.gu_part + (int64_t)nt * p.rows * p.DL + d : nullptr;
    InT* const gu_t = PART ? nullptr : p.gu + d;
    auto adjoint_half = [&](auto half, const float (&hbeg)[4]) {
      constexpr int t0 = decltype(half)::value;
      float hs[kHalf][4];
      {
        float hc[4] = {hbeg[0], hbeg[1], hbeg[2], hbeg[3]};
#pragma unroll
        for (int i = 0; i < kHalf; ++i) {
          const int t = t0 + i;
          if (FULL || t < p.T) {
            float dec[4], inb[4];
            unpack(sCoef[w][0][t][ng], dec);
            unpack(sCoef[w][1][t][ng], inb);
            const float uvt = sU[w][t][dl];
#pragma unroll
            for (int k = 0; k < 4; ++k) hc[k] = dec[k] * hc[k] + inb[k] * uvt;
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) hs[i][k] = hc[k];
        }
      }
#pragma unroll
      for (int i = kHalf - 1; i >= 0; --i) {
        const int t = t0 + i;
        if (FULL || t < p.T) {
          float dec[4], inb[4], outc[4];
          unpack(sCoef[w][0][t][ng], dec);
          unpack(sCoef[w][1][t][ng], inb);
          unpack(sCoef[w][2][t][ng], outc);
          const float uvt = sU[w][t][dl], gyt = sG[w][t][dl];
          float gup = 0.f, g12[12];   // Gin, Gout, Hp of the four states, summed over d
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            lam[k] += gyt * outc[k];
            gup += lam[k] * inb[k];
            g12[k] = lam[k] * uvt;
            g12[4 + k] = hs[i][k] * gyt;
            const float hprev = i > 0 ? hs[i - 1][k] : hbeg[k];
            g12[8 + k] = lam[k] * hprev;
            lam[k] *= dec[k];
          }
          dsum16(g12);
          gup = ngroup_sum(gup);
          const int64_t row = crow + (int64_t)t * p.H;
#pragma unroll
          for (int i = 0; i < 12; ++i) asm volatile("" : "+v"(g12[i]));   // formed here, selected below
          const float gv = pick12(g12, dl);
          if (gq_ok) gq[row * p.NS] = gv;
          if (act && dok && ng == (t & 3)) {
            if constexpr (PART) gu_f[row * p.DL] = gup;
            else rr::st(gu_t, row * p.DL, gup);
          }
        }
      }
    };
    adjoint_half(std::integral_constant<int, kHalf>{}, hmid);
    adjoint_half(std::integral_constant<int, 0>{}, hst);
    // DIRECT: chunk 0's wave ends with the adjoint of the initial state
    if (DIRECT && c == 0 && p.dh0 != nullptr && dok) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (nb + k < p.NS) p.dh0[sbase + state_idx<GLA>(d, nb + k, p.DL, p.NS)] = lam[k];
    }
  }
}

// y = sum over n-tiles of the forward partials.
__global__ void sum_tiles_kernel(const float* __restrict__ part, float* __restrict__ out,
                                 int64_t n, int tiles) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int j = 0; j < tiles; ++j) s += part[(int64_t)j * n + i];
  out[i] = s;
}

template <typename InT>
struct FinArgs {
  const float* g3;       // [3][ND][rows][NS]
  const float* gu_part;  // [NN][rows][DL] (NN > 1)
  const InT* step;       // delta / gates
  const InT* in_coef;    // B (SSD)
  const float* A;        // SSD
  int64_t a_sh, a_sn;
  InT* g_in;             // SSD dB  / GLA dk
  InT* g_out;            // SSD dC  / GLA dq
  InT* g_step;           // SSD d(delta) / GLA dgates
  InT* gu;               // du / dv (when NN > 1)
  float* gA_part;        // SSD: [H][nblk][NS]
  int64_t BL;            // B*L
  int H, DL, NS, ND, NN;
};

// Sum over the P lanes of a group (P = 16: a row, 32: two rows, 64: the
// wave); every lane of the group gets the sum.
template <int P>
__device__ __forceinline__ float group_sum(float v) {
  v = rr::row16_sum(v);
  if constexpr (P == 32) {
    const uint32_t x = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);   // rows 2k, 2k + 1
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (P == 64) {
    v = ngroup_sum(v);
  }
  return v;
}

// One workgroup = one head h and kFinRows consecutive (b, t) rows.  A group of
// P lanes takes one row (lanes over n, then over d for the du sum), so a wave
// takes 64 / P rows at a time: P = 16 for NS <= 16, 32 for NS <= 32, else 64
// (n strided by 64).
template <typename InT, bool GLA, int P>
__global__ __launch_bounds__(256) void r1_finalize_kernel(FinArgs<InT> p) {
  constexpr int G = 64 / P;   // rows per wave at a time
  __shared__ float sA[4][G][P == 64 ? 256 : P];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane / P, ln = lane % P;
  const int h = blockIdx.y;
  const int64_t rows = p.BL * p.H;
  const int64_t plane = (int64_t)p.ND * rows * p.NS;
  constexpr int QA = P == 64 ? 4 : 1;   // SSD dA partials of n = ln + P q
  float gacc[QA];
#pragma unroll
  for (int q = 0; q < QA; ++q) gacc[q] = 0.f;
  for (int r = w * G + sub; r < kFinRows; r += 4 * G) {
    const int64_t bt = (int64_t)blockIdx.x * kFinRows + r;
    if (bt >= p.BL) break;   // (uniform within the group; the groups after it stop too)
    const int64_t row = bt * p.H + h;
    const float sv = rr::ld(p.step, row);
    float acc = 0.f;
    for (int q = 0; q * P < p.NS; ++q) {
      const int n = q * P + ln;
      if (n < p.NS) {
        float gin = 0.f, gout = 0.f, hp = 0.f;
        for (int j = 0; j < p.ND; ++j) {
          const int64_t i = ((int64_t)j * rows + row) * p.NS + n;
          gin += p.g3[i];
          gout += p.g3[plane + i];
          hp += p.g3[2 * plane + i];
        }
        if (GLA) {
          rr::st(p.g_in, row * p.NS + n, gin);
          rr::st(p.g_out, row * p.NS + n, gout);
          acc += hp;
        } else {
          const float a = p.A[(int64_t)h * p.a_sh + (int64_t)n * p.a_sn];
          const float dec = expf(sv * a);
          rr::st(p.g_in, row * p.NS + n, sv * gin);
          rr::st(p.g_out, row * p.NS + n, gout);
          acc += a * dec * hp + rr::ld(p.in_coef, row * p.NS + n) * gin;
          if (q < QA) gacc[q] += sv * dec * hp;
        }
      }
    }
    acc = group_sum<P>(acc);
    if (ln == 0) rr::st(p.g_step, row, acc);
    if (p.NN > 1) {
      for (int d = ln; d < p.DL; d += P) {
        float s = 0.f;
        for (int j = 0; j < p.NN; ++j) s += p.gu_part[((int64_t)j * rows + row) * p.DL + d];
        rr::st(p.gu, row * p.DL + d, s);
      }
    }
  }
  if (!GLA) {
#pragma unroll
    for (int q = 0; q < QA; ++q) sA[w][sub][q * P + ln] = gacc[q];
    __syncthreads();
    for (int n = threadIdx.x; n < p.NS; n += 256) {
      float s = 0.f;
#pragma unroll
      for (int ww = 0; ww < 4; ++ww)
#pragma unroll
        for (int g = 0; g < G; ++g) s += sA[ww][g][n];
      p.gA_part[((int64_t)h * gridDim.x + blockIdx.x) * p.NS + n] = s;
    }
  }
}

// dA_neg[h, n] = the sum of part[h][j][n] over the nblk blocks j; per head
// (dA_sn == 0) dA_neg[h] = the sum over j and n.  One wave per output: lane l
// sums terms l, l + 64, ... in order, then a fixed butterfly sums the lanes
// (deterministic; every load of a lane is independent, so they overlap).
__global__ __launch_bounds__(256) void sum_gA_kernel(const float* __restrict__ part, float* __restrict__ dA, int H,
                                                     int NS, int nblk, int dA_sn) {
  const int o = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (o >= (dA_sn != 0 ? H * NS : H)) return;   // whole waves
  const int h = dA_sn != 0 ? o / NS : o, n0 = dA_sn != 0 ? o % NS : 0, nn = dA_sn != 0 ? 1 : NS;
  const int64_t terms = (int64_t)nn * nblk;
  const float* ph = part + (int64_t)h * nblk * NS;
  float s = 0.f;
#pragma unroll 4
  for (int64_t q = lane; q < terms; q += 64) s += ph[(q % nblk) * NS + n0 + q / nblk];
  s = rr::wave_sum(s);
  if (lane == 0) dA[o] = s;
}

// ------------------------------------------------------------------ host
struct Plan {
  int64_t T, nC, ND, NN, rows, nblk, groups;
  size_t off_y, off_g3, off_gu, off_gA, off_lam, fwd_bytes, bwd_bytes;
  size_t fwd_mapE, fwd_mapP, bwd_mapE, bwd_mapP;   // chunk maps of each pass
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

Plan make_plan(int64_t B, int64_t L, int64_t H, int64_t DL, int64_t NS, int64_t seg) {
  Plan q{};
  q.T = rr::chunk_len(L, seg);
  q.nC = q.T ? L / q.T : 0;
  q.ND = (DL + kTile - 1) / kTile;
  q.NN = (NS + kTile - 1) / kTile;
  q.rows = B * L * H;
  q.nblk = (B * L + kFinRows - 1) / kFinRows;
  q.groups = (q.nC + kChunkWaves - 1) / kChunkWaves;
  const size_t f = sizeof(float);
  const size_t mapE = align256(B * H * q.nC * DL * NS * f), mapP = align256(B * H * q.nC * NS * f);
  q.off_y = 0;
  q.fwd_bytes = q.NN > 1 ? align256(q.NN * q.rows * DL * f) : 0;
  q.fwd_mapE = q.fwd_bytes;
  q.fwd_mapP = q.fwd_mapE + mapE;
  q.fwd_bytes = q.fwd_mapP + mapP;
  q.off_g3 = 0;
  size_t o = align256(3 * q.ND * q.rows * NS * f);
  q.off_gu = o;
  o += q.NN > 1 ? align256(q.NN * q.rows * DL * f) : 0;
  q.off_gA = o;
  o += align256(H * q.nblk * NS * f);
  q.off_lam = o;
  o += align256(B * H * q.nC * DL * NS * f);
  q.bwd_mapE = o;
  o += mapE;
  q.bwd_mapP = o;
  o += mapP;
  q.bwd_bytes = o;
  return q;
}

int check_dims(const char* who, int64_t B, int64_t L, int64_t H, int64_t DL, int64_t NS,
               int64_t seg, int dtype, const char* lane_name) {
  if (B <= 0 || L <= 0 || H <= 0 || DL <= 0 || NS <= 0)
    return rr::fail(RR_EINVAL, std::string(who) + ": all dimensions must be positive");
  if (int rc = rr::check_segment_shape(L, seg, DL, lane_name)) return rc;
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, std::string(who) + ": unsupported dtype");
  if (B > 65535 || H > 65535)
    return rr::fail(RR_EUNSUPPORTED, std::string(who) + ": B and H must be <= 65535");
  if (B * L > ((int64_t)1 << 31) / kFinRows * kFinRows)
    return rr::fail(RR_EUNSUPPORTED, std::string(who) + ": B*L too large");
  return RR_OK;
}

template <typename InT, bool GLA>
int launch_fwd(Args<InT> a, const Plan& q, int64_t B, void* ws, hipStream_t s, float* y) {
  if (tile_grid(B, a.H, q.groups, q.ND * q.NN) >= ((int64_t)1 << 31))
    return rr::fail(RR_EUNSUPPORTED, "scan: too many (tile, chunk group) workgroups");
  const dim3 grid((unsigned)(q.ND * q.NN), (unsigned)a.H, (unsigned)B);
  const dim3 cgrid((unsigned)tile_grid(B, a.H, q.groups, q.ND * q.NN)), cblk(64 * kChunkWaves);
  a.mapE = reinterpret_cast<float*>(static_cast<char*>(ws) + q.fwd_mapE);
  a.mapP = reinterpret_cast<float*>(static_cast<char*>(ws) + q.fwd_mapP);
  hipLaunchKernelGGL((r1_fold_kernel<InT, GLA, kChunkWaves, false>), cgrid, cblk, 0, s, a);
  if (int rc = rr::check_launch("scan forward chunk maps")) return rc;
  if (q.T == kMaxT && q.nC <= kDirectMaxChunks) {   // short heads: the maps composed in the replay kernel
    hipLaunchKernelGGL((r1_out_kernel<InT, GLA, kChunkWaves, true, true>), cgrid, cblk, 0, s, a);
  } else {
    hipLaunchKernelGGL((r1_compose_kernel<GLA, false>), grid, dim3(64), 0, s, a.mapE, a.mapP, a.h0, a.ckpt, nullptr,
                       a.H, a.DL, a.NS, a.nC, a.NN);
    if (int rc = rr::check_launch("scan forward states")) return rc;
    if (q.T == kMaxT) hipLaunchKernelGGL((r1_out_kernel<InT, GLA, kChunkWaves, true, false>), cgrid, cblk, 0, s, a);
    else hipLaunchKernelGGL((r1_out_kernel<InT, GLA, kChunkWaves, false, false>), cgrid, cblk, 0, s, a);
  }
  if (int rc = rr::check_launch("scan forward outputs")) return rc;
  if (q.NN > 1) {
    const int64_t n = q.rows * a.DL;
    hipLaunchKernelGGL(sum_tiles_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       static_cast<const float*>(ws), y, n, (int)q.NN);
    if (int rc = rr::check_launch("scan forward tile sum")) return rc;
  }
  return RR_OK;
}

template <typename InT, bool GLA>
int launch_bwd(Args<InT> a, FinArgs<InT> f, const Plan& q, int64_t B, hipStream_t s,
               float* dA, int dA_sn) {
  if (tile_grid(B, a.H, q.groups, q.ND * q.NN) >= ((int64_t)1 << 31))
    return rr::fail(RR_EUNSUPPORTED, "scan: too many (tile, chunk group) workgroups");
  const dim3 grid((unsigned)(q.ND * q.NN), (unsigned)a.H, (unsigned)B);
  const dim3 cgrid((unsigned)tile_grid(B, a.H, q.groups, q.ND * q.NN)), cblk(64 * kChunkWaves);
  hipLaunchKernelGGL((r1_fold_kernel<InT, GLA, kChunkWaves, true>), cgrid, cblk, 0, s, a);
  if (int rc = rr::check_launch("scan backward chunk maps")) return rc;
  if (q.T == kMaxT && q.nC <= kDirectMaxChunks) {   // short heads: the maps composed in the replay kernel
    if (q.NN > 1) hipLaunchKernelGGL((r1_bwd_kernel<InT, GLA, kChunkWaves, true, true, true>), cgrid, cblk, 0, s, a);
    else hipLaunchKernelGGL((r1_bwd_kernel<InT, GLA, kChunkWaves, false, true, true>), cgrid, cblk, 0, s, a);
  } else {
    hipLaunchKernelGGL((r1_compose_kernel<GLA, true>), grid, dim3(64), 0, s, a.mapE, a.mapP, a.dfinal, a.lamws,
                       a.dh0, a.H, a.DL, a.NS, a.nC, a.NN);
    if (int rc = rr::check_launch("scan backward adjoints")) return rc;
    if (q.T == kMaxT) {
      if (q.NN > 1) hipLaunchKernelGGL((r1_bwd_kernel<InT, GLA, kChunkWaves, true, true, false>), cgrid, cblk, 0, s, a);
      else hipLaunchKernelGGL((r1_bwd_kernel<InT, GLA, kChunkWaves, false, true, false>), cgrid, cblk, 0, s, a);
    } else {
      if (q.NN > 1) hipLaunchKernelGGL((r1_bwd_kernel<InT, GLA, kChunkWaves, true, false, false>), cgrid, cblk, 0, s, a);
      else hipLaunchKernelGGL((r1_bwd_kernel<InT, GLA, kChunkWaves, false, false, false>), cgrid, cblk, 0, s, a);
    }
  }
  if (int rc = rr::check_launch("scan backward")) return rc;
  const dim3 fgrid((unsigned)q.nblk, (unsigned)a.H);
  if (a.NS <= 16)
    hipLaunchKernelGGL((r1_finalize_kernel<InT, GLA, 16>), fgrid, dim3(256), 0, s, f);
  else if (a.NS <= 32)
    hipLaunchKernelGGL((r1_finalize_kernel<InT, GLA, 32>), fgrid, dim3(256), 0, s, f);
  else
    hipLaunchKernelGGL((r1_finalize_kernel<InT, GLA, 64>), fgrid, dim3(256), 0, s, f);
  if (int rc = rr::check_launch("scan backward finalize")) return rc;
  if (!GLA) {
    const int n = dA_sn != 0 ? (int)(a.H * a.NS) : a.H;
    hipLaunchKernelGGL(sum_gA_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s,
                       f.gA_part, dA, a.H, a.NS, (int)q.nblk, dA_sn);
    if (int rc = rr::check_launch("scan backward dA")) return rc;
  }
  return RR_OK;
}

// SSD through the per-chunk kernels of ssd_dense.hip (a rate per (head, n), or
// fp32 / fp16 inputs, at T = 32): chunk maps, the walk over chunks, then every
// chunk's outputs or gradients at once.
rr::DenseArgs dense_args(const void* u, const void* delta, const void* Bm, const void* Cm, const float* A_neg,
                         int64_t A_stride_n, int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N, int64_t nC) {
  rr::DenseArgs d{};
  d.u = u;
  d.delta = delta;
  d.Bm = Bm;
  d.Cm = Cm;
  d.A = A_neg;
  d.a_sh = A_stride_n ? N : 1;
  d.a_sn = A_stride_n;
  d.B = (int)B; d.L = (int)L; d.H = (int)H; d.DH = (int)Dh; d.NS = (int)N; d.nC = (int)nC;
  return d;
}

int dense_fwd(rr::DenseArgs d, int dtype, const Plan& q, char* ws, float* ckpt, hipStream_t s) {
  d.mapE = reinterpret_cast<float*>(ws + q.fwd_mapE);
  d.mapP = reinterpret_cast<float*>(ws + q.fwd_mapP);
  d.ckpt = ckpt;
  if (int rc = rr::ssd_dense_launch(d, dtype, rr::kDenseMapsFwd, s)) return rc;
  if (int rc = rr::dense_compose(d.mapE, d.mapP, d.h0, ckpt, nullptr, d.B, d.H, d.DH, d.NS, d.nC, false, false, s))
    return rc;
  return rr::ssd_dense_launch(d, dtype, rr::kDenseOut, s);
}

int dense_bwd(rr::DenseArgs d, int dtype, const Plan& q, char* ws, const float* dfinal, float* dh0, float* dA,
              int dA_sn, hipStream_t s) {
  d.mapE = reinterpret_cast<float*>(ws + q.bwd_mapE);
  d.mapP = reinterpret_cast<float*>(ws + q.bwd_mapP);
  float* lam = reinterpret_cast<float*>(ws + q.off_lam);
  d.lamws = lam;
  d.gA_part = reinterpret_cast<float*>(ws + q.off_gA);   // H * (B * nC) * N floats: nblk == B * nC at T = 32
  if (int rc = rr::ssd_dense_launch(d, dtype, rr::kDenseMapsBwd, s)) return rc;
  if (int rc = rr::dense_compose(d.mapE, d.mapP, dfinal, lam, dh0, d.B, d.H, d.DH, d.NS, d.nC, true, false, s))
    return rc;
  if (int rc = rr::ssd_dense_launch(d, dtype, rr::kDenseGrad, s)) return rc;
  const int n = dA_sn != 0 ? d.H * d.NS : d.H;
  hipLaunchKernelGGL(sum_gA_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, d.gA_part, dA, d.H, d.NS,
                     d.B * d.nC, dA_sn);
  return rr::check_launch("ssd dense backward dA");
}

}  // namespace

// ====================================================================== SSD
extern "C" size_t rr_ssd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N,
                                         int64_t seg, int64_t A_stride_n, int dtype, int pass) {
  if (B <= 0 || L <= 0 || H <= 0 || Dh <= 0 || N <= 0 || rr::chunk_len(L, seg) == 0) return 0;
  if (rr::ssd2_supported(dtype, L, seg, Dh, N, A_stride_n) && (pass == 0 || rr::ssd2_bwd_supported(Dh, N)))
    return rr::ssd2_ws_bytes(B, H, L / 32, rr::chunked_mode(B, H, L / 32, Dh, N, pass), Dh, N, pass);
  const Plan q = make_plan(B, L, H, Dh, N, seg);
  return pass == 0 ? q.fwd_bytes : q.bwd_bytes;
}

extern "C" int64_t rr_ssd_workspace_extent(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N, int64_t seg,
                                           int64_t A_stride_n, int dtype, int pass) {
  if (B <= 0 || L <= 0 || H <= 0 || Dh <= 0 || N <= 0 || rr::chunk_len(L, seg) == 0 || (pass != 0 && pass != 1)) {
    rr::fail(RR_EINVAL, "rr_ssd_workspace_extent: invalid arguments");
    return -1;
  }
  if (!rr::ssd2_supported(dtype, L, seg, Dh, N, A_stride_n) || (pass == 1 && !rr::ssd2_bwd_supported(Dh, N))) return -1;
  const int64_t nC = L / 32;
  return rr::ssd2_ws_extent(B, H, nC, rr::chunked_mode(B, H, nC, Dh, N, pass), Dh, N, pass);
}

extern "C" int rr_ssd_fwd(const void* u, const void* delta, const void* Bm, const void* Cm,
                          const float* A_neg, int64_t A_stride_n, int dtype, int64_t B, int64_t L, int64_t H,
                          int64_t Dh, int64_t N, int64_t seg, const float* h0, float* y,
                          float* ckpt, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_dims("ssd_fwd", B, L, H, Dh, N, seg, dtype, "Dh")) return rc;
  if (N > 256) return rr::fail(RR_EUNSUPPORTED, "ssd_fwd: N > 256 is not supported");
  if (!u || !delta || !Bm || !Cm || !A_neg || !y || !ckpt)
    return rr::fail(RR_EINVAL, "ssd_fwd: null pointer argument");
  if (A_stride_n != 0 && A_stride_n != 1)
    return rr::fail(RR_EINVAL, "ssd_fwd: A_stride_n must be 0 or 1");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (rr::ssd2_supported(dtype, L, seg, Dh, N, A_stride_n)) {
    rr::ChunkArgs a{};
    a.u = static_cast<const uint16_t*>(u);
    a.delta = static_cast<const uint16_t*>(delta);
    a.Bm = static_cast<const uint16_t*>(Bm);
    a.Cm = static_cast<const uint16_t*>(Cm);
    a.A = A_neg;
    a.A_stride_h = 1;
    a.h0 = h0;
    a.y = y;
    a.ckpt = ckpt;
    a.B = (int)B; a.L = (int)L; a.H = (int)H; a.DH = (int)Dh; a.NS = (int)N; a.nC = (int)(L / 32);
    a.mode = rr::chunked_mode(B, H, a.nC, Dh, N, 0);
    a.R = a.mode == 0 ? a.nC : 1;
    const size_t need = rr::ssd2_ws_bytes(B, H, a.nC, a.mode, Dh, N, 0);
    if (need && (!workspace || workspace_bytes < need))
      return rr::fail(RR_EWORKSPACE, "ssd_fwd: workspace too small");
    rr::ssd2_carve_ws(a, workspace, B, 0);
    return rr::ssd2_fwd(a, B, s);
  }
  const Plan q = make_plan(B, L, H, Dh, N, seg);
  if (workspace_bytes < q.fwd_bytes || (q.fwd_bytes && !workspace))
    return rr::fail(RR_EWORKSPACE, "ssd_fwd: workspace too small");
  if (rr::ssd_dense_supported(q.T, Dh, N, B, H, q.nC)) {
    rr::DenseArgs d = dense_args(u, delta, Bm, Cm, A_neg, A_stride_n, B, L, H, Dh, N, q.nC);
    d.h0 = h0;
    d.y = y;
    return dense_fwd(d, dtype, q, static_cast<char*>(workspace), ckpt, s);
  }
  RR_DISPATCH_DTYPE(dtype, {
    Args<InT> a{};
    a.lane_in = static_cast<const InT*>(u);
    a.step = static_cast<const InT*>(delta);
    a.in_coef = static_cast<const InT*>(Bm);
    a.out_coef = static_cast<const InT*>(Cm);
    a.A = A_neg;
    a.a_sh = A_stride_n ? N : 1;
    a.a_sn = A_stride_n;
    a.h0 = h0;
    a.y = q.NN > 1 ? static_cast<float*>(workspace) : y;
    a.ckpt = ckpt;
    a.L = (int)L; a.H = (int)H; a.DL = (int)Dh; a.NS = (int)N; a.T = (int)q.T;
    a.Bsz = (int)B;
    a.nC = (int)q.nC; a.ND = (int)q.ND; a.NN = (int)q.NN; a.rows = q.rows;
    return launch_fwd<InT, false>(a, q, B, workspace, s, y);
  });
  return RR_OK;
}

extern "C" int rr_ssd_bwd(const float* dy, const float* dfinal, const void* u, const void* delta,
                          const void* Bm, const void* Cm, const float* A_neg, int64_t A_stride_n,
                          int dtype,
                          int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N, int64_t seg,
                          const float* h0, const float* ckpt, void* du, void* ddelta, void* dB,
                          void* dC, float* dA_neg, int64_t dA_stride_n, float* dh0, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (int rc = check_dims("ssd_bwd", B, L, H, Dh, N, seg, dtype, "Dh")) return rc;
  if (N > 256) return rr::fail(RR_EUNSUPPORTED, "ssd_bwd: N > 256 is not supported");
  if (!dy || !u || !delta || !Bm || !Cm || !A_neg || !ckpt || !du || !ddelta || !dB || !dC ||
      !dA_neg)
    return rr::fail(RR_EINVAL, "ssd_bwd: null pointer argument");
  if (A_stride_n != 0 && A_stride_n != 1)
    return rr::fail(RR_EINVAL, "ssd_bwd: A_stride_n must be 0 or 1");
  if (dA_stride_n != 0 && dA_stride_n != 1)
    return rr::fail(RR_EINVAL, "ssd_bwd: dA_stride_n must be 0 or 1");
  if (rr::ssd2_supported(dtype, L, seg, Dh, N, A_stride_n) && rr::ssd2_bwd_supported(Dh, N)) {
    const int nC = (int)(L / 32);
    const int mode = rr::chunked_mode(B, H, nC, Dh, N, 1);
    if (!workspace || workspace_bytes < rr::ssd2_ws_bytes(B, H, nC, mode, Dh, N, 1))
      return rr::fail(RR_EWORKSPACE, "ssd_bwd: workspace too small");
    rr::ChunkArgs a{};
    a.u = static_cast<const uint16_t*>(u);
    a.delta = static_cast<const uint16_t*>(delta);
    a.Bm = static_cast<const uint16_t*>(Bm);
    a.Cm = static_cast<const uint16_t*>(Cm);
    a.A = A_neg;
    a.A_stride_h = 1;
    a.h0 = h0;
    a.ckpt = const_cast<float*>(ckpt);
    a.dy = dy;
    a.dfinal = dfinal;
    a.du = static_cast<uint16_t*>(du);
    a.ddelta = static_cast<uint16_t*>(ddelta);
    a.dB = static_cast<uint16_t*>(dB);
    a.dC = static_cast<uint16_t*>(dC);
    a.dA = dA_neg;
    a.dA_sn = (int)dA_stride_n;
    a.dh0 = dh0;
    a.B = (int)B; a.L = (int)L; a.H = (int)H; a.DH = (int)Dh; a.NS = (int)N; a.nC = nC;
    a.mode = mode;
    a.R = rr::chunked_run(mode, nC);
    rr::ssd2_carve_ws(a, workspace, B, 1);
    return rr::ssd2_bwd(a, B, static_cast<hipStream_t>(stream));
  }
  const Plan q = make_plan(B, L, H, Dh, N, seg);
  if (workspace_bytes < q.bwd_bytes || !workspace)
    return rr::fail(RR_EWORKSPACE, "ssd_bwd: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (rr::ssd_dense_supported(q.T, Dh, N, B, H, q.nC)) {
    rr::DenseArgs d = dense_args(u, delta, Bm, Cm, A_neg, A_stride_n, B, L, H, Dh, N, q.nC);
    d.h0 = h0;
    d.ckpt = ckpt;
    d.dy = dy;
    d.du = du;
    d.ddelta = ddelta;
    d.dB = dB;
    d.dC = dC;
    return dense_bwd(d, dtype, q, ws, dfinal, dh0, dA_neg, (int)dA_stride_n, s);
  }
  RR_DISPATCH_DTYPE(dtype, {
    Args<InT> a{};
    a.lane_in = static_cast<const InT*>(u);
    a.step = static_cast<const InT*>(delta);
    a.in_coef = static_cast<const InT*>(Bm);
    a.out_coef = static_cast<const InT*>(Cm);
    a.A = A_neg;
    a.a_sh = A_stride_n ? N : 1;
    a.a_sn = A_stride_n;
    a.h0 = h0;
    a.dy = dy;
    a.dfinal = dfinal;
    a.ckpt = const_cast<float*>(ckpt);
    a.gu = static_cast<InT*>(du);
    a.gu_part = reinterpret_cast<float*>(ws + q.off_gu);
    a.g3 = reinterpret_cast<float*>(ws + q.off_g3);
    a.lamws = reinterpret_cast<float*>(ws + q.off_lam);
    a.mapE = reinterpret_cast<float*>(ws + q.bwd_mapE);
    a.mapP = reinterpret_cast<float*>(ws + q.bwd_mapP);
    a.dh0 = dh0;
    a.L = (int)L; a.H = (int)H; a.DL = (int)Dh; a.NS = (int)N; a.T = (int)q.T;
    a.Bsz = (int)B;
    a.nC = (int)q.nC; a.ND = (int)q.ND; a.NN = (int)q.NN; a.rows = q.rows;
    FinArgs<InT> f{};
    f.g3 = a.g3;
    f.gu_part = a.gu_part;
    f.step = a.step;
    f.in_coef = a.in_coef;
    f.A = A_neg;
    f.a_sh = A_stride_n ? N : 1;
    f.a_sn = A_stride_n;
    f.g_in = static_cast<InT*>(dB);
    f.g_out = static_cast<InT*>(dC);
    f.g_step = static_cast<InT*>(ddelta);
    f.gu = static_cast<InT*>(du);
    f.gA_part = reinterpret_cast<float*>(ws + q.off_gA);
    f.BL = B * L; f.H = (int)H; f.DL = (int)Dh; f.NS = (int)N; f.ND = (int)q.ND; f.NN = (int)q.NN;
    return launch_bwd<InT, false>(a, f, q, B, s, dA_neg, (int)dA_stride_n);
  });
  return RR_OK;
}

// ============================================== SSD backward, no allocation
// rr_ssd_bwd for callers that cannot allocate device memory: the workspace is
// `scratch`, a static device array of this library (one copy per device, held
// until the process ends), whose address is looked up once per device.  The
// SSD backward kernels write every workspace word before they read it (their
// results do not depend on its prior contents), so nothing is cleared between
// calls; calls that overlap on one device share the array and race.
namespace {
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;   // 16 MiB
constexpr int kNoAllocMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::atomic<void*> g_scratch_ptr[kNoAllocMaxDevices];

// Device address of `scratch` on the current device (nullptr with the error set).
void* scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) {
    rr::fail(RR_EHIP, "ssd_bwd_noalloc: no current HIP device");
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || addr == nullptr) {
      rr::fail(RR_EHIP, std::string("ssd_bwd_noalloc: hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev].store(addr, std::memory_order_release);
    p = addr;
  }
  return p;
}
}  // namespace

extern "C" int rr_ssd_bwd_noalloc(const float* dy, const float* dfinal, const void* u, const void* delta,
                                  const void* Bm, const void* Cm, const float* A_neg, int64_t A_stride_n,
                                  int dtype, int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N,
                                  int64_t seg, const float* h0, const float* ckpt, void* du, void* ddelta,
                                  void* dB, void* dC, float* dA_neg, int64_t dA_stride_n, float* dh0,
                                  void* stream) {
  if (int rc = check_dims("ssd_bwd_noalloc", B, L, H, Dh, N, seg, dtype, "Dh")) return rc;
  if (A_stride_n != 0 && A_stride_n != 1)
    return rr::fail(RR_EINVAL, "ssd_bwd_noalloc: A_stride_n must be 0 or 1");
  const size_t need = rr_ssd_workspace_bytes(B, L, H, Dh, N, seg, A_stride_n, dtype, 1);
  if (need > kNoAllocScratchBytes)
    return rr::fail(RR_EUNSUPPORTED, "ssd_bwd_noalloc: this call needs " + std::to_string(need) +
                                         " bytes of workspace, more than the library's " +
                                         std::to_string(kNoAllocScratchBytes) +
                                         "-byte device scratch; use rr_ssd_bwd with a caller workspace");
  void* ws = scratch_ptr();
  if (ws == nullptr) return RR_EHIP;
  return rr_ssd_bwd(dy, dfinal, u, delta, Bm, Cm, A_neg, A_stride_n, dtype, B, L, H, Dh, N, seg, h0, ckpt, du,
                    ddelta, dB, dC, dA_neg, dA_stride_n, dh0, ws, kNoAllocScratchBytes, stream);
}

// ====================================================================== GLA
namespace {
// Chunked-kernel arguments of a GLA call (u = v, delta = gates, Bm = k, Cm = q).
rr::ChunkArgs gla2_args(const void* qp, const void* kp, const void* vp, const void* gates, int64_t B,
                        int64_t L, int64_t H, int64_t Dh, const float* h0, int pass) {
  rr::ChunkArgs a{};
  a.B = (int)B;
  a.u = static_cast<const uint16_t*>(vp);
  a.delta = static_cast<const uint16_t*>(gates);
  a.Bm = static_cast<const uint16_t*>(kp);
  a.Cm = static_cast<const uint16_t*>(qp);
  a.h0 = h0;
  a.L = (int)L; a.H = (int)H; a.DH = (int)Dh; a.NS = (int)Dh; a.nC = (int)(L / 32);
  a.mode = rr::gla2_mode(B, H, a.nC, Dh, pass);
  a.R = a.mode == 0 ? a.nC : 1;   // whole-head mode (0): one run of nC chunks
  return a;
}
}  // namespace

namespace {
rr::GlaDenseArgs gla_dense_args(const void* qp, const void* kp, const void* vp, const void* gates, int64_t B,
                                int64_t L, int64_t H, int64_t Dh, int64_t nC) {
  rr::GlaDenseArgs d{};
  d.q = qp;
  d.k = kp;
  d.v = vp;
  d.g = gates;
  d.B = (int)B; d.L = (int)L; d.H = (int)H; d.D = (int)Dh; d.nC = (int)nC;
  return d;
}
}  // namespace

extern "C" size_t rr_gla_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh,
                                         int64_t seg, int dtype, int pass) {
  if (B <= 0 || L <= 0 || H <= 0 || Dh <= 0 || rr::chunk_len(L, seg) == 0) return 0;
  if (rr::gla2_supported(dtype, B, L, H, seg, Dh, pass)) return rr::gla2_ws_bytes(B, H, L / 32, Dh, pass);
  const Plan q = make_plan(B, L, H, Dh, Dh, seg);
  return pass == 0 ? q.fwd_bytes : q.bwd_bytes;
}

extern "C" int rr_gla_fwd(const void* qp, const void* kp, const void* vp, const void* gates,
                          int dtype, int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg,
                          const float* h0, float* y, float* ckpt, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (int rc = check_dims("gla_fwd", B, L, H, Dh, Dh, seg, dtype, "Dh")) return rc;
  if (!qp || !kp || !vp || !gates || !y || !ckpt)
    return rr::fail(RR_EINVAL, "gla_fwd: null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (rr::gla2_supported(dtype, B, L, H, seg, Dh, 0)) {
    rr::ChunkArgs a = gla2_args(qp, kp, vp, gates, B, L, H, Dh, h0, 0);
    a.y = y;
    a.ckpt = ckpt;
    const size_t need = rr::gla2_ws_bytes(B, H, a.nC, Dh, 0);
    if (need && (!workspace || workspace_bytes < need))
      return rr::fail(RR_EWORKSPACE, "gla_fwd: workspace too small");
    rr::gla2_carve_ws(a, workspace, B, 0);
    return rr::gla2_fwd(a, B, s);
  }
  const Plan q = make_plan(B, L, H, Dh, Dh, seg);
  if (workspace_bytes < q.fwd_bytes || (q.fwd_bytes && !workspace))
    return rr::fail(RR_EWORKSPACE, "gla_fwd: workspace too small");
  if (rr::gla_dense_supported(q.T, Dh, B, H, q.nC)) {
    rr::GlaDenseArgs d = gla_dense_args(qp, kp, vp, gates, B, L, H, Dh, q.nC);
    char* ws = static_cast<char*>(workspace);
    d.h0 = h0;
    d.y = y;
    d.ckpt = ckpt;
    d.mapE = reinterpret_cast<float*>(ws + q.fwd_mapE);
    d.mapP = reinterpret_cast<float*>(ws + q.fwd_mapP);
    if (int rc = rr::gla_dense_launch(d, dtype, rr::kDenseMapsFwd, s)) return rc;
    if (int rc = rr::dense_compose(d.mapE, d.mapP, h0, ckpt, nullptr, B, H, Dh, Dh, q.nC, false, true, s)) return rc;
    return rr::gla_dense_launch(d, dtype, rr::kDenseOut, s);
  }
  RR_DISPATCH_DTYPE(dtype, {
    Args<InT> a{};
    a.lane_in = static_cast<const InT*>(vp);
    a.step = static_cast<const InT*>(gates);
    a.in_coef = static_cast<const InT*>(kp);
    a.out_coef = static_cast<const InT*>(qp);
    a.h0 = h0;
    a.y = q.NN > 1 ? static_cast<float*>(workspace) : y;
    a.ckpt = ckpt;
    a.L = (int)L; a.H = (int)H; a.DL = (int)Dh; a.NS = (int)Dh; a.T = (int)q.T;
    a.Bsz = (int)B;
    a.nC = (int)q.nC; a.ND = (int)q.ND; a.NN = (int)q.NN; a.rows = q.rows;
    return launch_fwd<InT, true>(a, q, B, workspace, s, y);
  });
  return RR_OK;
}

extern "C" int rr_gla_bwd(const float* dy, const float* dfinal, const void* qp, const void* kp,
                          const void* vp, const void* gates, int dtype, int64_t B, int64_t L,
                          int64_t H, int64_t Dh, int64_t seg, const float* h0, const float* ckpt,
                          void* dq, void* dk, void* dv, void* dgates, float* dh0, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (int rc = check_dims("gla_bwd", B, L, H, Dh, Dh, seg, dtype, "Dh")) return rc;
  if (!dy || !qp || !kp || !vp || !gates || !ckpt || !dq || !dk || !dv || !dgates)
    return rr::fail(RR_EINVAL, "gla_bwd: null pointer argument");
  if (rr::gla2_supported(dtype, B, L, H, seg, Dh, 1)) {
    rr::ChunkArgs a = gla2_args(qp, kp, vp, gates, B, L, H, Dh, h0, 1);
    a.ckpt = const_cast<float*>(ckpt);
    a.dy = dy;
    a.dfinal = dfinal;
    a.du = static_cast<uint16_t*>(dv);
    a.ddelta = static_cast<uint16_t*>(dgates);
    a.dB = static_cast<uint16_t*>(dk);
    a.dC = static_cast<uint16_t*>(dq);
    a.dh0 = dh0;
    const size_t need = rr::gla2_ws_bytes(B, H, a.nC, Dh, 1);
    if (need && (!workspace || workspace_bytes < need))
      return rr::fail(RR_EWORKSPACE, "gla_bwd: workspace too small");
    rr::gla2_carve_ws(a, workspace, B, 1);
    return rr::gla2_bwd(a, B, static_cast<hipStream_t>(stream));
  }
  const Plan q = make_plan(B, L, H, Dh, Dh, seg);
  if (workspace_bytes < q.bwd_bytes || !workspace)
    return rr::fail(RR_EWORKSPACE, "gla_bwd: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (rr::gla_dense_supported(q.T, Dh, B, H, q.nC)) {
    rr::GlaDenseArgs d = gla_dense_args(qp, kp, vp, gates, B, L, H, Dh, q.nC);
    float* lam = reinterpret_cast<float*>(ws + q.off_lam);
    d.h0 = h0;
    d.ckpt = ckpt;
    d.lamws = lam;
    d.dy = dy;
    d.dq = dq;
    d.dk = dk;
    d.dv = dv;
    d.dg = dgates;
    d.mapE = reinterpret_cast<float*>(ws + q.bwd_mapE);
    d.mapP = reinterpret_cast<float*>(ws + q.bwd_mapP);
    if (int rc = rr::gla_dense_launch(d, dtype, rr::kDenseMapsBwd, s)) return rc;
    if (int rc = rr::dense_compose(d.mapE, d.mapP, dfinal, lam, dh0, B, H, Dh, Dh, q.nC, true, true, s)) return rc;
    return rr::gla_dense_launch(d, dtype, rr::kDenseGrad, s);
  }
  RR_DISPATCH_DTYPE(dtype, {
    Args<InT> a{};
    a.lane_in = static_cast<const InT*>(vp);
    a.step = static_cast<const InT*>(gates);
    a.in_coef = static_cast<const InT*>(kp);
    a.out_coef = static_cast<const InT*>(qp);
    a.h0 = h0;
    a.dy = dy;
    a.dfinal = dfinal;
    a.ckpt = const_cast<float*>(ckpt);
    a.gu = static_cast<InT*>(dv);
    a.gu_part = reinterpret_cast<float*>(ws + q.off_gu);
    a.g3 = reinterpret_cast<float*>(ws + q.off_g3);
    a.lamws = reinterpret_cast<float*>(ws + q.off_lam);
    a.mapE = reinterpret_cast<float*>(ws + q.bwd_mapE);
    a.mapP = reinterpret_cast<float*>(ws + q.bwd_mapP);
    a.dh0 = dh0;
    a.L = (int)L; a.H = (int)H; a.DL = (int)Dh; a.NS = (int)Dh; a.T = (int)q.T;
    a.Bsz = (int)B;
    a.nC = (int)q.nC; a.ND = (int)q.ND; a.NN = (int)q.NN; a.rows = q.rows;
    FinArgs<InT> f{};
    f.g3 = a.g3;
    f.gu_part = a.gu_part;
    f.step = a.step;
    f.g_in = static_cast<InT*>(dk);
    f.g_out = static_cast<InT*>(dq);
    f.g_step = static_cast<InT*>(dgates);
    f.gu = static_cast<InT*>(dv);
    f.BL = B * L; f.H = (int)H; f.DL = (int)Dh; f.NS = (int)Dh; f.ND = (int)q.ND; f.NN = (int)q.NN;
    return launch_bwd<InT, true>(a, f, q, B, s, nullptr, 1);
  });
  return RR_OK;
}
